// Host side of the Q4_K linear() path: the C ABI declared in include/q4k.h.
//
// Mirrors the reference's Weight / Ops::linear surface
// (model/qwen35/qwen35.hpp:29-37, model/qwen35/forward.cpp:51-70): a weight
// owns its device bytes plus a four-slot kernel cache indexed by phase, and
// linear() picks the phase from the packed batch's per-query row counts.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>


#include "../../include/q4k.h"
#include "q4k_internal.h"

using namespace q4k;

int q4k_internal_fail(int code, const char* msg);

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

}  // namespace

// Shared with the GGUF reader (q4k_gguf.cpp): records the thread's last error.
int q4k_internal_fail(int code, const char* msg) {
  return fail(code, "%s", msg);
}

namespace {

int hip_fail(hipError_t e, const char* what) {
  return fail(Q4K_EHIP, "%s: %s", what, hipGetErrorString(e));
}

#define Q4K_TRY_HIP(expr, what)            \
  do {                                     \
    hipError_t e_ = (expr);                \
    if (e_ != hipSuccess)                  \
      return hip_fail(e_, what);           \
  } while (0)

enum KernelKind : int { kNone = 0, kGemv = 1, kGemvGated = 2, kGemm = 3 };

// One resolved slot of Weight::kernels[4] (qwen35.hpp:29-32): which kernel
// family serves the phase, and its name for introspection.
struct Kernel {
  KernelKind kind = kNone;
  std::string name;
};

// Per-device staging workspace for activations (fp16 copy + row scales).
// Outgrown buffers are retired, not freed: a HIP graph captured earlier may
// still name them.  Growth is bounded by the largest m * k staged.
struct Workspace {
  std::mutex mu;
  _Float16* x = nullptr;  // staged activations, then the sub-block sums
  size_t x_elems = 0;
  float* scale = nullptr;
  size_t scale_elems = 0;
  float* part = nullptr;  // split-K GEMV slice partials
  size_t part_elems = 0;
  int* counters = nullptr;  // split-K GEMV group counters (zero between launches)
  size_t counter_elems = 0;
  uint8_t* pack = nullptr;  // decode pack of x (m <= 8)
  size_t pack_bytes = 0;
  uint8_t* normed = nullptr;  // q4k_mlp's RMS-normalised x when the norm is not fused
  size_t normed_bytes = 0;
  std::vector<void*> retired;
  // Fixed-size buffers in the no-allocation scratch: never grown; a call
  // that needs more fails (ensure_buffer).
  bool fixed = false;
};

Workspace g_ws[64];

// Launch timing (q4k_profile_enable / q4k_profile_query).
struct Profiler {
  std::mutex mu;
  bool on = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> events[5];

  void clear() {
    for (auto& v : events) {
      for (auto& e : v) {
        (void)hipEventDestroy(e.first);
        (void)hipEventDestroy(e.second);
      }
      v.clear();
    }
  }
};

Profiler g_prof;

thread_local DispatchEvents t_dispatch_events;

// Attaches a pair of events to the kernel dispatch made in its scope when
// profiling is enabled (see dispatch_events()).
struct LaunchTimer {
  hipEvent_t start = nullptr, stop = nullptr;
  int family;
  LaunchTimer(hipStream_t, int fam) : family(fam) {
    std::lock_guard<std::mutex> lock(g_prof.mu);
    if (!g_prof.on)
      return;
    if (hipEventCreate(&start) != hipSuccess || hipEventCreate(&stop) != hipSuccess) {
      start = stop = nullptr;
      return;
    }
    dispatch_events() = DispatchEvents{start, stop};
  }
  ~LaunchTimer() {
    if (!start)
      return;
    dispatch_events() = DispatchEvents{};
    std::lock_guard<std::mutex> lock(g_prof.mu);
    g_prof.events[family].emplace_back(start, stop);
  }
};

}  // namespace

DispatchEvents& q4k::dispatch_events() {
  return t_dispatch_events;
}

struct q4k_weight {
  int device = 0;
  uint32_t n = 0, k = 0, type = 0;
  uint8_t* data = nullptr;
  size_t bytes = 0;
  Kernel kernels[4];
};

namespace {

size_t q4k_bytes(uint32_t n, uint32_t k) {
  return (size_t)n * (k / 256) * kBlockBytes;
}

size_t type_bytes(uint32_t n, uint32_t k, uint32_t type) {
  return (size_t)n * (k / 256) * (size_t)type_block_bytes(type);
}

const char* type_name(uint32_t type) {
  switch (type) {
    case Q4K_GGML_TYPE_Q6_K:
      return "q6_k";
    case Q4K_GGML_TYPE_Q8_0:
      return "q8_0";
    case Q4K_GGML_TYPE_Q5_K:
      return "q5_k";
    case Q4K_GGML_TYPE_IQ4_XS:
      return "iq4_xs";
    default:
      return "q4_k";
  }
}

int check_shape(uint32_t n, uint32_t k, uint32_t type, size_t bytes) {
  if (type_block_bytes(type) == 0)
    return fail(Q4K_ETYPE, "unsupported ggml type %u (Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14, IQ4_XS = 23)", type);
  if (n == 0 || k == 0 || k % 256 != 0)
    return fail(Q4K_ESHAPE, "k must be a positive multiple of 256 (got k=%u, n=%u)", k, n);
  if (n % 16 != 0)
    return fail(Q4K_ESHAPE, "n must be a multiple of 16 (got %u)", n);
  if ((size_t)(k / 256) * kQ6TileBlockBytes > 0x7fffffffull / 16)
    return fail(Q4K_ESHAPE, "k too large (%u)", k);
  if (bytes != type_bytes(n, k, type))
    return fail(Q4K_ESHAPE, "byte count %zu does not match n=%u k=%u (expected %zu)", bytes, n, k, type_bytes(n, k, type));
  return Q4K_OK;
}

inline uint32_t swap_middle_bytes(uint32_t v) {
  return (v & 0xff0000ffu) | ((v & 0x0000ff00u) << 8) | ((v & 0x00ff0000u) >> 8);
}

// Host form of the tiled layout (q4k_internal.h); `forward` selects
// GGUF -> tiled, else tiled -> GGUF.  Both directions are a byte permutation.
void relayout(const uint8_t* src, uint8_t* dst, uint32_t n, uint32_t k, bool forward) {
  const uint32_t nb = k / 256;
  for (uint32_t c = 0; c < n / 16; ++c)
    for (uint32_t b = 0; b < nb; ++b) {
      const size_t tb = ((size_t)c * nb + b) * kTileBlockBytes;
      for (uint32_t i = 0; i < 16; ++i) {
        const size_t blk = ((size_t)(16 * c + i) * nb + b) * kBlockBytes;
        for (uint32_t j = 0; j < 16; ++j) {
          if (forward)
            dst[tb + kHeaderOffset + 16 * i + j] = src[blk + j];
          else
            dst[blk + j] = src[tb + kHeaderOffset + 16 * i + j];
        }
        for (uint32_t g = 0; g < 4; ++g)
          for (uint32_t h = 0; h < 2; ++h)
            for (uint32_t w = 0; w < 4; ++w) {
              const size_t qoff = blk + 16 + 32 * g + 16 * h + 4 * w;
              const size_t toff = tb + h * kSlabBytes + 16 * (16 * g + i) + 4 * w;
              uint32_t v;
              if (forward) {
                std::memcpy(&v, src + qoff, 4);
                v = swap_middle_bytes(v);
                std::memcpy(dst + toff, &v, 4);
              } else {
                std::memcpy(&v, src + toff, 4);
                v = swap_middle_bytes(v);
                std::memcpy(dst + qoff, &v, 4);
              }
            }
      }
    }
}

// Host form of the tiled layouts of the types other than Q4_K (encode_lane,
// q4k_internal.h): GGUF -> tiled.
void relayout_encode(const uint8_t* src, uint8_t* dst, uint32_t n, uint32_t k, uint32_t type) {
  const uint32_t nb = k / 256;
  const size_t bb = (size_t)type_block_bytes(type);
  for (uint32_t c = 0; c < n / 16; ++c)
    for (uint32_t b = 0; b < nb; ++b) {
      uint8_t* tb = dst + ((size_t)c * nb + b) * 16 * bb;
      for (int l = 0; l < 64; ++l)
        encode_lane(type, src + ((size_t)(16 * c + (l & 15)) * nb + b) * bb, tb, l);
    }
}

// Tiled -> GGUF for Q6_K (the layout tooling's inverse; dst zeroed first).
void relayout_q6_inverse(const uint8_t* src, uint8_t* dst, uint32_t n, uint32_t k) {
  const uint32_t nb = k / 256;
  for (uint32_t c = 0; c < n / 16; ++c)
    for (uint32_t b = 0; b < nb; ++b) {
      const size_t tb = ((size_t)c * nb + b) * kQ6TileBlockBytes;
      for (uint32_t l = 0; l < 64; ++l) {
        const uint32_t i = l & 15, g = l >> 4;
        uint8_t* out = dst + ((size_t)(16 * c + i) * nb + b) * kQ6BlockBytes;
        uint32_t wd[12] = {0};
        for (int s2 = 0; s2 < 3; ++s2)
          std::memcpy(wd + 4 * s2, src + tb + s2 * 1024 + 16 * l, 16);
        for (int o = 0; o < 32; ++o)
          for (int hf = 0; hf < 2; ++hf) {
            // Inverse of q6_quant's addressing for element e.
            const int e = q6_elem((int)g, o, hf), h = e >> 7, rr = e & 127, ll = rr & 31;
            const uint32_t v = q6_take(wd, o, hf);
            uint8_t& qb = out[64 * h + (rr & 32) + ll];
            qb = (rr & 64) ? (uint8_t)((qb & 0x0Fu) | ((v & 15u) << 4)) : (uint8_t)((qb & 0xF0u) | (v & 15u));
            uint8_t& hb = out[128 + 32 * h + ll];
            const int sh = 2 * (rr >> 5);
            hb = (uint8_t)((hb & ~(3u << sh)) | ((v >> 4) << sh));
          }
        for (int j = 0; j < 4; ++j)
          out[192 + 4 * g + j] = (uint8_t)(src[tb + kQ6ScaleOffset + 4 * l + j] ^ 0x80u);
        if (g == 0)
          std::memcpy(out + 208, src + tb + kQ6DOffset + 2 * i, 2);
      }
    }
}

// forward.cpp:52 with the decode flag accumulated as in forward.cpp:190.
uint32_t phase_of(const uint32_t* counts, uint32_t nq, uint32_t m, bool gated) {
  bool decode = true;
  if (counts) {
    for (uint32_t i = 0; i < nq; ++i)
      decode = decode && counts[i] <= Q4K_MAX_DECODE_ROWS;
  } else {
    decode = m <= Q4K_MAX_DECODE_ROWS;
  }
  return decode ? (gated ? Q4K_PHASE_GATED_DECODE : Q4K_PHASE_DECODE) : (m <= 8 ? Q4K_PHASE_PREFILL_SMALL : Q4K_PHASE_PREFILL);
}

int check_counts(const uint32_t* counts, uint32_t nq, uint32_t m) {
  if (!counts)
    return nq == 0 ? Q4K_OK : fail(Q4K_EINVAL, "query_counts is NULL but nqueries=%u", nq);
  if (nq == 0 || nq > Q4K_MAX_QUERIES)
    return fail(Q4K_EINVAL, "nqueries must be in [1, %u] (got %u)", Q4K_MAX_QUERIES, nq);
  uint64_t sum = 0;
  for (uint32_t i = 0; i < nq; ++i)
    sum += counts[i];
  if (sum != m)
    return fail(Q4K_EINVAL, "query counts sum to %llu but m=%u", (unsigned long long)sum, m);
  return Q4K_OK;
}

// Q4_K prefill with fewer output columns than this runs the GEMV per 8-row
// group (hi/lo activations, weights exact) instead of the GEMM, whose fp16
// activations and weights leave a per-row error near the 1e-3 bar when a row
// has few outputs to average over.  Batches of up to 24 rows keep the staged
// hi/lo GEMV.
constexpr uint32_t kGemmMinColumns = 256;
constexpr uint32_t kGemvSplitRows = 24;
// Longest row the staged Q4_K GEMV takes at up to 8 rows; longer rows go to
// the decode pack and the per-type GEMV.
constexpr uint32_t kStagedGemvMaxK = 12288;

// The kernel family each phase resolves to.  Decode-shaped phases (0, 2, 3)
// run the MFMA GEMV; prefill (1) runs the LDS-tiled MFMA GEMM, whose slot also
// serves prefill batches small enough for the GEMV (<= 48 rows) with the GEMV
// launch shape (run_linear) -- same arithmetic, lower latency.
Kernel& resolve(q4k_weight* w, uint32_t phase) {
  Kernel& k = w->kernels[phase];
  if (k.kind == kNone) {
    const char* suffix[] = {"decode", "prefill", "prefill_small", "gate_up_decode"};
    k.kind = phase == Q4K_PHASE_GATED_DECODE ? kGemvGated : phase == Q4K_PHASE_PREFILL ? kGemm : kGemv;
    const bool other = w->type != Q4K_GGML_TYPE_Q4_K;
    if (other && k.kind == kGemm)
      k.kind = kGemv;  // prefill of the other types: GEMV per 8-row group below 64 rows, the typed MFMA GEMM from 64
    if (k.kind == kGemm && w->n < kGemmMinColumns)
      k.kind = kGemv;  // narrow Q4_K outputs: the GEMV per 8-row group at every row count
    k.name = std::string(phase == Q4K_PHASE_GATED_DECODE ? "mlp_" : "linear_") + type_name(w->type) + "_k" + std::to_string(w->k) + "_n" +
             std::to_string(w->n) + "_" + suffix[phase] +
             "_mfma16x16x32";
  }
  return k;
}

Workspace& workspace(int device) {
  return g_ws[device & 63];
}

// Device allocation for workspace growth.  hipMalloc is not allowed while a
// stream captures a graph, and a failure there would look like a lack of
// memory: a call on a capturing stream that needs more workspace than the
// device already holds fails with Q4K_ECAPTURE instead, before allocating.
// Device allocations made for workspaces since the library was loaded
// (q4k_workspace_allocations).
std::atomic<uint64_t> g_ws_allocations{0};

int ws_alloc(hipStream_t stream, int device, void** p, size_t bytes, const char* what) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone)
    return fail(Q4K_ECAPTURE,
                "the %s must grow to %zu bytes on device %d, but the stream is capturing a graph and allocation is not allowed "
                "there: make one call of this shape (or a larger one) before the capture",
                what, bytes, device);
  if (hipMalloc(p, bytes) != hipSuccess) {
    *p = nullptr;
    return fail(Q4K_ENOMEM, "cannot allocate %zu-byte %s on device %d", bytes, what, device);
  }
  g_ws_allocations.fetch_add(1, std::memory_order_relaxed);
  return Q4K_OK;
}

// Grow-only device buffer (outgrown buffers are retired, not freed: a graph
// captured earlier may still name them).
template <typename T>
int ensure_buffer(hipStream_t stream, Workspace& ws, int device, T*& buf, size_t& have, size_t need, const char* what) {
  if (have >= need)
    return Q4K_OK;
  if (ws.fixed)
    return fail(Q4K_ESHAPE, "this call needs %zu bytes of %s; the no-allocation scratch of device %d holds %zu (q4k_linear_noalloc)",
                need * sizeof(T), what, device, have * sizeof(T));
  void* p = nullptr;
  int rc = ws_alloc(stream, device, &p, need * sizeof(T), what);
  if (rc)
    return rc;
  if (buf)
    ws.retired.push_back(buf);
  buf = static_cast<T*>(p);
  have = need;
  return Q4K_OK;
}

// Grows the device's staging buffers to `halves` fp16 values plus `rows` row scales.
int ensure_workspace(hipStream_t stream, Workspace& ws, int device, size_t halves, size_t rows) {
  int rc = ensure_buffer(stream, ws, device, ws.x, ws.x_elems, halves, "activation workspace");
  if (!rc)
    rc = ensure_buffer(stream, ws, device, ws.scale, ws.scale_elems, rows < 64 ? 64 : rows, "row-scale workspace");
  return rc;
}

// Split-K buffers.  New counters are zeroed once (synchronously, outside any
// capture: growth is refused there); every launch leaves them zero again.
int ensure_splitk_workspace(hipStream_t stream, Workspace& ws, int device, size_t part_floats, size_t groups) {
  int rc = ensure_buffer(stream, ws, device, ws.part, ws.part_elems, part_floats, "split-K workspace");
  if (rc || ws.counter_elems >= groups)
    return rc;
  if (ws.fixed)
    return fail(Q4K_ESHAPE, "this call needs %zu split-K counters; the no-allocation scratch of device %d holds %zu", groups, device,
                ws.counter_elems);
  const size_t n = groups < 1024 ? 1024 : groups;
  int* c = nullptr;
  rc = ws_alloc(stream, device, reinterpret_cast<void**>(&c), n * sizeof(int), "split-K counter array");
  if (rc)
    return rc;
  hipError_t e = hipMemset(c, 0, n * sizeof(int));
  if (e != hipSuccess) {
    (void)hipFree(c);
    return hip_fail(e, "hipMemset");
  }
  if (ws.counters)
    ws.retired.push_back(ws.counters);
  ws.counters = c;
  ws.counter_elems = n;
  return Q4K_OK;
}

// The pipelined GEMM of a shape with fewer tiles than CUs runs two
// K-segments per tile (gemm2_split_b): their accumulators and arrival
// counters live in the split-K workspace.
int device_cus(int device);

int gemm2_split_buffers(hipStream_t stream, Workspace& ws, int device, GemmArgs& a, bool gated) {
  if (!gemm2_split_b(a.m, a.n, a.nb, device_cus(device)))
    return Q4K_OK;
  size_t part_floats = 0, counters = 0;
  gemm2_split_workspace(a.m, a.n, gated, &part_floats, &counters);
  int rc = ensure_splitk_workspace(stream, ws, device, part_floats, counters);
  if (rc)
    return rc;
  if (ws.fixed)  // the scratch's counters start at zero for this launch (a fill kernel: capture-safe)
    Q4K_TRY_HIP(launch_fill_u32(stream, reinterpret_cast<uint32_t*>(ws.counters), 0u, (uint32_t)counters), "counter fill launch");
  a.part = ws.part;
  a.counters = ws.counters;
  return Q4K_OK;
}

// Packs x (m <= 8 rows) for the per-item and persistent GEMVs.
int stage_pack(hipStream_t stream, Workspace& ws, int device, const void* x, uint32_t dtype, uint32_t m, uint32_t k, DecodePack* pk) {
  const size_t nb = k / 256;
  int rc = ensure_buffer(stream, ws, device, ws.pack, ws.pack_bytes, nb * kPackBytesPerBlock, "decode pack");
  if (rc)
    return rc;
  pk->frag = reinterpret_cast<u4_t*>(ws.pack);
  pk->xs = reinterpret_cast<h4_t*>(ws.pack + nb * 8 * 64 * 16);
  pk->dsc = reinterpret_cast<float*>(ws.pack + nb * (8 * 64 * 16 + 64 * 8));
  LaunchTimer timer(stream, Q4K_KERNEL_STAGE);
  Q4K_TRY_HIP(launch_stage_pack(stream, x, (int)dtype, *pk, (int)m, (int)k), "stage_pack launch");
  return Q4K_OK;
}

// LM-head rows of a packed batch (native_ops.metal:12-15 with batch.hpp:25-29
// queryLogit): output row r reads input row start + count - samples +
// (r - logit) of the first query with samples whose logit range holds r.
// *rows receives the batch's total row count.
int logit_rows(const uint32_t* counts, const uint32_t* samples, uint32_t nqueries, GatherIndex* idx, uint32_t* rows) {
  uint32_t start[Q4K_MAX_QUERIES], logit[Q4K_MAX_QUERIES], nlogit = 0;
  int rc = q4k_pack_queries(counts, samples, nqueries, start, logit, rows, &nlogit);
  if (rc)
    return rc;
  if (nlogit > Q4K_MAX_LOGIT_ROWS)
    return fail(Q4K_EINVAL, "%u sampled rows exceed %u", nlogit, Q4K_MAX_LOGIT_ROWS);
  idx->rows = nlogit;
  for (uint32_t r = 0; r < nlogit; ++r) {
    uint32_t q = 0;
    while (!samples[q] || r >= logit[q] + samples[q])
      ++q;
    idx->src[r] = start[q] + counts[q] - samples[q] + (r - logit[q]);
  }
  return Q4K_OK;
}

bool overlaps(const void* a, size_t abytes, const void* b, size_t bbytes) {
  const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
  return a0 < b0 + bbytes && b0 < a0 + abytes;
}

// Compute units of each device (persistent-grid sizing), cached.
int device_cus(int device) {
  static int cus[64] = {0};
  int& c = cus[device & 63];
  if (c == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || v <= 0)
      v = 256;
    c = v;
  }
  return c;
}

int set_device(int device) {
  int cur = -1;
  Q4K_TRY_HIP(hipGetDevice(&cur), "hipGetDevice");
  if (cur != device)
    Q4K_TRY_HIP(hipSetDevice(device), "hipSetDevice");
  return Q4K_OK;
}

// One projection (phase already chosen) on the weight's device, with the
// device's workspace lock held.  restage == false reuses the staged x of the
// previous call, which must have been a projection of the same x with the
// same (m, k, n) under the same lock; the decode pack and split-K paths always
// stage (they are not reached by such pairs).
// Projection with weights of a type other than Q4_K (wu == nullptr): up to 63
// rows the GEMV per 8-row group (run_gemv_groups_locked); from 64 rows the
// GEMM below.
constexpr uint32_t kTypedGemmRows = 64;
// Prefill-sized batches with the other types (m >= 64): x staged in the GEMM
// order (fp16, power-of-two row scales, the attn/ffn norm folded in; only the
// m live rows are stored: the padded rows up to the 128-row tile keep whatever
// the workspace held, which no stored output reads, since each MFMA output row
// depends on its own A row only), then the type's MFMA GEMM, which dequantises the
// weights to the reference's prefill tile values in registers and applies the
// epilogue (row unscale, post 0/1/2, fp16 rounding) in place.
int run_typed_gemm_locked(hipStream_t stream, Workspace& ws, q4k_weight* w, const void* x, void* y, const void* aux, uint32_t m, uint32_t post,
                          uint32_t dtype, const float* norm_w, float eps) {
  const size_t rows = (size_t)gemm2_rows((int)m);
  int rc = ensure_workspace(stream, ws, w->device, rows * w->k, rows);
  if (rc)
    return rc;
  {
    LaunchTimer timer(stream, Q4K_KERNEL_STAGE);
    Q4K_TRY_HIP(launch_stage_x(stream, x, (int)dtype, ws.x, nullptr, ws.scale, (int)m, (int)w->k, kStageGemm, norm_w, eps), "stage_x launch");
  }
  GemmArgs a;
  a.w = w->data;
  a.xh = ws.x;
  a.rowscale = ws.scale;
  a.y = y;
  a.aux = aux;
  a.m = (int)m;
  a.n = (int)w->n;
  a.k = (int)w->k;
  a.nb = (int)(w->k / 256);
  a.post = (int)post;
  LaunchTimer timer(stream, Q4K_KERNEL_GEMM);
  Q4K_TRY_HIP(launch_typed_gemm(stream, a, w->type, (int)dtype, device_cus(w->device)), "typed gemm launch");
  return Q4K_OK;
}

// A path that packs x itself (split-K, decode pack) cannot fold a row's RMS
// norm into its staging: with a norm weight, x is normalised into the
// workspace first (one rms_norm launch, native_ops.metal:6-40) and the path
// reads that copy.
int prenorm(hipStream_t stream, Workspace& ws, int device, const void*& x, const float*& norm_w, float eps, uint32_t m, uint32_t k,
            uint32_t dtype) {
  if (!norm_w)
    return Q4K_OK;
  const size_t es = dtype == Q4K_DTYPE_F32 ? 4 : 2;
  int rc = ensure_buffer(stream, ws, device, ws.normed, ws.normed_bytes, (size_t)m * k * es, "normalised-activation buffer");
  if (rc)
    return rc;
  LaunchTimer timer(stream, Q4K_KERNEL_AUX);
  Q4K_TRY_HIP(launch_rms_norm(stream, x, norm_w, ws.normed, (int)m, (int)k, eps, (int)dtype, nullptr), "rms_norm launch");
  x = ws.normed;
  norm_w = nullptr;
  return Q4K_OK;
}

// Per group of up to 8 rows: the decode pack of the group's x (hi/lo fp16,
// per-(row, block) power-of-two scale), then the weight type's GEMV over the
// group's rows of y and aux.
int run_gemv_groups_locked(hipStream_t stream, Workspace& ws, q4k_weight* w, const void* x, void* y, const void* aux, uint32_t m, uint32_t post,
                           uint32_t dtype) {
  const size_t es = dtype == Q4K_DTYPE_F32 ? 4 : 2;
  for (uint32_t r0 = 0; r0 < m; r0 += 8) {
    const uint32_t mg = m - r0 < 8u ? m - r0 : 8u;
    const void* xg = static_cast<const uint8_t*>(x) + (size_t)r0 * w->k * es;
    GemvArgs a{};
    int rc = stage_pack(stream, ws, w->device, xg, dtype, mg, w->k, &a.pack);
    if (rc)
      return rc;
    a.w = w->data;
    a.x = xg;
    a.y = static_cast<uint8_t*>(y) + (size_t)r0 * w->n * es;
    a.aux = aux ? static_cast<const uint8_t*>(aux) + (size_t)r0 * w->n * es : nullptr;
    a.m = (int)mg;
    a.n = (int)w->n;
    a.k = (int)w->k;
    a.nb = (int)(w->k / 256);
    a.post = (int)post;
    a.rows = 2 * (int)mg;
    a.split = 1;
    LaunchTimer timer(stream, Q4K_KERNEL_GEMV);
    Q4K_TRY_HIP(launch_typed_gemv(stream, a, w->type, (int)dtype, device_cus(w->device)), "typed gemv launch");
  }
  return Q4K_OK;
}

// Outputs narrower than kGemmMinColumns take the GEMV groups at every row
// count, as with Q4_K (the per-row bar).
int run_typed_locked(hipStream_t stream, Workspace& ws, q4k_weight* w, const void* x, void* y, const void* aux, uint32_t m, uint32_t post,
                     uint32_t dtype, const float* norm_w, float eps) {
  if (m >= kTypedGemmRows && w->n >= kGemmMinColumns)
    return run_typed_gemm_locked(stream, ws, w, x, y, aux, m, post, dtype, norm_w, eps);
  int rc = prenorm(stream, ws, w->device, x, norm_w, eps, m, w->k, dtype);
  if (rc)
    return rc;
  return run_gemv_groups_locked(stream, ws, w, x, y, aux, m, post, dtype);
}

// norm_w != nullptr: the projection of rms_norm(x, norm_w) (forward.cpp:82,
// 114), folded into the activation staging where the path stages x.
int run_linear_locked(hipStream_t stream, Workspace& ws, q4k_weight* w, q4k_weight* wu, const void* x, void* y, const void* aux, uint32_t m,
                      uint32_t post, uint32_t dtype, uint32_t phase, bool restage, const float* norm_w = nullptr, float eps = 0.0f) {
  if (w->type != Q4K_GGML_TYPE_Q4_K) {
    if (wu)
      return fail(Q4K_ETYPE, "the fused gate/up kernel takes Q4_K weights");
    resolve(w, phase);
    return run_typed_locked(stream, ws, w, x, y, aux, m, post, dtype, norm_w, eps);
  }
  Kernel& kern = resolve(w, phase);
  if (wu)
    resolve(wu, phase);
  if (!wu && w->n < kGemmMinColumns && m > kGemvSplitRows) {
    int rc = prenorm(stream, ws, w->device, x, norm_w, eps, m, w->k, dtype);
    if (rc)
      return rc;
    return run_gemv_groups_locked(stream, ws, w, x, y, aux, m, post, dtype);
  }
  const bool gemv = kern.kind != kGemm || m <= 16u * kGemvMaxRowTiles;
  const bool split = gemv && gemv_split((int)m);
  const int rows = split ? 2 * (int)m : (int)m;
  SplitkPlan plan;
  if (gemv && gemv_splitk_plan((int)m, (int)w->n, (int)(w->k / 256), wu != nullptr, device_cus(w->device), &plan)) {
    // Split-K GEMV: each workgroup packs its own K-slice of x; partials in
    // the workspace.
    int rc = prenorm(stream, ws, w->device, x, norm_w, eps, m, w->k, dtype);
    if (!rc)
      rc = ensure_splitk_workspace(stream, ws, w->device, gemv_splitk_part_floats(plan), (size_t)plan.groups);
    if (rc)
      return rc;
    if (ws.fixed)  // the scratch's counters start at zero for this launch (a fill kernel: capture-safe)
      Q4K_TRY_HIP(launch_fill_u32(stream, reinterpret_cast<uint32_t*>(ws.counters), 0u, (uint32_t)plan.groups), "counter fill launch");
    GemvArgs a{};
    a.w = w->data;
    a.wu = wu ? wu->data : w->data;
    a.x = x;
    a.y = y;
    a.aux = aux;
    a.m = (int)m;
    a.n = (int)w->n;
    a.k = (int)w->k;
    a.nb = (int)(w->k / 256);
    a.post = (int)post;
    a.rows = 2 * (int)m;
    a.split = 1;
    LaunchTimer timer(stream, wu ? Q4K_KERNEL_GEMV_GATED : Q4K_KERNEL_GEMV);
    Q4K_TRY_HIP(launch_gemv_splitk(stream, a, (int)dtype, plan, ws.part, ws.counters), "gemv split-K launch");
    return Q4K_OK;
  }
  if (gemv && !wu && m <= 8 && w->k > kStagedGemvMaxK) {
    // Long rows with no split-K plan (K = 32768): the fragment staging
    // reduces each row in one workgroup, so the decode pack (parallel over
    // blocks) and the per-type GEMV take them (32 us for 8 rows x 32768 ->
    // 4096, against 41 us staged).
    int rc = prenorm(stream, ws, w->device, x, norm_w, eps, m, w->k, dtype);
    if (rc)
      return rc;
    return run_gemv_groups_locked(stream, ws, w, x, y, aux, m, post, dtype);
  }
  if (gemv && wu && gemv_gate_up_supported((int)m, (int)(w->k / 256), (int)w->n)) {
    // Fused gate/up GEMV: packs x in registers, no staging launch.
    GemvArgs a{};
    a.w = w->data;
    a.wu = wu->data;
    a.x = x;
    a.y = y;
    a.m = (int)m;
    a.n = (int)w->n;
    a.k = (int)w->k;
    a.nb = (int)(w->k / 256);
    a.rows = 2 * (int)m;
    a.split = 1;
    a.norm_w = norm_w;
    a.eps = eps;
    LaunchTimer timer(stream, Q4K_KERNEL_GEMV_GATED);
    Q4K_TRY_HIP(launch_gemv_gate_up(stream, a, (int)dtype, device_cus(w->device)), "gemv gate/up launch");
    return Q4K_OK;
  }
  if (gemv && !wu && q4k_persistent_supported((int)m, (int)(w->k / 256), (int)w->n, device_cus(w->device))) {
    // Wide plain projections (the LM head): the persistent GEMV, x fragments
    // resident in registers.
    GemvArgs a{};
    int rc = prenorm(stream, ws, w->device, x, norm_w, eps, m, w->k, dtype);
    if (!rc)
      rc = stage_pack(stream, ws, w->device, x, dtype, m, w->k, &a.pack);
    if (rc)
      return rc;
    a.w = w->data;
    a.x = x;
    a.y = y;
    a.aux = aux;
    a.m = (int)m;
    a.n = (int)w->n;
    a.k = (int)w->k;
    a.nb = (int)(w->k / 256);
    a.post = (int)post;
    a.rows = 2 * (int)m;
    a.split = 1;
    LaunchTimer timer(stream, Q4K_KERNEL_GEMV);
    Q4K_TRY_HIP(launch_q4k_persistent(stream, a, (int)dtype, device_cus(w->device)), "gemv persistent launch");
    return Q4K_OK;
  }
  const size_t ws_rows = gemv ? (size_t)((rows + 15) / 16) * 16 : (size_t)gemm2_rows((int)m);
  // xs (and, for single fp16 fragments, the residual plane after it) is
  // read 32 lanes at a time from its start; +128 halves of slack.
  const size_t xs_halves = gemv ? 2 * gemv_xs_halves(rows, (int)w->k) + 128 : 0;
  int rc = ensure_workspace(stream, ws, w->device, ws_rows * w->k + xs_halves, ws_rows);
  if (rc)
    return rc;
  _Float16* xs = ws.x + ws_rows * w->k;
  if (restage) {
    LaunchTimer timer(stream, Q4K_KERNEL_STAGE);
    const int mode = !gemv ? kStageGemm : split ? kStageFragSplit : kStageFrag;
    Q4K_TRY_HIP(launch_stage_x(stream, x, (int)dtype, ws.x, xs, ws.scale, (int)m, (int)w->k, mode, norm_w, eps), "stage_x launch");
  }
  if (gemv) {
    const RowsPlan rows_plan = gemv_rows_plan(rows, (int)(w->k / 256), (int)w->n, wu != nullptr, device_cus(w->device));
    if (rows_plan.slices > 1) {
      const size_t groups = (size_t)(w->n / (16 * rows_plan.tiles));
      rc = ensure_splitk_workspace(stream, ws, w->device, gemv_rows_part_floats(rows_plan, (int)w->n), groups);
      if (rc)
        return rc;
      if (ws.fixed)  // the scratch's counters start at zero for this launch (a fill kernel: capture-safe)
        Q4K_TRY_HIP(launch_fill_u32(stream, reinterpret_cast<uint32_t*>(ws.counters), 0u, (uint32_t)groups), "counter fill launch");
    }
    GemvArgs a;
    a.w = w->data;
    a.wu = wu ? wu->data : w->data;
    a.xf = ws.x;
    a.xs = xs;
    a.rowscale = ws.scale;
    a.y = y;
    a.aux = aux;
    a.m = (int)m;
    a.n = (int)w->n;
    a.k = (int)w->k;
    a.nb = (int)(w->k / 256);
    a.post = (int)post;
    a.rows = rows;
    a.split = split ? 1 : 0;
    if (rows_plan.slices > 1) {
      a.part = ws.part;
      a.counters = ws.counters;
    }
    LaunchTimer timer(stream, wu ? Q4K_KERNEL_GEMV_GATED : Q4K_KERNEL_GEMV);
    if (rows_plan.tiles > 0)
      Q4K_TRY_HIP(launch_gemv_rows(stream, a, (int)dtype, rows_plan, wu != nullptr), "gemv rows launch");
    else
      Q4K_TRY_HIP(launch_gemv(stream, a, (int)dtype, gemv_shape(rows, (int)w->n, a.nb, wu != nullptr, device_cus(w->device)), wu != nullptr),
                  "gemv launch");
  } else {
    GemmArgs a;
    a.w = w->data;
    a.xh = ws.x;
    a.rowscale = ws.scale;
    a.y = y;
    a.aux = aux;
    a.m = (int)m;
    a.n = (int)w->n;
    a.k = (int)w->k;
    a.nb = (int)(w->k / 256);
    a.post = (int)post;
    rc = gemm2_split_buffers(stream, ws, w->device, a, false);
    if (rc)
      return rc;
    LaunchTimer timer(stream, Q4K_KERNEL_GEMM);
    Q4K_TRY_HIP(launch_gemm2(stream, a, (int)dtype, device_cus(w->device)), "gemm launch");
  }
  return Q4K_OK;
}

int run_linear(hipStream_t stream, q4k_weight* w, q4k_weight* wu, const void* x, void* y, const void* aux, uint32_t m, uint32_t post, uint32_t dtype,
               uint32_t phase, const float* norm_w = nullptr, float eps = 0.0f) {
  Workspace& ws = workspace(w->device);
  std::lock_guard<std::mutex> lock(ws.mu);
  return run_linear_locked(stream, ws, w, wu, x, y, aux, m, post, dtype, phase, true, norm_w, eps);
}

}  // namespace

extern "C" {

const char* q4k_last_error(void) {
  return g_error.c_str();
}

int q4k_relayout_host(const void* gguf_bytes, void* tiled, uint32_t n, uint32_t k) {
  if (!gguf_bytes || !tiled)
    return fail(Q4K_EINVAL, "null buffer");
  int rc = check_shape(n, k, Q4K_GGML_TYPE_Q4_K, q4k_bytes(n, k));
  if (rc)
    return rc;
  relayout(static_cast<const uint8_t*>(gguf_bytes), static_cast<uint8_t*>(tiled), n, k, true);
  return Q4K_OK;
}

int q4k_unrelayout_host(const void* tiled, void* gguf_bytes, uint32_t n, uint32_t k) {
  if (!gguf_bytes || !tiled)
    return fail(Q4K_EINVAL, "null buffer");
  int rc = check_shape(n, k, Q4K_GGML_TYPE_Q4_K, q4k_bytes(n, k));
  if (rc)
    return rc;
  relayout(static_cast<const uint8_t*>(tiled), static_cast<uint8_t*>(gguf_bytes), n, k, false);
  return Q4K_OK;
}

int q4k_relayout_host_typed(const void* gguf_bytes, void* tiled, uint32_t n, uint32_t k, uint32_t ggml_type) {
  if (!gguf_bytes || !tiled)
    return fail(Q4K_EINVAL, "null buffer");
  int rc = check_shape(n, k, ggml_type, type_bytes(n, k, ggml_type));
  if (rc)
    return rc;
  if (ggml_type == Q4K_GGML_TYPE_Q4_K)
    relayout(static_cast<const uint8_t*>(gguf_bytes), static_cast<uint8_t*>(tiled), n, k, true);
  else
    relayout_encode(static_cast<const uint8_t*>(gguf_bytes), static_cast<uint8_t*>(tiled), n, k, ggml_type);
  return Q4K_OK;
}

int q4k_unrelayout_host_typed(const void* tiled, void* gguf_bytes, uint32_t n, uint32_t k, uint32_t ggml_type) {
  if (!gguf_bytes || !tiled)
    return fail(Q4K_EINVAL, "null buffer");
  int rc = check_shape(n, k, ggml_type, type_bytes(n, k, ggml_type));
  if (rc)
    return rc;
  if (ggml_type == Q4K_GGML_TYPE_Q4_K) {
    relayout(static_cast<const uint8_t*>(tiled), static_cast<uint8_t*>(gguf_bytes), n, k, false);
  } else if (ggml_type == Q4K_GGML_TYPE_Q6_K) {
    std::memset(gguf_bytes, 0, type_bytes(n, k, ggml_type));  // the inverse merges bit fields into place
    relayout_q6_inverse(static_cast<const uint8_t*>(tiled), static_cast<uint8_t*>(gguf_bytes), n, k);
  } else {
    return fail(Q4K_ETYPE, "the inverse re-layout covers Q4_K and Q6_K (got type %u)", ggml_type);
  }
  return Q4K_OK;
}

int q4k_weight_create(const void* gguf_bytes, size_t bytes, uint32_t n, uint32_t k, uint32_t ggml_type, int device, q4k_weight** out) {
  if (!out)
    return fail(Q4K_EINVAL, "out is NULL");
  *out = nullptr;
  if (!gguf_bytes)
    return fail(Q4K_EINVAL, "gguf_bytes is NULL");
  int rc = check_shape(n, k, ggml_type, bytes);
  if (rc)
    return rc;
  if (device < 0 || device > 63)
    return fail(Q4K_EINVAL, "bad device %d", device);
  rc = set_device(device);
  if (rc)
    return rc;
  std::vector<uint8_t> tiled(bytes);
  if (ggml_type == Q4K_GGML_TYPE_Q4_K)
    relayout(static_cast<const uint8_t*>(gguf_bytes), tiled.data(), n, k, true);
  else
    relayout_encode(static_cast<const uint8_t*>(gguf_bytes), tiled.data(), n, k, ggml_type);
  q4k_weight* w = new (std::nothrow) q4k_weight;
  if (!w)
    return fail(Q4K_ENOMEM, "host allocation failed");
  w->device = device;
  w->n = n;
  w->k = k;
  w->type = ggml_type;
  w->bytes = bytes;
  if (hipMalloc(&w->data, bytes) != hipSuccess) {
    delete w;
    return fail(Q4K_ENOMEM, "cannot allocate %zu bytes of weights on device %d", bytes, device);
  }
  hipError_t e = hipMemcpy(w->data, tiled.data(), bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(w->data);
    delete w;
    return hip_fail(e, "weight upload");
  }
  *out = w;
  return Q4K_OK;
}

int q4k_weight_create_from_device(const void* gguf_device_bytes, size_t bytes, uint32_t n, uint32_t k, uint32_t ggml_type, int device,
                                  void* stream, q4k_weight** out) {
  if (!out)
    return fail(Q4K_EINVAL, "out is NULL");
  *out = nullptr;
  if (!gguf_device_bytes)
    return fail(Q4K_EINVAL, "gguf_device_bytes is NULL");
  int rc = check_shape(n, k, ggml_type, bytes);
  if (rc)
    return rc;
  if (device < 0 || device > 63)
    return fail(Q4K_EINVAL, "bad device %d", device);
  rc = set_device(device);
  if (rc)
    return rc;
  q4k_weight* w = new (std::nothrow) q4k_weight;
  if (!w)
    return fail(Q4K_ENOMEM, "host allocation failed");
  w->device = device;
  w->n = n;
  w->k = k;
  w->type = ggml_type;
  w->bytes = bytes;
  if (hipMalloc(&w->data, bytes) != hipSuccess) {
    delete w;
    return fail(Q4K_ENOMEM, "cannot allocate %zu bytes of weights on device %d", bytes, device);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = ggml_type == Q4K_GGML_TYPE_Q4_K
                    ? launch_relayout(s, static_cast<const uint8_t*>(gguf_device_bytes), w->data, n, k)
                    : launch_typed_relayout(s, static_cast<const uint8_t*>(gguf_device_bytes), w->data, n, k, ggml_type);
  if (e == hipSuccess)
    e = hipStreamSynchronize(s);
  if (e != hipSuccess) {
    (void)hipFree(w->data);
    delete w;
    return hip_fail(e, "device relayout");
  }
  *out = w;
  return Q4K_OK;
}

int q4k_weight_destroy(q4k_weight* w) {
  if (!w)
    return Q4K_OK;
  int cur = -1;
  (void)hipGetDevice(&cur);
  if (cur != w->device)
    (void)hipSetDevice(w->device);
  hipError_t e = hipFree(w->data);
  if (cur != w->device && cur >= 0)
    (void)hipSetDevice(cur);
  delete w;
  return e == hipSuccess ? Q4K_OK : hip_fail(e, "hipFree(weight)");
}

int q4k_weight_info(const q4k_weight* w, uint32_t* n, uint32_t* k, uint64_t* device_bytes) {
  if (!w)
    return fail(Q4K_EINVAL, "weight is NULL");
  if (n)
    *n = w->n;
  if (k)
    *k = w->k;
  if (device_bytes)
    *device_bytes = w->bytes;
  return Q4K_OK;
}

int q4k_weight_kernel_name(const q4k_weight* w, uint32_t phase, char* buf, size_t buflen) {
  if (!w || !buf || buflen == 0)
    return fail(Q4K_EINVAL, "null argument");
  if (phase > 3)
    return fail(Q4K_EINVAL, "phase %u out of range", phase);
  std::snprintf(buf, buflen, "%s", w->kernels[phase].name.c_str());
  return Q4K_OK;
}

int q4k_weight_prepare(q4k_weight* w, uint32_t phase) {
  if (!w)
    return fail(Q4K_EINVAL, "weight is NULL");
  if (phase > 3)
    return fail(Q4K_EINVAL, "phase %u out of range", phase);
  resolve(w, phase);
  return Q4K_OK;
}

int q4k_select_phase(const uint32_t* query_counts, uint32_t nqueries, uint32_t m, int gated, uint32_t* phase) {
  if (!phase)
    return fail(Q4K_EINVAL, "phase is NULL");
  int rc = check_counts(query_counts, nqueries, m);
  if (rc)
    return rc;
  *phase = phase_of(query_counts, nqueries, m, gated != 0);
  return Q4K_OK;
}

}  // extern "C"

namespace {

// Argument checks of q4k_linear / q4k_linear_noalloc; *phase receives the
// batch's phase.
int check_linear(const q4k_weight* w, const void* x, const void* y, const void* aux, uint32_t m, const uint32_t* query_counts,
                 uint32_t nqueries, uint32_t post, uint32_t dtype, uint32_t* phase) {
  if (!w)
    return fail(Q4K_EINVAL, "weight is NULL");
  if (dtype > Q4K_DTYPE_F16)
    return fail(Q4K_EINVAL, "bad dtype %u", dtype);
  if (post > Q4K_POST_GATE)
    return fail(Q4K_EINVAL, "bad post code %u", post);
  if (m == 0)
    return fail(Q4K_ESHAPE, "m must be positive");
  if (!x || !y)
    return fail(Q4K_EINVAL, "x and y must be non-NULL");
  if (post != Q4K_POST_STORE && !aux)
    return fail(Q4K_EINVAL, "post %u needs aux", post);
  int rc = check_counts(query_counts, nqueries, m);
  if (rc)
    return rc;
  const size_t es = dtype == Q4K_DTYPE_F32 ? 4 : 2;
  if (overlaps(x, (size_t)m * w->k * es, y, (size_t)m * w->n * es))
    return fail(Q4K_EALIAS, "x must not overlap y");
  if (aux && aux != y && overlaps(aux, (size_t)m * w->n * es, y, (size_t)m * w->n * es))
    return fail(Q4K_EALIAS, "aux must be y itself or disjoint from it");
  *phase = phase_of(query_counts, nqueries, m, false);
  if (*phase != Q4K_PHASE_PREFILL && m > 16u * kGemvMaxRowTiles)
    return fail(Q4K_ESHAPE, "decode batch of %u rows exceeds %d", m, 16 * kGemvMaxRowTiles);
  return Q4K_OK;
}

// ---- the no-allocation entry point (q4k_linear_noalloc) -------------------
// Its workspace lives in `scratch`, a file-scope device array that every GPU
// the library runs on holds until the process ends.  In host code the name
// `scratch` is a host-side stand-in, not a device address: the device
// address of each GPU's copy comes from hipGetSymbolAddress, taken once per
// device at that device's first call (with the device current), and only
// that address is used (kernel arguments, fills).
constexpr size_t kScratchBytes = 120ull << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// Fixed regions of the scratch: decode pack, split-K partials and counters,
// row scales; the rest holds the staged activations.
constexpr size_t kScrPackBytes = 2ull << 20;
constexpr size_t kScrPartBytes = 64ull << 20;  // two K-segments of a GEMM of up to 256 tiles
constexpr size_t kScrCounterBytes = 16ull << 10;
constexpr size_t kScrScaleBytes = 256ull << 10;
constexpr size_t kScrXBytes = kScratchBytes - kScrPackBytes - kScrPartBytes - kScrCounterBytes - kScrScaleBytes;

struct ScratchWorkspace {
  Workspace ws;
  bool ready = false;
};
ScratchWorkspace g_scratch[64];
std::mutex g_scratch_setup;

// The device's scratch workspace, set up on first use (device current).
int scratch_workspace(int device, Workspace** out) {
  ScratchWorkspace& sw = g_scratch[device & 63];
  std::lock_guard<std::mutex> lock(g_scratch_setup);
  if (!sw.ready) {
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess)
      return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!ptr)
      return fail(Q4K_EHIP, "hipGetSymbolAddress(scratch) returned no address on device %d", device);
    uint8_t* b = static_cast<uint8_t*>(ptr);
    Workspace& ws = sw.ws;
    ws.fixed = true;
    ws.pack = b;
    ws.pack_bytes = kScrPackBytes;
    b += kScrPackBytes;
    ws.part = reinterpret_cast<float*>(b);
    ws.part_elems = kScrPartBytes / sizeof(float);
    b += kScrPartBytes;
    ws.counters = reinterpret_cast<int*>(b);
    ws.counter_elems = kScrCounterBytes / sizeof(int);
    b += kScrCounterBytes;
    ws.scale = reinterpret_cast<float*>(b);
    ws.scale_elems = kScrScaleBytes / sizeof(float);
    b += kScrScaleBytes;
    ws.x = reinterpret_cast<_Float16*>(b);
    ws.x_elems = kScrXBytes / sizeof(_Float16);
    sw.ready = true;
  }
  *out = &sw.ws;
  return Q4K_OK;
}

}  // namespace

extern "C" {

int q4k_linear_noalloc(void* stream, q4k_weight* w, const void* x, void* y, const void* aux, uint32_t m, const uint32_t* query_counts,
                       uint32_t nqueries, uint32_t post, uint32_t dtype) {
  uint32_t phase = 0;
  int rc = check_linear(w, x, y, aux, m, query_counts, nqueries, post, dtype, &phase);
  if (rc)
    return rc;
  rc = set_device(w->device);
  if (rc)
    return rc;
  Workspace* ws = nullptr;
  rc = scratch_workspace(w->device, &ws);
  if (rc)
    return rc;
  std::lock_guard<std::mutex> lock(ws->mu);
  return run_linear_locked(static_cast<hipStream_t>(stream), *ws, w, nullptr, x, y, aux, m, post, dtype, phase, true);
}

int q4k_linear(void* stream, q4k_weight* w, const void* x, void* y, const void* aux, uint32_t m, const uint32_t* query_counts, uint32_t nqueries,
               uint32_t post, uint32_t dtype) {
  uint32_t phase = 0;
  int rc = check_linear(w, x, y, aux, m, query_counts, nqueries, post, dtype, &phase);
  if (rc)
    return rc;
  rc = set_device(w->device);
  if (rc)
    return rc;
  return run_linear(static_cast<hipStream_t>(stream), w, nullptr, x, y, aux, m, post, dtype, phase);
}

int q4k_linear_norm(void* stream, q4k_weight* w, const float* norm_w, float eps, const void* x, void* y, const void* aux, uint32_t m,
                    const uint32_t* query_counts, uint32_t nqueries, uint32_t post, uint32_t dtype) {
  if (!norm_w)
    return fail(Q4K_EINVAL, "norm_w is NULL");
  if (!(eps >= 0.0f))
    return fail(Q4K_EINVAL, "eps must be a non-negative number");
  uint32_t phase = 0;
  int rc = check_linear(w, x, y, aux, m, query_counts, nqueries, post, dtype, &phase);
  if (rc)
    return rc;
  if (aux && aux == x)
    return fail(Q4K_EALIAS, "aux must not be x");
  rc = set_device(w->device);
  if (rc)
    return rc;
  return run_linear(static_cast<hipStream_t>(stream), w, nullptr, x, y, aux, m, post, dtype, phase, norm_w, eps);
}

}  // extern "C"

namespace {

// The gated projection with an optional RMS norm of x (q4k_mlp's ffn_norm).
int mlp_gate_up_impl(void* stream, q4k_weight* wg, q4k_weight* wu, const void* x, void* y, uint32_t m, const uint32_t* query_counts,
                     uint32_t nqueries, uint32_t dtype, const float* norm_w, float eps);

}  // namespace

extern "C" {

int q4k_mlp_gate_up(void* stream, q4k_weight* wg, q4k_weight* wu, const void* x, void* y, uint32_t m, const uint32_t* query_counts,
                    uint32_t nqueries, uint32_t dtype) {
  return mlp_gate_up_impl(stream, wg, wu, x, y, m, query_counts, nqueries, dtype, nullptr, 0.0f);
}

}  // extern "C"

namespace {

int mlp_gate_up_impl(void* stream, q4k_weight* wg, q4k_weight* wu, const void* x, void* y, uint32_t m, const uint32_t* query_counts,
                     uint32_t nqueries, uint32_t dtype, const float* norm_w, float eps) {
  if (!wg || !wu)
    return fail(Q4K_EINVAL, "gate and up weights must be non-NULL");
  if (wg->n != wu->n || wg->k != wu->k || wg->device != wu->device)
    return fail(Q4K_ESHAPE, "gate (%ux%u) and up (%ux%u) weights differ", wg->n, wg->k, wu->n, wu->k);
  if (dtype > Q4K_DTYPE_F16)
    return fail(Q4K_EINVAL, "bad dtype %u", dtype);
  if (m == 0)
    return fail(Q4K_ESHAPE, "m must be positive");
  if (!x || !y)
    return fail(Q4K_EINVAL, "x and y must be non-NULL");
  int rc = check_counts(query_counts, nqueries, m);
  if (rc)
    return rc;
  const size_t es = dtype == Q4K_DTYPE_F32 ? 4 : 2;
  if (overlaps(x, (size_t)m * wg->k * es, y, (size_t)m * wg->n * es))
    return fail(Q4K_EALIAS, "x must not overlap y");
  rc = set_device(wg->device);
  if (rc)
    return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint32_t phase = phase_of(query_counts, nqueries, m, true);
  const bool q4 = wg->type == Q4K_GGML_TYPE_Q4_K && wu->type == Q4K_GGML_TYPE_Q4_K;
  if (phase == Q4K_PHASE_GATED_DECODE && m > 16u * kGemvMaxRowTiles)
    return fail(Q4K_ESHAPE, "decode batch of %u rows exceeds %d", m, 16 * kGemvMaxRowTiles);
  if (phase == Q4K_PHASE_GATED_DECODE && q4)
    return run_linear(s, wg, wu, x, y, nullptr, m, Q4K_POST_STORE, dtype, phase, norm_w, eps);
  if (phase == Q4K_PHASE_GATED_DECODE && wg->type == wu->type && typed_gate_up_supported(wg->type, (int)m, (int)(wg->k / 256), (int)wg->n)) {
    // The fused gate/up GEMV of a type with one in the reference
    // (fused_kernels.metal:80-200): one launch, x packed in registers.
    Workspace& ws = workspace(wg->device);
    std::lock_guard<std::mutex> lock(ws.mu);
    resolve(wg, phase);
    resolve(wu, phase);
    GemvArgs a{};
    a.w = wg->data;
    a.wu = wu->data;
    a.x = x;
    a.y = y;
    a.m = (int)m;
    a.n = (int)wg->n;
    a.k = (int)wg->k;
    a.nb = (int)(wg->k / 256);
    a.rows = 2 * (int)m;
    a.split = 1;
    a.norm_w = norm_w;
    a.eps = eps;
    LaunchTimer timer(s, Q4K_KERNEL_GEMV_GATED);
    Q4K_TRY_HIP(launch_typed_gate_up(s, a, wg->type, (int)dtype, device_cus(wg->device)), "typed gate/up launch");
    return Q4K_OK;
  }
  Workspace& ws = workspace(wg->device);
  std::lock_guard<std::mutex> lock(ws.mu);
  if (q4 && resolve(wg, phase).kind == kGemm && m > 16u * kGemvMaxRowTiles && gemm2_supported((int)m, (int)wg->n)) {
    // Both projections on the pipelined GEMM: one gated launch over x staged
    // once computes SiLU(gate) * up with the two-call form's roundings (the
    // same buffer bit for bit), without storing the gate and reading it back.
    resolve(wu, phase);
    const size_t rows = (size_t)gemm2_rows((int)m);
    rc = ensure_workspace(s, ws, wg->device, rows * wg->k, rows);
    if (rc)
      return rc;
    {
      LaunchTimer timer(s, Q4K_KERNEL_STAGE);
      Q4K_TRY_HIP(launch_stage_x(s, x, (int)dtype, ws.x, nullptr, ws.scale, (int)m, (int)wg->k, kStageGemm, norm_w, eps), "stage_x launch");
    }
    GemmArgs a;
    a.w = wg->data;
    a.wu = wu->data;
    a.xh = ws.x;
    a.rowscale = ws.scale;
    a.y = y;
    a.aux = nullptr;
    a.m = (int)m;
    a.n = (int)wg->n;
    a.k = (int)wg->k;
    a.nb = (int)(wg->k / 256);
    a.post = Q4K_POST_GATE;
    rc = gemm2_split_buffers(s, ws, wg->device, a, true);
    if (rc)
      return rc;
    LaunchTimer timer(s, Q4K_KERNEL_GEMM);
    Q4K_TRY_HIP(launch_gemm2_gated(s, a, (int)dtype, device_cus(wg->device)), "gated gemm launch");
    return Q4K_OK;
  }
  // forward.cpp:116-118: gate -> y (post 0), then up with aux = y, post 2, in
  // place.  Both read the same x: it is staged once (with the norm, if any),
  // under one hold of the workspace lock.
  rc = run_linear_locked(s, ws, wg, nullptr, x, y, nullptr, m, Q4K_POST_STORE, dtype, phase, true, norm_w, eps);
  if (rc)
    return rc;
  // The Q4_K projection of a Q4_K pair reuses the staged x; other types pack their own.
  return run_linear_locked(s, ws, wu, nullptr, x, y, y, m, Q4K_POST_GATE, dtype, phase, !q4, norm_w, eps);
}

}  // namespace

extern "C" {

int q4k_mlp(void* stream, q4k_weight* wg, q4k_weight* wu, q4k_weight* wd, const float* norm_w, float eps, const void* x, void* gate, void* hidden,
            uint32_t m, const uint32_t* query_counts, uint32_t nqueries, uint32_t dtype) {
  if (!wg || !wu || !wd)
    return fail(Q4K_EINVAL, "gate, up and down weights must be non-NULL");
  if (wg->n != wu->n || wg->k != wu->k || wg->device != wu->device)
    return fail(Q4K_ESHAPE, "gate (%ux%u) and up (%ux%u) weights differ", wg->n, wg->k, wu->n, wu->k);
  if (wd->k != wg->n || wd->n != wg->k || wd->device != wg->device)
    return fail(Q4K_ESHAPE, "down weight %ux%u does not map the %u gate outputs back to %u", wd->n, wd->k, wg->n, wg->k);
  if (dtype > Q4K_DTYPE_F16)
    return fail(Q4K_EINVAL, "bad dtype %u", dtype);
  if (m == 0)
    return fail(Q4K_ESHAPE, "m must be positive");
  if (!x || !gate || !hidden)
    return fail(Q4K_EINVAL, "x, gate and hidden must be non-NULL");
  if (norm_w && !(eps >= 0.0f))
    return fail(Q4K_EINVAL, "eps must be a non-negative number");
  int rc = check_counts(query_counts, nqueries, m);
  if (rc)
    return rc;
  const size_t es = dtype == Q4K_DTYPE_F32 ? 4 : 2;
  const size_t xb = (size_t)m * wg->k * es, gb = (size_t)m * wg->n * es, hb = (size_t)m * wd->n * es;
  if (overlaps(x, xb, gate, gb) || overlaps(gate, gb, hidden, hb))
    return fail(Q4K_EALIAS, "the gate buffer must not overlap x or hidden");
  if (x != hidden && overlaps(x, xb, hidden, hb))
    return fail(Q4K_EALIAS, "x must equal hidden or not overlap it");
  rc = set_device(wg->device);
  if (rc)
    return rc;
  // forward.cpp:114-119 as two calls: the ffn_norm (inside the fused gate/up
  // GEMV for decode passes, folded into the activation staging of the
  // gate/up projections otherwise) and gate/up into the gate buffer, then
  // down with the residual added in place.  (Stream order: the gate/up
  // launches have read all of x before the down projection writes hidden, so
  // x may be hidden.)
  rc = mlp_gate_up_impl(stream, wg, wu, x, gate, m, query_counts, nqueries, dtype, norm_w, eps);
  if (rc)
    return rc;
  return q4k_linear(stream, wd, gate, hidden, hidden, m, query_counts, nqueries, Q4K_POST_ADD, dtype);
}

int q4k_workspace_allocations(uint64_t* count) {
  if (!count)
    return fail(Q4K_EINVAL, "null argument");
  *count = g_ws_allocations.load(std::memory_order_relaxed);
  return Q4K_OK;
}

int q4k_profile_enable(int on) {
  std::lock_guard<std::mutex> lock(g_prof.mu);
  if (on)
    g_prof.clear();
  g_prof.on = on != 0;
  return Q4K_OK;
}

int q4k_mfma_ceiling(void* stream, int device, uint32_t iters, double* tflops) {
  if (!tflops || iters == 0)
    return fail(Q4K_EINVAL, "tflops must be non-NULL and iters positive");
  int rc = set_device(device);
  if (rc)
    return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int blocks = device_cus(device);
  float* out = nullptr;
  Q4K_TRY_HIP(hipMalloc(&out, (size_t)blocks * 256 * sizeof(float)), "hipMalloc");
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t err = hipEventCreate(&e0);
  if (err == hipSuccess)
    err = hipEventCreate(&e1);
  if (err == hipSuccess)
    err = launch_mfma_ceiling(s, out, blocks, (int)(iters < 64 ? iters : 64));  // warm-up
  if (err == hipSuccess)
    err = hipEventRecord(e0, s);
  if (err == hipSuccess)
    err = launch_mfma_ceiling(s, out, blocks, (int)iters);
  if (err == hipSuccess)
    err = hipEventRecord(e1, s);
  if (err == hipSuccess)
    err = hipEventSynchronize(e1);
  float ms = 0.0f;
  if (err == hipSuccess)
    err = hipEventElapsedTime(&ms, e0, e1);
  if (e0)
    (void)hipEventDestroy(e0);
  if (e1)
    (void)hipEventDestroy(e1);
  (void)hipFree(out);
  if (err != hipSuccess)
    return fail(Q4K_EHIP, "mfma ceiling: %s", hipGetErrorString(err));
  const double flop = 2.0 * 16 * 16 * 32 * 32.0 * iters * 4.0 * blocks;
  *tflops = ms > 0.0f ? flop / (ms * 1e-3) / 1e12 : 0.0;
  return Q4K_OK;
}

int q4k_read_ceiling(void* stream, int device, const void* const* buffers, uint32_t count, uint64_t bytes, uint32_t reps, double* gbs) {
  if (!gbs || !buffers || count == 0 || reps == 0 || bytes == 0 || bytes % 16 != 0)
    return fail(Q4K_EINVAL, "gbs and buffers must be non-NULL; count, reps and bytes (a multiple of 16) positive");
  for (uint32_t i = 0; i < count; ++i)
    if (!buffers[i] || reinterpret_cast<uintptr_t>(buffers[i]) % 16 != 0)
      return fail(Q4K_EINVAL, "buffer %u is NULL or not 16-byte aligned", i);
  int rc = set_device(device);
  if (rc)
    return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // 32 workgroups per CU: the fastest grid measured (57 MB reads: 5.93 TB/s,
  // against 5.46 with 16, 5.34 with 8 and 5.26 with 4).
  const int blocks = 32 * device_cus(device);
  uint32_t* out = nullptr;
  Q4K_TRY_HIP(hipMalloc(&out, (size_t)blocks * sizeof(uint32_t)), "hipMalloc");
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t err = hipEventCreate(&e0);
  if (err == hipSuccess)
    err = hipEventCreate(&e1);
  for (uint32_t i = 0; i < count && err == hipSuccess; ++i)  // warm-up: one pass over every buffer
    err = launch_stream_read(s, buffers[i], bytes, out, blocks);
  if (err == hipSuccess)
    err = hipEventRecord(e0, s);
  for (uint32_t r = 0; r < reps && err == hipSuccess; ++r)
    err = launch_stream_read(s, buffers[r % count], bytes, out, blocks);
  if (err == hipSuccess)
    err = hipEventRecord(e1, s);
  if (err == hipSuccess)
    err = hipEventSynchronize(e1);
  float ms = 0.0f;
  if (err == hipSuccess)
    err = hipEventElapsedTime(&ms, e0, e1);
  if (e0)
    (void)hipEventDestroy(e0);
  if (e1)
    (void)hipEventDestroy(e1);
  (void)hipFree(out);
  if (err != hipSuccess)
    return fail(Q4K_EHIP, "read ceiling: %s", hipGetErrorString(err));
  *gbs = ms > 0.0f ? (double)bytes * reps / (ms * 1e-3) / 1e9 : 0.0;
  return Q4K_OK;
}

int q4k_profile_query(uint32_t kernel, uint32_t* launches, double* total_ms, double* min_ms, double* max_ms) {
  if (kernel > Q4K_KERNEL_AUX)
    return fail(Q4K_EINVAL, "kernel family %u out of range", kernel);
  std::lock_guard<std::mutex> lock(g_prof.mu);
  double total = 0.0, lo = 0.0, hi = 0.0;
  uint32_t count = 0;
  for (auto& e : g_prof.events[kernel]) {
    Q4K_TRY_HIP(hipEventSynchronize(e.second), "hipEventSynchronize");
    float ms = 0.0f;
    Q4K_TRY_HIP(hipEventElapsedTime(&ms, e.first, e.second), "hipEventElapsedTime");
    total += ms;
    lo = count == 0 ? ms : (ms < lo ? ms : lo);
    hi = count == 0 ? ms : (ms > hi ? ms : hi);
    ++count;
  }
  if (launches)
    *launches = count;
  if (total_ms)
    *total_ms = total;
  if (min_ms)
    *min_ms = lo;
  if (max_ms)
    *max_ms = hi;
  return Q4K_OK;
}

int q4k_pack_queries(const uint32_t* counts, const uint32_t* samples, uint32_t nqueries, uint32_t* start, uint32_t* logit, uint32_t* rows,
                     uint32_t* logit_rows) {
  if (!counts || !start || !logit)
    return fail(Q4K_EINVAL, "null argument");
  if (nqueries > Q4K_MAX_QUERIES)
    return fail(Q4K_EINVAL, "at most %u queries (got %u)", Q4K_MAX_QUERIES, nqueries);
  uint64_t r = 0, l = 0;
  for (uint32_t i = 0; i < nqueries; ++i) {
    if (samples && samples[i] > counts[i])
      return fail(Q4K_EINVAL, "query %u samples %u rows but has %u", i, samples[i], counts[i]);
    start[i] = (uint32_t)r;
    logit[i] = (uint32_t)l;
    l += samples ? samples[i] : 0u;
    r += counts[i];
    if (r > 0xffffffffull)
      return fail(Q4K_EINVAL, "row count overflows 32 bits");
  }
  if (rows)
    *rows = (uint32_t)r;
  if (logit_rows)
    *logit_rows = (uint32_t)l;
  return Q4K_OK;
}

int q4k_gather_rows(void* stream, const void* x, void* out, uint32_t k, const uint32_t* counts, const uint32_t* samples, uint32_t nqueries,
                    uint32_t dtype, uint32_t* rows_out) {
  if (!x || !out || !counts || !samples)
    return fail(Q4K_EINVAL, "null argument");
  if (dtype > Q4K_DTYPE_F16)
    return fail(Q4K_EINVAL, "bad dtype %u", dtype);
  if (k == 0)
    return fail(Q4K_ESHAPE, "k must be positive");
  GatherIndex idx;
  uint32_t rows = 0;
  int rc = logit_rows(counts, samples, nqueries, &idx, &rows);
  if (rc)
    return rc;
  if (rows_out)
    *rows_out = idx.rows;
  const size_t es = dtype == Q4K_DTYPE_F32 ? 4 : 2;
  if (overlaps(x, (size_t)rows * k * es, out, (size_t)idx.rows * k * es))
    return fail(Q4K_EALIAS, "out must not overlap x");
  Q4K_TRY_HIP(launch_gather(static_cast<hipStream_t>(stream), x, out, (int)k, (int)dtype, idx), "gather launch");
  return Q4K_OK;
}

int q4k_embedding(void* stream, const q4k_weight* table, const int32_t* ids, uint32_t rows, void* y, uint32_t dtype) {
  if (!table || !ids || !y)
    return fail(Q4K_EINVAL, "null argument");
  if (dtype > Q4K_DTYPE_F16)
    return fail(Q4K_EINVAL, "bad dtype %u", dtype);
  if (table->type != Q4K_GGML_TYPE_Q4_K)
    return fail(Q4K_ETYPE, "the embedding table must be Q4_K (embedding_q4_k)");
  const size_t es = dtype == Q4K_DTYPE_F32 ? 4 : 2;
  if (overlaps(ids, (size_t)rows * 4, y, (size_t)rows * table->k * es))
    return fail(Q4K_EALIAS, "y must not overlap ids");
  int rc = set_device(table->device);
  if (rc)
    return rc;
  LaunchTimer timer(static_cast<hipStream_t>(stream), Q4K_KERNEL_AUX);
  Q4K_TRY_HIP(launch_embedding(static_cast<hipStream_t>(stream), table->data, ids, y, (int)rows, (int)table->n, (int)table->k, (int)dtype),
              "embedding launch");
  return Q4K_OK;
}

int q4k_embedding_batch(void* stream, const q4k_weight* table, const int32_t* tokens, uint32_t capacity, const uint32_t* counts,
                        const uint32_t* positions, const uint32_t* slots, uint32_t nqueries, void* y, uint32_t dtype, uint32_t* rows_out) {
  if (!table || !tokens || !counts || !positions || !slots || !y)
    return fail(Q4K_EINVAL, "null argument");
  if (dtype > Q4K_DTYPE_F16)
    return fail(Q4K_EINVAL, "bad dtype %u", dtype);
  if (table->type != Q4K_GGML_TYPE_Q4_K)
    return fail(Q4K_ETYPE, "the embedding table must be Q4_K (embedding_q4_k)");
  if (nqueries == 0 || nqueries > kEmbedMaxQueries)
    return fail(Q4K_ESHAPE, "nqueries must be 1..%u (got %u)", kEmbedMaxQueries, nqueries);
  EmbedQueries qs{};
  qs.n = nqueries;
  qs.capacity = capacity;
  uint64_t rows = 0;
  uint32_t max_slot = 0;
  for (uint32_t q = 0; q < nqueries; ++q) {
    if ((uint64_t)positions[q] + counts[q] > capacity)
      return fail(Q4K_ESHAPE, "query %u: position %u + count %u exceeds the capacity %u", q, positions[q], counts[q], capacity);
    qs.start[q] = (uint32_t)rows;
    qs.count[q] = counts[q];
    qs.position[q] = positions[q];
    qs.slot[q] = slots[q];
    rows += counts[q];
    max_slot = slots[q] > max_slot ? slots[q] : max_slot;
  }
  if (rows == 0 || rows > 65535)
    return fail(Q4K_ESHAPE, "the batch must have 1..65535 rows (got %llu)", (unsigned long long)rows);
  if (((uint64_t)max_slot + 1) * capacity > 0x7fffffffull)
    return fail(Q4K_ESHAPE, "slot %u x capacity %u exceeds the token buffer's 32-bit index", max_slot, capacity);
  if (rows_out)
    *rows_out = (uint32_t)rows;
  const size_t es = dtype == Q4K_DTYPE_F32 ? 4 : 2;
  if (overlaps(tokens, ((size_t)max_slot + 1) * capacity * 4, y, (size_t)rows * table->k * es))
    return fail(Q4K_EALIAS, "y must not overlap tokens");
  int rc = set_device(table->device);
  if (rc)
    return rc;
  LaunchTimer timer(static_cast<hipStream_t>(stream), Q4K_KERNEL_AUX);
  Q4K_TRY_HIP(launch_embedding_batch(static_cast<hipStream_t>(stream), table->data, tokens, qs, y, (int)rows, (int)table->n, (int)table->k,
                                     (int)dtype),
              "embedding launch");
  return Q4K_OK;
}

int q4k_rms_norm(void* stream, const void* x, const float* w, void* y, uint32_t m, uint32_t k, float eps, uint32_t dtype) {
  if (!x || !w || !y)
    return fail(Q4K_EINVAL, "null argument");
  if (dtype > Q4K_DTYPE_F16)
    return fail(Q4K_EINVAL, "bad dtype %u", dtype);
  if (k == 0)
    return fail(Q4K_ESHAPE, "k must be positive");
  if (!(eps >= 0.0f))
    return fail(Q4K_EINVAL, "eps must be a non-negative number");
  const size_t es = dtype == Q4K_DTYPE_F32 ? 4 : 2;
  if (x != y && overlaps(x, (size_t)m * k * es, y, (size_t)m * k * es))
    return fail(Q4K_EALIAS, "y must equal x or not overlap it");
  LaunchTimer timer(static_cast<hipStream_t>(stream), Q4K_KERNEL_AUX);
  Q4K_TRY_HIP(launch_rms_norm(static_cast<hipStream_t>(stream), x, w, y, (int)m, (int)k, eps, (int)dtype, nullptr), "rms_norm launch");
  return Q4K_OK;
}

int q4k_rms_norm_gather(void* stream, const void* x, const float* w, void* out, uint32_t k, const uint32_t* counts, const uint32_t* samples,
                        uint32_t nqueries, float eps, uint32_t dtype, uint32_t* rows_out) {
  if (!x || !w || !out || !counts || !samples)
    return fail(Q4K_EINVAL, "null argument");
  if (dtype > Q4K_DTYPE_F16)
    return fail(Q4K_EINVAL, "bad dtype %u", dtype);
  if (k == 0)
    return fail(Q4K_ESHAPE, "k must be positive");
  if (!(eps >= 0.0f))
    return fail(Q4K_EINVAL, "eps must be a non-negative number");
  GatherIndex idx;
  uint32_t rows = 0;
  int rc = logit_rows(counts, samples, nqueries, &idx, &rows);
  if (rc)
    return rc;
  if (rows_out)
    *rows_out = idx.rows;
  const size_t es = dtype == Q4K_DTYPE_F32 ? 4 : 2;
  if (overlaps(x, (size_t)rows * k * es, out, (size_t)idx.rows * k * es))
    return fail(Q4K_EALIAS, "out must not overlap x");
  LaunchTimer timer(static_cast<hipStream_t>(stream), Q4K_KERNEL_AUX);
  Q4K_TRY_HIP(launch_rms_norm(static_cast<hipStream_t>(stream), x, w, out, (int)idx.rows, (int)k, eps, (int)dtype, &idx), "rms_norm_gather launch");
  return Q4K_OK;
}

}  // extern "C"
