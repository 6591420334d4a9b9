// Internal interface between the C-ABI host code (q4k_api.hip) and the
// kernels (q4k_kernels.hip).  Not installed; the public surface is include/q4k.h.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace q4k {

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

// ---- device weight layout --------------------------------------------------
// GGUF stores row n as k/256 consecutive 144-byte block_q4_K records
// (d fp16 @0, dmin fp16 @2, 12 packed 6-bit scale/min bytes @4, 128 quant
// bytes @16).  The device copy groups 16 consecutive rows ("column tile" c)
// and, for each 256-element block b, stores the 16 records of that tile as one
// 2304-byte "tile-block" at ((c * nb) + b) * 2304:
//   [0, 1024)     slab 0: lane l = 16*g + i holds quant bytes 32g..32g+15 of row 16c+i
//   [1024, 2048)  slab 1: lane l holds quant bytes 32g+16..32g+31 of row 16c+i
//   [2048, 2304)  row 16c+i's 16 header bytes at 2048 + 16i (unchanged)
// Within each 4-byte word of a slab the two middle bytes are swapped, so that
// masking a word with 0x000F000F yields the low nibbles of two *consecutive*
// quant bytes.  A wave reads a whole slab with one fully-contiguous 16-byte
// load per lane, and the lane order is the B-operand order of
// v_mfma_f32_16x16x32_f16 (column = lane % 16, k-group = lane / 16).
// The byte count is unchanged: 144 bytes per 256 weights.
constexpr int kTileN = 16;
constexpr int kBlockBytes = 144;
constexpr int kTileBlockBytes = kTileN * kBlockBytes;  // 2304
constexpr int kSlabBytes = 1024;
constexpr int kHeaderOffset = 2048;

// ---- block_q6_K device layout ----------------------------------------------
// GGUF stores row n as k/256 consecutive 210-byte block_q6_K records (ql[128]
// @0, qh[64] @128, int8 scales[16] @192, d fp16 @208; weight = d * sc * (q - 32)
// with a 6-bit q).  The device copy uses the same 16-row column tiles; tile-
// block (c, b) is 3360 bytes at ((c * nb) + b) * 3360:
//   [0, 3072)     three slabs: lane l = 16g + i (row 16c + i) holds its quant
//                 dwords 4s..4s+3 at s * 1024 + 16 l
//   [3072, 3328)  lane l's scale dword at 3072 + 4 l: scales 4g..4g+3 of row
//                 16c + i, each stored as sc + 128 (the byte sc ^ 0x80)
//   [3328, 3360)  d of rows 16c..16c+15
// Lane l covers elements 64g + [0, 64) of its row in the decode pack's order:
// B-operand dword o = 4 fs + t of MFMA fs holds elements
// e = 64g + 32 (fs / 4) + 8 (fs % 4) + 2t + {0, 1} (low half, high half), all
// in sub-block 4g + o / 8.  The twelve dwords are four triples (A, B, C) =
// dwords 3a..3a+2 for outputs o = 8a + r; per 16-bit half, r = 0, 2, 4 sit at
// bits 4..9 of A, B, C; r = 1, 3, 5 at bits 10..15; r = 6 takes its low four
// bits from bits 0..3 of A and its top two from bits 0..1 of B; r = 7 from
// bits 0..3 of C and bits 2..3 of B.  Same byte count: 210 per 256 weights.
constexpr int kQ6BlockBytes = 210;
constexpr int kQ6TileBlockBytes = kTileN * kQ6BlockBytes;  // 3360
constexpr int kQ6ScaleOffset = 3072;
constexpr int kQ6DOffset = 3328;

// 6-bit quant (0..63) of element e of a GGUF block_q6_K
// (backend/metal/kernel/quant_linear.metal:69-86 addressing).
__host__ __device__ inline uint32_t q6_quant(const uint8_t* blk, int e) {
  const int h = e >> 7, rr = e & 127, l = rr & 31;
  const uint32_t q = blk[64 * h + (rr & 32) + l];
  const uint32_t lo = (rr & 64) ? (q >> 4) : (q & 15u);
  return lo | (((uint32_t)(blk[128 + 32 * h + l] >> (2 * (rr >> 5))) & 3u) << 4);
}

// Element of block b's lane-group g for output dword o, half hf.
__host__ __device__ inline int q6_elem(int g, int o, int hf) {
  const int fs = o >> 2, t = o & 3;
  return 64 * g + 32 * (fs >> 2) + 8 * (fs & 3) + 2 * t + hf;
}

// Writes / reads the 6-bit quant of (o, hf) in a lane's twelve dwords.
__host__ __device__ inline void q6_place(uint32_t* wd, int o, int hf, uint32_t v) {
  const int a = o >> 3, r = o & 7, sh = 16 * hf;
  uint32_t* A = wd + 3 * a;
  switch (r) {
    case 6:
      A[0] |= (v & 15u) << sh;
      A[1] |= (v >> 4) << sh;
      break;
    case 7:
      A[2] |= (v & 15u) << sh;
      A[1] |= (v >> 4) << (2 + sh);
      break;
    default:
      A[r >> 1] |= v << ((r & 1 ? 10 : 4) + sh);
  }
}

__host__ __device__ inline uint32_t q6_take(const uint32_t* wd, int o, int hf) {
  const int a = o >> 3, r = o & 7, sh = 16 * hf;
  const uint32_t* A = wd + 3 * a;
  switch (r) {
    case 6:
      return ((A[0] >> sh) & 15u) | (((A[1] >> sh) & 3u) << 4);
    case 7:
      return ((A[2] >> sh) & 15u) | (((A[1] >> (2 + sh)) & 3u) << 4);
    default:
      return (A[r >> 1] >> ((r & 1 ? 10 : 4) + sh)) & 63u;
  }
}

// Rows of a GEMV call are padded to 16-row MFMA tiles; the GEMV handles up to
// kGemvMaxRowTiles of them (48 rows: the 8 x 5 decode rows of the reference).
constexpr int kGemvMaxRowTiles = 3;

enum Dtype : int { kF32 = 0, kF16 = 1 };

// Decode pack: the MFMA operands of x (m <= 8 rows) for the streaming and
// split-K GEMVs (layout in q4k_kernels.hip, stage_pack_kernel).
struct DecodePack {
  u4_t* frag = nullptr;  // [nb][8][64] x 16 B
  h4_t* xs = nullptr;    // [nb][64] x 8 B
  float* dsc = nullptr;  // [nb][8]
};
constexpr size_t kPackBytesPerBlock = 8 * 64 * 16 + 64 * 8 + 8 * 4;

struct GemvArgs {
  const uint8_t* w;       // tiled weights (gate weights when gated)
  const uint8_t* wu;      // up weights when gated, else unused
  const _Float16* xf;     // staged activations, fragment order
  const _Float16* xs;     // staged sub-block sums / 32, min-term fragment order
  const float* rowscale;  // per-row power-of-two unscale factor
  const void* x;          // caller's activations [m, k]
  DecodePack pack;        // packed operands of x (streaming and split-K GEMVs)
  void* y;
  const void* aux;
  int m, n, k, nb, post;
  int rows;  // staged fragment rows: 2m when split (rows m.. hold the low parts), else m
  int split;
  // Fused gate/up GEMV only: when non-null, x is RMS-normalised first,
  // x * rsqrt(sum(x^2) / k + eps) * norm_w (native_ops.metal:6-40).
  const float* norm_w = nullptr;
  float eps = 0.0f;
};

struct GemmArgs {
  const uint8_t* w;
  const _Float16* xh;  // staged activations, row-major [m, k]
  const float* rowscale;
  void* y;
  const void* aux;
  int m, n, k, nb, post;
};

struct GatherIndex {
  uint32_t rows;
  uint32_t src[64];
};

// Activation staging layouts.
enum StageMode : int {
  kStageRowMajor = 0,  // fp16 [m, k] (GEMM A operand)
  kStageFrag = 1,      // fp16 in GEMV fragment order, m rows
  kStageFragSplit = 2, // fragment order, rows [0, m) = hi, rows [m, 2m) = lo
  kStageGemm = 3       // fp16 in the pipelined GEMM's order (gemm_frag_offset), no xs
};

// Stage x [m, k] (fp32 or fp16) as fp16 scaled by a per-row power of two
// (so rows with |x| beyond the fp16 range stay finite); rowscale[r] receives
// the factor that undoes the scaling.  In the split mode each scaled value v
// is carried as hi = fp16(v) plus lo = fp16(v - hi), about 22 significant bits.
// The fragment modes also write xs: each 32-element sub-block's sum of the
// scaled values, divided by 32 (so it stays within fp16), hi/lo like x.
hipError_t launch_stage_x(hipStream_t s, const void* x, int dtype, _Float16* xo, _Float16* xs, float* rowscale, int m, int k, int mode);
hipError_t launch_stage_pack(hipStream_t s, const void* x, int dtype, const DecodePack& pk, int m, int k);

// Halves of the sub-block-sum fragments for `rows` staged rows: per 16-row
// tile and block, 32 lanes x 4 halves.
inline size_t gemv_xs_halves(int rows, int k) {
  return (size_t)((rows + 15) / 16) * (k / 256) * 128;
}

// GEMV rows that the fragment layout holds for m activation rows: the split
// (hi + lo) form while it fits the kernel's row tiles (2m <= 48), else m.
inline bool gemv_split(int m) {
  return 2 * m <= 48;
}

// Launch geometry of the GEMV: 16-row tiles of activations, 16-column tiles
// of weights per workgroup, waves per workgroup (each takes 1/waves of K).
struct GemvShape {
  int row_tiles = 1, tiles = 1, waves = 8;
};
// rows = staged fragment rows (2m when split).  The environment variables
// Q4K_GEMV_TILES (1 or 2) and Q4K_GEMV_WAVES (4, 8 or 16) override the
// column tiles and waves per workgroup, for tuning.
GemvShape gemv_shape(int rows, int n, int nb, bool gated);

// Streaming GEMV (LDS ring, persistent workgroups) for one row tile and the
// block counts it is instantiated for; `cus` = compute units of the device.
bool gemv_stream_supported(int rows, int nb, int n, bool gated, int cus);
hipError_t launch_gemv_stream(hipStream_t s, const GemvArgs& a, int dtype, bool gated, int cus);

// Fused gate/up GEMV for m <= 8 rows and K = 4096 that packs x itself (no
// staging launch); reads a.x, a.w, a.wu (and a.norm_w when set) and writes a.y.
bool gemv_gate_up_supported(int m, int nb, int n);
hipError_t launch_gemv_gate_up(hipStream_t s, const GemvArgs& a, int dtype, int cus);

// Split-K GEMV for m <= 8 (see q4k_gemv_splitk_kernel): a plan picks an
// instance for (n, nb); the launch needs `part` (gemv_splitk_part_floats
// floats) and `counters` (plan.groups ints, zero before the first launch;
// every launch leaves them zero).  Calls sharing the buffers must not overlap.
struct SplitkPlan {
  int inst = 0, groups = 0, ks = 0, mt = 0, grid = 0;
};
bool gemv_splitk_plan(int m, int n, int nb, bool gated, int cus, SplitkPlan* plan);
size_t gemv_splitk_part_floats(const SplitkPlan& plan);
hipError_t launch_gemv_splitk(hipStream_t s, const GemvArgs& a, int dtype, const SplitkPlan& plan, float* part, int* counters);

// GEMV for m <= 48.
hipError_t launch_gemv(hipStream_t s, const GemvArgs& a, int dtype, const GemvShape& shape, bool gated);

hipError_t launch_gemm(hipStream_t s, const GemmArgs& a, int dtype);

// Pipelined GEMM: xh holds the activations staged in the GEMM order
// (kStageGemm) for gemm2_rows(m) rows; N a multiple of 256.
bool gemm2_supported(int m, int n);
int gemm2_rows(int m);
hipError_t launch_gemm2(hipStream_t s, const GemmArgs& a, int dtype, int cus);

// One MFMA-ceiling launch: `blocks` workgroups of 4 waves, each wave issuing
// 32 * iters v_mfma_f32_16x16x32_f16 (16384 FLOP each); out holds blocks * 256 floats.
hipError_t launch_mfma_ceiling(hipStream_t s, float* out, int blocks, int iters);

hipError_t launch_gather(hipStream_t s, const void* x, void* out, int k, int dtype, const GatherIndex& idx);

// Token embedding from a tiled Q4_K table (n rows of k): y[t] = row ids[t].
hipError_t launch_embedding(hipStream_t s, const uint8_t* w, const int32_t* ids, void* y, int rows, int n, int k, int dtype);

// RMS norm of `rows` rows of k (idx == nullptr: row r reads x row r;
// otherwise x row idx->src[r]).
hipError_t launch_rms_norm(hipStream_t s, const void* x, const float* w, void* y, int rows, int k, float eps, int dtype, const GatherIndex* idx);

// Device-side GGUF -> tiled re-layout (src and dst are device buffers).
hipError_t launch_relayout(hipStream_t s, const uint8_t* src, uint8_t* dst, uint32_t n, uint32_t k);

// Q6_K GEMV for m <= 8 rows: a.w = tiled Q6_K weights, a.pack = the decode
// pack of x (launch_stage_pack), post 0/1/2 on a.y / a.aux.
hipError_t launch_q6k_gemv(hipStream_t s, const GemvArgs& a, int dtype, int cus);

// Device-side GGUF -> tiled re-layout of block_q6_K weights.
hipError_t launch_q6k_relayout(hipStream_t s, const uint8_t* src, uint8_t* dst, uint32_t n, uint32_t k);

// ---- dispatch --------------------------------------------------------------
// Events attached to the calling thread's next kernel dispatches (both null
// unless launch profiling is on).  hipExtLaunchKernel stamps them with the
// dispatch's own begin and end times, so the measured duration is the
// kernel's execution (as a kernel-trace profiler reports it), without the
// host launch overhead that stream-ordered event records would include.
struct DispatchEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
DispatchEvents& dispatch_events();

template <typename... P, typename... A>
hipError_t dispatch(void (*kernel)(P...), dim3 grid, dim3 block, hipStream_t s, A... args) {
  const DispatchEvents& e = dispatch_events();
  hipExtLaunchKernelGGL(kernel, grid, block, 0, s, e.start, e.stop, 0, static_cast<P>(args)...);
  return hipGetLastError();
}

}  // namespace q4k
