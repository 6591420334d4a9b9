// Q4_K linear() kernels for gfx950 (MI355X / CDNA4), and the other GGUF
// weight types on the same surface.
//
//  stage_x_kernel, stage_gemm_kernel, stage_pack_kernel
//                   activations -> fp16 operands with power-of-two scales
//  q4k_gemv_kernel  staged decode GEMV (up to 48 rows), optionally gated
//  q4k_gemv_gate_up_kernel   fused gate/up decode GEMV, x packed in registers
//  q4k_gemv_splitk_kernel    split-K decode GEMV (K = 12288)
//  typed_gemv_kernel, typed_gemv_persistent_kernel, typed_gate_up_kernel
//                   decode GEMVs over a format policy (Q6_K, Q8_0, Q5_K,
//                   IQ4_XS; Q4_K for the wide LM head)
//  q4k_gemm2_kernel, typed_gemm_kernel
//                   pipelined prefill GEMMs on v_mfma_f32_16x16x32_f16
//  gather_rows_kernel, relayout_kernel, typed_relayout_kernel
//  embedding_kernel, embedding_batch_kernel, rms_norm_kernel
//                   the path's neighbours in a pass (token embedding
//                   gather-dequant, RMS norm / LM-head rms_norm_gather)
//
// Reference semantics: backend/metal/kernel/quant_linear.metal and
// backend/metal/kernel/fused_kernels.metal.
#include <float.h>
#include <hip/hip_runtime.h>
#include <stdlib.h>

#include "q4k_device.h"

namespace q4k {
namespace {

// ----------------------------------------------------------------------------
// Activation staging.  One workgroup per row.  Rows of up to 256 * 8 * kStageRegChunks
// elements are held in registers between the max reduction and the
// conversion (one read of x); longer rows are read twice.
// ----------------------------------------------------------------------------
constexpr int kStageRegChunks = 6;

__device__ __forceinline__ float block_max_256(float mx) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    mx = fmaxf(mx, __shfl_xor(mx, off));
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0)
    red[threadIdx.x >> 6] = mx;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Maximum of mx and sum of ss over the 256 threads (one barrier).
__device__ __forceinline__ void block_max_sum_256(float& mx, float& ss) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, off));
    ss += __shfl_xor(ss, off);
  }
  __shared__ float red[2][4];
  if ((threadIdx.x & 63) == 0) {
    red[0][threadIdx.x >> 6] = mx;
    red[1][threadIdx.x >> 6] = ss;
  }
  __syncthreads();
  mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  ss = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
}

// Fused RMS norm of a staged row (native_ops.metal:6-40): the staging
// kernels multiply each element by its weight w[k] as it is read, sum the
// squares of the unweighted elements, and fold rsqrt(sum / k + eps) into the
// power-of-two conversion scale.
struct RowNorm {
  const float* w = nullptr;
  float eps = 0.0f;
};

// Converts and stores one 8-element chunk; all 256 threads of the workgroup
// must call it together (the sub-block sum is reduced over 4 lanes).
template <int MODE>
__device__ __forceinline__ void stage_store(_Float16* xo, _Float16* xs, _Float16* xe, int row, int c, bool live, int m, int k, int nb,
                                            const float* v, float up) {
  h8_t hi, lo;
  float sum = 0.0f, res = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float t = v[i] * up;
    hi[i] = (_Float16)t;
    const float r = t - (float)hi[i];
    lo[i] = (_Float16)r;
    sum += t;
    res += r;
  }
  if (live) {
    *reinterpret_cast<h8_t*>(xo + frag_offset(row, c, nb)) = hi;
    if (MODE == kStageFragSplit)
      *reinterpret_cast<h8_t*>(xo + frag_offset(m + row, c, nb)) = lo;
  }
  // Chunks 4q..4q+3 (lanes 4q..4q+3) form one sub-block.
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  res += __shfl_xor(res, 1);
  res += __shfl_xor(res, 2);
  if (live && (c & 3) == 0) {
    const float s32 = sum * 0.03125f;
    const _Float16 sh = (_Float16)s32;
    const int b = c >> 5, j = (c >> 2) & 7;
    xs[xs_offset(row, b, j, nb)] = sh;
    if (MODE == kStageFragSplit)
      xs[xs_offset(m + row, b, j, nb)] = (_Float16)(s32 - (float)sh);
    // The sub-block's sum of fp16 rounding residuals (the mean-quant
    // correction's A operand; |.| <= 32 half-ulps of 2^15), zero for hi/lo
    // fragments, whose low parts carry the residuals.
    if (MODE == kStageFrag) {
      xe[xs_offset(row, b, j, nb)] = (_Float16)res;
    } else {
      xe[xs_offset(row, b, j, nb)] = (_Float16)0.0f;
      xe[xs_offset(m + row, b, j, nb)] = (_Float16)0.0f;
    }
  }
}

// Loads chunk c (8 elements) of row xr; with NORM, multiplies each element by
// its norm weight and adds the squares of the unweighted elements to ss.
template <bool NORM, typename InT>
__device__ __forceinline__ void load8_norm(const InT* xr, const float* nw, int c, float* v, float& ss) {
  load8(xr + (size_t)c * 8, v);
  if (NORM) {
    float w8[8];
    load8(nw + (size_t)c * 8, w8);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ss = fmaf(v[i], v[i], ss);
      v[i] *= w8[i];
    }
  }
}

template <typename InT, int MODE, bool NORM>
__global__ __launch_bounds__(256) void stage_x_kernel(const InT* __restrict__ x, _Float16* __restrict__ xo, _Float16* __restrict__ xs,
                                                      float* __restrict__ rowscale, int m, int k, RowNorm nrm) {
  const int row = blockIdx.x;
  const InT* xr = x + (size_t)row * k;
  const int chunks = k >> 3, nb = k >> 8;
  const bool in_regs = chunks <= 256 * kStageRegChunks;
  // The residual sums' plane follows the sub-block sums (of m rows, or 2m
  // for hi/lo fragments, whose residual sums are written as zeros).
  _Float16* const xe = xs + xs_plane_halves(MODE == kStageFragSplit ? 2 * m : m, nb);
  float v[kStageRegChunks][8] = {};
  float mx = 0.0f, ss = 0.0f;
  if (in_regs) {
#pragma unroll
    for (int j = 0; j < kStageRegChunks; ++j) {
      const int c = threadIdx.x + 256 * j;
      if (c < chunks) {
        load8_norm<NORM>(xr, nrm.w, c, v[j], ss);
#pragma unroll
        for (int i = 0; i < 8; ++i)
          mx = fmaxf(mx, fabsf(v[j][i]));
      }
    }
  } else {
    for (int c = threadIdx.x; c < chunks; c += 256) {
      float t[8];
      load8_norm<NORM>(xr, nrm.w, c, t, ss);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        mx = fmaxf(mx, fabsf(t[i]));
    }
  }
  float r = 1.0f;
  if (NORM) {
    block_max_sum_256(mx, ss);
    r = 1.0f / sqrtf(ss / (float)k + nrm.eps);
    mx *= r;
  } else {
    mx = block_max_256(mx);
  }
  float up, down;
  pow2_scale(mx, up, down);
  if (threadIdx.x == 0)
    rowscale[row] = down;
  const float cs = NORM ? up * r : up;
  if (in_regs) {
#pragma unroll
    for (int j = 0; j < kStageRegChunks; ++j) {
      const int c = threadIdx.x + 256 * j;
      if (256 * j < chunks)  // uniform: whole groups of 4 lanes take part
        stage_store<MODE>(xo, xs, xe, row, c, c < chunks, m, k, nb, v[j], cs);
    }
  } else {
    for (int c0 = 0; c0 < chunks; c0 += 256) {
      const int c = c0 + threadIdx.x;
      float t[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      float unused = 0.0f;
      if (c < chunks)
        load8_norm<NORM>(xr, nrm.w, c, t, unused);
      stage_store<MODE>(xo, xs, xe, row, c, c < chunks, m, k, nb, t, cs);
    }
  }
}

// ----------------------------------------------------------------------------
// Decode pack (m <= 8): x converted once into the MFMA operands of the
// persistent and per-item GEMVs, per 256-element block b:
//   frag[b][s][l]  16 B: A fragment s (v_mfma_f32_16x16x32_f16) of lane l =
//                  16g + i: elements 64g + 32 (s / 4) + 8 (s % 4) + [0, 8)
//                  of row i (i < 8: high fp16 parts, i >= 8: low parts of
//                  row i - 8; zero for rows >= m);
//   xs[b][l]       8 B: min-term A operand (v_mfma_f32_16x16x16_f16) of lane
//                  l = 16G + i: sub-block sums / 32 of sub-blocks 4G..4G+3
//                  (high / low parts as above; zero for G >= 2);
//   dsc[b][r]      float: unscale factor of row r in block b.
// Each (row, block) is scaled by a power of two that puts its largest
// magnitude in [2^14, 2^15); hi + lo carries about 22 significant bits.
// One 64-thread workgroup per (block, row); lane l holds elements 4l..4l+3.
// ----------------------------------------------------------------------------
// Packs the four elements v of lane l (elements 4l..4l+3 of row r of one
// block) into the block's fragments frag_b [8][64], min-term operands xs_b
// [64] and unscale factors dsc_b [8]; the 64 lanes of one wave call it
// together.  The pointers may be global or LDS.
__device__ __forceinline__ void pack_block_row(const float (&v)[4], int r, int l, u4_t* frag_b, h4_t* xs_b, float* dsc_b) {
  const float amax = max64_lanes(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  float up = 1.0f, down = 1.0f;
  if (amax > 0.0f && amax <= FLT_MAX) {
    int ex;
    frexpf(amax, &ex);
    ex = ex < -80 ? -80 : ex;
    up = ldexpf(1.0f, 15 - ex);
    down = ldexpf(1.0f, ex - 15);
  }
  const float t0 = v[0] * up, t1 = v[1] * up, t2 = v[2] * up, t3 = v[3] * up;
  const h2_t h01 = __builtin_bit_cast(h2_t, __builtin_amdgcn_cvt_pkrtz(t0, t1));
  const h2_t h23 = __builtin_bit_cast(h2_t, __builtin_amdgcn_cvt_pkrtz(t2, t3));
  const h2_t l01 = __builtin_bit_cast(h2_t, __builtin_amdgcn_cvt_pkrtz(t0 - (float)h01[0], t1 - (float)h01[1]));
  const h2_t l23 = __builtin_bit_cast(h2_t, __builtin_amdgcn_cvt_pkrtz(t2 - (float)h23[0], t3 - (float)h23[1]));
  // Element e = 4l: lane group g = e / 64, fragment s = 4 ((e / 32) & 1) +
  // (e / 8) & 3, half offset e & 7 (0 or 4).
  const int e = 4 * l, g = e >> 6, fs = 4 * ((e >> 5) & 1) + ((e >> 3) & 3), h0 = e & 7;
  uint2* fh = reinterpret_cast<uint2*>(reinterpret_cast<_Float16*>(frag_b + fs * 64 + 16 * g + r) + h0);
  uint2* fl = reinterpret_cast<uint2*>(reinterpret_cast<_Float16*>(frag_b + fs * 64 + 16 * g + r + 8) + h0);
  *fh = uint2{__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23)};
  *fl = uint2{__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23)};
  // Sub-block j = l / 8: eight lanes.
  const float sum = sum8_lanes((t0 + t1) + (t2 + t3));
  _Float16* xsh = reinterpret_cast<_Float16*>(xs_b);
  if ((l & 7) == 0) {
    const int j = l >> 3;
    const float s32 = sum * 0.03125f;
    const _Float16 sh = (_Float16)s32;
    xsh[(16 * (j >> 2) + r) * 4 + (j & 3)] = sh;
    xsh[(16 * (j >> 2) + r + 8) * 4 + (j & 3)] = (_Float16)(s32 - (float)sh);
  }
  if (r == 0 && l < 32)  // lanes 32..63 of the min-term operand
    xs_b[32 + l] = h4_t{(_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
  if (l == 0)
    dsc_b[r] = down;
}

// GEMM staging (kStageGemm) with 8 rows per workgroup: thread t converts row
// t / 32 of the workgroup's 8, chunks (8 elements) t % 32 + 32 j.  The 8
// rows' 16-byte pieces of one fragment lane group are one 128-byte line, so
// every line is written whole by one workgroup (row-per-workgroup staging
// leaves 8 workgroups, on different XCDs, writing 16 bytes of each line).
// TPR threads per row (32, or 64 for long rows: 512 threads per workgroup).
// CPT > 0: the row's K / (8 TPR) <= CPT chunks per thread stay in registers
// between the maximum and the conversion; CPT == 0: x is read twice.  With
// 64 threads per row the 8 pieces of a line come from 8 waves at different
// times, and lines left the L2 partly written (1.38 x the output bytes
// written at K = 12288): those rows pass their pieces through LDS, half of
// the chunks at a time, and 8 consecutive lanes then store each line whole.
// Reduction over the lanes of one staged row: lanes 0..31 and 32..63 of a
// wave are two rows (TPR = 32), or the whole wave is one (TPR = 64).
template <int TPR, bool MAX>
__device__ __forceinline__ float row_reduce(float v) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  v = op(v, dpp_f<kDppQuadSwap1>(v));
  v = op(v, dpp_f<kDppQuadSwap2>(v));
  v = op(v, dpp_f<kDppHalfMirror>(v));
  v = op(v, dpp_f<kDppRowMirror>(v));
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)), r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)), r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return TPR == 64 ? op(op(r0, r1), op(r2, r3)) : (threadIdx.x & 63) < 32 ? op(r0, r1) : op(r2, r3);
}

template <typename InT, int CPT, int TPR, bool NORM>
__global__ __launch_bounds__(8 * TPR) void stage_gemm_kernel(const InT* __restrict__ x, _Float16* __restrict__ xo, float* __restrict__ rowscale,
                                                             int m, int k, RowNorm nrm) {
  static_assert(TPR == 32 || TPR == 64, "one row per half wave or per wave");
  const int t = threadIdx.x, q = t & (TPR - 1);
  const int row = blockIdx.x * 8 + t / TPR;
  const bool live = row < m;
  const int nb = k >> 8, cpt = (k >> 3) / TPR;
  const InT* xr = x + (size_t)(live ? row : 0) * k;
  float v[CPT > 0 ? CPT : 1][8];
  float mx = 0.0f, ss = 0.0f;
#pragma unroll
  for (int j = 0; j < (CPT > 0 ? CPT : 1); ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      v[j][i] = 0.0f;
  if (CPT > 0) {
#pragma unroll
    for (int j = 0; j < CPT; ++j)
      if (live && j < cpt)
        load8_norm<NORM>(xr, nrm.w, q + TPR * j, v[j], ss);
#pragma unroll
    for (int j = 0; j < CPT; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        mx = fmaxf(mx, fabsf(v[j][i]));
  } else if (live) {
    for (int j = 0; j < cpt; ++j) {
      float w[8];
      load8_norm<NORM>(xr, nrm.w, q + TPR * j, w, ss);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        mx = fmaxf(mx, fabsf(w[i]));
    }
  }
  mx = row_reduce<TPR, true>(mx);
  float r = 1.0f;
  if (NORM) {
    r = 1.0f / sqrtf(row_reduce<TPR, false>(ss) / (float)k + nrm.eps);
    mx *= r;
  }
  float up, down;
  pow2_scale(mx, up, down);
  // Rows past m write nothing; with the LDS path their waves stay for its
  // barriers.
  if (!live && !(CPT > 0 && TPR == 64))
    return;
  if (q == 0 && live)
    rowscale[row] = down;
  const float cs = NORM ? up * r : up;
  auto put = [&](int j, const float* w) {
    h8_t h;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      h[i] = (_Float16)(w[i] * cs);
    *reinterpret_cast<h8_t*>(xo + gemm_frag_offset(row, q + TPR * j, nb)) = h;
  };
  if constexpr (CPT > 0 && TPR == 64) {
    // LDS piece (chunk, row of the 8) at 16 (8 chunk + row); CPT / 2 chunks
    // of every thread per half.
    constexpr int HALF = (CPT + 1) / 2;
    __shared__ __attribute__((aligned(16))) h8_t piece[HALF * TPR * 8];
    const int r8 = t / TPR;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      if (hf)
        __syncthreads();  // the first half's stores have read their pieces
#pragma unroll
      for (int jj = 0; jj < HALF; ++jj) {
        const int j = hf * HALF + jj;
        if (j < CPT && j < cpt) {
          h8_t h;
#pragma unroll
          for (int i = 0; i < 8; ++i)
            h[i] = (_Float16)(v[j][i] * cs);
          piece[(jj * TPR + q) * 8 + r8] = h;
        }
      }
      __syncthreads();
      // Thread t stores piece (chunk (t / 8) + 64 i of the half, row t % 8):
      // lanes 8c .. 8c + 7 write one whole line.
      const int pr = t & 7, pc = t >> 3;
      const int prow = blockIdx.x * 8 + pr;
#pragma unroll
      for (int i = 0; i < HALF; ++i) {
        const int jj = i, j = hf * HALF + jj, c = pc + TPR * j;
        if (j < CPT && j < cpt && prow < m)
          *reinterpret_cast<h8_t*>(xo + gemm_frag_offset(prow, c, nb)) = piece[(jj * TPR + pc) * 8 + pr];
      }
    }
  } else if (CPT > 0) {
#pragma unroll
    for (int j = 0; j < (CPT > 0 ? CPT : 1); ++j)
      if (j < cpt)
        put(j, v[j]);
  } else {
    for (int j = 0; j < cpt; ++j) {
      float w[8];
      float unused = 0.0f;
      load8_norm<NORM>(xr, nrm.w, q + TPR * j, w, unused);
      put(j, w);
    }
  }
}

template <typename InT>
__global__ __launch_bounds__(64) void stage_pack_kernel(const InT* __restrict__ x, u4_t* __restrict__ frag, h4_t* __restrict__ xs,
                                                        float* __restrict__ dsc, int m, int k) {
  const int b = blockIdx.x >> 3, r = blockIdx.x & 7, l = threadIdx.x;
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (r < m) {
    const InT* p = x + (size_t)r * k + (size_t)b * 256 + 4 * l;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v[e] = (float)p[e];
  }
  pack_block_row(v, r, l, frag + (size_t)b * 8 * 64, xs + (size_t)b * 64, dsc + (size_t)b * 8);
}

// ----------------------------------------------------------------------------
// GEMV (decode / small prefill / gated decode).
//
// Workgroup = W waves over T column tiles (16T output columns); the K blocks
// are split into W contiguous ranges, one per wave, and the partial sums are
// reduced through LDS.  Per tile-block a wave issues three fully contiguous
// 16-byte loads per lane (two quant slabs + header) and, per 16-row tile of
// activations, 8 MFMAs with B = q*sc (exact fp16) plus one 16x16x16 MFMA of
// the sub-block sums against 32*m_j, then acc += d * C_q - dmin * C_m in fp32
// -- the decode form of quant_linear.metal:288-302 with the integer parts on
// the matrix core.
// ----------------------------------------------------------------------------
template <int T, int NM>
struct TileWords {
  u4_t q0[NM][T], q1[NM][T], hd[NM][T];
};

template <int T, int NM>
__device__ __forceinline__ void load_tile_words(TileWords<T, NM>& tw, const GemvArgs& a, int ct0, int b, int nb, int lane, int col) {
#pragma unroll
  for (int mi = 0; mi < NM; ++mi)
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint8_t* p = (mi ? a.wu : a.w) + ((size_t)(ct0 + t) * nb + b) * kTileBlockBytes;
      tw.q0[mi][t] = *reinterpret_cast<const u4_t*>(p + 16 * lane);
      tw.q1[mi][t] = *reinterpret_cast<const u4_t*>(p + kSlabBytes + 16 * lane);
      tw.hd[mi][t] = *reinterpret_cast<const u4_t*>(p + kHeaderOffset + 16 * col);
    }
}

// BPW > 0: every wave owns exactly BPW blocks (nb == W * BPW) and issues all of
// their weight loads at once; BPW == 0: any split, with a one-block prefetch.
template <int RT, int T, int W, int BPW, bool GATED, typename OutT>
__global__ __launch_bounds__(64 * W) void q4k_gemv_kernel(GemvArgs a) {
  constexpr int NM = GATED ? 2 : 1;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, col = lane & 15;
  const int nb = a.nb;
  const int ct0 = blockIdx.x * T;
  const int b0 = nb * wave / W, b1 = nb * (wave + 1) / W;

  f4_t acc[NM][T][RT];
#pragma unroll
  for (int mi = 0; mi < NM; ++mi)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
        acc[mi][t][rt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // Dead activation rows (>= a.rows, inside the padded 16-row tiles) are
  // loaded unmasked: in a matrix product a garbage A row only reaches its own
  // C row, which the epilogue never reads.  Branch-free loads keep the vmcnt
  // waits exact.
  // The min-term operand: lanes 0..31 the sub-block sums / 32, lanes 32..63
  // (k = 8..15) the sub-blocks' sums of fp16 rounding residuals from the
  // plane after them (zeros for hi/lo rows), as in the rows GEMV.
  const h4_t* const xsrc = reinterpret_cast<const h4_t*>(a.xs + (lane >= 32 ? xs_plane_halves(a.rows, nb) : 0));
  auto load_x = [&](h8_t (&xa)[RT][8], h4_t (&xsa)[RT], int b) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const h8_t* xp = reinterpret_cast<const h8_t*>(a.xf) + (size_t)(rt * nb + b) * 8 * 64 + lane;
#pragma unroll
      for (int s = 0; s < 8; ++s)
        xa[rt][s] = xp[s * 64];
      xsa[rt] = xsrc[(size_t)(rt * nb + b) * 32 + (lane & 31)];
    }
  };
  auto compute = [&](const TileWords<T, NM>& cur, const h8_t (&xa)[RT][8], const h4_t (&xsa)[RT]) {
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const BlockConsts kc = block_consts(cur.hd[mi][t], g);
        f4_t cq[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          cq[rt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const u4_t q = u < 2 ? cur.q0[mi][t] : cur.q1[mi][t];
          const uint32_t wa = q[2 * (u & 1)], wb = q[2 * (u & 1) + 1];
          const h8_t blo = quant_times_scale(wa, wb, 0x000F000Fu, 0x64006400u, kc.mul_lo, kc.add_lo);
          const h8_t bhi = quant_times_scale(wa, wb, 0x00F000F0u, 0x64006400u, kc.mul_hi, kc.add_hi);
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            cq[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[rt][u], blo, cq[rt], 0, 0, 0);
            cq[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[rt][4 + u], bhi, cq[rt], 0, 0, 0);
          }
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          // mean-quant correction of the fp16 rounding (k = 8 + j; single
          // fp16 rows, m >= 25, need at least two row tiles: one holds only
          // hi/lo rows), then the min term: sum_j (xs_j / 32) * (32 m_j)
          if constexpr (RT >= 2)
            cq[rt] = __builtin_amdgcn_mfma_f32_16x16x16f16(xsa[rt], kc.bsc, cq[rt], 0, 0, 0);
          const f4_t cm = __builtin_amdgcn_mfma_f32_16x16x16f16(xsa[rt], kc.bmin, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 4; ++v)
            acc[mi][t][rt][v] = fmaf(kc.d, cq[rt][v], fmaf(-kc.dmin, cm[v], acc[mi][t][rt][v]));
        }
      }
  };

  if constexpr (BPW > 0) {
    // Issue order for the in-order vmcnt counter: block 0's activations, all
    // BPW blocks' weights, then each later block's activations just in time.
    TileWords<T, NM> tw[BPW];
    h8_t xa[RT][8];
    h4_t xsa[RT];
    load_x(xa, xsa, b0);
#pragma unroll
    for (int j = 0; j < BPW; ++j)
      load_tile_words(tw[j], a, ct0, b0 + j, nb, lane, col);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
      if (j > 0)
        load_x(xa, xsa, b0 + j);
      compute(tw[j], xa, xsa);
    }
  } else {
    TileWords<T, NM> cur, next;
    if (b0 < b1)
      load_tile_words(cur, a, ct0, b0, nb, lane, col);
    for (int b = b0; b < b1; ++b) {
      h8_t xa[RT][8];
      h4_t xsa[RT];
      load_x(xa, xsa, b);
      __builtin_amdgcn_sched_barrier(0);
      if (b + 1 < b1)
        load_tile_words(next, a, ct0, b + 1, nb, lane, col);
      __builtin_amdgcn_sched_barrier(0);
      compute(cur, xa, xsa);
      cur = next;
    }
  }

  // Cross-wave reduction through LDS in [wave][matrix][tile][row][column]
  // order (the C fragment of lane l is rows 4*(l/16)+v, column l%16).
  constexpr int ROWS = RT * 16;
  __shared__ float red[W][NM][T][ROWS][16];
#pragma unroll
  for (int mi = 0; mi < NM; ++mi)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          red[wave][mi][t][rt * 16 + 4 * g + v][col] = acc[mi][t][rt][v];
  __syncthreads();

  // Epilogue: one thread per output (row, column); split rows add their low half.
  OutT* y = reinterpret_cast<OutT*>(a.y);
  const OutT* aux = reinterpret_cast<const OutT*>(a.aux);
  for (int item = tid; item < a.m * 16 * T; item += 64 * W) {
    const int row = item / (16 * T), c = item % (16 * T), t = c >> 4, cc = c & 15;
    float s[NM];
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < W; ++w)
        v += red[w][mi][t][row][cc];
      if (a.split) {
#pragma unroll
        for (int w = 0; w < W; ++w)
          v += red[w][mi][t][a.m + row][cc];
      }
      s[mi] = v;
    }
    const float scale = a.rowscale[row];
    const size_t o = (size_t)row * a.n + (size_t)(ct0 + t) * 16 + cc;
    float out;
    if (GATED) {
      float gv = s[0] * scale, uv = s[NM - 1] * scale;
      if (sizeof(OutT) == 2) {
        gv = round_half(gv);
        uv = round_half(uv);
      }
      out = silu(gv) * uv;
    } else {
      float acc_v = s[0] * scale;
      if (sizeof(OutT) == 2)
        acc_v = round_half(acc_v);
      out = a.post == 1 ? acc_v + load_elem(aux, o) : a.post == 2 ? silu(load_elem(aux, o)) * acc_v : acc_v;
    }
    store_elem(y, o, out);
  }
}

// ----------------------------------------------------------------------------
// Load helpers of the GEMVs that stream weights through LDS.
// ----------------------------------------------------------------------------

// ----------------------------------------------------------------------------
// Fused gate/up GEMV with in-register activation packing (m <= 8 rows, K =
// 4096, N = 16 T x workgroups: one item of T column tiles per workgroup).
//
// Wave w owns K-blocks bw, bw + 1 (bw = 2 ((w + b) % 8), rotated so that the
// workgroups of one L2 read different parts of x first) of the workgroup's T
// column tiles of both matrices: U = 4T tile-blocks ("units").  It loads its
// two blocks of x (one coalesced 1 KB load per (block, row)), then keeps two
// units in flight ahead of the pair it computes (per unit the 16-byte header
// row of the lane's column and the two quant slabs, 16 B per lane).  No
// staging launch precedes it: while
// the first units are in flight the wave turns its blocks of x into the MFMA
// operands in registers, with the same arithmetic as the decode pack
// (pack_block_row):
//  - x passes through LDS so that lane 16g + i holds elements
//    64g + 32 (i / 8) + [0, 32) of row i % 8 (rows >= m read as zero);
//  - each (row, block) is scaled by a power of two that puts its largest
//    magnitude in [2^14, 2^15) and split into hi = h(t), lo = h(t - hi);
//  - lanes i and i ^ 8 (one DPP row rotation) trade halves so that lanes
//    i < 8 hold the high parts of elements 64g + [0, 64) of row i and lanes
//    i >= 8 the low parts: the A fragments of v_mfma_f32_16x16x32_f16, rows
//    8..15 carrying the low parts;
//  - each lane's 32 elements are one sub-block; their sums / 32 (hi / lo)
//    are gathered into the min-term operand of v_mfma_f32_16x16x16_f16.
// Units are computed two at a time, their instruction streams interleaved.
// The partial sums of a unit are unscaled and accumulated in registers; hi
// and lo rows are combined (lanes l, l + 32) and the eight waves' sums are
// added in wave order through LDS before the SiLU(gate) * up epilogue.  The
// kernel is bound by its vector ALU: about 135 VALU instructions per unit
// and 500 for the pack, two waves per SIMD.
// ----------------------------------------------------------------------------
constexpr int kDppRowRor8 = 0x128;  // lane i <- lane (i + 8) % 16 within 16 lanes

template <int BANKS>
__device__ __forceinline__ uint32_t ror8_into(uint32_t old, uint32_t src) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)src, kDppRowRor8, 0xF, BANKS, false);
}

// Registers of one packed x block: A fragments, min-term operand and the
// unscale factors of this lane's C rows (4g + v) & 7.
struct XBlock {
  h8_t frag[8];
  h4_t xs;
  float dv[4];
};

// Converts the 32 values t0 (elements 64g + 32 (i / 8) + [0, 32) of row i % 8,
// lane 16g + i) of one block into the block's operands.
__device__ __forceinline__ void pack_x_regs(const float (&xv)[32], int lane, XBlock& xb) {
  const int g = lane >> 4, i = lane & 15, half = i >> 3;
  // Largest magnitude of the (row, block): own 32, the partner half, the four
  // lane groups.
  float mx = 0.0f;
#pragma unroll
  for (int e = 0; e < 32; ++e)
    mx = fmaxf(mx, fabsf(xv[e]));
  mx = fmaxf(mx, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, mx), kDppRowRor8, 0xF, 0xF, false)));
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  float up = 1.0f, down = 1.0f;
  if (mx > 0.0f && mx <= FLT_MAX) {
    int ex;
    frexpf(mx, &ex);
    ex = ex < -80 ? -80 : ex;
    up = ldexpf(1.0f, 15 - ex);
    down = ldexpf(1.0f, ex - 15);
  }
  uint32_t hw[16], lw[16];
  float sum = 0.0f;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const float t0 = xv[2 * v] * up, t1 = xv[2 * v + 1] * up;
    sum += t0 + t1;
    const h2_t h = __builtin_bit_cast(h2_t, __builtin_amdgcn_cvt_pkrtz(t0, t1));
    hw[v] = __builtin_bit_cast(uint32_t, h);
    lw[v] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(t0 - (float)h[0], t1 - (float)h[1]));
  }
  // Fragments 0..3 (elements 64g + [0, 32)): own high parts in lanes i < 8,
  // the partner's low parts in lanes i >= 8 (banks 2, 3 take the rotation).
  // Fragments 4..7 (64g + [32, 64)): the partner's high parts in lanes i < 8,
  // own low parts in lanes i >= 8.
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    u4_t f0, f1;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      f0[v] = ror8_into<0xC>(hw[4 * s + v], lw[4 * s + v]);
      f1[v] = ror8_into<0x3>(lw[4 * s + v], hw[4 * s + v]);
    }
    xb.frag[s] = __builtin_bit_cast(h8_t, f0);
    xb.frag[4 + s] = __builtin_bit_cast(h8_t, f1);
  }
  // Sub-block sums / 32 as (hi, lo) halves; lane 16G + r (G < 2) gathers
  // sub-blocks 4G + c (c = 0..3) of row r % 8 from lanes 16 (2G + c / 2) +
  // r % 8 + 8 (c % 2), taking the high halves for r < 8 and the low for r >= 8.
  const float s32 = sum * 0.03125f;
  const _Float16 sh = (_Float16)s32;
  const _Float16 sl = (_Float16)(s32 - (float)sh);
  const uint32_t shl = (uint32_t)__builtin_bit_cast(uint16_t, sh) | ((uint32_t)__builtin_bit_cast(uint16_t, sl) << 16);
  const int G = g & 1, r8 = i & 7;
  uint32_t got[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    got[c] = (uint32_t)__shfl((int)shl, 16 * (2 * G + (c >> 1)) + r8 + 8 * (c & 1));
  const uint32_t sel = half ? 0x07060302u : 0x05040100u;  // low or high halves of a pair of dwords
  const uint32_t x01 = __builtin_amdgcn_perm(got[1], got[0], sel), x23 = __builtin_amdgcn_perm(got[3], got[2], sel);
  xb.xs = g < 2 ? __builtin_bit_cast(h4_t, uint2{x01, x23}) : h4_t{(_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
  // Unscale factors of C rows 4 (g & 1) + v (the same in every lane of a row).
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float d0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, down), v));
    const float d1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, down), 4 + v));
    xb.dv[v] = (g & 1) ? d1 : d0;
  }
}

// x of wave w, re-ordered for the register pack: [block][lane][32 + 4]
// floats (the 4-float pad makes the 16-byte reads of 16 lanes hit 64
// distinct banks), BPW blocks per wave.  The partial sums reuse the wave's
// own region at the end.
constexpr int kGuXRow = 36;
template <int BPW>
constexpr int gu_wave_floats() {
  return BPW * 64 * kGuXRow;
}

// The x of one item of the fused gate/up GEMV, packed: wave w loads K-blocks
// bw, bw + 1 of all 8 rows (one coalesced load per (block, row), lane l
// holding elements 4l..4l+3; rows >= m read row 0 and are zeroed), calls
// issue_first() once its x has landed, and turns its blocks into MFMA
// operands in registers (through its LDS region).  NORM: x
// is RMS-normalised on the way in (native_ops.metal:6-40, the norm
// forward.cpp:114 applies before the MLP): the 8 waves hold all of x between
// them, so each row's sum of squares is their partial sums (ssq [wave][row])
// added after one barrier, and every element becomes
// (x * rsqrt(sum / k + eps)) * w before the pack.
template <typename OutT, bool NORM, int W, int BPW, typename Issue>
__device__ __forceinline__ void gate_up_pack_x(const GemvArgs& a, float* xl, float (*ssq)[8], int bw, XBlock (&xb)[BPW],
                                               Issue&& issue_first) {
  constexpr int kXRow = kGuXRow;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  float xv[BPW][8][4];
#pragma unroll
  for (int j = 0; j < BPW; ++j)
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const OutT* p = reinterpret_cast<const OutT*>(a.x) + (size_t)(r < a.m ? r : 0) * a.k + (size_t)(bw + j) * 256 + 4 * lane;
      if (sizeof(OutT) == 4) {
        const f4_t v4 = *reinterpret_cast<const f4_t*>(p);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          xv[j][r][e] = v4[e];
      } else {
        const h4_t v4 = *reinterpret_cast<const h4_t*>(p);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          xv[j][r][e] = (float)v4[e];
      }
    }
  f4_t nw[BPW];
  if constexpr (NORM) {
#pragma unroll
    for (int j = 0; j < BPW; ++j)
      nw[j] = *reinterpret_cast<const f4_t*>(a.norm_w + (size_t)(bw + j) * 256 + 4 * lane);
  }
  __builtin_amdgcn_sched_barrier(0);

  if constexpr (NORM) {
    float ss[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      ss[r] = 0.0f;
#pragma unroll
      for (int j = 0; j < BPW; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          ss[r] = fmaf(xv[j][r][e], xv[j][r][e], ss[r]);
#pragma unroll
      for (int off = 32; off > 0; off >>= 1)
        ss[r] += __shfl_xor(ss[r], off);
    }
    if (lane < 8) {
      float v = ss[0];
#pragma unroll
      for (int r = 1; r < 8; ++r)
        v = lane == r ? ss[r] : v;
      ssq[wave][lane] = v;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      float tot = 0.0f;
#pragma unroll
      for (int w = 0; w < W; ++w)
        tot += ssq[w][r];
      const float scale = 1.0f / sqrtf(tot / (float)a.k + a.eps);
#pragma unroll
      for (int j = 0; j < BPW; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          xv[j][r][e] = (xv[j][r][e] * scale) * nw[j][e];
    }
  }
  // Element e = 4 lane of row r goes to pack lane 16 (e / 64) + r + 8 ((e / 32) & 1),
  // float (e & 31) of its 32.
  float* const xw = xl + (size_t)wave * gu_wave_floats<BPW>();
  const int dl = 16 * (lane >> 4) + 8 * ((lane >> 3) & 1), doff = 4 * (lane & 7);
#pragma unroll
  for (int j = 0; j < BPW; ++j)
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      f4_t v4;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v4[e] = r < a.m ? xv[j][r][e] : 0.0f;
      *reinterpret_cast<f4_t*>(xw + (j * 64 + dl + r) * kXRow + doff) = v4;
    }
  // The first weight loads go out once x has landed, not with it: issued
  // together, every wave's first units queue ahead of the x of later
  // workgroups (measured: kernel 15.0 against 15.6 us at config 1).  The
  // LDS transposition and the register pack below run under them.
  __builtin_amdgcn_sched_barrier(0);
  issue_first();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
    float t32[32];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const f4_t v4 = *reinterpret_cast<const f4_t*>(xw + (j * 64 + lane) * kXRow + 4 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        t32[4 * c + e] = v4[e];
    }
    pack_x_regs(t32, lane, xb[j]);
  }
}

// The end of an item: C row 4g + v of each (matrix, tile) pair, lanes g < 2
// adding the low part held 32 lanes up, goes to the wave's LDS region; the
// eight waves' sums are added in wave order and SiLU(gate) * up is stored.
template <int T, typename OutT, int W, int BPW>
__device__ __forceinline__ void gate_up_finish(const GemvArgs& a, float* xl, const f4_t (&acc)[2 * T], int item) {
  constexpr int MT = 2 * T, WF = gu_wave_floats<BPW>();
  static_assert(MT * 8 * 16 <= WF, "partials fit the x region");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, col = lane & 15;
  float* const xw = xl + (size_t)wave * WF;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float tot = acc[mt][v] + __shfl_xor(acc[mt][v], 32);
      if (g < 2)
        xw[(mt * 8 + 4 * g + v) * 16 + col] = tot;
    }
  __syncthreads();
  OutT* y = reinterpret_cast<OutT*>(a.y);
  constexpr int EPI = 16 * T;
  for (int o = tid; o < a.m * EPI; o += 64 * W) {
    const int row = o / EPI, c = o % EPI, t = c >> 4, cc = c & 15;
    float gv = 0.0f, uv = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      gv += xl[w * WF + (t * 8 + row) * 16 + cc];
      uv += xl[w * WF + ((T + t) * 8 + row) * 16 + cc];
    }
    if (sizeof(OutT) == 2) {
      gv = round_half(gv);
      uv = round_half(uv);
    }
    store_elem(y, (size_t)row * a.n + ((size_t)item * T + t) * 16 + cc, silu(gv) * uv);
  }
}

// One item (T column tiles of both matrices) of the fused gate/up GEMV, by the
// 8 waves of the workgroup.
template <int T, typename OutT, bool NORM, int W, int BPW>
__device__ __forceinline__ void gate_up_item(const GemvArgs& a, float* xl, float (*ssq)[8], int item) {
  constexpr int NM = 2, MT = NM * T, U = BPW * MT;
  static_assert(W * BPW == 16, "the waves cover the 16 blocks of K = 4096");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, col = lane & 15;
  const int nb = a.nb, bw = ((wave + item) % W) * BPW;
  const size_t tile_bytes = (size_t)nb * kTileBlockBytes;

  // Units are loaded into registers DQ ahead of the one being computed
  // (header dword, then the two quant slabs; the scheduling barriers keep
  // the issue order: x first, then unit by unit, the first units once x has
  // landed).  A shallow window keeps the memory queues short, so x and each
  // wave's next unit arrive early; issuing more units ahead measured slower
  // (they queue ahead of the x of later workgroups).
  // Units are loaded into registers two ahead of the pair being computed:
  // the header row of the lane's own column (16 bytes; four lanes share
  // one row), then the two quant slabs.  The scheduling barriers keep the
  // issue order: x first, then unit by unit, the first units once x has
  // landed.  A shallow window keeps the memory queues short, so x and each
  // wave's next units arrive early (deeper windows measured no faster).
  constexpr int DQ = 2;
  static_assert(U % 2 == 0 && MT % 2 == 0, "pairs of units within one block");
  u4_t hdr[U], q0[U], q1[U];
  auto issue_unit = [&](int u) {
    const int j = u / MT, mt = u - j * MT, mi = mt / T, t = mt - mi * T;
    const uint8_t* src = (mi ? a.wu : a.w) + ((size_t)item * T + t) * tile_bytes + (size_t)(bw + j) * kTileBlockBytes;
    hdr[u] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src + kHeaderOffset) + col);
    q0[u] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src) + lane);
    q1[u] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src + kSlabBytes) + lane);
    __builtin_amdgcn_sched_barrier(0);
  };
  XBlock xb[BPW];
  gate_up_pack_x<OutT, NORM, W, BPW>(a, xl, ssq, bw, xb, [&] {
#pragma unroll
    for (int u = 0; u < (DQ < U ? DQ : U); ++u)
      issue_unit(u);
  });

  f4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    acc[mt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
  // Two units per step, their instruction streams interleaved: the block
  // constants, nibble decode, MFMA chains and accumulator updates of two
  // independent tile-blocks of one K-block.  Units 2p + 2, 2p + 3 are
  // loaded during step p.
#pragma unroll
  for (int p = 0; p < U / 2; ++p) {
    const int u0 = 2 * p, j = u0 / MT, mt0 = u0 - j * MT;
    __builtin_amdgcn_sched_barrier(0);
    if (u0 + DQ < U) {
      issue_unit(u0 + 2);
      issue_unit(u0 + 3);
    }
    BlockConsts kc[2];
#pragma unroll
    for (int e = 0; e < 2; ++e)
      kc[e] = block_consts(hdr[u0 + e], g);
    f4_t cl[2], ch[2], cm[2];
#pragma unroll
    for (int e = 0; e < 2; ++e)
      cl[e] = ch[e] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const u4_t qq = s < 2 ? q0[u0 + e] : q1[u0 + e];
        const uint32_t wa = qq[2 * (s & 1)], wb = qq[2 * (s & 1) + 1];
        const h8_t blo = quant_times_scale(wa, wb, 0x000F000Fu, 0x64006400u, kc[e].mul_lo, kc[e].add_lo);
        const h8_t bhi = quant_times_scale(wa, wb, 0x00F000F0u, 0x64006400u, kc[e].mul_hi, kc[e].add_hi);
        cl[e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xb[j].frag[s], blo, cl[e], 0, 0, 0);
        ch[e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xb[j].frag[4 + s], bhi, ch[e], 0, 0, 0);
      }
#pragma unroll
    for (int e = 0; e < 2; ++e)
      cm[e] = __builtin_amdgcn_mfma_f32_16x16x16f16(xb[j].xs, kc[e].bmin, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        acc[mt0 + e][v] += fmaf(kc[e].d, cl[e][v] + ch[e][v], -kc[e].dmin * cm[e][v]) * xb[j].dv[v];
  }
  gate_up_finish<T, OutT, W, BPW>(a, xl, acc, item);
}

template <int T, typename OutT, bool NORM, int W>
__global__ __launch_bounds__(64 * W) void q4k_gemv_gate_up_kernel(GemvArgs a) {
  constexpr int BPW = 16 / W;
  __shared__ __attribute__((aligned(16))) float xl[W * gu_wave_floats<BPW>()];
  __shared__ float ssq[W][8];
  gate_up_item<T, OutT, NORM, W, BPW>(a, xl, ssq, blockIdx.x);
}

// ----------------------------------------------------------------------------
// GEMV for staged activations of 17..48 fragment rows (the decode pass of a
// speculative batch, up to 8 queries x 5 rows), K = 2048 .. 12288.
//
// The work split of the fused gate/up GEMV over the staged fp16 fragments
// (stage_x_kernel, one power-of-two scale per row; split rows carry the low
// parts) of the RT row tiles: workgroup = one item of T column tiles of NM
// matrices (NM = 2: gate and up), 8 waves; wave w owns K-blocks bw ..
// bw + BPW - 1 (bw = BPW ((w + item) % 8)) of the item's NM T (matrix, tile)
// pairs, U = BPW NM T units.  The wave loads a block's fragments for all RT
// row tiles once (RT x 8 KB from the staging) and every unit of that block
// multiplies them: RT x 8 v_mfma_f32_16x16x32_f16 and RT min-term MFMAs per
// tile-block dequantised once.  A CU thus reads the staged x once per T
// column tiles of NM matrices; the one-tile GEMV reads it once per column
// tile, and at M = 40 its gated launch was bound by those reads (768
// workgroups x 384 KB).  Units stream two ahead as in the fused gate/up
// GEMV; a block's fragments replace the previous block's after its units
// (one L2 round trip per block and wave, which the SIMD's other wave
// covers).  The 8 waves' partial sums meet in LDS in wave order.
// KS > 1 K-slices: workgroup b takes slice b % KS (blocks 8 BPW of them) of
// column group b / KS, so that KS times fewer column groups, each of KS
// times more column tiles, read all of x; each slice's workgroup writes its
// sums (written through to memory) and the last of the KS to arrive (a
// per-group counter, reset by it) adds them in slice order and runs the
// epilogue.  No workgroup waits for another.
// ----------------------------------------------------------------------------
template <int NM, int T, int RT, int BPW, typename OutT, int KS = 1>
__global__ __launch_bounds__(512) void q4k_gemv_rows_kernel(GemvArgs a) {
  constexpr int W = 8, MT = NM * T, U = BPW * MT, ROWS = 16 * RT, DQ = 2;
  __shared__ float red[W][MT][ROWS][16];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, col = lane & 15;
  const int item = blockIdx.x / KS, ks = blockIdx.x % KS, nb = a.nb;
  const int bw = ks * (W * BPW) + BPW * ((wave + item) % W);
  const size_t tile_bytes = (size_t)nb * kTileBlockBytes;

  u4_t hdr[U], q0[U], q1[U];
  auto issue_unit = [&](int u) {
    const int j = u / MT, mt = u - j * MT, mi = mt / T, t = mt - mi * T;
    const uint8_t* src = (mi ? a.wu : a.w) + ((size_t)item * T + t) * tile_bytes + (size_t)(bw + j) * kTileBlockBytes;
    hdr[u] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src + kHeaderOffset) + col);
    q0[u] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src) + lane);
    q1[u] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src + kSlabBytes) + lane);
    __builtin_amdgcn_sched_barrier(0);
  };
  // Dead fragment rows (>= a.rows inside the last row tile) are loaded as
  // they are: a garbage A row reaches only its own C row, never stored.
  h8_t xa[RT][8];
  // The min-term MFMA's A operand: lanes 0..31 (k = 0..7) the sub-block sums
  // / 32; lanes 32..63 (k = 8..15) the sub-blocks' sums of fp16 rounding
  // residuals, from the plane after the sums that stage_x_kernel writes
  // (zeros for hi/lo fragments).  Each of the two MFMAs that read it has a
  // zero B operand for the other half's k.
  h4_t xsa[RT];
  const h4_t* const xsrc = reinterpret_cast<const h4_t*>(a.xs + (lane >= 32 ? xs_plane_halves(a.rows, nb) : 0));
  auto load_x = [&](int b) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const h8_t* xp = reinterpret_cast<const h8_t*>(a.xf) + (size_t)(rt * nb + b) * 8 * 64 + lane;
#pragma unroll
      for (int s = 0; s < 8; ++s)
        xa[rt][s] = xp[s * 64];
      xsa[rt] = xsrc[(size_t)(rt * nb + b) * 32 + (lane & 31)];
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  load_x(bw);
#pragma unroll
  for (int u = 0; u < (DQ < U ? DQ : U); ++u)
    issue_unit(u);

  f4_t acc[MT][RT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
      acc[mt][rt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int j = u / MT, mt = u - j * MT;
    __builtin_amdgcn_sched_barrier(0);
    if (u > 0 && mt == 0)
      load_x(bw + j);
    if (u + DQ < U)
      issue_unit(u + DQ);
    const BlockConsts kc = block_consts(hdr[u], g);
    f4_t cq[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
      cq[rt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u4_t qq = s < 2 ? q0[u] : q1[u];
      const uint32_t wa = qq[2 * (s & 1)], wb = qq[2 * (s & 1) + 1];
      const h8_t blo = quant_times_scale(wa, wb, 0x000F000Fu, 0x64006400u, kc.mul_lo, kc.add_lo);
      const h8_t bhi = quant_times_scale(wa, wb, 0x00F000F0u, 0x64006400u, kc.mul_hi, kc.add_hi);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        cq[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[rt][s], blo, cq[rt], 0, 0, 0);
        cq[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[rt][4 + s], bhi, cq[rt], 0, 0, 0);
      }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      // Mean-quant correction of the fp16 rounding: sum_j E_j * 7.5 sc_j
      // (k = 8 + j), E_j = the sub-block's sum of rounding residuals: the
      // part of the q-term's error common to every column.
      if constexpr (RT >= 2)
        cq[rt] = __builtin_amdgcn_mfma_f32_16x16x16f16(xsa[rt], kc.bsc, cq[rt], 0, 0, 0);
      // min term: sum_j (xs_j / 32) * (32 m_j), k = sub-block
      const f4_t cm = __builtin_amdgcn_mfma_f32_16x16x16f16(xsa[rt], kc.bmin, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
      for (int v = 0; v < 4; ++v)
        acc[mt][rt][v] = fmaf(kc.d, cq[rt][v], fmaf(-kc.dmin, cm[v], acc[mt][rt][v]));
      // Each unit's sums are folded here: otherwise the compiler defers the
      // folds and keeps every unit's MFMA results live.
      asm volatile("" : "+v"(acc[mt][rt]));
    }
  }

  // C fragment of lane l: rows 4 (l / 16) + v of each row tile, column l % 16.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        red[wave][mt][rt * 16 + 4 * g + v][col] = acc[mt][rt][v];
  __syncthreads();
  OutT* y = reinterpret_cast<OutT*>(a.y);
  const OutT* aux = reinterpret_cast<const OutT*>(a.aux);
  constexpr int EPI = 16 * T;
  // This workgroup's sum of output o (row o / EPI, column o % EPI) of
  // matrix mi: the waves in order, then (split rows) the low parts.
  auto wave_sum = [&](int o, int mi) {
    const int row = o / EPI, c = o % EPI, t = c >> 4, cc = c & 15;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w)
      v += red[w][mi * T + t][row][cc];
    if (a.split) {
#pragma unroll
      for (int w = 0; w < W; ++w)
        v += red[w][mi * T + t][a.m + row][cc];
    }
    return v;
  };
  // K-slices: outputs of slice k2 of matrix mi at part + ((item KS + k2) NM
  // + mi) ROWS EPI + o.  Per thread at most PER outputs (o = tid + 512 r).
  constexpr int PER = (ROWS * EPI + 64 * W - 1) / (64 * W);
  float sl[PER][NM];
  if constexpr (KS > 1) {
    float* const mine = a.part + ((size_t)item * KS + ks) * NM * ROWS * EPI;
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int o = tid + r * 64 * W;
      if (o < a.m * EPI) {
#pragma unroll
        for (int mi = 0; mi < NM; ++mi)
          store_coherent(mine + mi * ROWS * EPI + o, wave_sum(o, mi));
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0)
      s_last = count_arrival(&a.counters[item]) == KS - 1;
    __syncthreads();
    if (!s_last)
      return;
    // Every slice's sums, loaded together, then added in slice order.
    float pv[PER][NM][KS];
    const float* const grp = a.part + (size_t)item * KS * NM * ROWS * EPI;
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int o0 = tid + r * 64 * W, o = o0 < a.m * EPI ? o0 : 0;
#pragma unroll
      for (int mi = 0; mi < NM; ++mi)
#pragma unroll
        for (int k2 = 0; k2 < KS; ++k2)
          pv[r][mi][k2] = load_coherent(grp + (k2 * NM + mi) * ROWS * EPI + o);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int r = 0; r < PER; ++r)
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) {
        float v = 0.0f;
#pragma unroll
        for (int k2 = 0; k2 < KS; ++k2) {
          hold(pv[r][mi][k2]);
          v += pv[r][mi][k2];
        }
        sl[r][mi] = v;
      }
    if (tid == 0)
      reset_counter(&a.counters[item]);  // ready for the next launch
  }
#pragma unroll
  for (int r = 0; r < PER; ++r) {
    const int o = tid + r * 64 * W;
    if (o >= a.m * EPI)
      break;
    const int row = o / EPI, c = o % EPI, t = c >> 4, cc = c & 15;
    float s[NM];
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
      s[mi] = (KS > 1 ? sl[r][mi] : wave_sum(o, mi)) * a.rowscale[row];
    const size_t off = (size_t)row * a.n + ((size_t)item * T + t) * 16 + cc;
    float out;
    if (NM == 2) {
      float gv = s[0], uv = s[NM - 1];
      if (sizeof(OutT) == 2) {
        gv = round_half(gv);
        uv = round_half(uv);
      }
      out = silu(gv) * uv;
    } else {
      float acc_v = s[0];
      if (sizeof(OutT) == 2)
        acc_v = round_half(acc_v);
      out = a.post == 1 ? acc_v + load_elem(aux, off) : a.post == 2 ? silu(load_elem(aux, off)) * acc_v : acc_v;
    }
    store_elem(y, off, out);
  }
}

// ----------------------------------------------------------------------------
// Split-K GEMV (m <= 8 rows, split hi/lo into one 16-row activation tile).
//
// Each CU of a persistent launch would otherwise pull all of x from L2 (32 MB
// across the chip for m = 8, K = 4096, fp32) before its first MFMA.  Here
// workgroup b covers column group `grp` (T tiles of NM matrices) over one
// K-slice `ks` of BPS blocks, so it reads only its slice of x:
//  1. the workgroup converts its slice of x once into LDS: A fragments
//     (fp16 high parts in rows 0..7, low parts in rows 8..15, per-(row, slice)
//     power-of-two scale) and the min-term fragments (sub-block sums / 32);
//  2. wave w owns (matrix, tile) pairs w, w + 8, ... (PW of them) and streams
//     their tile-blocks of the slice through a private LDS ring with DP
//     block-steps in flight; a block-step is PW independent MFMA chains
//     over one set of A fragments;
//  3. each wave writes its slice partials (hi + lo rows combined, unscaled)
//     to the workspace; the last workgroup of the group to arrive (a device-
//     scope counter, reset by that workgroup) sums the KS slices in slice
//     order and runs the epilogue.  No workgroup ever waits for another.
// Workgroups of one group are placed on one XCD (workgroup b runs on XCD
// b % 8), so their partials meet in one L2.
// ----------------------------------------------------------------------------
// Bytes of LDS one split-K slice uses.
// The slice of x as read: one row of one block per (block, row) pair, 1 KB
// of fp32 (512 B of fp16) at a stride of 1040 B, so that the 8 rows' 128-byte
// reads of the pack fall in different banks.
constexpr int kSplitkStageStride = 1040;
template <int NM, int T, int BPS, int DP>
constexpr int splitk_lds_bytes() {
  return 8 * DP * (NM * T / 8) * kTileBlockBytes + BPS * 8 * 64 * 16 + BPS * 64 * 8 + BPS * 8 * 4 + BPS * 8 * kSplitkStageStride;
}

// One workgroup's K-slice ks of column group grp (see above), over LDS of
// splitk_lds_bytes().
template <int NM, int T, int KS, int BPS, int DP, typename OutT>
__device__ __forceinline__ void splitk_slice(const GemvArgs& a, uint8_t* lds, int* s_last, float* __restrict__ part, int* __restrict__ counters,
                                             int grp, int ks) {
  constexpr int W = 8, MT = NM * T, PW = MT / W;
  static_assert(MT % W == 0, "whole (matrix, tile) pairs per wave");
  // LDS: the rings, then the slice's decode pack (fragments, min-term
  // operands, unscale factors: the same layout as in global memory).
  constexpr int kFragBytes = BPS * 8 * 64 * 16;  // [BPS][8 fragments][64 lanes] x 16 B
  constexpr int kXsBytes = BPS * 64 * 8;         // [BPS][64 lanes] x 4 halves
  constexpr int kDscBytes = BPS * 8 * 4;         // [BPS][8 rows]
  constexpr int kStageBytes = BPS * 8 * kSplitkStageStride;  // the slice of x as read, per (block, row) pair
  constexpr int kSlots = DP * PW;                // ring slots per wave
  constexpr int kRingBytes = W * kSlots * kTileBlockBytes;
  static_assert(kRingBytes + kFragBytes + kXsBytes + kDscBytes + kStageBytes == splitk_lds_bytes<NM, T, BPS, DP>(), "LDS layout");
  uint8_t* const stage = lds + kRingBytes + kFragBytes + kXsBytes + kDscBytes;
  u4_t* const xf = reinterpret_cast<u4_t*>(lds + kRingBytes);
  _Float16* const xs = reinterpret_cast<_Float16*>(lds + kRingBytes + kFragBytes);
  const float* const dscl = reinterpret_cast<const float*>(lds + kRingBytes + kFragBytes + kXsBytes);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, col = lane & 15;
  const int nb = a.nb, kb0 = ks * BPS;
  uint8_t* const ring = lds + (size_t)wave * kSlots * kTileBlockBytes;
  const uint32_t ring0 = lds_addr(ring);
  const uint32_t voff16 = 16u * (uint32_t)lane, voff4 = 4u * (uint32_t)lane;

  // Block-step i of this wave: block kb0 + i of each of its PW pairs, into
  // slot group i % DP.  Steps past the end re-load the last one (L2 hits),
  // so every step issues exactly 3 * PW loads.
  auto issue = [&](int i) {
    __builtin_amdgcn_sched_barrier(0);
    const int bb = i < BPS ? i : BPS - 1;
    const int sg = i % DP;
#pragma unroll
    for (int pw = 0; pw < PW; ++pw) {
      const int mt = wave + W * pw, mi = mt / T, t = mt - mi * T;
      const size_t ct = (size_t)grp * T + t;
      const uint8_t* src = uniform_ptr((mi ? a.wu : a.w) + (ct * nb + kb0 + bb) * kTileBlockBytes);
      const uint32_t l = __builtin_amdgcn_readfirstlane(ring0 + (uint32_t)(sg * PW + pw) * kTileBlockBytes);
      lds_dma16<0>(src, voff16, l);
      lds_dma16<kSlabBytes>(src, voff16, l);
      lds_dma4<kHeaderOffset>(src, voff4, l);
    }
  };

  // 1. The workgroup packs its slice of x into LDS (the decode pack layout,
  // see stage_pack_kernel): wave w converts (block, row) pairs w, w + 8, ...
  // of the slice.  The slice arrives by LDS DMA like the weights, issued
  // before them; a wait that leaves the weight loads in flight
  // (vmcnt(3 * PW * DP)) then covers x alone.  (Compiler-visible loads of x
  // would be waited for with vmcnt(0): the compiler does not count the
  // weight DMAs, so that wait would also cover the first weight steps.)
  constexpr int PPW = BPS * 8 / W;  // (block, row) pairs per wave
  static_assert(BPS * 8 % W == 0, "whole pairs per wave");
  static_assert(3 * PW * DP <= 63, "vmcnt range");
  const OutT* const xin = reinterpret_cast<const OutT*>(a.x);
  const bool live = (wave & 7) < a.m;  // row (wave + 8j) & 7 of every pair of this wave
  if (live) {
#pragma unroll
    for (int j = 0; j < PPW; ++j) {
      const int pr = wave + W * j, r = pr & 7;
      const OutT* src = xin + (size_t)r * a.k + (size_t)(kb0 + (pr >> 3)) * 256;
      const uint32_t l = __builtin_amdgcn_readfirstlane(lds_addr(stage + (size_t)pr * kSplitkStageStride));
      if (sizeof(OutT) == 4) {
        lds_dma16<0>(uniform_ptr(reinterpret_cast<const uint8_t*>(src)), voff16, l);
      } else {
        lds_dma4<0>(uniform_ptr(reinterpret_cast<const uint8_t*>(src)), voff4, l);
        lds_dma4<256>(uniform_ptr(reinterpret_cast<const uint8_t*>(src)), voff4, l);
      }
    }
  }
  __builtin_amdgcn_s_barrier();  // the workgroup's x requests ahead of its weight requests
#pragma unroll
  for (int i = 0; i < DP; ++i)
    issue(i);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * PW * DP) : "memory");
  __syncthreads();
  // Wave w < BPS packs block w of the slice, all 8 rows, as the fused gate/up
  // GEMV packs its blocks: lane 16 g + 8 h + r takes elements 64 g + 32 h +
  // [0, 32) of row r (128 contiguous bytes of the stage), so that the row
  // maximum and the sub-block sums are mostly in-lane, and writes the block's
  // fragments, min-term operands and unscale factors to LDS.  Rows >= m are
  // zero.
  static_assert(BPS <= W, "one block per packing wave");
  if (wave < BPS) {
    const int r = lane & 7, e0 = 64 * (lane >> 4) + 32 * ((lane >> 3) & 1);
    const uint8_t* src = stage + (size_t)(8 * wave + r) * kSplitkStageStride;
    float t32[32];
    if (sizeof(OutT) == 4) {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const f4_t v4 = *reinterpret_cast<const f4_t*>(src + 4 * e0 + 16 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          t32[4 * c + e] = v4[e];
      }
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const h8_t v8 = *reinterpret_cast<const h8_t*>(src + 2 * e0 + 16 * c);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          t32[8 * c + e] = (float)v8[e];
      }
    }
    if (r >= a.m) {
#pragma unroll
      for (int e = 0; e < 32; ++e)
        t32[e] = 0.0f;
    }
    XBlock xb;
    pack_x_regs(t32, lane, xb);
#pragma unroll
    for (int f = 0; f < 8; ++f)
      xf[((size_t)wave * 8 + f) * 64 + lane] = __builtin_bit_cast(u4_t, xb.frag[f]);
    reinterpret_cast<h4_t*>(xs)[(size_t)wave * 64 + lane] = xb.xs;
    if (lane == 0 || lane == 16) {
#pragma unroll
      for (int v = 0; v < 4; ++v)
        const_cast<float*>(dscl)[wave * 8 + (lane >> 2) + v] = xb.dv[v];
    }
  }
  __syncthreads();

  // 2. Stream the slice's tile-blocks of this wave's pairs.
  f4_t acc[PW];
#pragma unroll
  for (int pw = 0; pw < PW; ++pw)
    acc[pw] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < BPS; ++i) {
    // 3 * PW loads per step: with DP steps outstanding, this marks step i.
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * PW * (DP - 1)) : "memory");
    const u4_t* sl = reinterpret_cast<const u4_t*>(ring + (size_t)(i % DP) * PW * kTileBlockBytes);
    u4_t q0[PW], q1[PW], hd[PW];
#pragma unroll
    for (int pw = 0; pw < PW; ++pw) {
      const u4_t* su = sl + pw * (kTileBlockBytes / 16);
      q0[pw] = su[lane];
      q1[pw] = su[kSlabBytes / 16 + lane];
      hd[pw] = su[kHeaderOffset / 16 + col];
    }
    h8_t xa[8];
#pragma unroll
    for (int f = 0; f < 8; ++f)
      xa[f] = __builtin_bit_cast(h8_t, xf[(i * 8 + f) * 64 + lane]);
    const h4_t xsa = *reinterpret_cast<const h4_t*>(xs + (i * 64 + lane) * 4);
    // Unscale factors of this lane's C rows (4g + v) & 7 in block i.
    const f4_t dv = *reinterpret_cast<const f4_t*>(dscl + i * 8 + 4 * (g & 1));
    // The step is in registers: its slots take the step DP ahead.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    issue(i + DP);
#pragma unroll
    for (int pw = 0; pw < PW; ++pw) {
      const BlockConsts kc = block_consts(hd[pw], g);
      f4_t cl = f4_t{0.0f, 0.0f, 0.0f, 0.0f}, ch = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const u4_t qq = u < 2 ? q0[pw] : q1[pw];
        const uint32_t wa = qq[2 * (u & 1)], wb = qq[2 * (u & 1) + 1];
        const h8_t blo = quant_times_scale(wa, wb, 0x000F000Fu, 0x64006400u, kc.mul_lo, kc.add_lo);
        const h8_t bhi = quant_times_scale(wa, wb, 0x00F000F0u, 0x64006400u, kc.mul_hi, kc.add_hi);
        cl = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[u], blo, cl, 0, 0, 0);
        ch = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[4 + u], bhi, ch, 0, 0, 0);
      }
      const f4_t cm = __builtin_amdgcn_mfma_f32_16x16x16f16(xsa, kc.bmin, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
      for (int v = 0; v < 4; ++v)
        acc[pw][v] += fmaf(kc.d, cl[v] + ch[v], -kc.dmin * cm[v]) * dv[v];
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // 3. Slice partials: C row r (lanes g < 2) plus its low part r + 8 (lanes
  // g + 2), unscaled; layout [grp][ks][mt][8 rows][16 columns].  They are
  // written through to memory (system-coherent stores) and read back the
  // same way, so no cache of any XCD needs flushing; the counter is a
  // device-scope atomic.
#pragma unroll
  for (int pw = 0; pw < PW; ++pw) {
    const int mt = wave + W * pw;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float tot = acc[pw][v] + __shfl_xor(acc[pw][v], 32);
      const int row = 4 * g + v;
      if (g < 2 && row < a.m)
        store_coherent(part + ((((size_t)grp * KS + ks) * MT + mt) * 8 + row) * 16 + col, tot);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0)
    *s_last = count_arrival(&counters[grp]) == KS - 1;
  __syncthreads();
  if (!*s_last)
    return;
  OutT* y = reinterpret_cast<OutT*>(a.y);
  const OutT* aux = reinterpret_cast<const OutT*>(a.aux);
  constexpr int EPI = 16 * T;  // outputs per row of a group
  // The outputs of the group this thread finishes (at most PER of them), with
  // all their loads (the KS slice partials, and aux) issued before a single
  // wait: the reduction costs one memory round trip, not two per output.
  constexpr int PER = (8 * EPI + 64 * W - 1) / (64 * W);
  float pv[PER][NM][KS], av[PER];
  size_t offs[PER];
#pragma unroll
  for (int r = 0; r < PER; ++r) {
    const int o0 = tid + r * 64 * W, o = o0 < a.m * EPI ? o0 : 0;
    const int row = o / EPI, c = o % EPI, t = c >> 4, cc = c & 15;
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
#pragma unroll
      for (int k2 = 0; k2 < KS; ++k2)
        pv[r][mi][k2] = load_coherent(part + ((((size_t)grp * KS + k2) * MT + mi * T + t) * 8 + row) * 16 + cc);
    offs[r] = (size_t)row * a.n + ((size_t)grp * T + t) * 16 + cc;
    av[r] = NM == 1 && a.post != 0 ? load_elem(aux, offs[r]) : 0.0f;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int r = 0; r < PER; ++r) {
    if (tid + r * 64 * W >= a.m * EPI)
      break;
    float sm[NM];
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
      float v = 0.0f;
#pragma unroll
      for (int k2 = 0; k2 < KS; ++k2) {
        hold(pv[r][mi][k2]);
        v += pv[r][mi][k2];
      }
      sm[mi] = v;
    }
    float out;
    if (NM == 2) {
      float gv = sm[0], uv = sm[NM - 1];
      if (sizeof(OutT) == 2) {
        gv = round_half(gv);
        uv = round_half(uv);
      }
      out = silu(gv) * uv;
    } else {
      float acc_v = sm[0];
      if (sizeof(OutT) == 2)
        acc_v = round_half(acc_v);
      out = a.post == 1 ? acc_v + av[r] : a.post == 2 ? silu(av[r]) * acc_v : acc_v;
    }
    store_elem(y, offs[r], out);
  }
  if (tid == 0)
    reset_counter(&counters[grp]);  // ready for the next launch
}

// Workgroup b: slice (b / 8) % KS of group (b % 8) + 8 ((b / 8) / KS), so the
// KS slices of a group run on one XCD (b % 8).
template <int NM, int T, int KS, int BPS, int DP, typename OutT>
__global__ __launch_bounds__(512) void q4k_gemv_splitk_kernel(GemvArgs a, float* __restrict__ part, int* __restrict__ counters) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[splitk_lds_bytes<NM, T, BPS, DP>()];
  __shared__ int s_last;
  const int sidx = (int)blockIdx.x >> 3;
  splitk_slice<NM, T, KS, BPS, DP, OutT>(a, lds, &s_last, part, counters, ((int)blockIdx.x & 7) + 8 * (sidx / KS), sidx % KS);
}


// ----------------------------------------------------------------------------
// Pipelined GEMM (prefill, N a multiple of 256).
//
// Workgroup tile 128 rows x 256 columns, 4 waves; wave w owns columns
// [64w, 64w + 64) (4 column tiles) of all 128 rows (8 row tiles), so every
// weight element is dequantised once per workgroup and each A fragment read
// from LDS feeds 4 column tiles.  K runs in u-steps of v_mfma_f32_16x16x32_f16
// pairs: u-step t = 4 * block + u covers, in every row, elements
// 64g + 8u + [0, 8) (low nibbles, fragment u) and 64g + 32 + 8u + [0, 8)
// (high nibbles, fragment 4 + u) of the block, for lane groups g.
//  - A: the activations, staged in the GEMM order (gemm_frag_offset: one
//    contiguous 16 KB run per (row block, u-step)), stream through a
//    5-slot LDS ring shared by the 4 waves (16 KB per u-step: 8 row tiles
//    x 2 fragments), loaded with global_load_lds_dwordx4 four u-steps ahead;
//    one barrier per u-step.
//  - B: each wave streams the tile-blocks of its 4 column tiles through a
//    private 2-block LDS ring (one block ahead) and dequantises in
//    registers to h(d*sc*q - dmin*m), the fp32 expression rounded to fp16
//    once (the reference's prefill tile value, quant_linear.metal:43,45).
// Loads: per u-step a wave issues its 4 fragments of A(t + 4) and, at the
// first u-step of a block, the 4 tile-blocks (12 loads) of the next block,
// one fragment (and one tile-block) per column group so that the load
// issue is spread over the step.
// ----------------------------------------------------------------------------
constexpr int kG2M = 128, kG2N = 256, kG2AS = 5, kG2AD = 4;  // A ring slots, A distance
// Time of one 128-column tile (two column tiles per wave) in tenths of a
// 256-column tile's, for the choice between the two tilings.
constexpr int kGemmNarrowTileTime = 6;
constexpr int kG2ASlot = 16 * 1024;                    // 8 row tiles x 2 fragments x 1 KB
constexpr int kG2BWave = 2 * 4 * kTileBlockBytes;      // per wave: 2 blocks x 4 tile-blocks

// Epilogue of a 128 x 64 wave tile.  Lane (col, g) holds rows 16 rt + 4 g + v
// of column col of each column tile.  The aux loads (post 1 / 2) run one row
// tile ahead of the stores: those of row tile rt + 1 are issued before the
// stores of row tile rt, so their latency overlaps the previous tile's stores
// instead of being paid once per row tile (rows differ, so an aux that is y
// itself is read before it is written).  A tile wholly inside m (FULL) has no
// per-row checks.  CT column tiles per wave, of which the first nct lie
// inside n.
template <typename OutT, int POST, bool FULL, int CT = 4>
__device__ __forceinline__ void gemm2_epilogue(const GemmArgs& a, const f4_t (&acc)[8][CT], int mt0, int ct0, int lane, int nct = CT,
                                               float* lrs = nullptr) {
  OutT* y = reinterpret_cast<OutT*>(a.y);
  const OutT* aux = reinterpret_cast<const OutT*>(a.aux);
  const int g = lane >> 4, col = lane & 15;
  const int row0 = mt0 * 16 + 4 * g;
  constexpr bool full = FULL;
  // Row scales exist for the padded rows (the staging buffers cover whole
  // 128-row tiles), so these 16-byte loads stay in bounds.
  // Row scales of the 8 row tiles up front and the aux of row tile rt + 1
  // loaded under the stores of row tile rt (two buffers).  With more than
  // four column tiles per wave the registers of all that do not fit beside
  // the six-tile loop's: the wave stages the tile's 128 row scales in its own
  // LDS (lrs, its B ring, idle once its loads have landed) with one load and
  // reads each row tile's from there, and loads each row tile's aux just
  // before it.
  constexpr bool ahead = CT <= 4;
  f4_t rs[8];
  if constexpr (ahead) {
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
      rs[rt] = *reinterpret_cast<const f4_t*>(a.rowscale + row0 + 16 * rt);
  } else {
    *reinterpret_cast<float2*>(lrs + 2 * lane) = *reinterpret_cast<const float2*>(a.rowscale + mt0 * 16 + 2 * lane);
  }
  const size_t col0 = (size_t)ct0 * 16 + col;
  float av[2][4][CT];
  auto load_aux = [&](int rt, float (&dst)[4][CT]) {
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        const int row = row0 + 16 * rt + v;
        dst[v][c] = (full || row < a.m) && c < nct ? load_elem(aux, (size_t)row * a.n + col0 + 16 * c) : 0.0f;
      }
  };
  if (POST != 0 && ahead)
    load_aux(0, av[0]);
#pragma unroll
  for (int rt = 0; rt < 8; ++rt) {
    if (POST != 0 && ahead && rt + 1 < 8)
      load_aux(rt + 1, av[(rt + 1) & 1]);
    if (POST != 0 && !ahead)
      load_aux(rt, av[0]);
    if constexpr (!ahead)
      rs[rt] = *reinterpret_cast<const f4_t*>(lrs + 16 * rt + 4 * g);
    const float (&cur)[4][CT] = av[ahead ? rt & 1 : 0];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = row0 + 16 * rt + v;
      if (!full && row >= a.m)
        continue;
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        if (c >= nct)
          continue;
        float acc_v = acc[rt][c][v] * rs[rt][v];
        if (sizeof(OutT) == 2)
          acc_v = round_half(acc_v);
        float out = POST == 1 ? acc_v + cur[v][c] : POST == 2 ? silu(cur[v][c]) * acc_v : acc_v;
        // The fp32 value is formed before any conversion to fp16: fused into
        // the conversion (v_fma_mix) the product would round once instead of
        // twice, as the reference's half(silu(g) * u) does.
        asm("" : "+v"(out));
        store_elem(y, (size_t)row * a.n + col0 + 16 * c, out);
      }
    }
  }
}

// Epilogue of the gated GEMM's wave tile of 128 rows and CT / 2 output column
// tiles: the gate tiles (columns 0 .. CT / 2 - 1 of acc) and the up tiles
// (the rest) of the same output column tiles combine as in the two-call
// form: SiLU(gate) * up, each of gate and up first unscaled and, for fp16
// outputs, rounded to fp16 (the gate value the first call stores, the up
// value the second call's epilogue forms).  nct of the output tiles lie
// inside n.
template <typename OutT, bool FULL, int CT = 4>
__device__ __forceinline__ void gemm2_epilogue_gated(const GemmArgs& a, const f4_t (&acc)[8][CT], int mt0, int ct0, int lane, int nct) {
  constexpr int H = CT / 2;  // output tiles: gate columns 0 .. H - 1, up columns H .. CT - 1
  OutT* y = reinterpret_cast<OutT*>(a.y);
  const int g = lane >> 4, col = lane & 15;
  const int row0 = mt0 * 16 + 4 * g;
  f4_t rs[8];
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
    rs[rt] = *reinterpret_cast<const f4_t*>(a.rowscale + row0 + 16 * rt);
  const size_t col0 = (size_t)ct0 * 16 + col;
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = row0 + 16 * rt + v;
      if (!FULL && row >= a.m)
        continue;
#pragma unroll
      for (int c = 0; c < H; ++c) {
        if (c >= nct)
          continue;
        float gv = acc[rt][c][v] * rs[rt][v], uv = acc[rt][H + c][v] * rs[rt][v];
        if (sizeof(OutT) == 2) {
          gv = round_half(gv);
          uv = round_half(uv);
        }
        float out = silu(gv) * uv;
        asm("" : "+v"(out));  // the fp32 value first, as in the post-2 epilogue
        store_elem(y, (size_t)row * a.n + col0 + 16 * c, out);
      }
    }
}

// Tile order of the persistent GEMMs.  Workgroup b runs on XCD b % 8 (the
// dispatcher deals workgroups to the eight XCDs in turn).  In the plain order
// tile t = b + i * grid has column block t % tiles_x, so an XCD owns whole
// column blocks and streams the A operand of every row block.  With rg > 0
// the tile grid is cut into 8 rectangles of tiles_y / rg row blocks by
// tiles_x / (8 / rg) column blocks, one per XCD, and the XCD's workgroups
// take its tiles column by column, so that the tiles running together on one
// XCD share the A of a few row blocks and the B of a few column blocks in
// that XCD's L2.
struct TileMap {
  int tiles_x, tiles;  // column blocks, all tiles
  int rg;              // 0: plain order; else row groups (8 / rg column groups)
  int rows, cols;      // rectangle of one XCD (rg > 0)
};

__device__ __forceinline__ int tile_count(const TileMap& m) {
  if (m.rg == 0)
    return ((int)blockIdx.x < m.tiles) ? (m.tiles - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
  const int per = (int)gridDim.x >> 3, j = (int)blockIdx.x >> 3;
  const int rect = m.rows * m.cols;
  return j < rect ? (rect - 1 - j) / per + 1 : 0;
}

// The i-th tile of this workgroup as (column block, row block).
__device__ __forceinline__ void tile_at(const TileMap& m, int i, int& bx, int& by) {
  if (m.rg == 0) {
    const int t = (int)blockIdx.x + i * (int)gridDim.x;
    bx = t % m.tiles_x;
    by = t / m.tiles_x;
    return;
  }
  const int x = (int)blockIdx.x & 7, per = (int)gridDim.x >> 3;
  const int l = ((int)blockIdx.x >> 3) + i * per;
  const int cg = 8 / m.rg;
  by = (x / cg) * m.rows + l % m.rows;
  bx = (x % cg) * m.cols + l / m.rows;
}

// One 128 x 256 output tile (column block bx, row block by).  Column tiles
// at or past ntiles = n / 16 (a last, partial column block) load the last
// column tile (in bounds) and store nothing.  GATED: the workgroup's 128
// output columns of the gated GEMM; wave w takes output column tiles
// ct0 = 8 bx + 2 w and ct0 + 1, whose gate tiles are its B columns 0, 1 and
// whose up tiles (a.wu) are its columns 2, 3.
template <typename OutT, bool GATED, bool SPLIT>
__device__ __forceinline__ void gemm2_tile(const GemmArgs& a, uint8_t* lds, int bx, int by, int ntiles, int kb0, int nbr, int item,
                                           int* s_last) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, col = lane & 15;
  // Blocks [kb0, kb0 + nbr) of K (all of them unless SPLIT); u-steps and
  // ring positions count from kb0.
  const int nb = a.nb, steps = 4 * nbr;
  const int mt0 = by * (kG2M / 16);                         // first row tile
  const int ct0 = GATED ? bx * 8 + 2 * wave : bx * (kG2N / 16) + 4 * wave;  // this wave's first column tile
  const uint32_t aring = lds_addr(lds);
  uint8_t* const bring = lds + kG2AS * kG2ASlot + wave * kG2BWave;
  const uint32_t bring0 = lds_addr(bring);
  const uint32_t voff16 = 16u * (uint32_t)lane, voff4 = 4u * (uint32_t)lane;
  const _Float16* const xh = a.xh;

  // A(t, i): fragment i of this wave's 4 (of the 16) fragments of u-step t
  // (clamped to the last u-step past the end).
  auto issue_a = [&](int t, int i) {
    const int tc = t < steps ? t : steps - 1;
    const int b = kb0 + (tc >> 2), u = tc & 3;
    const int f = 4 * wave + i;
    const _Float16* src = xh + ((((size_t)by * nb + b) * 4 + u) * 16 + f) * 512;
    const uint32_t l = __builtin_amdgcn_readfirstlane(aring + (uint32_t)(t % kG2AS) * kG2ASlot + (uint32_t)f * 1024);
    lds_dma16<0>(uniform_ptr(reinterpret_cast<const uint8_t*>(src)), voff16, l);
  };
  // B(blk, c): tile-block c of block blk (clamped) into ring half blk & 1.
  auto issue_b = [&](int blk, int c) {
    const int bc = kb0 + (blk < nbr ? blk : nbr - 1);
    const int cc = GATED ? ct0 + (c & 1) : ct0 + c;
    const int ct = cc < ntiles ? cc : ntiles - 1;
    const uint8_t* const wm = GATED && c >= 2 ? a.wu : a.w;
    const uint8_t* src = uniform_ptr(wm + ((size_t)ct * nb + bc) * kTileBlockBytes);
    const uint32_t l = __builtin_amdgcn_readfirstlane(bring0 + (uint32_t)((blk & 1) * 4 + c) * kTileBlockBytes);
    lds_dma16<0>(src, voff16, l);
    lds_dma16<kSlabBytes>(src, voff16, l);
    lds_dma4<kHeaderOffset>(src, voff4, l);
  };

  // Block constants of the 4 column tiles, in fp32, from the 4 headers (this
  // lane's column) of one block: for sub-block 2g (low nibbles) d * sc * 2^24
  // and -dmin * m, for sub-block 2g + 1 (high nibbles) d * sc * 2^20 and
  // -dmin * m.  All are exact in fp32 (11-bit d times a 6-bit field, times a
  // power of two).
  float dsl[4], csl[4], dsh[4], csh[4];
  auto block_const = [&](int c, const u4_t& hd) {
    uint32_t p0, p1;
    scale_min_packed(hd, g, p0, p1);
    const float d = half_bits_to_float(hd.x & 0xffffu), dmin = half_bits_to_float(hd.x >> 16);
    dsl[c] = d * (float)(p0 & 0xffu) * 0x1p24f;
    csl[c] = -dmin * (float)((p0 >> 16) & 0xffu);
    dsh[c] = d * (float)(p1 & 0xffu) * 0x1p20f;
    csh[c] = -dmin * (float)((p1 >> 16) & 0xffu);
  };
  // B fragments of column tile c from its two raw words (words 2(u & 1),
  // 2(u & 1) + 1 of slab u / 2 for u-step u), with the block constants: the
  // reference's prefill tile value h(d * sc * q - dmin * m), formed in fp32
  // and rounded to fp16 once (quant_linear.metal:43,45), bit for bit.
  // w & 0x000F000F puts two low nibbles into the low bits of two fp16
  // halves: the denormals q * 2^-24 (w & 0x00F000F0: 16 q * 2^-24 for two
  // high nibbles).  One v_fma_mix_f32 per weight, which takes fp16 denormal
  // sources at their exact value, forms q * (d * sc * 2^24) - dmin * m (2^20
  // for the high nibbles) with the product exact and one rounding to fp32,
  // and one v_cvt_pk_f16_f32 per pair rounds to fp16.  The empty asm keeps
  // the fp32 results apart from the conversion: fused, they become
  // v_fma_mixlo/mixhi_f16 pairs writing the two halves of one register, a
  // dependent chain that measured 6 % slower.  The nibble masks live in
  // registers, as plain values that the scheduler sees as vector ALU work.
  uint32_t m_lo = 0x000F000Fu, m_hi = 0x00F000F0u;
  asm volatile("" : "+v"(m_lo), "+v"(m_hi));
  auto dequant_words = [&](int c, uint2 wv, h8_t& blo, h8_t& bhi) {
    const uint32_t lw[4] = {wv.x, wv.x >> 8, wv.y, wv.y >> 8};
    u4_t lo, hi;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const h2_t ql = as_h2(lw[e] & m_lo);
      const h2_t qh = as_h2(lw[e] & m_hi);
      float a0 = __builtin_fmaf((float)ql[0], dsl[c], csl[c]), a1 = __builtin_fmaf((float)ql[1], dsl[c], csl[c]);
      float b0 = __builtin_fmaf((float)qh[0], dsh[c], csh[c]), b1 = __builtin_fmaf((float)qh[1], dsh[c], csh[c]);
      asm("" : "+v"(a0), "+v"(a1), "+v"(b0), "+v"(b1));
      lo[e] = as_u32(h2_t{(_Float16)a0, (_Float16)a1});
      hi[e] = as_u32(h2_t{(_Float16)b0, (_Float16)b1});
    }
    blo = __builtin_bit_cast(h8_t, lo);
    bhi = __builtin_bit_cast(h8_t, hi);
  };

  // Accumulators: 32 MFMA tiles, zeroed and pinned to AGPRs (the loop-carried
  // values then stay in AGPRs instead of being copied through VGPRs).
  f4_t acc[8][4];
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      acc[rt][c] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
      asm volatile("" : "+a"(acc[rt][c]));
    }

#pragma unroll
  for (int c = 0; c < 4; ++c)
    issue_b(0, c);
#pragma unroll
  for (int t = 0; t < kG2AD; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      issue_a(t, i);
  // B(0) and A(0) landed: A(1..3) (12 loads) were issued after them.
  asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  // Dequantisation runs one column behind the MFMAs: column c of u-step
  // t + 1 is dequantised under the MFMAs of column c + 1 of u-step t, and
  // column 3 under those of column 0 of u-step t + 1 (from words kept in
  // wv3), so that every column's MFMAs have vector work to cover.  At the
  // last u-step of a block the next block's constants of column c are
  // computed under column c's MFMAs, after column 3 of the current u-step
  // (old constants) was dequantised and before column c's first use.
  h8_t bclo[4], bchi[4];  // dequantised B fragments of the current u-step
  uint2 wv3;              // raw words of column 3 for the current u-step
  {
    u4_t hd[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      hd[c] = *reinterpret_cast<const u4_t*>(bring + c * kTileBlockBytes + kHeaderOffset + 16 * col);
      block_const(c, hd[c]);
    }
#pragma unroll
    for (int c = 0; c < 3; ++c)
      dequant_words(c, *reinterpret_cast<const uint2*>(bring + c * kTileBlockBytes + 16 * lane), bclo[c], bchi[c]);
    wv3 = *reinterpret_cast<const uint2*>(bring + 3 * kTileBlockBytes + 16 * lane);
  }
  // A in the loop: this wave's 4 fragments of u-step t are 4 consecutive KB
  // at xa + 16 KB * t of the staging and at 4 KB * wave of ring slot t % 5;
  // fragment i is the instruction offset 1 KB * i.  The ring addresses of
  // the slot read (ar) and written (aw) roll instead of being recomputed.
  const uint8_t* const xa = reinterpret_cast<const uint8_t*>(xh) + ((size_t)by * nb * 64 + (size_t)kb0 * 64 + 4 * wave) * 1024;
  const uint32_t aend = aring + kG2AS * kG2ASlot;
  uint32_t ar = aring, aw = aring + kG2AD * kG2ASlot + 4096u * (uint32_t)wave;
  for (int blk = 0; blk < nbr; ++blk) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = 4 * blk + u;
      const int ta = t + kG2AD < steps ? t + kG2AD : steps - 1;
      const uint8_t* const asrc = uniform_ptr(xa + (size_t)ta * 16384);
      // Own loads issued after A(t) (during u-steps t - 4 .. t - 1, in the
      // order of the column groups below): 15 at u = 0 (the 3 of B tile 3
      // that follow A(t) at u-step t - 4, then 3 x 4), 24 at u = 1, 2, 3.
      // At u = 3 B(blk + 1), issued at u-step t - 3 after A(t), must have
      // landed too: 8 loads follow it.  (A(0) is waited for in the prologue.)
      if (u == 0)
        asm volatile("s_waitcnt vmcnt(15)" ::: "memory");
      else if (u == 3)
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
      __syncthreads();  // A(t) of every wave landed; u-step t - 1 fully read
      __builtin_amdgcn_sched_barrier(0);
      // LDS reads of the step: the 16 A fragments of u-step t ([row tile][low,
      // high]), then (u = 3) the headers of the next block, then the raw B
      // words of u-step t + 1.  At u = 3 that is the next block, whose B
      // landed before A(t) (issued at u = 0).
      const int bn = u == 3 ? blk + 1 : blk, un = (u + 1) & 3;
      const uint8_t* aslot = lds + (ar - aring);
      h8_t af[16];
#pragma unroll
      for (int i = 0; i < 16; ++i)
        af[i] = *reinterpret_cast<const h8_t*>(aslot + i * 1024 + 16 * lane);
      const uint8_t* bslot = bring + (size_t)((bn & 1) * 4) * kTileBlockBytes;
      u4_t hd[4];
      if (u == 3) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          hd[c] = *reinterpret_cast<const u4_t*>(bslot + c * kTileBlockBytes + kHeaderOffset + 16 * col);
      }
      uint2 wv[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        wv[c] = *reinterpret_cast<const uint2*>(bslot + c * kTileBlockBytes + (un >> 1) * kSlabBytes + 16 * lane + 8 * (un & 1));
      __builtin_amdgcn_sched_barrier(0);
      // Column tile c: its 16 MFMAs of u-step t, then its B fragments of
      // u-step t + 1 replace the ones just consumed.  The dequantisation of
      // column c runs under the MFMAs of column c + 1.
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (c == 0)
          dequant_words(3, wv3, bclo[3], bchi[3]);  // column 3 of this u-step
        // Low-nibble fragments over the 8 row tiles, then the high ones:
        // neighbouring MFMAs are independent.
#pragma unroll
        for (int rt = 0; rt < 8; ++rt)
          acc[rt][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[2 * rt], bclo[c], acc[rt][c], 0, 0, 0);
#pragma unroll
        for (int rt = 0; rt < 8; ++rt)
          acc[rt][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[2 * rt + 1], bchi[c], acc[rt][c], 0, 0, 0);
        if (u == 3)
          block_const(c, hd[c]);
        if (c > 0)
          dequant_words(c - 1, wv[c - 1], bclo[c - 1], bchi[c - 1]);
        // The loads of the column group, spread over the step: fragment c
        // of A(t + 4) and, at u = 0, tile-block c of B(blk + 1).
        if (c == 0)
          lds_dma16<0>(asrc, voff16, aw);
        else if (c == 1)
          lds_dma16<1024>(asrc, voff16, aw);
        else if (c == 2)
          lds_dma16<2048>(asrc, voff16, aw);
        else
          lds_dma16<3072>(asrc, voff16, aw);
        if (u == 0)
          issue_b(blk + 1, c);
      }
      wv3 = wv[3];
      ar = ar + kG2ASlot == aend ? aring : ar + kG2ASlot;
      aw = aw + kG2ASlot >= aend ? aw + kG2ASlot - kG2AS * kG2ASlot : aw + kG2ASlot;
      // Schedule of the step: the LDS reads first, then each MFMA followed
      // by a share of the vector work (the next step's dequantisation, and
      // at u = 3 the next block's constants), so that no vector work is
      // left after the last MFMA.
      if (u == 3) {
        __builtin_amdgcn_sched_group_barrier(0x100, 24, 0);
#pragma unroll
        for (int i = 0; i < 64; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        }
      } else {
        __builtin_amdgcn_sched_group_barrier(0x100, 20, 0);
#pragma unroll
        for (int i = 0; i < 64; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        }
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // Pin the accumulators to AGPRs at the loop exit, so that the epilogue's
  // element reads do not pull copies of them into the loop.
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      asm volatile("" : "+a"(acc[rt][c]));

  if constexpr (SPLIT) {
    // Two K-segments per tile (items 2 tile, 2 tile + 1).  A segment that
    // finds the other already arrived (its accumulators in memory and the
    // counter at 1) stores nothing; otherwise it stores its accumulators
    // (written through to memory), counts its arrival, and the second to
    // arrive adds the other's and runs the epilogue.  fp32 addition
    // commutes, so the result does not depend on which segment is last.
    constexpr size_t kWaveFloats = 32 * 64 * 4;
    int* const ctr = &a.counters[item >> 1];
    if (tid == 0)
      *s_last = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) != 0;
    __syncthreads();
    if (!*s_last) {
      float* const mine = a.part + ((size_t)item * 4 + wave) * kWaveFloats + 4 * lane;
#pragma unroll
      for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          store_coherent4(mine + (rt * 4 + c) * 256, acc[rt][c]);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (tid == 0)
        *s_last = count_arrival(ctr) == 1;
      __syncthreads();
      if (!*s_last)
        return;
    }
    const float* const other = a.part + ((size_t)(item ^ 1) * 4 + wave) * kWaveFloats + 4 * lane;
    f4_t pv[8][4];
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        pv[rt][c] = load_coherent4(other + (rt * 4 + c) * 256);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        hold(pv[rt][c]);
        acc[rt][c] += pv[rt][c];
      }
    if (tid == 0)
      reset_counter(ctr);  // ready for the next launch
  }

  // One straight-line epilogue per (post code, tile inside m or not).
  const bool full = mt0 * 16 + kG2M <= a.m;
  if constexpr (GATED) {
    const int nct2 = ntiles - ct0 >= 2 ? 2 : ntiles - ct0 > 0 ? ntiles - ct0 : 0;
    full ? gemm2_epilogue_gated<OutT, true>(a, acc, mt0, ct0, lane, nct2) : gemm2_epilogue_gated<OutT, false>(a, acc, mt0, ct0, lane, nct2);
    return;
  }
  const int nct = ntiles - ct0 >= 4 ? 4 : ntiles - ct0 > 0 ? ntiles - ct0 : 0;
  if (a.post == 0)
    full ? gemm2_epilogue<OutT, 0, true>(a, acc, mt0, ct0, lane, nct) : gemm2_epilogue<OutT, 0, false>(a, acc, mt0, ct0, lane, nct);
  else if (a.post == 1)
    full ? gemm2_epilogue<OutT, 1, true>(a, acc, mt0, ct0, lane, nct) : gemm2_epilogue<OutT, 1, false>(a, acc, mt0, ct0, lane, nct);
  else
    full ? gemm2_epilogue<OutT, 2, true>(a, acc, mt0, ct0, lane, nct) : gemm2_epilogue<OutT, 2, false>(a, acc, mt0, ct0, lane, nct);
}

// Persistent launch: workgroup b takes its tiles in the order of the tile
// map.  Consecutive tiles of a workgroup reuse its LDS rings; a barrier
// separates the last reads of one tile from the first loads of the next.
// SPLIT: items 2 t and 2 t + 1 are the two K-segments of tile t (plain tile
// order): with a.split_q > 0 workgroup t < tiles takes segment 0 of tile t
// and workgroup tiles + r segments 1 of tiles r, r + R, ... (R workgroups
// past the tiles), else the workgroups take the items in turn.
template <typename OutT, bool GATED, bool SPLIT = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void q4k_gemm2_kernel(GemmArgs a, TileMap map) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kG2AS * kG2ASlot + 4 * kG2BWave];
  __shared__ int s_last;
  if constexpr (SPLIT) {
    // This workgroup's items: first, first + step, ... below 2 x tiles (one
    // call site of the tile body, which is inlined).
    const int b = a.split_b, tiles = map.tiles, g = (int)blockIdx.x;
    int first = g, step = (int)gridDim.x;
    if (a.split_q > 0) {
      first = g < tiles ? 2 * g : 2 * (g - tiles) + 1;
      step = g < tiles ? 2 * tiles : 2 * ((int)gridDim.x - tiles);
    }
    for (int it = first; it < 2 * tiles; it += step) {
      if (it != first)
        __syncthreads();
      const int tile = it >> 1, ks = it & 1;
      gemm2_tile<OutT, GATED, true>(a, lds, tile % map.tiles_x, tile / map.tiles_x, a.n / 16, ks ? b : 0, ks ? a.nb - b : b, it, &s_last);
    }
  } else {
    const int count = tile_count(map);
    for (int i = 0; i < count; ++i) {
      if (i > 0)
        __syncthreads();
      int bx, by;
      tile_at(map, i, bx, by);
      gemm2_tile<OutT, GATED, false>(a, lds, bx, by, a.n / 16, 0, a.nb, 0, &s_last);
    }
  }
}

// ----------------------------------------------------------------------------
// Measured MFMA ceiling: the GEMM's instruction (v_mfma_f32_16x16x32_f16) back
// to back, 32 independent accumulators per wave, one wave per SIMD, operands
// in registers -- the rate a kernel of this instruction can reach on the box
// (clock under a dense MFMA load included).  The result is stored so that
// nothing is dead; its value is meaningless.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void mfma_ceiling_kernel(float* out, int iters) {
  const int lane = threadIdx.x & 63;
  f4_t acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    acc[i] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    asm volatile("" : "+a"(acc[i]));
  }
  h8_t a0, a1, b0, b1;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a0[i] = (_Float16)(0.001f * (float)(lane + i));
    a1[i] = (_Float16)(0.002f * (float)(lane - i));
    b0[i] = (_Float16)(0.003f * (float)(i - lane));
    b1[i] = (_Float16)(0.004f * (float)(i + 1));
  }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 32; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(i & 1 ? a1 : a0, i & 2 ? b1 : b0, acc[i], 0, 0, 0);
  }
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    asm volatile("" : "+a"(acc[i]));
    sum += acc[i][0] + acc[i][3];
  }
  out[(size_t)blockIdx.x * 256 + threadIdx.x] = sum;
}

// ----------------------------------------------------------------------------
// Measured streaming-read ceiling: a plain read of n16 16-byte words with
// non-temporal loads (as the GEMVs stream their weights), up to four in
// flight per lane, over the grid the caller gives.  The xor of each lane's words is stored only
// if it hits a fixed value, which keeps the loads alive without a store
// stream of its own.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void stream_read_kernel(const u4_t* __restrict__ p, size_t n16, uint32_t* out) {
  const size_t stride = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u4_t a = __builtin_nontemporal_load(p + i), b = __builtin_nontemporal_load(p + i + stride);
    const u4_t c = __builtin_nontemporal_load(p + i + 2 * stride), d = __builtin_nontemporal_load(p + i + 3 * stride);
    acc ^= (a.x ^ a.y ^ a.z ^ a.w) ^ (b.x ^ b.y ^ b.z ^ b.w) ^ (c.x ^ c.y ^ c.z ^ c.w) ^ (d.x ^ d.y ^ d.z ^ d.w);
  }
  for (; i < n16; i += stride) {
    const u4_t a = __builtin_nontemporal_load(p + i);
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (acc == 0x9E3779B9u)
    out[blockIdx.x] = acc;
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* __restrict__ p, uint32_t v, uint32_t n) {
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256)
    p[i] = v;
}

// ----------------------------------------------------------------------------
// Row gather and device re-layout.
// ----------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void gather_rows_kernel(const T* __restrict__ x, T* __restrict__ out, int k, GatherIndex idx) {
  const int r = blockIdx.x;
  const T* src = x + (size_t)idx.src[r] * k;
  T* dst = out + (size_t)r * k;
  for (int i = threadIdx.x; i < k; i += 256)
    dst[i] = src[i];
}


// ----------------------------------------------------------------------------
// Token embedding (quant_linear.metal:572-591, embedding_q4_k): output row t
// is row ids[t] of a Q4_K table kept in the tiled device layout, dequantised.
// One 256-thread workgroup per (block, row); thread e forms element e of the
// block from its byte (e / 64) * 32 + e % 32 (high nibble when e & 32) and
// sub-block e / 32, as (d * sc) * q - dmin * m with each product and the
// difference rounded once (no contraction; the CPU oracle's order).  Ids
// outside [0, n) give a zero row.
// ----------------------------------------------------------------------------
template <typename OutT>
__device__ __forceinline__ void embedding_elem(const uint8_t* __restrict__ w, int id, OutT* __restrict__ y, int n, int nb, int t, int b, int e) {
#pragma clang fp contract(off)
  float v = 0.0f;
  if (id >= 0 && id < n) {
    const int i = id & 15;
    const uint8_t* tb = w + ((size_t)(id >> 4) * nb + b) * kTileBlockBytes;
    const uint8_t* hd = tb + kHeaderOffset + 16 * i;
    const uint8_t* q12 = hd + 4;
    // 6-bit scale and min of sub-block j (quant_linear.metal:12-20).
    const int j = e >> 5;
    uint32_t sc, mn;
    if (j < 4) {
      sc = q12[j] & 63u;
      mn = q12[j + 4] & 63u;
    } else {
      sc = (q12[j + 4] & 15u) | ((uint32_t)(q12[j - 4] >> 6) << 4);
      mn = (uint32_t)(q12[j + 4] >> 4) | ((uint32_t)(q12[j] >> 6) << 4);
    }
    // Quant byte p of the GGUF record: lane 16 (p / 32) + i of slab (p / 16) & 1,
    // word (p / 4) & 3, with the word's two middle bytes swapped.
    const int p = (e >> 6) * 32 + (e & 31), o = p & 31, bw = o & 3;
    const int sbw = bw == 1 ? 2 : bw == 2 ? 1 : bw;
    const uint8_t qb = tb[(o >> 4) * kSlabBytes + 16 * (16 * (p >> 5) + i) + (o & 12) + sbw];
    const uint32_t q = (e & 32) ? (uint32_t)(qb >> 4) : (uint32_t)(qb & 15);
    const float d = half_bits_to_float((uint32_t)hd[0] | ((uint32_t)hd[1] << 8));
    const float dmin = half_bits_to_float((uint32_t)hd[2] | ((uint32_t)hd[3] << 8));
    const float dsc = d * (float)sc;
    const float val = dsc * (float)q;
    const float mterm = dmin * (float)mn;
    v = val - mterm;
  }
  store_elem(y, (size_t)t * nb * 256 + (size_t)b * 256 + e, v);
}

template <typename OutT>
__global__ __launch_bounds__(256) void embedding_kernel(const uint8_t* __restrict__ w, const int32_t* __restrict__ ids, OutT* __restrict__ y, int n,
                                                        int nb) {
  embedding_elem(w, ids[blockIdx.y], y, n, nb, (int)blockIdx.y, (int)blockIdx.x, (int)threadIdx.x);
}

// The same over a packed batch, each row's token resolved in the kernel
// (quant_linear.metal:577-584 mode 0 with queryRow, batch.hpp:19-23): row t
// belongs to the first query q with t < start[q] + count[q] and takes the
// request buffer's token tokens[slot[q] * capacity + position[q] + t -
// start[q]].
template <typename OutT>
__global__ __launch_bounds__(256) void embedding_batch_kernel(const uint8_t* __restrict__ w, const int32_t* __restrict__ tokens, OutT* __restrict__ y,
                                                              int n, int nb, EmbedQueries qs) {
  const uint32_t t = blockIdx.y;
  uint32_t q = 0;
  while (q + 1 < qs.n && t >= qs.start[q] + qs.count[q])
    ++q;
  const int id = tokens[(size_t)qs.slot[q] * qs.capacity + qs.position[q] + (t - qs.start[q])];
  embedding_elem(w, id, y, n, nb, (int)t, (int)blockIdx.x, (int)threadIdx.x);
}

// ----------------------------------------------------------------------------
// RMS norm (native_ops.metal:6-40): y[r] = x[s] * rsqrt(sum(x[s]^2) / k + eps)
// * w, s = idx.src[r] for rms_norm_gather (the LM-head rows, batch.hpp:25-29)
// or s = r.  One 256-thread workgroup per output row; fp32 sum of squares
// (wave shuffle reduction, then across the 4 waves).  Rows of up to
// 256 * kNormRegs elements stay in registers between the two passes (one
// read of x); longer rows are read again.
// ----------------------------------------------------------------------------
constexpr int kNormRegs = 16;

template <typename T>
__global__ __launch_bounds__(256) void rms_norm_kernel(const T* __restrict__ x, const float* __restrict__ w, T* y, int k, float eps, GatherIndex idx,
                                                       int gather) {
  __shared__ float part[4];
  const int r = blockIdx.x, tid = threadIdx.x;
  const T* xr = x + (size_t)(gather ? idx.src[r] : (uint32_t)r) * k;
  float v[kNormRegs];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormRegs; ++i) {
    const int d = tid + 256 * i;
    v[i] = d < k ? (float)xr[d] : 0.0f;
    ss = fmaf(v[i], v[i], ss);
  }
  for (int d = tid + 256 * kNormRegs; d < k; d += 256) {
    const float t = (float)xr[d];
    ss = fmaf(t, t, ss);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    ss += __shfl_xor(ss, off);
  if ((tid & 63) == 0)
    part[tid >> 6] = ss;
  __syncthreads();
  const float total = (part[0] + part[1]) + (part[2] + part[3]);
  const float scale = 1.0f / sqrtf(total / (float)k + eps);
  T* yr = y + (size_t)r * k;
#pragma unroll
  for (int i = 0; i < kNormRegs; ++i) {
    const int d = tid + 256 * i;
    if (d < k)
      yr[d] = (T)((v[i] * scale) * w[d]);
  }
  for (int d = tid + 256 * kNormRegs; d < k; d += 256)
    yr[d] = (T)(((float)xr[d] * scale) * w[d]);
}

__device__ __forceinline__ uint32_t swap_middle_bytes(uint32_t v) {
  return (v & 0xff0000ffu) | ((v & 0x0000ff00u) << 8) | ((v & 0x00ff0000u) >> 8);
}

// One workgroup of 64 lanes per tile-block.
__global__ __launch_bounds__(64) void relayout_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t n, uint32_t nb) {
  const size_t tb = blockIdx.x;
  const uint32_t c = (uint32_t)(tb / nb), b = (uint32_t)(tb % nb);
  const int lane = threadIdx.x, i = lane & 15, g = lane >> 4;
  const uint8_t* blk = src + ((size_t)(16 * c + i) * nb + b) * kBlockBytes;
  uint8_t* out = dst + tb * kTileBlockBytes;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint8_t* q = blk + 16 + 32 * g + 16 * h;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = swap_middle_bytes((uint32_t)q[4 * j] | ((uint32_t)q[4 * j + 1] << 8) | ((uint32_t)q[4 * j + 2] << 16) | ((uint32_t)q[4 * j + 3] << 24));
    *reinterpret_cast<u4_t*>(out + h * kSlabBytes + 16 * lane) = u4_t{w[0], w[1], w[2], w[3]};
  }
  if (g == 0) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = (uint32_t)blk[4 * j] | ((uint32_t)blk[4 * j + 1] << 8) | ((uint32_t)blk[4 * j + 2] << 16) | ((uint32_t)blk[4 * j + 3] << 24);
    *reinterpret_cast<u4_t*>(out + kHeaderOffset + 16 * i) = u4_t{w[0], w[1], w[2], w[3]};
  }
}

// ----------------------------------------------------------------------------
// The other GGUF types on the same linear() surface: Q6_K (the LM head of real
// files, mixed-type down projections), Q8_0, Q5_K and IQ4_XS
// (quant_linear.metal:50-115 dequant, :329-570 decode GEMVs, :620-662 shapes;
// fused_kernels.metal:80-200).
//
// GEMV for m <= 8 rows (decode, small prefill, LM head) over the decode pack
// of x (hi / lo fp16 rows 0..7 / 8..15, per-(row, block) power-of-two scale;
// the sub-block sums for the Q5_K min term).  A format policy F supplies the
// per-lane registers of one tile-block (U), their loads, and `mac`: the eight
// B operands of v_mfma_f32_16x16x32_f16 in fp16, the MFMAs, and the tile-
// block's contribution scaled into the lane's four accumulator rows:
//   Q6_K   (q - 32) * sc per dword: (w & 0x03F003F0) | 0x6400 = 1024 + 16q for
//          two quants stored at bits 4..9 of each half, one v_pk_fma_f16 with
//          (sc / 16, -96 sc); d * row unscale after the MFMAs.
//   Q8_0   q * d per dword: v_perm_b32 of two biased bytes with 0x64 bytes is
//          1024 + 128 + q; v_pk_add_f16 -1152 leaves q, v_pk_mul_f16 by the
//          record's d (one rounding); row unscale after the MFMAs.
//   Q5_K   the Q4_K nibble decode with the fifth bit or'ed into the fp16 bias
//          (16 for low nibbles, 256 for high ones), q * sc exact (<= 1953), the
//          min term on a 16x16x16 MFMA of the sub-block sums.
//   IQ4_XS codebook lookup of four indices per v_perm_b32 pair (entries 0..7,
//          8..15, selected by bit 3 with v_bfi_b32), biased bytes to fp16 as for
//          Q8_0, one v_pk_fma_f16 with (ls - 32, -1152 (ls - 32)).
// Products above 2048 in magnitude (Q6_K, IQ4_XS) and q * d (Q8_0) are
// rounded once to fp16; the reference's prefill tiles round every dequantised
// weight to fp16 (quant_linear.metal:65,83,98,112).
//
// Workgroup = 8 waves; wave w takes blocks w, w + 8, ...  The persistent form
// (K = 4096, 16 blocks: two per wave) keeps each wave's x fragments in
// registers and streams every item (T column tiles) it owns through one
// register window that runs across item boundaries; partial sums alternate
// between two LDS buffers, one barrier per item.  The other form (any K)
// takes one item per workgroup, double-buffers the next block's x fragments
// and streams its T tile-blocks per block through a window DQ deep.
// ----------------------------------------------------------------------------

struct XF {
  h8_t f[8];
  float dv[4];
  h4_t xs;
};

template <bool MIN>
__device__ __forceinline__ void load_xf(XF& xf, const DecodePack& pk, size_t b, int lane) {
  const u4_t* fr = pk.frag + b * 8 * 64 + lane;
#pragma unroll
  for (int fs = 0; fs < 8; ++fs)
    xf.f[fs] = __builtin_bit_cast(h8_t, fr[fs * 64]);
  const float* ds = pk.dsc + b * 8 + 4 * ((lane >> 4) & 1);
#pragma unroll
  for (int v = 0; v < 4; ++v)
    xf.dv[v] = ds[v];
  if constexpr (MIN)
    xf.xs = pk.xs[b * 64 + lane];
}

__device__ __forceinline__ h2_t h2_splat(float v) {
  return h2_t{(_Float16)v, (_Float16)v};
}

// Outputs o = 8a .. 8a+7 of Q6_K triple (A, B, C) times their scale: b0 = MFMA
// 2a's four B dwords, b1 = MFMA 2a + 1's (layout in q4k_internal.h).
__device__ __forceinline__ void q6_triple(uint32_t A, uint32_t B, uint32_t C, h2_t mul, h2_t add, h8_t& b0, h8_t& b1) {
  const uint32_t m6 = 0x03F003F0u, m4 = 0x00F000F0u, m2 = 0x03000300u, magic = 0x64006400u;
  const uint32_t o0 = and_or(A, m6, magic), o1 = and_or(A >> 6, m6, magic);
  const uint32_t o2 = and_or(B, m6, magic), o3 = and_or(B >> 6, m6, magic);
  const uint32_t o4 = and_or(C, m6, magic), o5 = and_or(C >> 6, m6, magic);
  const uint32_t o6 = and_or(A << 4, m4, and_or(B << 8, m2, magic));
  const uint32_t o7 = and_or(C << 4, m4, and_or(B << 6, m2, magic));
  auto f = [&](uint32_t o) { return as_u32(__builtin_elementwise_fma(as_h2(o), mul, add)); };
  b0 = __builtin_bit_cast(h8_t, u4_t{f(o0), f(o1), f(o2), f(o3)});
  b1 = __builtin_bit_cast(h8_t, u4_t{f(o4), f(o5), f(o6), f(o7)});
}

// Each policy also names the shape of its persistent form: kPW waves (16:
// one block of x each, within 128 VGPRs, four waves per SIMD; 8: two blocks
// each, two waves per SIMD) and kPT column tiles per item, the measured best
// that does not spill.
struct FmtQ6K {
  static constexpr int kTB = kQ6TileBlockBytes;
  static constexpr bool kMin = false;
  static constexpr int kPW = 16, kPT = 2;
  struct U {
    u4_t s0, s1, s2;
    uint32_t sc, d;
  };
  static __device__ __forceinline__ void load(U& u, const uint8_t* src, int lane) {
    u.s0 = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src) + lane);
    u.s1 = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src + 1024) + lane);
    u.s2 = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src + 2048) + lane);
    u.sc = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(src + kQ6ScaleOffset) + lane);
    u.d = *(reinterpret_cast<const uint16_t*>(src + kQ6DOffset) + (lane & 15));
  }
  static __device__ __forceinline__ void mac(const U& u, const XF& x, int, f4_t& acc) {
    const float d = half_bits_to_float(u.d & 0xffffu);
    f4_t c0 = f4_t{0.0f, 0.0f, 0.0f, 0.0f}, c1 = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // Triple tr = dwords 3tr..3tr+2 of the lane's twelve (named directly: a
    // local array of them is not always kept in registers).
    auto triple = [&](int tr, uint32_t A, uint32_t B, uint32_t C) {
      // fp16 1152 + sc -> sc / 16 (exact), and -96 sc.
      const uint32_t sel = 0x04000400u | (uint32_t)tr | ((uint32_t)tr << 16);
      const h2_t p = as_h2(__builtin_amdgcn_perm(0x64646464u, u.sc, sel));
      const h2_t mul = __builtin_elementwise_fma(p, h2_splat(0.0625f), h2_splat(-72.0f));
      const h2_t add = mul * h2_splat(-1536.0f);
      h8_t b0, b1;
      q6_triple(A, B, C, mul, add, b0, b1);
      c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(x.f[2 * tr], b0, c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(x.f[2 * tr + 1], b1, c1, 0, 0, 0);
    };
    triple(0, u.s0[0], u.s0[1], u.s0[2]);
    triple(1, u.s0[3], u.s1[0], u.s1[1]);
    triple(2, u.s1[2], u.s1[3], u.s2[0]);
    triple(3, u.s2[1], u.s2[2], u.s2[3]);
#pragma unroll
    for (int v = 0; v < 4; ++v)
      acc[v] = fmaf(c0[v] + c1[v], d * x.dv[v], acc[v]);
  }
};

struct FmtQ8_0 {
  static constexpr int kTB = kTileN * kQ8BlockBytes;
  static constexpr bool kMin = false;
  static constexpr int kPW = 16, kPT = 2;
  struct U {
    u4_t s[4];
    uint32_t d;
  };
  static __device__ __forceinline__ void load(U& u, const uint8_t* src, int lane) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      u.s[j] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src + 1024 * j) + lane);
    u.d = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(src + 4096) + lane);
  }
  static __device__ __forceinline__ void mac(const U& u, const XF& x, int, f4_t& acc) {
    // d of the lane's two records, each in both halves.
    const h2_t d0 = as_h2(__builtin_amdgcn_perm(u.d, u.d, 0x01000100u)), d1 = as_h2(__builtin_amdgcn_perm(u.d, u.d, 0x03020302u));
    const h2_t k1152 = h2_splat(-1152.0f);
    f4_t c0 = f4_t{0.0f, 0.0f, 0.0f, 0.0f}, c1 = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int fs = 0; fs < 8; ++fs) {
      const u4_t sl = u.s[fs >> 1];
      const uint32_t w0 = sl[2 * (fs & 1)], w1 = sl[2 * (fs & 1) + 1];
      const h2_t d = fs < 4 ? d0 : d1;
      auto q = [&](uint32_t w, uint32_t sel) { return as_u32((as_h2(__builtin_amdgcn_perm(0x64646464u, w, sel)) + k1152) * d); };
      const h8_t b = __builtin_bit_cast(h8_t, u4_t{q(w0, 0x04010400u), q(w0, 0x04030402u), q(w1, 0x04010400u), q(w1, 0x04030402u)});
      if (fs & 1)
        c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(x.f[fs], b, c1, 0, 0, 0);
      else
        c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(x.f[fs], b, c0, 0, 0, 0);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v)
      acc[v] = fmaf(c0[v] + c1[v], x.dv[v], acc[v]);
  }
};

struct FmtQ5K {
  static constexpr int kTB = kTileN * kQ5BlockBytes;
  static constexpr bool kMin = true;
  static constexpr int kPW = 8, kPT = 2;
  struct U {
    u4_t q0, q1, hd;
    uint32_t h0, h1;
  };
  static __device__ __forceinline__ void load(U& u, const uint8_t* src, int lane) {
    u.q0 = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src) + lane);
    u.q1 = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src + kSlabBytes) + lane);
    u.hd = *(reinterpret_cast<const u4_t*>(src + kHeaderOffset) + (lane & 15));
    typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
    const u2_t h = __builtin_nontemporal_load(reinterpret_cast<const u2_t*>(src + 2304) + lane);
    u.h0 = h[0];
    u.h1 = h[1];
  }
  // Fifth bits of B dword k (= 4 (fs % 4) + t) moved to bit P of each half,
  // or'ed with the fp16 bias 0x6400.
  template <int P>
  static __device__ __forceinline__ uint32_t bias(uint32_t h, int k) {
    const uint32_t moved = k < P ? h << (P - k) : h >> (k - P);
    return and_or(moved, (1u << P) | (1u << (16 + P)), 0x64006400u);
  }
  static __device__ __forceinline__ void mac(const U& u, const XF& x, int lane, f4_t& acc) {
    const BlockConsts kc = block_consts(u.hd, lane >> 4);
    f4_t cl = f4_t{0.0f, 0.0f, 0.0f, 0.0f}, ch = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u4_t qq = s < 2 ? u.q0 : u.q1;
      const uint32_t wa = qq[2 * (s & 1)], wb = qq[2 * (s & 1) + 1];
      const uint32_t src[4] = {wa, wa >> 8, wb, wb >> 8};
      u4_t lo, hi;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        lo[t] = as_u32(__builtin_elementwise_fma(as_h2(and_or(src[t], 0x000F000Fu, bias<4>(u.h0, 4 * s + t))), kc.mul_lo, kc.add_lo));
        hi[t] = as_u32(__builtin_elementwise_fma(as_h2(and_or(src[t], 0x00F000F0u, bias<8>(u.h1, 4 * s + t))), kc.mul_hi, kc.add_hi));
      }
      cl = __builtin_amdgcn_mfma_f32_16x16x32_f16(x.f[s], __builtin_bit_cast(h8_t, lo), cl, 0, 0, 0);
      ch = __builtin_amdgcn_mfma_f32_16x16x32_f16(x.f[4 + s], __builtin_bit_cast(h8_t, hi), ch, 0, 0, 0);
    }
    const f4_t cm = __builtin_amdgcn_mfma_f32_16x16x16f16(x.xs, kc.bmin, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < 4; ++v)
      acc[v] += fmaf(kc.d, cl[v] + ch[v], -kc.dmin * cm[v]) * x.dv[v];
  }
};

// Q4_K itself in the same form (the tiled layout of q4k_internal.h), for the
// wide decode projections (the LM head) the persistent form serves best.
struct FmtQ4K {
  static constexpr int kTB = kTileBlockBytes;
  static constexpr bool kMin = true;
  static constexpr int kPW = 16, kPT = 2;
  struct U {
    u4_t q0, q1, hd;
  };
  static __device__ __forceinline__ void load(U& u, const uint8_t* src, int lane) {
    u.q0 = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src) + lane);
    u.q1 = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src + kSlabBytes) + lane);
    u.hd = *(reinterpret_cast<const u4_t*>(src + kHeaderOffset) + (lane & 15));
  }
  static __device__ __forceinline__ void mac(const U& u, const XF& x, int lane, f4_t& acc) {
    const BlockConsts kc = block_consts(u.hd, lane >> 4);
    f4_t cl = f4_t{0.0f, 0.0f, 0.0f, 0.0f}, ch = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u4_t qq = s < 2 ? u.q0 : u.q1;
      const uint32_t wa = qq[2 * (s & 1)], wb = qq[2 * (s & 1) + 1];
      const h8_t blo = quant_times_scale(wa, wb, 0x000F000Fu, 0x64006400u, kc.mul_lo, kc.add_lo);
      const h8_t bhi = quant_times_scale(wa, wb, 0x00F000F0u, 0x64006400u, kc.mul_hi, kc.add_hi);
      cl = __builtin_amdgcn_mfma_f32_16x16x32_f16(x.f[s], blo, cl, 0, 0, 0);
      ch = __builtin_amdgcn_mfma_f32_16x16x32_f16(x.f[4 + s], bhi, ch, 0, 0, 0);
    }
    const f4_t cm = __builtin_amdgcn_mfma_f32_16x16x16f16(x.xs, kc.bmin, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < 4; ++v)
      acc[v] += fmaf(kc.d, cl[v] + ch[v], -kc.dmin * cm[v]) * x.dv[v];
  }
};

struct FmtIQ4XS {
  static constexpr int kTB = kTileN * kIQ4BlockBytes;
  static constexpr bool kMin = false;
  static constexpr int kPW = 16, kPT = 2;
  struct U {
    u4_t q0, q1;
    uint2 hd;
  };
  static __device__ __forceinline__ void load(U& u, const uint8_t* src, int lane) {
    u.q0 = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src) + lane);
    u.q1 = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(src + 1024) + lane);
    u.hd = *(reinterpret_cast<const uint2*>(src + 2048) + (lane & 15));
  }
  // Codebook entries (iq4nl, quant_linear.metal:5) + 128 as bytes, four per word.
  static constexpr uint32_t kT0 = 0x3F2D1801u, kT1 = 0x766A5D4Fu, kT2 = 0xA6998D81u, kT3 = 0xF1D9C5B5u;
  // Four codebook bytes for the four 4-bit indices at bits 0..3 of each byte of w.
  static __device__ __forceinline__ uint32_t lookup(uint32_t w) {
    const uint32_t t = w & 0x07070707u;
    const uint32_t a = __builtin_amdgcn_perm(kT1, kT0, t), b = __builtin_amdgcn_perm(kT3, kT2, t);
    // Selector byte 0x0C gives 0x00, 0x0D gives 0xFF: a byte mask of bit 3.
    const uint32_t m = __builtin_amdgcn_perm(0u, 0u, and_or(w >> 3, 0x01010101u, 0x0C0C0C0Cu));
    return (m & b) | (~m & a);
  }
  // The same for the indices at bits 4..7 of each byte.  Bit 3 of index b is
  // bit 7 of byte b, which selectors 8..11 turn into a byte mask directly
  // (0x00 or 0xFF from bit 15 / 31 of the second source, bit 15 / 31 of the
  // first): bytes 1, 3 from w, bytes 0, 2 from w << 8.
  static __device__ __forceinline__ uint32_t lookup_hi(uint32_t w) {
    const uint32_t t = (w >> 4) & 0x07070707u;
    const uint32_t a = __builtin_amdgcn_perm(kT1, kT0, t), b = __builtin_amdgcn_perm(kT3, kT2, t);
    const uint32_t m = __builtin_amdgcn_perm(w << 8, w, 0x090B080Au);
    return (m & b) | (~m & a);
  }
  static __device__ __forceinline__ void mac(const U& u, const XF& x, int lane, f4_t& acc) {
    const int g = lane >> 4;
    const uint32_t sh = u.hd.x >> 16, sl = u.hd.y;
    const float d = half_bits_to_float(u.hd.x & 0xffffu);
    // ls - 32 of sub-blocks 2g (MFMAs 0..3) and 2g + 1 (MFMAs 4..7).
    const int j0 = 2 * g;
    const int ls0 = (int)(((sl >> (4 * j0)) & 15u) | (((sh >> (2 * j0)) & 3u) << 4)) - 32;
    const int ls1 = (int)(((sl >> (4 * j0 + 4)) & 15u) | (((sh >> (2 * j0 + 2)) & 3u) << 4)) - 32;
    const h2_t mul0 = h2_splat((float)ls0), mul1 = h2_splat((float)ls1);
    const h2_t add0 = mul0 * h2_splat(-1152.0f), add1 = mul1 * h2_splat(-1152.0f);
    f4_t c0 = f4_t{0.0f, 0.0f, 0.0f, 0.0f}, c1 = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int fs = 0; fs < 8; ++fs) {
      const uint32_t w = (fs < 4 ? u.q0 : u.q1)[fs & 3];
      const uint32_t vlo = lookup(w), vhi = lookup_hi(w);
      const h2_t mul = fs < 4 ? mul0 : mul1, add = fs < 4 ? add0 : add1;
      auto f = [&](uint32_t v, uint32_t sel) {
        return as_u32(__builtin_elementwise_fma(as_h2(__builtin_amdgcn_perm(0x64646464u, v, sel)), mul, add));
      };
      const h8_t b = __builtin_bit_cast(h8_t, u4_t{f(vlo, 0x04010400u), f(vlo, 0x04030402u), f(vhi, 0x04010400u), f(vhi, 0x04030402u)});
      if (fs & 1)
        c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(x.f[fs], b, c1, 0, 0, 0);
      else
        c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(x.f[fs], b, c0, 0, 0, 0);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v)
      acc[v] = fmaf(c0[v] + c1[v], d * x.dv[v], acc[v]);
  }
};

template <typename OutT, int W = 8>
__device__ __forceinline__ void typed_epilogue(const GemvArgs& a, const float* part, int t_count, int tile0, int ntiles) {
  OutT* y = reinterpret_cast<OutT*>(a.y);
  const OutT* aux = reinterpret_cast<const OutT*>(a.aux);
  const int tid = threadIdx.x;
  for (int o = tid; o < a.m * 16 * t_count; o += 64 * W) {
    const int row = o / (16 * t_count), c = o % (16 * t_count), t = c >> 4, cc = c & 15;
    if (tile0 + t >= ntiles)
      continue;
    float acc_v = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w)
      acc_v += part[((w * t_count + t) * 8 + row) * 16 + cc];
    if (sizeof(OutT) == 2)
      acc_v = round_half(acc_v);
    const size_t off = (size_t)row * a.n + (size_t)(tile0 + t) * 16 + cc;
    const float out = a.post == 1 ? acc_v + load_elem(aux, off) : a.post == 2 ? silu(load_elem(aux, off)) * acc_v : acc_v;
    store_elem(y, off, out);
  }
}

// Fused gate/up GEMV of a weight type with a fused decode kernel in the
// reference (Q5_K, IQ4_XS: fused_kernels.metal:80-143, 145-200): the Q4_K
// item's x packing and epilogue (gate_up_pack_x, gate_up_finish) around the
// type's tile-block units (F::load, F::mac), two units in flight per wave.
template <class F, int T, typename OutT, bool NORM>
__device__ __forceinline__ void typed_gate_up_item(const GemvArgs& a, float* xl, float (*ssq)[8], int item) {
  constexpr int W = 8, BPW = 2, NM = 2, MT = NM * T, U = BPW * MT, DQ = 2;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nb = a.nb, bw = ((wave + item) % W) * BPW;
  const size_t tile_bytes = (size_t)nb * F::kTB;
  typename F::U un[U];
  auto issue_unit = [&](int u) {
    const int j = u / MT, mt = u - j * MT, mi = mt / T, t = mt - mi * T;
    F::load(un[u], (mi ? a.wu : a.w) + ((size_t)item * T + t) * tile_bytes + (size_t)(bw + j) * F::kTB, lane);
    __builtin_amdgcn_sched_barrier(0);
  };
  XBlock xb[BPW];
  gate_up_pack_x<OutT, NORM, W, BPW>(a, xl, ssq, bw, xb, [&] {
#pragma unroll
    for (int u = 0; u < (DQ < U ? DQ : U); ++u)
      issue_unit(u);
  });
  XF xf[BPW];
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
#pragma unroll
    for (int s = 0; s < 8; ++s)
      xf[j].f[s] = xb[j].frag[s];
    xf[j].xs = xb[j].xs;
#pragma unroll
    for (int v = 0; v < 4; ++v)
      xf[j].dv[v] = xb[j].dv[v];
  }
  f4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    acc[mt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int j = u / MT, mt = u - j * MT;
    __builtin_amdgcn_sched_barrier(0);
    if (u + DQ < U)
      issue_unit(u + DQ);
    F::mac(un[u], xf[j], lane, acc[mt]);
  }
  gate_up_finish<T, OutT, W, BPW>(a, xl, acc, item);
}

template <class F, int T, typename OutT, bool NORM>
__global__ __launch_bounds__(512) void typed_gate_up_kernel(GemvArgs a) {
  __shared__ __attribute__((aligned(16))) float xl[8 * gu_wave_floats<2>()];
  __shared__ float ssq[8][8];
  typed_gate_up_item<F, T, OutT, NORM>(a, xl, ssq, blockIdx.x);
}

template <class F, int T, int DQ, typename OutT>
__global__ __launch_bounds__(512) void typed_gemv_kernel(GemvArgs a) {
  constexpr int W = 8;
  static_assert(DQ <= T || T == 1, "window");
  constexpr int D = DQ < T ? DQ : T;
  __shared__ float part[W][T][8][16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, col = lane & 15;
  const int nb = a.nb, ntiles = a.n >> 4, tile0 = blockIdx.x * T;
  const size_t tile_bytes = (size_t)nb * F::kTB;
  const int nbw = wave < nb ? (nb - 1 - wave) / W + 1 : 0;

  typename F::U ring[T];
  auto issue = [&](int t, int bi) {
    const int tile = tile0 + t < ntiles ? tile0 + t : ntiles - 1;
    F::load(ring[t], a.w + (size_t)tile * tile_bytes + (size_t)(wave + W * bi) * F::kTB, lane);
  };
  f4_t acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t)
    acc[t] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
  if (nbw > 0) {
    XF xc, xn;
    load_xf<F::kMin>(xc, a.pack, (size_t)wave, lane);
#pragma unroll
    for (int t = 0; t < D; ++t)
      issue(t, 0);
    for (int bi = 0; bi < nbw; ++bi) {
      const bool more = bi + 1 < nbw;
      if (more)
        load_xf<F::kMin>(xn, a.pack, (size_t)(wave + W * (bi + 1)), lane);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        // Take slot t before the window's next issue, which may reuse it.
        const typename F::U cur = ring[t];
        const int tn = t + D;
        if (tn < T)
          issue(tn, bi);
        else if (more)
          issue(tn - T, bi + 1);
        F::mac(cur, xc, lane, acc[t]);
      }
      if (more)
        xc = xn;
    }
  }
  // C row 4g + v: lanes g < 2 add the low parts held 32 lanes up.
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float tot = acc[t][v] + __shfl_xor(acc[t][v], 32);
      if (g < 2)
        part[wave][t][4 * g + v][col] = tot;
    }
  __syncthreads();
  typed_epilogue<OutT>(a, &part[0][0][0][0], T, tile0, ntiles);
}

template <class F, int T, int DQ, int W, typename OutT>
__global__ __launch_bounds__(64 * W) void typed_gemv_persistent_kernel(GemvArgs a, int items) {
  constexpr int BPW = 16 / W, U = BPW * T;
  static_assert(W * BPW == 16 && DQ <= U, "16 blocks; window");
  __shared__ float part[2][W][T][8][16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, col = lane & 15;
  const int ntiles = a.n >> 4;
  const size_t tile_bytes = (size_t)(W * BPW) * F::kTB;
  int item = blockIdx.x;
  if (item >= items)
    return;

  XF xf[BPW];
#pragma unroll
  for (int j = 0; j < BPW; ++j)
    load_xf<F::kMin>(xf[j], a.pack, (size_t)(wave + W * j), lane);
  typename F::U ring[U];
  auto issue = [&](int u, int it) {
    const int j = u / T, t = u - j * T;
    const int tile = it * T + t < ntiles ? it * T + t : ntiles - 1;
    F::load(ring[u], a.w + (size_t)tile * tile_bytes + (size_t)(wave + W * j) * F::kTB, lane);
  };
#pragma unroll
  for (int u = 0; u < DQ; ++u)
    issue(u, item);
  for (int it = 0; item < items; ++it, item += gridDim.x) {
    const int next = item + (int)gridDim.x;
    f4_t acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t)
      acc[t] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = u / T, t = u - j * T;
      const typename F::U cur = ring[u];
      if (u + DQ < U)
        issue(u + DQ, item);
      else if (next < items)
        issue(u + DQ - U, next);
      F::mac(cur, xf[j], lane, acc[t]);
    }
    float(*pb)[T][8][16] = part[it & 1];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float tot = acc[t][v] + __shfl_xor(acc[t][v], 32);
        if (g < 2)
          pb[wave][t][4 * g + v][col] = tot;
      }
    __syncthreads();
    typed_epilogue<OutT, W>(a, &pb[0][0][0][0], T, item * T, ntiles);
  }
}

// ----------------------------------------------------------------------------
// Prefill GEMM for the other weight types (Q5_K, Q6_K, Q8_0, IQ4_XS).
//
// The pipelined GEMM of the Q4_K path with its B operand taken from a policy
// of the type's tile-block (layouts in q4k_internal.h): the same A ring over
// the activations in the GEMM staging order, a private 2-block B ring per
// wave filled by LDS-DMA, and per u-step u the B fragments of MFMA fs = u
// (low) and fs = 4 + u (high) of each column tile dequantised in registers to
// the reference's prefill tile value (quant_linear.metal:49-115): its fp32
// expression rounded once to fp16, bit for bit.
//   Q5_K   h(d*sc*(q + 16h) - dmin*m): q + 16h as an fp16 denormal (as the
//          Q4_K nibbles), then one fp32 fma with d*sc*2^24 and -dmin*m (both
//          exact), the single fp32 rounding of the reference's expression.
//   Q6_K   h(d*sc*(q - 32)): the product has at most 23 significant bits, so
//          fma(64 + q, d*sc, -96 d*sc) is exact.
//   Q8_0   h(d*q): 19 bits; one fp16 multiply rounds the exact product once.
//   IQ4_XS h(d*(ls - 32)*v): 23 bits; fma(1152 + v, dl, -1152 dl) is exact.
// Per type: kCT column tiles per wave and kAS A ring slots (A loaded kAS - 1
// u-steps ahead), so that both rings fit the 160 KB of LDS; kNL DMA loads per
// tile-block; kVPM vector instructions scheduled after each MFMA (measured:
// 2 for Q5_K, Q6_K and Q8_0, 3-5 percent faster than 3 or 4 at M = 2048; 4
// for IQ4_XS).  Column tiles past n (a multiple of 16, not of the
// workgroup's width) load the last tile and store nothing.  Wrappers set
// other widths: Narrow (2 tiles), Mid (3), Six (6, with a 3-slot A ring;
// also the gated Q4_K GEMM, GATED), and TgQ8_0W streams Q8_0's B in half
// tile-blocks so that four tiles fit.
// ----------------------------------------------------------------------------

// Bit `from` (and from + 16) of h moved to bit `to` (and to + 16).
__device__ __forceinline__ uint32_t move_bits(uint32_t h, int from, int to) {
  return from >= to ? h >> (from - to) : h << (to - from);
}

// Two fp16 pairs from four fp32 values, each rounded once: the four values
// are formed before either conversion (the empty asm keeps them apart from
// it), so that no conversion directly follows the v_fma_mix that wrote its
// source (that adjacency costs two wait states).
__device__ __forceinline__ void pack_h2x2(float a0, float a1, float b0, float b1, uint32_t& lo, uint32_t& hi) {
  asm("" : "+v"(a0), "+v"(a1), "+v"(b0), "+v"(b1));
  lo = as_u32(h2_t{(_Float16)a0, (_Float16)a1});
  hi = as_u32(h2_t{(_Float16)b0, (_Float16)b1});
}

__device__ __forceinline__ uint32_t lds_u32(const uint8_t* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}

struct TgQ5K {
  static constexpr int kTB = kTileN * kQ5BlockBytes, kCT = 4, kAS = 4, kNL = 5, kVPM = 2;
  struct R {
    u4_t hd;
    uint2 h;
  };
  struct K {
    float dl, cl, dh, ch;
    uint32_t h0, h1;
  };
  struct W {
    uint2 q;
  };
  static __device__ __forceinline__ void issue(const uint8_t* src, uint32_t v16, uint32_t v4, uint32_t l, int) {
    lds_dma16<0>(src, v16, l);
    lds_dma16<kSlabBytes>(src, v16, l);
    lds_dma4<kHeaderOffset>(src, v4, l);
    lds_dma4<2304>(src, v4, l);
    lds_dma4<2560>(src, v4, l);
  }
  static __device__ __forceinline__ void raw(R& r, const uint8_t* tb, int lane) {
    r.hd = *reinterpret_cast<const u4_t*>(tb + kHeaderOffset + 16 * (lane & 15));
    r.h = *reinterpret_cast<const uint2*>(tb + 2304 + 8 * lane);
  }
  // Sub-blocks 2g (low nibbles) and 2g + 1 (high nibbles): d * sc times
  // 2^24 (2^20), and -dmin * m.
  static __device__ __forceinline__ void consts(K& k, const R& r, int lane) {
    uint32_t p0, p1;
    scale_min_packed(r.hd, lane >> 4, p0, p1);
    const float d = half_bits_to_float(r.hd.x & 0xffffu), dm = half_bits_to_float(r.hd.x >> 16);
    k.dl = d * (float)(p0 & 0xffu) * 0x1p24f;
    k.cl = -dm * (float)((p0 >> 16) & 0xffu);
    k.dh = d * (float)(p1 & 0xffu) * 0x1p20f;
    k.ch = -dm * (float)((p1 >> 16) & 0xffu);
    k.h0 = r.h.x;
    k.h1 = r.h.y;
  }
  static __device__ __forceinline__ void words(W& w, const uint8_t* tb, int u, int lane) {
    w.q = *reinterpret_cast<const uint2*>(tb + (u >> 1) * kSlabBytes + 16 * lane + 8 * (u & 1));
  }
  // B dword t of MFMA u (low nibbles): fifth bits at bit 4u + t (+16) of h0;
  // of MFMA 4 + u (high nibbles): the same bits of h1.  The value is the fp16
  // denormal (q + 16h) * 2^-24 (low nibble at bit 0, fifth bit at bit 4) or
  // (q + 16h) * 2^-20 (nibble at bits 4..7, fifth bit at bit 8).
  static __device__ __forceinline__ void dequant(const K& k, const W& w, int u, h8_t& blo, h8_t& bhi) {
    const uint32_t lw[4] = {w.q.x, w.q.x >> 8, w.q.y, w.q.y >> 8};
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const h2_t ql = as_h2(and_or(lw[t], 0x000F000Fu, move_bits(k.h0, 4 * u + t, 4) & 0x00100010u));
      const h2_t qh = as_h2(and_or(lw[t], 0x00F000F0u, move_bits(k.h1, 4 * u + t, 8) & 0x01000100u));
      pack_h2x2(__builtin_fmaf((float)ql[0], k.dl, k.cl), __builtin_fmaf((float)ql[1], k.dl, k.cl), __builtin_fmaf((float)qh[0], k.dh, k.ch),
                __builtin_fmaf((float)qh[1], k.dh, k.ch), lo[t], hi[t]);
    }
    blo = __builtin_bit_cast(h8_t, u4_t{lo[0], lo[1], lo[2], lo[3]});
    bhi = __builtin_bit_cast(h8_t, u4_t{hi[0], hi[1], hi[2], hi[3]});
  }
};

struct TgQ6K {
  static constexpr int kTB = kQ6TileBlockBytes, kCT = 4, kAS = 3, kNL = 5, kVPM = 2;
  struct R {
    uint32_t sc, d;
  };
  // d * sc of the lane's four scale bytes (MFMAs u and 4 + u take bytes u / 2
  // and 2 + u / 2), formed once per block.
  struct K {
    float ds[4];
  };
  // Triples u / 2 (MFMA u) and 2 + u / 2 (MFMA 4 + u); C only for odd u.
  struct W {
    uint32_t a0, b0, c0, a1, b1, c1;
  };
  static __device__ __forceinline__ void issue(const uint8_t* src, uint32_t v16, uint32_t v4, uint32_t l, int lane) {
    lds_dma16<0>(src, v16, l);
    lds_dma16<1024>(src, v16, l);
    lds_dma16<2048>(src, v16, l);
    lds_dma4<kQ6ScaleOffset>(src, v4, l);
    if (lane < 8)  // the 16 rows' d: 32 bytes
      lds_dma4<kQ6DOffset>(src, v4, l);
  }
  static __device__ __forceinline__ void raw(R& r, const uint8_t* tb, int lane) {
    r.sc = lds_u32(tb + kQ6ScaleOffset + 4 * lane);
    r.d = *reinterpret_cast<const uint16_t*>(tb + kQ6DOffset + 2 * (lane & 15));
  }
  // Scale byte i is stored sc + 128: d * sc = fma(sc + 128, d, -128 d), exact.
  static __device__ __forceinline__ void consts(K& k, const R& r, int) {
    const float d = half_bits_to_float(r.d), m128 = -128.0f * d;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      k.ds[i] = __builtin_fmaf((float)((r.sc >> (8 * i)) & 0xffu), d, m128);
  }
  static __device__ __forceinline__ uint32_t dword(const uint8_t* tb, int j, int lane) {
    return lds_u32(tb + (j >> 2) * 1024 + 16 * lane + 4 * (j & 3));
  }
  static __device__ __forceinline__ void words(W& w, const uint8_t* tb, int u, int lane) {
    const int a = 3 * (u >> 1);
    w.a0 = dword(tb, a, lane);
    w.b0 = dword(tb, a + 1, lane);
    w.a1 = dword(tb, a + 6, lane);
    w.b1 = dword(tb, a + 7, lane);
    w.c0 = (u & 1) ? dword(tb, a + 2, lane) : 0u;
    w.c1 = (u & 1) ? dword(tb, a + 8, lane) : 0u;
  }
  // Outputs 8a + 4p .. 8a + 4p + 3 of triple (A, B, C) (p = u & 1) as fp16
  // 64 + q (bias 0x5400: bit 4 of a half is 1), then d*sc*(q - 32) exactly.
  static __device__ __forceinline__ h8_t triple(uint32_t A, uint32_t B, uint32_t C, int p, float ds) {
    const uint32_t m6 = 0x03F003F0u, m4 = 0x00F000F0u, m2 = 0x03000300u, bias = 0x54005400u;
    uint32_t o[4];
    if (p == 0) {
      o[0] = and_or(A, m6, bias);
      o[1] = and_or(A >> 6, m6, bias);
      o[2] = and_or(B, m6, bias);
      o[3] = and_or(B >> 6, m6, bias);
    } else {
      o[0] = and_or(C, m6, bias);
      o[1] = and_or(C >> 6, m6, bias);
      o[2] = and_or(A << 4, m4, and_or(B << 8, m2, bias));
      o[3] = and_or(C << 4, m4, and_or(B << 6, m2, bias));
    }
    const float c = -96.0f * ds;
    uint32_t r[4];
#pragma unroll
    for (int t = 0; t < 4; t += 2) {
      const h2_t q = as_h2(o[t]), p = as_h2(o[t + 1]);
      pack_h2x2(__builtin_fmaf((float)q[0], ds, c), __builtin_fmaf((float)q[1], ds, c), __builtin_fmaf((float)p[0], ds, c),
                __builtin_fmaf((float)p[1], ds, c), r[t], r[t + 1]);
    }
    return __builtin_bit_cast(h8_t, u4_t{r[0], r[1], r[2], r[3]});
  }
  // Scale of MFMA u: byte u / 2 of the lane's scale dword; of MFMA 4 + u:
  // byte 2 + u / 2.
  static __device__ __forceinline__ void dequant(const K& k, const W& w, int u, h8_t& blo, h8_t& bhi) {
    blo = triple(w.a0, w.b0, w.c0, u & 1, k.ds[u >> 1]);
    bhi = triple(w.a1, w.b1, w.c1, u & 1, k.ds[2 + (u >> 1)]);
  }
};

struct TgQ8_0 {
  static constexpr int kTB = kTileN * kQ8BlockBytes, kCT = 2, kAS = 5, kNL = 5, kVPM = 2;
  struct R {
    uint32_t dd;
  };
  struct K {
    h2_t dl, dh;
  };
  struct W {
    uint2 lo, hi;
  };
  static __device__ __forceinline__ void issue(const uint8_t* src, uint32_t v16, uint32_t v4, uint32_t l, int) {
    lds_dma16<0>(src, v16, l);
    lds_dma16<1024>(src, v16, l);
    lds_dma16<2048>(src, v16, l);
    lds_dma16<3072>(src, v16, l);
    lds_dma4<0>(src + 4096, v4, l + 4096);  // past the instruction offset's range
  }
  static __device__ __forceinline__ void raw(R& r, const uint8_t* tb, int lane) {
    r.dd = lds_u32(tb + 4096 + 4 * lane);
  }
  // d of records 2g (MFMAs 0..3) and 2g + 1 (MFMAs 4..7), in both halves.
  static __device__ __forceinline__ void consts(K& k, const R& r, int) {
    k.dl = as_h2(__builtin_amdgcn_perm(r.dd, r.dd, 0x01000100u));
    k.dh = as_h2(__builtin_amdgcn_perm(r.dd, r.dd, 0x03020302u));
  }
  static __device__ __forceinline__ void words(W& w, const uint8_t* tb, int u, int lane) {
    w.lo = *reinterpret_cast<const uint2*>(tb + (u >> 1) * 1024 + 16 * lane + 8 * (u & 1));
    w.hi = *reinterpret_cast<const uint2*>(tb + (2 + (u >> 1)) * 1024 + 16 * lane + 8 * (u & 1));
  }
  // Byte q ^ 0x80 as fp16 1024 + (q + 128), minus 1152 (exact), times d.
  static __device__ __forceinline__ h8_t frag(uint2 v, h2_t d) {
    auto q = [&](uint32_t x, uint32_t sel) { return as_u32((as_h2(__builtin_amdgcn_perm(0x64646464u, x, sel)) + h2_splat(-1152.0f)) * d); };
    return __builtin_bit_cast(h8_t, u4_t{q(v.x, 0x04010400u), q(v.x, 0x04030402u), q(v.y, 0x04010400u), q(v.y, 0x04030402u)});
  }
  static __device__ __forceinline__ void dequant(const K& k, const W& w, int, h8_t& blo, h8_t& bhi) {
    blo = frag(w.lo, k.dl);
    bhi = frag(w.hi, k.dh);
  }
};

// Q8_0 with four column tiles per wave: two blocks of its 4352-byte
// tile-blocks per column do not fit beside an A ring, so B streams in half
// tile-blocks through three half-slots per column (typed_gemm_tile_half).
// Half 0 of a tile-block holds the quant slabs of u-steps 0, 1 (slabs 0 and
// 2: the low and high MFMA fragments) and the d row, half 1 the slabs of
// u-steps 2, 3 (slabs 1 and 3).  A half-slot: [low slab 1 KB][high slab
// 1 KB][d row 256 B].
struct TgQ8_0W : TgQ8_0 {
  static constexpr int kCT = 4, kAS = 3, kHS = 2304, kL0 = 3, kL1 = 2;
  static constexpr bool kHalf = true;
  static __device__ __forceinline__ void issue_half0(const uint8_t* src, uint32_t v16, uint32_t v4, uint32_t l) {
    lds_dma16<0>(src, v16, l);
    lds_dma16<1024>(src + 1024, v16, l);  // slab 2 into [1 KB, 2 KB)
    lds_dma4<0>(src + 4096, v4, l + 2048);
  }
  static __device__ __forceinline__ void issue_half1(const uint8_t* src, uint32_t v16, uint32_t l) {
    lds_dma16<0>(src + 1024, v16, l);     // slab 1
    lds_dma16<1024>(src + 2048, v16, l);  // slab 3 into [1 KB, 2 KB)
  }
  static __device__ __forceinline__ void raw_half(R& r, const uint8_t* hs, int lane) {
    r.dd = lds_u32(hs + 2048 + 4 * lane);
  }
  static __device__ __forceinline__ void words_half(W& w, const uint8_t* hs, int u, int lane) {
    w.lo = *reinterpret_cast<const uint2*>(hs + 16 * lane + 8 * (u & 1));
    w.hi = *reinterpret_cast<const uint2*>(hs + 1024 + 16 * lane + 8 * (u & 1));
  }
};

template <class P, class = void>
struct TgIsHalf {
  static constexpr bool value = false;
};
template <class P>
struct TgIsHalf<P, decltype((void)P::kHalf)> {
  static constexpr bool value = P::kHalf;
};

struct TgIQ4XS {
  static constexpr int kTB = kTileN * kIQ4BlockBytes, kCT = 4, kAS = 5, kNL = 3, kVPM = 4;
  struct R {
    uint2 hd;
  };
  struct K {
    float dl, cl, dh, ch;
  };
  struct W {
    uint32_t lo, hi;
  };
  static __device__ __forceinline__ void issue(const uint8_t* src, uint32_t v16, uint32_t v4, uint32_t l, int lane) {
    lds_dma16<0>(src, v16, l);
    lds_dma16<1024>(src, v16, l);
    if (lane < 32)  // the 16 rows' 8-byte headers: 128 bytes
      lds_dma4<2048>(src, v4, l);
  }
  static __device__ __forceinline__ void raw(R& r, const uint8_t* tb, int lane) {
    r.hd = *reinterpret_cast<const uint2*>(tb + 2048 + 8 * (lane & 15));
  }
  // Sub-blocks 2g (MFMAs 0..3) and 2g + 1 (4..7): dl = d * (ls - 32) and
  // -1152 dl, both exact.
  static __device__ __forceinline__ void consts(K& k, const R& r, int lane) {
    const int j = 2 * (lane >> 4);
    const uint32_t sh = r.hd.x >> 16, sl = r.hd.y;
    const float d = half_bits_to_float(r.hd.x & 0xffffu);
    const int ls0 = (int)(((sl >> (4 * j)) & 15u) | (((sh >> (2 * j)) & 3u) << 4));
    const int ls1 = (int)(((sl >> (4 * j + 4)) & 15u) | (((sh >> (2 * j + 2)) & 3u) << 4));
    k.dl = d * (float)(ls0 - 32);
    k.cl = -1152.0f * k.dl;
    k.dh = d * (float)(ls1 - 32);
    k.ch = -1152.0f * k.dh;
  }
  static __device__ __forceinline__ void words(W& w, const uint8_t* tb, int u, int lane) {
    w.lo = lds_u32(tb + 16 * lane + 4 * u);
    w.hi = lds_u32(tb + 1024 + 16 * lane + 4 * u);
  }
  // Codebook value + 128 per byte (FmtIQ4XS::lookup) as fp16 1152 + v, then
  // dl * v exactly.
  static __device__ __forceinline__ h8_t frag(uint32_t wq, float dl, float cl) {
    const uint32_t vlo = FmtIQ4XS::lookup(wq), vhi = FmtIQ4XS::lookup_hi(wq);
    const uint32_t p[4] = {__builtin_amdgcn_perm(0x64646464u, vlo, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, vlo, 0x04030402u),
                           __builtin_amdgcn_perm(0x64646464u, vhi, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, vhi, 0x04030402u)};
    uint32_t r[4];
#pragma unroll
    for (int t = 0; t < 4; t += 2) {
      const h2_t v = as_h2(p[t]), w = as_h2(p[t + 1]);
      pack_h2x2(__builtin_fmaf((float)v[0], dl, cl), __builtin_fmaf((float)v[1], dl, cl), __builtin_fmaf((float)w[0], dl, cl),
                __builtin_fmaf((float)w[1], dl, cl), r[t], r[t + 1]);
    }
    return __builtin_bit_cast(h8_t, u4_t{r[0], r[1], r[2], r[3]});
  }
  static __device__ __forceinline__ void dequant(const K& k, const W& w, int, h8_t& blo, h8_t& bhi) {
    blo = frag(w.lo, k.dl, k.cl);
    bhi = frag(w.hi, k.dh, k.ch);
  }
};

// Q4_K on the same template, two column tiles per wave (128 columns per
// workgroup): for prefill grids that the 256-column Q4_K GEMM leaves short of
// the CUs.  The dequantisation is that GEMM's (fp16 denormal nibbles, one
// fp32 fma with d*sc*2^24 or d*sc*2^20 and -dmin*m): the reference's value
// exactly.
struct TgQ4K {
  static constexpr int kTB = kTileBlockBytes, kCT = 2, kAS = 5, kNL = 3, kVPM = 2;
  struct R {
    u4_t hd;
  };
  struct K {
    float dl, cl, dh, ch;
  };
  struct W {
    uint2 q;
  };
  static __device__ __forceinline__ void issue(const uint8_t* src, uint32_t v16, uint32_t v4, uint32_t l, int) {
    lds_dma16<0>(src, v16, l);
    lds_dma16<kSlabBytes>(src, v16, l);
    lds_dma4<kHeaderOffset>(src, v4, l);
  }
  static __device__ __forceinline__ void raw(R& r, const uint8_t* tb, int lane) {
    r.hd = *reinterpret_cast<const u4_t*>(tb + kHeaderOffset + 16 * (lane & 15));
  }
  static __device__ __forceinline__ void consts(K& k, const R& r, int lane) {
    uint32_t p0, p1;
    scale_min_packed(r.hd, lane >> 4, p0, p1);
    const float d = half_bits_to_float(r.hd.x & 0xffffu), dm = half_bits_to_float(r.hd.x >> 16);
    k.dl = d * (float)(p0 & 0xffu) * 0x1p24f;
    k.cl = -dm * (float)((p0 >> 16) & 0xffu);
    k.dh = d * (float)(p1 & 0xffu) * 0x1p20f;
    k.ch = -dm * (float)((p1 >> 16) & 0xffu);
  }
  static __device__ __forceinline__ void words(W& w, const uint8_t* tb, int u, int lane) {
    w.q = *reinterpret_cast<const uint2*>(tb + (u >> 1) * kSlabBytes + 16 * lane + 8 * (u & 1));
  }
  static __device__ __forceinline__ void dequant(const K& k, const W& w, int, h8_t& blo, h8_t& bhi) {
    const uint32_t lw[4] = {w.q.x, w.q.x >> 8, w.q.y, w.q.y >> 8};
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const h2_t ql = as_h2(lw[t] & 0x000F000Fu), qh = as_h2(lw[t] & 0x00F000F0u);
      pack_h2x2(__builtin_fmaf((float)ql[0], k.dl, k.cl), __builtin_fmaf((float)ql[1], k.dl, k.cl), __builtin_fmaf((float)qh[0], k.dh, k.ch),
                __builtin_fmaf((float)qh[1], k.dh, k.ch), lo[t], hi[t]);
    }
    blo = __builtin_bit_cast(h8_t, u4_t{lo[0], lo[1], lo[2], lo[3]});
    bhi = __builtin_bit_cast(h8_t, u4_t{hi[0], hi[1], hi[2], hi[3]});
  }
};

// A policy with two column tiles per wave (128 columns per workgroup) and a
// 5-slot A ring, for grids the 4-tile form leaves short of the CUs.
template <class P>
struct Narrow : P {
  static constexpr int kCT = 2, kAS = 5;
};

// Three column tiles per wave (192 columns per workgroup): the B ring is
// three quarters of the 4-tile form's, which leaves LDS for a deeper A ring
// (Q6_K: 5 slots instead of 3) or more MFMAs per A fragment read (Q8_0).
template <class P, int AS>
struct Mid : P {
  static constexpr int kCT = 3, kAS = AS;
};

// Six column tiles per wave (384 columns per workgroup, or 192 output
// columns of the gated GEMM: three gate and three up tiles) with a 3-slot A
// ring (156 KB of LDS with Q4_K, 150 KB with IQ4_XS): each A fragment read
// from LDS feeds six column tiles.
template <class P>
struct Six : P {
  static constexpr int kCT = 6, kAS = 3;
};
// IQ4_XS: six vector instructions per MFMA in the schedule (with 2 to 5 the
// plain GEMM's epilogue spills two VGPRs around the loop).
template <>
struct Six<TgIQ4XS> : TgIQ4XS {
  static constexpr int kCT = 6, kAS = 3, kVPM = 6;
};

// Load accounting of the typed GEMM.  A wave issues per u-step its 4 A
// fragments of A(t + kAS - 1) spread over its kCT column groups, each group's
// share followed, at u = 0, by the kNL loads of that column's tile-block of
// the next block.  vmcnt is in order, so A(t) has landed once no more than
// the loads issued after its last fragment are outstanding.
constexpr int tg_mod4(int v) {
  return ((v % 4) + 4) % 4;
}
constexpr int tg_step_loads(int u, int ct, int nl) {
  return 4 + (u == 0 ? ct * nl : 0);
}
// Loads issued after A(t)'s last fragment (issued at u-step t - ad) up to the
// top of u-step t, u = t % 4; at u = 3 also no more than the 8 loads of
// u-steps 1 and 2, which follow the next block's B (issued at u = 0).
constexpr int tg_wait(int u, int ad, int ct, int nl) {
  int n = tg_mod4(u - ad) == 0 ? nl : 0;
  for (int j = 1; j < ad; ++j)
    n += tg_step_loads(tg_mod4(u - j), ct, nl);
  return u == 3 && n > 8 ? 8 : n;
}
// In the first block A(1 .. ad - 1) come from the prologue (after B(0), before
// any u-step): the steady-state wait must not exceed the loads that really
// follow them there.  (A(0) is waited for by the prologue itself.)
constexpr bool tg_first_block_ok(int ad, int ct, int nl) {
  for (int t = 1; t < ad && t < 4; ++t) {
    int after = 4 * (ad - 1 - t);
    for (int s = 0; s < t; ++s)
      after += tg_step_loads(s % 4, ct, nl);
    if (after < tg_wait(t, ad, ct, nl))
      return false;
  }
  return true;
}

template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One 128 x (64 kCT) output tile (column block bx, row block by); ntiles =
// n / 16.  The step structure is the Q4_K GEMM's: the LDS reads of a u-step
// first (the 16 A fragments, at u = 3 the next block's per-column data, the
// raw B words of u-step t + 1), then per column tile its 16 MFMAs with the
// dequantisation of the previous column for u-step t + 1 under them (the
// last column's under the first column of the next u-step).
// GATED: the gated GEMM (SiLU(gate) * up of a.w and a.wu): the wave's
// columns 0 .. CT / 2 - 1 are output column tiles ct0 .. of the gate matrix,
// the others the same tiles of the up matrix; ct0 counts output tiles.
template <class P, typename OutT, bool GATED = false>
__device__ __forceinline__ void typed_gemm_tile(const GemmArgs& a, uint8_t* lds, int bx, int by, int ntiles) {
  constexpr int CT = P::kCT, AS = P::kAS, AD = AS - 1, NL = P::kNL, TB = P::kTB;
  constexpr int OT = GATED ? CT / 2 : CT;  // output column tiles per wave
  static_assert(tg_first_block_ok(AD, CT, NL), "first-block load accounting");
  static_assert(!GATED || CT % 2 == 0, "gate and up tiles in pairs");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nb = a.nb, steps = 4 * nb;
  const int mt0 = by * (kG2M / 16);
  const int ct0 = bx * (4 * OT) + OT * wave;
  const uint32_t aring = lds_addr(lds);
  uint8_t* const bring = lds + AS * kG2ASlot + wave * (2 * CT * TB);
  const uint32_t bring0 = lds_addr(bring);
  const uint32_t voff16 = 16u * (uint32_t)lane, voff4 = 4u * (uint32_t)lane;
  // A: this wave's 4 fragments of u-step t are 4 consecutive KB at
  // xa + 16 KB * t of the staging and at 4 KB * wave of ring slot t % AS;
  // fragment i is the instruction offset 1 KB * i.  The ring addresses of
  // the slot read (ar) and written (aw) roll from step to step.
  const uint8_t* const xa = uniform_ptr(reinterpret_cast<const uint8_t*>(a.xh) + ((size_t)by * nb * 64 + 4 * (size_t)wave) * 1024);
  const uint32_t aend = aring + AS * kG2ASlot;
  auto frag_a = [&](const uint8_t* src, uint32_t l, int i) {
    if (i == 0)
      lds_dma16<0>(src, voff16, l);
    else if (i == 1)
      lds_dma16<1024>(src, voff16, l);
    else if (i == 2)
      lds_dma16<2048>(src, voff16, l);
    else
      lds_dma16<3072>(src, voff16, l);
  };
  // B: column c's tile-blocks start at wcol[c] (column tiles past n read the
  // last one); block blk goes to ring half blk & 1.
  const uint8_t* wcol[CT];
#pragma unroll
  for (int c = 0; c < CT; ++c) {
    const int oc = ct0 + (GATED ? c % OT : c);
    wcol[c] = uniform_ptr((GATED && c >= OT ? a.wu : a.w) + (size_t)(oc < ntiles ? oc : ntiles - 1) * nb * TB);
  }
  auto issue_b = [&](int blk, int c) {
    const int bc = blk < nb ? blk : nb - 1;
    const uint32_t l = __builtin_amdgcn_readfirstlane(bring0 + (uint32_t)((blk & 1) * CT + c) * TB);
    P::issue(wcol[c] + (size_t)bc * TB, voff16, voff4, l, lane);
  };

  f4_t acc[8][CT];
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      acc[rt][c] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
      asm volatile("" : "+a"(acc[rt][c]));
    }

#pragma unroll
  for (int c = 0; c < CT; ++c)
    issue_b(0, c);
#pragma unroll
  for (int t = 0; t < AD; ++t) {
    const uint8_t* src = xa + (size_t)(t < steps ? t : steps - 1) * 16384;
    const uint32_t l = aring + (uint32_t)t * kG2ASlot + 4096u * (uint32_t)wave;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      frag_a(src, l, i);
  }
  vm_wait<4 * (AD - 1)>();  // B(0) and A(0)
  typename P::K kk[CT];
  h8_t bclo[CT], bchi[CT];
  typename P::W wl;  // raw words of the last column for the current u-step
  {
    typename P::R r[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c)
      P::raw(r[c], bring + c * TB, lane);
#pragma unroll
    for (int c = 0; c < CT; ++c)
      P::consts(kk[c], r[c], lane);
#pragma unroll
    for (int c = 0; c < CT - 1; ++c) {
      typename P::W w;
      P::words(w, bring + c * TB, 0, lane);
      P::dequant(kk[c], w, 0, bclo[c], bchi[c]);
    }
    P::words(wl, bring + (CT - 1) * TB, 0, lane);
  }
  uint32_t ar = aring, aw = aring + AD * kG2ASlot + 4096u * (uint32_t)wave;
  for (int blk = 0; blk < nb; ++blk) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = 4 * blk + u;
      const int ta = t + AD < steps ? t + AD : steps - 1;
      const uint8_t* const asrc = xa + (size_t)ta * 16384;
      if (u == 0)
        vm_wait<tg_wait(0, AD, CT, NL)>();
      else if (u == 1)
        vm_wait<tg_wait(1, AD, CT, NL)>();
      else if (u == 2)
        vm_wait<tg_wait(2, AD, CT, NL)>();
      else
        vm_wait<tg_wait(3, AD, CT, NL)>();
      __syncthreads();  // A(t) of every wave landed; u-step t - 1 fully read
      __builtin_amdgcn_sched_barrier(0);
      const int bn = u == 3 ? blk + 1 : blk, un = (u + 1) & 3;
      const uint8_t* aslot = lds + (ar - aring);
      h8_t af[16];
#pragma unroll
      for (int i = 0; i < 16; ++i)
        af[i] = *reinterpret_cast<const h8_t*>(aslot + i * 1024 + 16 * lane);
      const uint8_t* bslot = bring + (size_t)((bn & 1) * CT) * TB;
      typename P::R r[CT];
      if (u == 3) {
#pragma unroll
        for (int c = 0; c < CT; ++c)
          P::raw(r[c], bslot + c * TB, lane);
      }
      typename P::W wv[CT];
#pragma unroll
      for (int c = 0; c < CT; ++c)
        P::words(wv[c], bslot + c * TB, un, lane);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        if (c == 0)
          P::dequant(kk[CT - 1], wl, u, bclo[CT - 1], bchi[CT - 1]);
#pragma unroll
        for (int rt = 0; rt < 8; ++rt)
          acc[rt][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[2 * rt], bclo[c], acc[rt][c], 0, 0, 0);
#pragma unroll
        for (int rt = 0; rt < 8; ++rt)
          acc[rt][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[2 * rt + 1], bchi[c], acc[rt][c], 0, 0, 0);
        if (u == 3)
          P::consts(kk[c], r[c], lane);
        if (c > 0)
          P::dequant(kk[c - 1], wv[c - 1], un, bclo[c - 1], bchi[c - 1]);
#pragma unroll
        for (int i = 4 * c / CT; i < 4 * (c + 1) / CT; ++i)
          frag_a(asrc, aw, i);
        if (u == 0)
          issue_b(blk + 1, c);
      }
      wl = wv[CT - 1];
      ar = ar + kG2ASlot == aend ? aring : ar + kG2ASlot;
      aw = aw + kG2ASlot >= aend ? aw + kG2ASlot - AS * kG2ASlot : aw + kG2ASlot;
      __builtin_amdgcn_sched_group_barrier(0x100, 64, 0);
#pragma unroll
      for (int i = 0; i < 16 * CT; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, P::kVPM, 0);
      }
    }
  }
  vm_wait<0>();
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
#pragma unroll
    for (int c = 0; c < CT; ++c)
      asm volatile("" : "+a"(acc[rt][c]));

  const bool full = mt0 * 16 + kG2M <= a.m;
  if constexpr (GATED) {
    const int nct2 = ntiles - ct0 >= OT ? OT : ntiles - ct0 > 0 ? ntiles - ct0 : 0;
    full ? gemm2_epilogue_gated<OutT, true, CT>(a, acc, mt0, ct0, lane, nct2) : gemm2_epilogue_gated<OutT, false, CT>(a, acc, mt0, ct0, lane, nct2);
    return;
  }
  const int nct = ntiles - ct0 >= CT ? CT : ntiles - ct0 > 0 ? ntiles - ct0 : 0;
  float* const lrs = reinterpret_cast<float*>(bring);  // this wave's B ring: its loads have landed
  if (a.post == 0)
    full ? gemm2_epilogue<OutT, 0, true, CT>(a, acc, mt0, ct0, lane, nct, lrs) : gemm2_epilogue<OutT, 0, false, CT>(a, acc, mt0, ct0, lane, nct, lrs);
  else if (a.post == 1)
    full ? gemm2_epilogue<OutT, 1, true, CT>(a, acc, mt0, ct0, lane, nct, lrs) : gemm2_epilogue<OutT, 1, false, CT>(a, acc, mt0, ct0, lane, nct, lrs);
  else
    full ? gemm2_epilogue<OutT, 2, true, CT>(a, acc, mt0, ct0, lane, nct, lrs) : gemm2_epilogue<OutT, 2, false, CT>(a, acc, mt0, ct0, lane, nct, lrs);
}

// typed_gemm_tile with B in half tile-blocks (policies with kHalf): per
// column three half-slots, half h (half h % 2 of block h / 2) in slot h % 3.
// Half 1 of block blk + 1 is issued at u-step 1 of block blk into the slot of
// half 0 of blk (last read at u-step 0), half 0 of block blk + 2 at u-step 3
// into the slot of half 1 of blk (last read at u-step 2); each is read three
// or four u-steps after its issue.  The A ring has kAS = 3 slots (A two
// u-steps ahead).  Loads in issue order per u-step and column group c: A
// fragment c of A(t + 2), then at u = 1 column c's half 1 (kL1 loads), at
// u = 3 its half 0 (kL0 loads).  Every half read at u-step t was issued
// before A(t), so the wait for A(t) covers it: the loads after A(t)'s last
// fragment are column 3's half of u-step t - 2 and all of u-step t - 1, that
// is 4 + CT kL0 (u = 0), kL0 + 4 (u = 1), 4 + CT kL1 (u = 2), kL1 + 4
// (u = 3); at u-step 1 of the first block only A(2) follows A(1) (the
// prologue issues no B after it), so the wait there is 4.
template <class P, typename OutT>
__device__ __forceinline__ void typed_gemm_tile_half(const GemmArgs& a, uint8_t* lds, int bx, int by, int ntiles) {
  constexpr int CT = P::kCT, AS = P::kAS, AD = AS - 1, TB = P::kTB, HS = P::kHS, L0 = P::kL0, L1 = P::kL1;
  static_assert(AD == 2 && CT == 4, "the wait counts below assume A two u-steps ahead and four column groups");
  constexpr int W0 = 4 + CT * L0, W1 = L0 + 4, W2 = 4 + CT * L1, W3 = L1 + 4;
  static_assert(W0 < 64 && W2 < 64, "vmcnt field");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nb = a.nb, steps = 4 * nb;
  const int mt0 = by * (kG2M / 16);
  const int ct0 = bx * (4 * CT) + CT * wave;
  const uint32_t aring = lds_addr(lds);
  uint8_t* const bring = lds + AS * kG2ASlot + wave * (3 * CT * HS);
  const uint32_t bring0 = lds_addr(bring);
  const uint32_t voff16 = 16u * (uint32_t)lane, voff4 = 4u * (uint32_t)lane;
  const uint8_t* const xa = uniform_ptr(reinterpret_cast<const uint8_t*>(a.xh) + ((size_t)by * nb * 64 + 4 * (size_t)wave) * 1024);
  const uint32_t aend = aring + AS * kG2ASlot;
  auto frag_a = [&](const uint8_t* src, uint32_t l, int i) {
    if (i == 0)
      lds_dma16<0>(src, voff16, l);
    else if (i == 1)
      lds_dma16<1024>(src, voff16, l);
    else if (i == 2)
      lds_dma16<2048>(src, voff16, l);
    else
      lds_dma16<3072>(src, voff16, l);
  };
  const uint8_t* wcol[CT];
#pragma unroll
  for (int c = 0; c < CT; ++c)
    wcol[c] = uniform_ptr(a.w + (size_t)(ct0 + c < ntiles ? ct0 + c : ntiles - 1) * nb * TB);
  // Half s of block blk (clamped to the last block) of column c into slot sl.
  auto issue_half = [&](int blk, int s, int c, int sl) {
    const int bc = blk < nb ? blk : nb - 1;
    const uint32_t l = __builtin_amdgcn_readfirstlane(bring0 + (uint32_t)((sl * CT + c) * HS));
    if (s == 0)
      P::issue_half0(wcol[c] + (size_t)bc * TB, voff16, voff4, l);
    else
      P::issue_half1(wcol[c] + (size_t)bc * TB, voff16, l);
  };
  auto hslot = [&](int sl, int c) { return bring + (size_t)(sl * CT + c) * HS; };

  f4_t acc[8][CT];
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      acc[rt][c] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
      asm volatile("" : "+a"(acc[rt][c]));
    }

  // Prologue: half 0 and 1 of block 0 and half 0 of block 1 into slots 0, 1,
  // 2, then A(0), A(1); everything but A(1) waited for.
#pragma unroll
  for (int c = 0; c < CT; ++c)
    issue_half(0, 0, c, 0);
#pragma unroll
  for (int c = 0; c < CT; ++c)
    issue_half(0, 1, c, 1);
#pragma unroll
  for (int c = 0; c < CT; ++c)
    issue_half(1, 0, c, 2);
#pragma unroll
  for (int t = 0; t < AD; ++t) {
    const uint8_t* src = xa + (size_t)(t < steps ? t : steps - 1) * 16384;
    const uint32_t l = aring + (uint32_t)t * kG2ASlot + 4096u * (uint32_t)wave;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      frag_a(src, l, i);
  }
  vm_wait<4>();
  typename P::K kk[CT];
  h8_t bclo[CT], bchi[CT];
  typename P::W wl;
  {
    typename P::R r[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c)
      P::raw_half(r[c], hslot(0, c), lane);
#pragma unroll
    for (int c = 0; c < CT; ++c)
      P::consts(kk[c], r[c], lane);
#pragma unroll
    for (int c = 0; c < CT - 1; ++c) {
      typename P::W w;
      P::words_half(w, hslot(0, c), 0, lane);
      P::dequant(kk[c], w, 0, bclo[c], bchi[c]);
    }
    P::words_half(wl, hslot(0, CT - 1), 0, lane);
  }
  uint32_t ar = aring, aw = aring + AD * kG2ASlot + 4096u * (uint32_t)wave;
  // Slots of half 0 and half 1 of block blk and of half 0 of block blk + 1.
  int s0 = 0, s1 = 1, s2 = 2;
  for (int blk = 0; blk < nb; ++blk) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = 4 * blk + u;
      const int ta = t + AD < steps ? t + AD : steps - 1;
      const uint8_t* const asrc = xa + (size_t)ta * 16384;
      if (u == 0)
        vm_wait<W0>();
      else if (u == 1) {
        if (blk == 0)
          vm_wait<4>();
        else
          vm_wait<W1>();
      } else if (u == 2)
        vm_wait<W2>();
      else
        vm_wait<W3>();
      __syncthreads();  // A(t) of every wave landed; u-step t - 1 fully read
      __builtin_amdgcn_sched_barrier(0);
      const int un = (u + 1) & 3;
      const int ws = u == 0 ? s0 : u == 3 ? s2 : s1;  // slot of the words of u-step t + 1
      const uint8_t* aslot = lds + (ar - aring);
      h8_t af[16];
#pragma unroll
      for (int i = 0; i < 16; ++i)
        af[i] = *reinterpret_cast<const h8_t*>(aslot + i * 1024 + 16 * lane);
      typename P::R r[CT];
      if (u == 3) {
#pragma unroll
        for (int c = 0; c < CT; ++c)
          P::raw_half(r[c], hslot(s2, c), lane);
      }
      typename P::W wv[CT];
#pragma unroll
      for (int c = 0; c < CT; ++c)
        P::words_half(wv[c], hslot(ws, c), un, lane);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        if (c == 0)
          P::dequant(kk[CT - 1], wl, u, bclo[CT - 1], bchi[CT - 1]);
#pragma unroll
        for (int rt = 0; rt < 8; ++rt)
          acc[rt][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[2 * rt], bclo[c], acc[rt][c], 0, 0, 0);
#pragma unroll
        for (int rt = 0; rt < 8; ++rt)
          acc[rt][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[2 * rt + 1], bchi[c], acc[rt][c], 0, 0, 0);
        if (u == 3)
          P::consts(kk[c], r[c], lane);
        if (c > 0)
          P::dequant(kk[c - 1], wv[c - 1], un, bclo[c - 1], bchi[c - 1]);
        frag_a(asrc, aw, c);
        if (u == 1)
          issue_half(blk + 1, 1, c, s0);
        else if (u == 3)
          issue_half(blk + 2, 0, c, s1);
      }
      wl = wv[CT - 1];
      ar = ar + kG2ASlot == aend ? aring : ar + kG2ASlot;
      aw = aw + kG2ASlot >= aend ? aw + kG2ASlot - AS * kG2ASlot : aw + kG2ASlot;
      __builtin_amdgcn_sched_group_barrier(0x100, 64, 0);
#pragma unroll
      for (int i = 0; i < 16 * CT; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, P::kVPM, 0);
      }
    }
    const int sn = s2;
    s2 = s1;
    s1 = s0;
    s0 = sn;
  }
  vm_wait<0>();
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
#pragma unroll
    for (int c = 0; c < CT; ++c)
      asm volatile("" : "+a"(acc[rt][c]));

  const bool full = mt0 * 16 + kG2M <= a.m;
  const int nct = ntiles - ct0 >= CT ? CT : ntiles - ct0 > 0 ? ntiles - ct0 : 0;
  if (a.post == 0)
    full ? gemm2_epilogue<OutT, 0, true, CT>(a, acc, mt0, ct0, lane, nct) : gemm2_epilogue<OutT, 0, false, CT>(a, acc, mt0, ct0, lane, nct);
  else if (a.post == 1)
    full ? gemm2_epilogue<OutT, 1, true, CT>(a, acc, mt0, ct0, lane, nct) : gemm2_epilogue<OutT, 1, false, CT>(a, acc, mt0, ct0, lane, nct);
  else
    full ? gemm2_epilogue<OutT, 2, true, CT>(a, acc, mt0, ct0, lane, nct) : gemm2_epilogue<OutT, 2, false, CT>(a, acc, mt0, ct0, lane, nct);
}

template <class P>
constexpr int tg_lds_bytes() {
  if constexpr (TgIsHalf<P>::value)
    return P::kAS * kG2ASlot + 4 * 3 * P::kCT * P::kHS;
  else
    return P::kAS * kG2ASlot + 4 * 2 * P::kCT * P::kTB;
}

// Persistent over the (column block, row block) tiles, as the Q4_K GEMM.
template <class P, typename OutT, bool GATED = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void typed_gemm_kernel(GemmArgs a, TileMap map, int ntiles) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[tg_lds_bytes<P>()];
  static_assert(tg_lds_bytes<P>() <= 160 * 1024, "LDS of one workgroup");
  const int count = tile_count(map);
  for (int i = 0; i < count; ++i) {
    if (i > 0)
      __syncthreads();
    int bx, by;
    tile_at(map, i, bx, by);
    if constexpr (TgIsHalf<P>::value)
      typed_gemm_tile_half<P, OutT>(a, lds, bx, by, ntiles);
    else
      typed_gemm_tile<P, OutT, GATED>(a, lds, bx, by, ntiles);
  }
}

// One workgroup of 64 lanes per tile-block (encode_lane, q4k_internal.h).
__global__ __launch_bounds__(64) void typed_relayout_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t nb, uint32_t type) {
  const size_t tb = blockIdx.x;
  const uint32_t c = (uint32_t)(tb / nb), b = (uint32_t)(tb % nb);
  const int lane = threadIdx.x;
  const size_t bb = (size_t)type_block_bytes(type);
  encode_lane(type, src + ((size_t)(16 * c + (lane & 15)) * nb + b) * bb, dst + tb * 16 * bb, lane);
}

int env_int(const char* name, int fallback) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : fallback;
}

template <int RT, int T, int W, int BPW, bool GATED>
hipError_t gemv_launch(hipStream_t s, const GemvArgs& a, int dtype) {
  const dim3 grid((unsigned)(a.n / (16 * T))), block(64 * W);
  if (dtype == kF32)
    (void)dispatch(q4k_gemv_kernel<RT, T, W, BPW, GATED, float>, grid, block, s, a);
  else
    (void)dispatch(q4k_gemv_kernel<RT, T, W, BPW, GATED, _Float16>, grid, block, s, a);
  return hipGetLastError();
}

// One row tile: the block count per wave is fixed at compile time when the
// waves split nb evenly into at most 4 blocks each.
template <int T, bool GATED>
hipError_t gemv_one_row_tile(hipStream_t s, const GemvArgs& a, int dtype, int waves) {
  static const bool generic = env_int("Q4K_GEMV_GENERIC", 0) != 0;
  const int bpw = !generic && a.nb % waves == 0 ? a.nb / waves : 0;
  if (waves == 16) {
    if (bpw == 1)
      return gemv_launch<1, T, 16, 1, GATED>(s, a, dtype);
    if constexpr (T == 1 && !GATED) {  // the other BPW=3 instances spill
      if (bpw == 3)
        return gemv_launch<1, T, 16, 3, GATED>(s, a, dtype);
    }
    return gemv_launch<1, T, 16, 0, GATED>(s, a, dtype);
  }
  if (waves == 8) {
    if (bpw == 2)
      return gemv_launch<1, T, 8, 2, GATED>(s, a, dtype);
    return gemv_launch<1, T, 8, 0, GATED>(s, a, dtype);
  }
  if (bpw == 4)
    return gemv_launch<1, T, 4, 4, GATED>(s, a, dtype);
  return gemv_launch<1, T, 4, 0, GATED>(s, a, dtype);
}

template <int RT, bool GATED>
hipError_t gemv_multi_row_tile(hipStream_t s, const GemvArgs& a, int dtype, int waves, int tiles) {
  if constexpr (!GATED) {
    if (tiles == 2)
      return gemv_launch<RT, 2, 4, 0, false>(s, a, dtype);
  }
  if (waves >= 8)
    return gemv_launch<RT, 1, 8, 0, GATED>(s, a, dtype);
  return gemv_launch<RT, 1, 4, 0, GATED>(s, a, dtype);
}

// Instances kept within the register file (no spills): 16 waves only with
// one row tile; two column tiles only with one row tile and no gate/up pair.
template <bool GATED>
hipError_t gemv_dispatch(hipStream_t s, const GemvArgs& a, int dtype, const GemvShape& shape) {
  if (shape.row_tiles == 1) {
    if constexpr (!GATED) {
      if (shape.tiles == 2)
        return gemv_one_row_tile<2, false>(s, a, dtype, shape.waves);
    }
    return gemv_one_row_tile<1, GATED>(s, a, dtype, shape.waves);
  }
  if (shape.row_tiles == 2)
    return gemv_multi_row_tile<2, GATED>(s, a, dtype, shape.waves, shape.tiles);
  return gemv_multi_row_tile<3, GATED>(s, a, dtype, shape.waves, shape.tiles);
}

}  // namespace

namespace {

// Split-K instances: (NM, T, KS, BPS, DP).  A group is T column tiles of NM
// matrices; KS slices of BPS blocks each.
struct SplitkInst {
  int nm, t, ks, bps;
};
constexpr SplitkInst kSplitk[] = {
    {1, 8, 8, 6},  // K = 12288 (nb = 48), N a multiple of 1024: 8 tiles x 8 slices of 6 blocks
};

template <int NM, int T, int KS, int BPS, int DP>
hipError_t splitk_launch(hipStream_t s, const GemvArgs& a, int dtype, int grid, float* part, int* counters) {
  if (dtype == kF32)
    (void)dispatch(q4k_gemv_splitk_kernel<NM, T, KS, BPS, DP, float>, dim3((unsigned)grid), dim3(512), s, a, part, counters);
  else
    (void)dispatch(q4k_gemv_splitk_kernel<NM, T, KS, BPS, DP, _Float16>, dim3((unsigned)grid), dim3(512), s, a, part, counters);
  return hipGetLastError();
}

}  // namespace

bool gemv_splitk_plan(int m, int n, int nb, bool gated, int cus, SplitkPlan* plan) {
  static const int forced = env_int("Q4K_GEMV_SPLITK", -1);  // -1 auto, -2 off, else instance
  if (forced == -2 || m < 1 || m > 8 || n % 16 != 0)
    return false;
  const int tiles = n / 16, nm = gated ? 2 : 1;
  int best = -1, best_grid = 0;
  for (int i = 0; i < (int)(sizeof(kSplitk) / sizeof(kSplitk[0])); ++i) {
    const SplitkInst& c = kSplitk[i];
    if (forced >= 0 && i != forced)
      continue;
    if (c.nm != nm || c.ks * c.bps != nb || tiles % c.t != 0 || (tiles / c.t) % 8 != 0)
      continue;
    const int grid = tiles / c.t * c.ks;
    // Prefer the largest grid that fills at most one workgroup per CU, then
    // the smallest grid above that.
    const bool fits = grid <= cus, best_fits = best_grid <= cus;
    if (best < 0 || (fits && (!best_fits || grid > best_grid)) || (!fits && !best_fits && grid < best_grid)) {
      best = i;
      best_grid = grid;
    }
  }
  if (best < 0)
    return false;
  const SplitkInst& c = kSplitk[best];
  plan->inst = best;
  plan->groups = tiles / c.t;
  plan->ks = c.ks;
  plan->mt = c.nm * c.t;
  plan->grid = best_grid;
  return true;
}

size_t gemv_splitk_part_floats(const SplitkPlan& plan) {
  return (size_t)plan.groups * plan.ks * plan.mt * 8 * 16;
}

hipError_t launch_gemv_splitk(hipStream_t s, const GemvArgs& a, int dtype, const SplitkPlan& plan, float* part, int* counters) {
  (void)plan.inst;  // one instance
  // Two block-steps in flight per wave: measured faster than four (shorter
  // memory queues, as for the fused gate/up GEMV).
  return splitk_launch<1, 8, 8, 6, 2>(s, a, dtype, plan.grid, part, counters);
}

// Column tiles per workgroup of the rows GEMV (0: not this kernel).  Gated
// pairs at K = 4096 take 3 (one workgroup per CU at N = 12288): at M = 40
// 19.4 us against 26.7 on the one-tile GEMV.  Plain projections with K =
// 12288 take the most of 3, 2, 1 that still gives every CU a workgroup, or
// 1 (M = 40, N = 4096: 19.1 against 20.5 us).  Plain projections at K = 4096
// stay on the staged GEMV, which already splits K over 8 waves with two
// column tiles where that fills the CUs (measured as fast or faster).
RowsPlan gemv_rows_plan(int rows, int nb, int n, bool gated, int cus) {
  static const int forced = env_int("Q4K_GEMV_ROWS", -1);  // -1 auto, 0 off, 1..3 column tiles
  static const int slices_env = env_int("Q4K_GEMV_ROWS_SLICES", -1);  // -1 auto, 1 one slice, 3 three
  RowsPlan p;
  if (forced == 0 || rows <= 16 || rows > 16 * kGemvMaxRowTiles || n % 16 != 0)
    return p;
  const int ctiles = n / 16;
  if (gated) {
    if (nb != 16)
      return p;
    const int t = forced > 0 ? forced : 3;
    if (ctiles % t == 0 && (forced > 0 || ctiles / t >= cus))
      p.tiles = t;
    return p;
  }
  if (nb != 48 && !(forced > 0 && nb == 16))
    return p;
  // K = 12288: three K-slices of 4 column tiles when the column groups fill
  // the CUs in one round -- each CU then reads a third of x for 4 column
  // tiles instead of all of it for one (M = 40, N = 4096: 64 groups x 3).
  const bool slices_ok = nb == 48 && forced <= 0 && ctiles % 4 == 0 && (ctiles / 4) * 3 <= cus;
  if (slices_env == 3 ? nb == 48 && ctiles % 4 == 0 : slices_env != 1 && slices_ok) {
    p.tiles = 4;
    p.slices = 3;
    return p;
  }
  if (forced > 0) {
    if (ctiles % forced == 0)
      p.tiles = forced;
    return p;
  }
  p.tiles = 1;
  for (int t = 3; t >= 1; --t)
    if (ctiles % t == 0 && ctiles / t >= cus) {
      p.tiles = t;
      break;
    }
  return p;
}

size_t gemv_rows_part_floats(const RowsPlan& p, int n) {
  return p.slices > 1 ? (size_t)(n / (16 * p.tiles)) * p.slices * (16 * kGemvMaxRowTiles) * (16 * p.tiles) : 0;
}

template <int NM, int T, int RT, int BPW, int KS = 1>
hipError_t gemv_rows_launch(hipStream_t s, const GemvArgs& a, int dtype) {
  const dim3 grid((unsigned)(a.n / (16 * T) * KS)), block(512);
  if (dtype == kF32)
    (void)dispatch(q4k_gemv_rows_kernel<NM, T, RT, BPW, float, KS>, grid, block, s, a);
  else
    (void)dispatch(q4k_gemv_rows_kernel<NM, T, RT, BPW, _Float16, KS>, grid, block, s, a);
  return hipGetLastError();
}

// K = 4096 (2 blocks per wave) and, for plain projections, K = 12288 (6).
template <int NM, int T, int RT>
hipError_t gemv_rows_bpw(hipStream_t s, const GemvArgs& a, int dtype) {
  if (a.nb == 16)
    return gemv_rows_launch<NM, T, RT, 2>(s, a, dtype);
  if constexpr (NM == 1) {
    if (a.nb == 48)
      return gemv_rows_launch<NM, T, RT, 6>(s, a, dtype);
  }
  return hipErrorInvalidValue;
}

template <int NM, int T>
hipError_t gemv_rows_rt(hipStream_t s, const GemvArgs& a, int dtype) {
  return a.rows <= 32 ? gemv_rows_bpw<NM, T, 2>(s, a, dtype) : gemv_rows_bpw<NM, T, 3>(s, a, dtype);
}

hipError_t launch_gemv_rows(hipStream_t s, const GemvArgs& a, int dtype, const RowsPlan& p, bool gated) {
  const int tiles = p.tiles;
  if (a.rows <= 16 || a.rows > 16 * kGemvMaxRowTiles || (a.nb != 16 && a.nb != 48) || tiles < 1 || a.n % (16 * tiles) != 0 ||
      a.rows != (a.split ? 2 * a.m : a.m))
    return hipErrorInvalidValue;
  if (p.slices != 1) {
    // K = 12288: three K-slices of four column tiles (2 blocks per wave).
    // (Two slices of two column tiles, 3 blocks per wave and all 256 CUs,
    // measured the same config-2 pass: 78.9-81.3 against 79.4-79.7 us.)
    if (gated || p.slices != 3 || tiles != 4 || a.nb != 48 || !a.part || !a.counters)
      return hipErrorInvalidValue;
    return a.rows <= 32 ? gemv_rows_launch<1, 4, 2, 2, 3>(s, a, dtype) : gemv_rows_launch<1, 4, 3, 2, 3>(s, a, dtype);
  }
  if (gated) {
    if (a.nb != 16)
      return hipErrorInvalidValue;
    switch (tiles) {
      case 3: return gemv_rows_rt<2, 3>(s, a, dtype);
      case 2: return gemv_rows_rt<2, 2>(s, a, dtype);
      case 1: return gemv_rows_rt<2, 1>(s, a, dtype);
      default: return hipErrorInvalidValue;
    }
  }
  switch (tiles) {
    case 3: return gemv_rows_rt<1, 3>(s, a, dtype);
    case 2: return gemv_rows_rt<1, 2>(s, a, dtype);
    case 1: return gemv_rows_rt<1, 1>(s, a, dtype);
    default: return hipErrorInvalidValue;
  }
}

bool gemv_gate_up_supported(int m, int nb, int n) {
  static const bool enabled = env_int("Q4K_GEMV_GATE_UP", 1) != 0;
  return enabled && m >= 1 && m <= 8 && nb == 16 && n % 16 == 0;
}

// Eight waves per workgroup, two K-blocks each.  (Sixteen waves of one
// block each need more than their 128 registers and spill.)
constexpr int kGuWaves = 8;

template <int T, bool NORM>
hipError_t gate_up_launch(hipStream_t s, const GemvArgs& a, int dtype, unsigned grid) {
  if (dtype == kF32)
    (void)dispatch(q4k_gemv_gate_up_kernel<T, float, NORM, kGuWaves>, dim3(grid), dim3(64 * kGuWaves), s, a);
  else
    (void)dispatch(q4k_gemv_gate_up_kernel<T, _Float16, NORM, kGuWaves>, dim3(grid), dim3(64 * kGuWaves), s, a);
  return hipGetLastError();
}

hipError_t launch_gemv_gate_up(hipStream_t s, const GemvArgs& a, int dtype, int cus) {
  // Three column tiles per workgroup while that still gives every CU one
  // workgroup (N = 12288: 256); otherwise one.
  const int ctiles = a.n / 16;
  const bool t3 = ctiles % 3 == 0 && ctiles / 3 >= cus;
  const unsigned grid = (unsigned)(t3 ? ctiles / 3 : ctiles);
  if (a.norm_w)
    return t3 ? gate_up_launch<3, true>(s, a, dtype, grid) : gate_up_launch<1, true>(s, a, dtype, grid);
  return t3 ? gate_up_launch<3, false>(s, a, dtype, grid) : gate_up_launch<1, false>(s, a, dtype, grid);
}

bool typed_gate_up_supported(uint32_t type, int m, int nb, int n) {
  static const bool enabled = env_int("Q4K_GEMV_GATE_UP", 1) != 0;
  return enabled && (type == kTypeQ5_K || type == kTypeIQ4_XS) && m >= 1 && m <= 8 && nb == 16 && n % 16 == 0;
}

template <class F, int T, bool NORM>
hipError_t typed_gate_up_launch(hipStream_t s, const GemvArgs& a, int dtype, unsigned grid) {
  if (dtype == kF32)
    (void)dispatch(typed_gate_up_kernel<F, T, float, NORM>, dim3(grid), dim3(512), s, a);
  else
    (void)dispatch(typed_gate_up_kernel<F, T, _Float16, NORM>, dim3(grid), dim3(512), s, a);
  return hipGetLastError();
}

template <class F>
hipError_t typed_gate_up_dispatch(hipStream_t s, const GemvArgs& a, int dtype, int cus) {
  // Column tiles per workgroup as for Q4_K.
  const int ctiles = a.n / 16;
  const bool t3 = ctiles % 3 == 0 && ctiles / 3 >= cus;
  const unsigned grid = (unsigned)(t3 ? ctiles / 3 : ctiles);
  if (a.norm_w)
    return t3 ? typed_gate_up_launch<F, 3, true>(s, a, dtype, grid) : typed_gate_up_launch<F, 1, true>(s, a, dtype, grid);
  return t3 ? typed_gate_up_launch<F, 3, false>(s, a, dtype, grid) : typed_gate_up_launch<F, 1, false>(s, a, dtype, grid);
}

hipError_t launch_typed_gate_up(hipStream_t s, const GemvArgs& a, uint32_t type, int dtype, int cus) {
  if (a.m < 1 || a.m > 8 || a.nb != 16 || a.n % 16 != 0)
    return hipErrorInvalidValue;
  switch (type) {
    case kTypeQ5_K:
      return typed_gate_up_dispatch<FmtQ5K>(s, a, dtype, cus);
    case kTypeIQ4_XS:
      return typed_gate_up_dispatch<FmtIQ4XS>(s, a, dtype, cus);
    default:
      return hipErrorInvalidValue;
  }
}

template <typename InT, bool NORM>
hipError_t stage_launch(hipStream_t s, const InT* x, _Float16* xo, _Float16* xs, float* rowscale, int m, int k, int mode, RowNorm nrm) {
  const dim3 grid((unsigned)m), block(256);
  if (mode == kStageFrag)
    (void)dispatch(stage_x_kernel<InT, kStageFrag, NORM>, grid, block, s, x, xo, xs, rowscale, m, k, nrm);
  else if (mode == kStageGemm && k / 256 <= 16)
    (void)dispatch(stage_gemm_kernel<InT, 16, 32, NORM>, dim3((unsigned)((m + 7) / 8)), block, s, x, xo, rowscale, m, k, nrm);
  else if (mode == kStageGemm && k % 512 == 0 && k / 512 <= 24)  // K <= 12288: one read of x, 64 threads per row
    (void)dispatch(stage_gemm_kernel<InT, 24, 64, NORM>, dim3((unsigned)((m + 7) / 8)), dim3(512), s, x, xo, rowscale, m, k, nrm);
  else if (mode == kStageGemm)
    (void)dispatch(stage_gemm_kernel<InT, 0, 32, NORM>, dim3((unsigned)((m + 7) / 8)), block, s, x, xo, rowscale, m, k, nrm);
  else
    (void)dispatch(stage_x_kernel<InT, kStageFragSplit, NORM>, grid, block, s, x, xo, xs, rowscale, m, k, nrm);
  return hipGetLastError();
}

hipError_t launch_stage_pack(hipStream_t s, const void* x, int dtype, const DecodePack& pk, int m, int k) {
  const dim3 grid((unsigned)(k / 256 * 8)), block(64);
  if (dtype == kF32)
    (void)dispatch(stage_pack_kernel<float>, grid, block, s, static_cast<const float*>(x), pk.frag, pk.xs, pk.dsc, m, k);
  else
    (void)dispatch(stage_pack_kernel<_Float16>, grid, block, s, static_cast<const _Float16*>(x), pk.frag, pk.xs, pk.dsc, m, k);
  return hipGetLastError();
}

hipError_t launch_stage_x(hipStream_t s, const void* x, int dtype, _Float16* xo, _Float16* xs, float* rowscale, int m, int k, int mode,
                          const float* norm_w, float eps) {
  if (m <= 0)
    return hipSuccess;
  RowNorm nrm;
  nrm.w = norm_w;
  nrm.eps = eps;
  if (dtype == kF32)
    return norm_w ? stage_launch<float, true>(s, static_cast<const float*>(x), xo, xs, rowscale, m, k, mode, nrm)
                  : stage_launch<float, false>(s, static_cast<const float*>(x), xo, xs, rowscale, m, k, mode, nrm);
  return norm_w ? stage_launch<_Float16, true>(s, static_cast<const _Float16*>(x), xo, xs, rowscale, m, k, mode, nrm)
                : stage_launch<_Float16, false>(s, static_cast<const _Float16*>(x), xo, xs, rowscale, m, k, mode, nrm);
}

GemvShape gemv_shape(int rows, int n, int nb, bool gated, int cus) {
  GemvShape sh;
  sh.row_tiles = rows <= 16 ? 1 : rows <= 32 ? 2 : 3;
  // One 16-column tile per workgroup (two for very wide outputs, one row tile,
  // no gate/up pair), and enough waves per workgroup -- each taking 1/waves
  // of K -- for about 12-16 resident waves per CU across the grid.
  const int ctiles = n / 16;
  static const int env_tiles = env_int("Q4K_GEMV_TILES", 0), env_waves = env_int("Q4K_GEMV_WAVES", 0);
  sh.tiles = (sh.row_tiles == 1 && !gated && n % 32 == 0 && ctiles >= 4096) ? 2 : 1;
  // More than one row tile: each workgroup reads all of the staged x (its
  // launches fit about 4 us + 14 us per MB of x a CU reads).  Between one
  // and two workgroups per CU, two column tiles per workgroup (4 waves) take
  // one round with half the x reads per tile: at M = 40, N = 6144 (the QKV
  // projection, 384 tiles) 11.7 us against 14.6.  Narrower outputs lose CUs
  // that way (N = 4096: 12.5 against 9.4 us), and gate/up pairs, three
  // workgroups per CU, measured 34.3 against 26.7 us (three tiles: 27.9).
  if (sh.row_tiles > 1 && !gated && ctiles % 2 == 0 && ctiles > cus && ctiles <= 2 * cus)
    sh.tiles = 2;
  if (env_tiles == 1 || (env_tiles == 2 && sh.row_tiles == 1 && !gated && n % 32 == 0))
    sh.tiles = env_tiles;
  const int groups = ctiles / sh.tiles;
  int waves = groups >= 1024 ? 4 : groups >= 512 ? 4 : groups >= 320 ? 8 : 16;
  if (env_waves == 4 || env_waves == 8 || env_waves == 16)
    waves = env_waves;
  while (waves > 4 && waves > nb)
    waves >>= 1;
  if (sh.row_tiles > 1 && waves > 8)
    waves = 8;
  sh.waves = waves;
  return sh;
}

hipError_t launch_gemv(hipStream_t s, const GemvArgs& a, int dtype, const GemvShape& shape, bool gated) {
  if (shape.row_tiles < 1 || shape.row_tiles > kGemvMaxRowTiles || a.n % (16 * shape.tiles) != 0 || a.rows > 16 * shape.row_tiles ||
      a.rows != (a.split ? 2 * a.m : a.m))
    return hipErrorInvalidValue;
  return gated ? gemv_dispatch<true>(s, a, dtype, shape) : gemv_dispatch<false>(s, a, dtype, shape);
}

bool gemm2_supported(int m, int n) {
  return n > 0 && n % 16 == 0 && m > 0;
}

int gemm2_rows(int m) {
  return (m + kG2M - 1) / kG2M * kG2M;
}

hipError_t launch_stream_read(hipStream_t s, const void* p, size_t bytes, uint32_t* out, int blocks) {
  (void)dispatch(stream_read_kernel, dim3((unsigned)blocks), dim3(256), s, static_cast<const u4_t*>(p), bytes / 16, out);
  return hipGetLastError();
}

hipError_t launch_mfma_ceiling(hipStream_t s, float* out, int blocks, int iters) {
  hipLaunchKernelGGL(mfma_ceiling_kernel, dim3((unsigned)blocks), dim3(256), 0, s, out, iters);
  return hipGetLastError();
}

// The tile map of a persistent GEMM launch of `grid` workgroups over a
// tiles_y x tiles_x tile grid: the XCD rectangles when the grid deals the
// same number of workgroups to each XCD and the rectangles divide the grid
// (Q4K_GEMM_XCD_ROWS: row groups, default 4; 0 keeps the plain order).
TileMap make_tile_map(int tiles_x, int tiles_y, int grid) {
  static const int rg_env = env_int("Q4K_GEMM_XCD_ROWS", 4);
  TileMap m{tiles_x, tiles_x * tiles_y, 0, 0, 0};
  const int rg = rg_env == 1 || rg_env == 2 || rg_env == 4 || rg_env == 8 ? rg_env : 0;
  if (rg && grid % 8 == 0 && tiles_y % rg == 0 && tiles_x % (8 / rg) == 0) {
    m.rg = rg;
    m.rows = tiles_y / rg;
    m.cols = tiles_x / (8 / rg);
  }
  return m;
}

template <class P, bool GATED = false>
hipError_t typed_gemm_launch(hipStream_t s, const GemmArgs& a, int dtype, int cus);

// Rounds of workgroups (tiles / CUs, rounded up) of the 256-column and
// 128-column tilings, weighted by the time of one tile of each.
bool gemm2_narrow(int tiles256, int tiles128, int cus) {
  static const int forced = env_int("Q4K_GEMM_NARROW", -1);  // -1 auto, 0 off, 1 always
  if (forced >= 0)
    return forced == 1;
  const int r4 = (tiles256 + cus - 1) / cus, r2 = (tiles128 + cus - 1) / cus;
  return r2 * kGemmNarrowTileTime < r4 * 10;
}

// 192 columns per workgroup (the typed template's Q4_K policy with three
// column tiles per wave) when the 256-column tiles leave CUs idle and the
// 192-column ones fill between three quarters of the CUs and all of them in
// one round.  At M = 821 the N = 6144 projection (168 256-column tiles, 224
// of 192) measured 55.0 us against 59.6 in K-segments and 64.3 unsplit; the
// N = 4096 one (154 tiles) 59.4 against 51.5 on 128 columns, which it keeps.
// The accumulation order and the dequantised values are those of the
// 256-column GEMM, and the K-split defers to this rule, so the gated GEMM
// stays bit-identical to the two-call form.  Q4K_GEMM_MID: -1 auto, 0
// never, 1 always (for the plain Q4_K GEMM).
static bool gemm2_mid(int m, int n, int cus) {
  static const int forced = env_int("Q4K_GEMM_MID", -1);
  if (forced >= 0)
    return forced == 1;
  const int tiles_y = (m + kG2M - 1) / kG2M;
  const int t4 = (n + kG2N - 1) / kG2N * tiles_y, t3 = (n / 16 + 11) / 12 * tiles_y;
  return t4 < cus && t3 <= cus && 4 * t3 >= 3 * cus;
}

// Segments 1 per workgroup on the CUs that `tiles` workgroups leave free.
static int split_segments_per_wg(int tiles, int cus) {
  const int free = cus - tiles;
  return (tiles + free - 1) / free;
}

// K-split of the pipelined GEMM when its 256-column tiles leave CUs idle:
// segment 0 of each tile (blocks [0, b)) on a workgroup of its own, segments
// 1 (the other nb - b blocks) q to a workgroup on the CUs the tiles leave
// free, q = tiles / free CUs rounded up.
//  - q = 1 (the tiles fill at most half the CUs) and K >= 8192: two halves
//    (b = nb / 2).  At M = 821 the K = 12288 down projection (112 tiles)
//    measured 113.6 us against 123.9 on the 128-column template; longer
//    segments 0 (b = 27, 30: 119.0, 128.0 us) do not pay for the exchange
//    they hide.  At K = 4096 the 112-tile O projection measured 56.0 us split
//    against 50.4 on the template, which it keeps.
//  - q >= 2 and K >= 4096: b = q nb / (q + 1) rounded up, so that the q
//    segments 1 of a workgroup take no longer than one segment 0.  The
//    N = 6144 projection's 168 tiles at M = 821 (b = 11) measured 58.9-60.9
//    us for b = 10..13 against 64.3 unsplit: the segments 0 run at 5.4 us
//    per block against 4.0 unsplit, so that 252 workgroups gain only 8 %
//    over 168.
// Returns b, or 0 for no split.  Q4K_GEMM2_SPLIT=0 turns the split off;
// Q4K_GEMM2_SPLIT_B forces b (for every shape with tiles < CUs and b < nb).
int gemm2_split_b(int m, int n, int nb, int cus) {
  static const int on = env_int("Q4K_GEMM2_SPLIT", 1);
  static const int b_env = env_int("Q4K_GEMM2_SPLIT_B", 0);
  const int tiles = ((n + kG2N - 1) / kG2N) * ((m + kG2M - 1) / kG2M);
  if (!on || tiles >= cus || gemm2_mid(m, n, cus))
    return 0;
  if (b_env > 0)
    return b_env < nb ? b_env : 0;
  const int q = split_segments_per_wg(tiles, cus);
  if (q == 1)
    return nb >= 32 ? nb / 2 : 0;
  return nb >= 16 ? (q * nb + q) / (q + 1) : 0;
}

void gemm2_split_workspace(int m, int n, bool gated, size_t* part_floats, size_t* counters) {
  const int tiles_x = gated ? (n / 16 + 7) / 8 : (n + kG2N - 1) / kG2N, tiles = tiles_x * ((m + kG2M - 1) / kG2M);
  *part_floats = (size_t)2 * tiles * 4 * 32 * 64 * 4;
  *counters = (size_t)tiles;
}

namespace {
// Segments 0 one per workgroup and segments 1 q per workgroup past them
// when the launch's own tiles leave CUs free, else both dealt round robin
// (the gated GEMM, twice the plain GEMM's tiles, takes the plain GEMM's b).
template <bool GATED>
hipError_t gemm2_split_launch(hipStream_t s, GemmArgs a, int dtype, int tiles_x, int tiles_y, int cus, int b) {
  const int tiles = tiles_x * tiles_y;
  a.split_b = b;
  a.split_q = tiles < cus ? split_segments_per_wg(tiles, cus) : 0;
  const int grid = a.split_q > 0 ? tiles + (tiles + a.split_q - 1) / a.split_q : (2 * tiles < cus ? 2 * tiles : cus);
  const TileMap map{tiles_x, tiles, 0, 0, 0};
  if (dtype == kF32)
    (void)dispatch(q4k_gemm2_kernel<float, GATED, true>, dim3((unsigned)grid), dim3(256), s, a, map);
  else
    (void)dispatch(q4k_gemm2_kernel<_Float16, GATED, true>, dim3((unsigned)grid), dim3(256), s, a, map);
  return hipGetLastError();
}
}  // namespace

// Six column tiles per wave (384 columns per workgroup) for a plain GEMM
// when its rounds of workgroups over the CUs take no longer than those of
// the 256-column tiling, a 384-column tile counted as 1.375 of a 256-column
// one (at M = 2048, N = 12288, K = 4096: Q4_K 182.6 us against 199-202 with
// four tiles per wave, IQ4_XS 208-210 against 224-225).  Q4K_GEMM_SIX: -1
// auto, 0 never, 1 always (the Q4_K and IQ4_XS GEMMs).
static bool gemm_six(int tiles256, int tiles384, int cus) {
  static const int forced = env_int("Q4K_GEMM_SIX", -1);
  if (forced >= 0)
    return forced == 1;
  const int r4 = (tiles256 + cus - 1) / cus, r6 = (tiles384 + cus - 1) / cus;
  return 11 * r6 <= 8 * r4;
}

hipError_t launch_gemm2(hipStream_t s, const GemmArgs& a, int dtype, int cus) {
  if (!gemm2_supported(a.m, a.n) || a.nb < 1)
    return hipErrorInvalidValue;
  const int tiles_x = (a.n + kG2N - 1) / kG2N, tiles_y = (a.m + kG2M - 1) / kG2M, tiles = tiles_x * tiles_y;
  if (const int b = gemm2_split_b(a.m, a.n, a.nb, cus)) {
    if (!a.part || !a.counters)
      return hipErrorInvalidValue;
    return gemm2_split_launch<false>(s, a, dtype, tiles_x, tiles_y, cus, b);
  }
  if (gemm2_mid(a.m, a.n, cus))
    return typed_gemm_launch<Mid<TgQ4K, 5>>(s, a, dtype, cus);
  if (gemm_six(tiles, ((a.n / 16 + 23) / 24) * tiles_y, cus))
    return typed_gemm_launch<Six<TgQ4K>>(s, a, dtype, cus);
  if (gemm2_narrow(tiles, ((a.n / 16 + 7) / 8) * tiles_y, cus))
    return typed_gemm_launch<TgQ4K>(s, a, dtype, cus);
  static const int persist = env_int("Q4K_GEMM2_PERSIST", 1);
  const int grid = persist && tiles > cus ? cus : tiles;
  const TileMap map = make_tile_map(tiles_x, tiles_y, grid);
  const dim3 block(256);
  if (dtype == kF32)
    (void)dispatch(q4k_gemm2_kernel<float, false>, dim3((unsigned)grid), block, s, a, map);
  else
    (void)dispatch(q4k_gemm2_kernel<_Float16, false>, dim3((unsigned)grid), block, s, a, map);
  return hipGetLastError();
}

// The gated GEMM on the typed template with six B column tiles per wave
// (three gate and three up tiles: 192 output columns per workgroup, against
// 128 for q4k_gemm2_kernel) when its rounds of workgroups over the CUs take
// no longer, a 192-column tile counted as 1.375 of a 128-column one (at
// M = 2048, N = 12288, K = 4096 the plain GEMM measured 182.6 us with six
// column tiles per wave against 199-202 us with four).  Its accumulation
// order and dequantised values are those of q4k_gemm2_kernel, so it stays
// bit-identical to the gate-then-up calls.  Q4K_GEMM_GATED_SIX: -1 auto, 0
// never, 1 always.
static bool gemm2_gated_six(int tiles128, int tiles192, int cus) {
  static const int forced = env_int("Q4K_GEMM_GATED_SIX", -1);
  if (forced >= 0)
    return forced == 1;
  const int r4 = (tiles128 + cus - 1) / cus, r6 = (tiles192 + cus - 1) / cus;
  return 11 * r6 <= 8 * r4;
}

hipError_t launch_gemm2_gated(hipStream_t s, const GemmArgs& a, int dtype, int cus) {
  if (!gemm2_supported(a.m, a.n) || a.nb < 1 || !a.wu)
    return hipErrorInvalidValue;
  // 128 output columns (256 B columns: gate and up) per tile.
  const int tiles_x = (a.n / 16 + 7) / 8, tiles_y = (a.m + kG2M - 1) / kG2M, tiles = tiles_x * tiles_y;
  // K-segments exactly when, and where, the plain GEMM of this shape splits,
  // so that the gated launch stays bit-identical to the gate-then-up calls.
  if (const int b = gemm2_split_b(a.m, a.n, a.nb, cus)) {
    if (!a.part || !a.counters)
      return hipErrorInvalidValue;
    return gemm2_split_launch<true>(s, a, dtype, tiles_x, tiles_y, cus, b);
  }
  if (gemm2_gated_six(tiles, ((a.n / 16 + 11) / 12) * tiles_y, cus))
    return typed_gemm_launch<Six<TgQ4K>, true>(s, a, dtype, cus);
  const int grid = tiles > cus ? cus : tiles;
  const TileMap map = make_tile_map(tiles_x, tiles_y, grid);
  const dim3 block(256);
  if (dtype == kF32)
    (void)dispatch(q4k_gemm2_kernel<float, true>, dim3((unsigned)grid), block, s, a, map);
  else
    (void)dispatch(q4k_gemm2_kernel<_Float16, true>, dim3((unsigned)grid), block, s, a, map);
  return hipGetLastError();
}

hipError_t launch_fill_u32(hipStream_t s, uint32_t* p, uint32_t v, uint32_t n) {
  if (n == 0)
    return hipSuccess;
  const unsigned grid = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
  (void)dispatch(fill_u32_kernel, dim3(grid), dim3(256), s, p, v, n);
  return hipGetLastError();
}

hipError_t launch_gather(hipStream_t s, const void* x, void* out, int k, int dtype, const GatherIndex& idx) {
  if (idx.rows == 0)
    return hipSuccess;
  const dim3 grid(idx.rows), block(256);
  if (dtype == kF32)
    (void)dispatch(gather_rows_kernel<float>, grid, block, s, static_cast<const float*>(x), static_cast<float*>(out), k, idx);
  else
    (void)dispatch(gather_rows_kernel<_Float16>, grid, block, s, static_cast<const _Float16*>(x), static_cast<_Float16*>(out), k, idx);
  return hipGetLastError();
}

hipError_t launch_embedding_batch(hipStream_t s, const uint8_t* w, const int32_t* tokens, const EmbedQueries& qs, void* y, int rows, int n, int k,
                                  int dtype) {
  if (rows == 0)
    return hipSuccess;
  const dim3 grid((unsigned)(k / 256), (unsigned)rows), block(256);
  if (dtype == kF32)
    (void)dispatch(embedding_batch_kernel<float>, grid, block, s, w, tokens, static_cast<float*>(y), n, k / 256, qs);
  else
    (void)dispatch(embedding_batch_kernel<_Float16>, grid, block, s, w, tokens, static_cast<_Float16*>(y), n, k / 256, qs);
  return hipGetLastError();
}

hipError_t launch_embedding(hipStream_t s, const uint8_t* w, const int32_t* ids, void* y, int rows, int n, int k, int dtype) {
  if (rows == 0)
    return hipSuccess;
  const dim3 grid((unsigned)(k / 256), (unsigned)rows), block(256);
  if (dtype == kF32)
    (void)dispatch(embedding_kernel<float>, grid, block, s, w, ids, static_cast<float*>(y), n, k / 256);
  else
    (void)dispatch(embedding_kernel<_Float16>, grid, block, s, w, ids, static_cast<_Float16*>(y), n, k / 256);
  return hipGetLastError();
}

hipError_t launch_rms_norm(hipStream_t s, const void* x, const float* w, void* y, int rows, int k, float eps, int dtype, const GatherIndex* idx) {
  if (rows == 0)
    return hipSuccess;
  GatherIndex gi{};
  if (idx)
    gi = *idx;
  const dim3 grid((unsigned)rows), block(256);
  if (dtype == kF32)
    (void)dispatch(rms_norm_kernel<float>, grid, block, s, static_cast<const float*>(x), w, static_cast<float*>(y), k, eps, gi, idx ? 1 : 0);
  else
    (void)dispatch(rms_norm_kernel<_Float16>, grid, block, s, static_cast<const _Float16*>(x), w, static_cast<_Float16*>(y), k, eps, gi,
                   idx ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_relayout(hipStream_t s, const uint8_t* src, uint8_t* dst, uint32_t n, uint32_t k) {
  const uint32_t nb = k / 256;
  const size_t tiles = (size_t)(n / 16) * nb;
  if (tiles == 0)
    return hipSuccess;
  (void)dispatch(relayout_kernel, dim3((unsigned)tiles), dim3(64), s, src, dst, n, nb);
  return hipGetLastError();
}

template <class F, int T, int DQ>
hipError_t typed_gemv_launch(hipStream_t s, const GemvArgs& a, int dtype) {
  const int ntiles = a.n / 16;
  const dim3 grid((unsigned)((ntiles + T - 1) / T)), block(512);
  if (dtype == kF32)
    (void)dispatch(typed_gemv_kernel<F, T, DQ, float>, grid, block, s, a);
  else
    (void)dispatch(typed_gemv_kernel<F, T, DQ, _Float16>, grid, block, s, a);
  return hipGetLastError();
}

template <class F, int T, int DQ, int W = 8>
hipError_t typed_persistent_launch(hipStream_t s, const GemvArgs& a, int dtype, int cus) {
  const int items = (a.n / 16 + T - 1) / T;
  const dim3 grid((unsigned)(items < cus ? items : cus)), block(64 * W);
  if (dtype == kF32)
    (void)dispatch(typed_gemv_persistent_kernel<F, T, DQ, W, float>, grid, block, s, a, items);
  else
    (void)dispatch(typed_gemv_persistent_kernel<F, T, DQ, W, _Float16>, grid, block, s, a, items);
  return hipGetLastError();
}

// K = 4096 with at least 16 column tiles per CU: the persistent form
// (F::kPW waves, F::kPT tiles per item).  Otherwise column tiles per
// workgroup: the most (of 4, 2, 1) that still gives every CU at least two
// workgroups.
template <class F>
hipError_t typed_gemv_dispatch(hipStream_t s, const GemvArgs& a, int dtype, int cus) {
  const int ntiles = a.n / 16;
  static const int persistent = env_int("Q6K_GEMV_PERSISTENT", -1);  // -1 auto, 0 off, 1 on
  if (a.nb == 16 && persistent != 0 && (persistent > 0 || ntiles >= 16 * cus))
    return typed_persistent_launch<F, F::kPT, 2, F::kPW>(s, a, dtype, cus);
  static const int forced = env_int("Q6K_GEMV_TILES", 0);
  const int t = forced == 1 || forced == 2 || forced == 4 ? forced : ntiles >= 8 * cus ? 4 : ntiles >= 4 * cus ? 2 : 1;
  if (t == 4)
    return typed_gemv_launch<F, 4, 2>(s, a, dtype);
  if (t == 2)
    return typed_gemv_launch<F, 2, 2>(s, a, dtype);
  return typed_gemv_launch<F, 1, 2>(s, a, dtype);
}

// The Q4_K LM-head shape (K = 4096, at least 16 column tiles per CU, m <= 8)
// on the persistent form.
bool q4k_persistent_supported(int m, int nb, int n, int cus) {
  static const int on = env_int("Q4K_GEMV_PERSISTENT", 1);
  return on && m >= 1 && m <= 8 && nb == 16 && n % 16 == 0 && n / 16 >= 16 * cus;
}

hipError_t launch_q4k_persistent(hipStream_t s, const GemvArgs& a, int dtype, int cus) {
  return typed_persistent_launch<FmtQ4K, FmtQ4K::kPT, 2, FmtQ4K::kPW>(s, a, dtype, cus);
}

hipError_t launch_typed_gemv(hipStream_t s, const GemvArgs& a, uint32_t type, int dtype, int cus) {
  switch (type) {
    case kTypeQ4_K:
      return typed_gemv_dispatch<FmtQ4K>(s, a, dtype, cus);
    case kTypeQ6_K:
      return typed_gemv_dispatch<FmtQ6K>(s, a, dtype, cus);
    case kTypeQ8_0:
      return typed_gemv_dispatch<FmtQ8_0>(s, a, dtype, cus);
    case kTypeQ5_K:
      return typed_gemv_dispatch<FmtQ5K>(s, a, dtype, cus);
    case kTypeIQ4_XS:
      return typed_gemv_dispatch<FmtIQ4XS>(s, a, dtype, cus);
    default:
      return hipErrorInvalidValue;
  }
}

template <class P, bool GATED>
hipError_t typed_gemm_launch(hipStream_t s, const GemmArgs& a, int dtype, int cus) {
  constexpr int OT = GATED ? P::kCT / 2 : P::kCT;  // output column tiles per wave
  const int ntiles = a.n / 16, tiles_x = (ntiles + 4 * OT - 1) / (4 * OT);
  const int tiles_y = (a.m + kG2M - 1) / kG2M, tiles = tiles_x * tiles_y;
  const int g = tiles > cus ? cus : tiles;
  const TileMap map = make_tile_map(tiles_x, tiles_y, g);
  const dim3 grid((unsigned)g), block(256);
  if (dtype == kF32)
    (void)dispatch(typed_gemm_kernel<P, float, GATED>, grid, block, s, a, map, ntiles);
  else
    (void)dispatch(typed_gemm_kernel<P, _Float16, GATED>, grid, block, s, a, map, ntiles);
  return hipGetLastError();
}

bool typed_gemm_supported(uint32_t type, int m, int n) {
  const bool served = type == kTypeQ5_K || type == kTypeQ6_K || type == kTypeQ8_0 || type == kTypeIQ4_XS;
  return served && m > 0 && n > 0 && n % 16 == 0;
}

// Rounds of workgroups of the 192-column Q8_0 tiling against the 128-column
// one, each weighted by its columns per tile.
static bool q8_mid(int ntiles, int tiles_y, int cus) {
  static const int forced = env_int("Q4K_TYPED_MID", -1);
  if (forced >= 0)
    return forced == 1;
  const int r3 = ((ntiles + 11) / 12 * tiles_y + cus - 1) / cus, r2 = ((ntiles + 7) / 8 * tiles_y + cus - 1) / cus;
  return 3 * r3 <= 2 * r2;
}

// Four column tiles per wave with B in half tile-blocks (TgQ8_0W) where its
// rounds of workgroups over the CUs take no longer than those of the three-
// and two-tile forms, each round weighted by the time of one tile of that
// form: at M = 2048 a 192-column tile took 0.80 and a 128-column tile 0.61 of
// a 256-column tile's time (N = 12288, K = 4096: 190.6 us against 202.1 with
// three tiles per wave; N = 4096, K = 12288: 178.6 against 219.0 with two).
// Q4K_TYPED_Q8W: -1 auto, 0 never, 1 always; Q4K_TYPED_MID set (0 or 1)
// turns the auto choice of this form off as well.
static bool q8_wide(int ntiles, int tiles_y, int cus) {
  static const int forced = env_int("Q4K_TYPED_Q8W", -1);
  static const int mid = env_int("Q4K_TYPED_MID", -1);
  if (forced >= 0)
    return forced == 1;
  if (mid >= 0)
    return false;
  auto rounds = [&](int cols) { return ((ntiles * 16 + cols - 1) / cols * tiles_y + cus - 1) / cus; };
  const int r4 = rounds(256), r3 = rounds(192), r2 = rounds(128);
  return 100 * r4 <= 80 * r3 && 100 * r4 <= 61 * r2;
}

hipError_t launch_typed_gemm(hipStream_t s, const GemmArgs& a, uint32_t type, int dtype, int cus) {
  if (!typed_gemm_supported(type, a.m, a.n) || a.nb < 1)
    return hipErrorInvalidValue;
  const int ntiles = a.n / 16, tiles_y = (a.m + kG2M - 1) / kG2M;
  const bool narrow = gemm2_narrow(((ntiles + 15) / 16) * tiles_y, ((ntiles + 7) / 8) * tiles_y, cus);
  switch (type) {
    case kTypeQ5_K:
      return narrow ? typed_gemm_launch<Narrow<TgQ5K>>(s, a, dtype, cus) : typed_gemm_launch<TgQ5K>(s, a, dtype, cus);
    case kTypeQ6_K:
      return narrow ? typed_gemm_launch<Narrow<TgQ6K>>(s, a, dtype, cus) : typed_gemm_launch<TgQ6K>(s, a, dtype, cus);
    case kTypeQ8_0:
      // Four column tiles per wave on the half tile-block ring (q8_wide), or
      // two (two blocks of its tile-blocks per column fit beside an A ring),
      // or three where the 192-column grid takes no more time in rounds:
      // three tiles read each A fragment for half as many MFMAs again (at
      // M = 2048 the N = 12288 GEMM measured 211 instead of 243 us; Q6_K and
      // Q5_K measured slower with three, also with a 5-slot A ring).
      // Q4K_TYPED_MID: -1 auto, 0 never, 1 always.
      if (q8_wide(ntiles, tiles_y, cus))
        return typed_gemm_launch<TgQ8_0W>(s, a, dtype, cus);
      if (q8_mid(ntiles, tiles_y, cus))
        return typed_gemm_launch<Mid<TgQ8_0, 3>>(s, a, dtype, cus);
      return typed_gemm_launch<TgQ8_0>(s, a, dtype, cus);
    default:
      if (gemm_six(((ntiles + 15) / 16) * tiles_y, ((ntiles + 23) / 24) * tiles_y, cus))
        return typed_gemm_launch<Six<TgIQ4XS>>(s, a, dtype, cus);
      return narrow ? typed_gemm_launch<Narrow<TgIQ4XS>>(s, a, dtype, cus) : typed_gemm_launch<TgIQ4XS>(s, a, dtype, cus);
  }
}

hipError_t launch_typed_relayout(hipStream_t s, const uint8_t* src, uint8_t* dst, uint32_t n, uint32_t k, uint32_t type) {
  const uint32_t nb = k / 256;
  const size_t tiles = (size_t)(n / 16) * nb;
  if (tiles == 0)
    return hipSuccess;
  if (type_block_bytes(type) == 0 || type == kTypeQ4_K)
    return hipErrorInvalidValue;
  (void)dispatch(typed_relayout_kernel, dim3((unsigned)tiles), dim3(64), s, src, dst, nb, type);
  return hipGetLastError();
}

}  // namespace q4k
