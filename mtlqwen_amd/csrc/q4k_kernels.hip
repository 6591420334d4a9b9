// Q4_K linear() kernels for gfx950 (MI355X / CDNA4).
//
//  stage_x_kernel   activations -> fp16 with a per-row power-of-two scale
//  q4k_gemv_kernel  decode-shaped (m <= 48) GEMV on v_mfma_f32_16x16x32_f16,
//                   optionally fused gate/up with the SiLU(gate)*up epilogue
//  q4k_gemm_kernel  prefill-shaped GEMM: Q4_K tiles dequantised to fp16 in LDS,
//                   v_mfma_f32_32x32x16_f16, fp32 accumulation, post 0/1/2
//  gather_rows_kernel, relayout_kernel
//
// Reference semantics: backend/metal/kernel/quant_linear.metal (Q4_K parts)
// and backend/metal/kernel/fused_kernels.metal:11-78.
#include <float.h>
#include <hip/hip_runtime.h>
#include <stdlib.h>

#include "q4k_internal.h"

namespace q4k {
namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef float f16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float silu(float g) {
  return g / (1.0f + expf(-g));
}

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ float round_half(float v) {
  return (float)(_Float16)v;
}

template <typename T>
__device__ __forceinline__ float load_elem(const T* p, size_t i) {
  return (float)p[i];
}

template <typename T>
__device__ __forceinline__ void store_elem(T* p, size_t i, float v) {
  p[i] = (T)v;
}

// Loads 8 consecutive activations as fp32.
__device__ __forceinline__ void load8(const float* p, float* v) {
  f4_t a = *reinterpret_cast<const f4_t*>(p), b = *reinterpret_cast<const f4_t*>(p + 4);
  v[0] = a[0], v[1] = a[1], v[2] = a[2], v[3] = a[3], v[4] = b[0], v[5] = b[1], v[6] = b[2], v[7] = b[3];
}

__device__ __forceinline__ void load8(const _Float16* p, float* v) {
  h8_t a = *reinterpret_cast<const h8_t*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    v[i] = (float)a[i];
}

// Scales and mins of sub-blocks 2g and 2g+1 from the three packed words of a
// block header (quant_linear.metal:12-20, taken four bytes at a time).
__device__ __forceinline__ void scale_min_pair(u4_t hd, int g, uint32_t& sc0, uint32_t& m0, uint32_t& sc1, uint32_t& m1) {
  const uint32_t sh = 16u * (uint32_t)(g & 1);
  const uint32_t a = hd.y >> sh, b = hd.z >> sh, c = hd.w >> sh;
  if (g < 2) {
    sc0 = a & 63u;
    sc1 = (a >> 8) & 63u;
    m0 = b & 63u;
    m1 = (b >> 8) & 63u;
  } else {
    sc0 = (c & 15u) | ((a >> 2) & 0x30u);
    sc1 = ((c >> 8) & 15u) | ((a >> 10) & 0x30u);
    m0 = ((c >> 4) & 15u) | ((b >> 2) & 0x30u);
    m1 = ((c >> 12) & 15u) | ((b >> 10) & 0x30u);
  }
}

// (a & mask) | bits in one v_and_or_b32.  Written as asm because gfx9 VOP3
// encodings cannot take the two literal constants the compiler would
// otherwise need, so it splits the expression into v_and + v_or.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(mask), "v"(bits));
  return r;
}

__device__ __forceinline__ h2_t as_h2(uint32_t v) {
  return __builtin_bit_cast(h2_t, v);
}

__device__ __forceinline__ uint32_t as_u32(h2_t v) {
  return __builtin_bit_cast(uint32_t, v);
}

// Eight quants of one slab pair as exact fp16 products q * sc.
// (w & mask) | 0x6400 is the fp16 value 1024 + q (low nibble, mask 0x000F) or
// 1024 + 16q (high nibble, mask 0x00F0); one fused multiply-add with
// (sc, -1024 sc) or (sc/16, -64 sc) leaves q*sc <= 945, exact in fp16.
__device__ __forceinline__ h8_t quant_times_scale(uint32_t wa, uint32_t wb, uint32_t mask, uint32_t bias, h2_t mul, h2_t add) {
  const uint32_t wa8 = wa >> 8, wb8 = wb >> 8;
  const h2_t v0 = __builtin_elementwise_fma(as_h2(and_or(wa, mask, bias)), mul, add);
  const h2_t v1 = __builtin_elementwise_fma(as_h2(and_or(wa8, mask, bias)), mul, add);
  const h2_t v2 = __builtin_elementwise_fma(as_h2(and_or(wb, mask, bias)), mul, add);
  const h2_t v3 = __builtin_elementwise_fma(as_h2(and_or(wb8, mask, bias)), mul, add);
  return __builtin_bit_cast(h8_t, u4_t{as_u32(v0), as_u32(v1), as_u32(v2), as_u32(v3)});
}

// Per-lane constants of one tile-block header for lane group g: the fp16
// multipliers of the low / high nibbles (sub-blocks 2g, 2g+1) and the min
// fragment 32 * m_{4g..4g+3} (zero for g >= 2: k = 8..15 of the 16x16x16 MFMA
// are unused).  quant_linear.metal:12-20 unpacking, two fields at a time.
struct BlockConsts {
  float d, dmin;
  h2_t mul_lo, add_lo, mul_hi, add_hi;
  h4_t bmin;
};

__device__ __forceinline__ BlockConsts block_consts(u4_t hd, int g) {
  BlockConsts k;
  k.d = half_bits_to_float(hd.x & 0xffffu);
  k.dmin = half_bits_to_float(hd.x >> 16);
  const uint32_t sh = 16u * (uint32_t)(g & 1);
  const uint32_t a = hd.y >> sh, c = hd.w >> sh;
  // bytes 0, 1 = sc_{2g}, sc_{2g+1} (both forms computed, then selected:
  // lanes of one wave take both sides of the g < 2 split)
  const uint32_t sc_direct = a & 0x3F3Fu, sc_packed = (c & 0x0F0Fu) | ((a >> 2) & 0x3030u);
  const uint32_t scp = g < 2 ? sc_direct : sc_packed;
  const h2_t k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
  const h2_t kneg1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
  // perm(0x64646464, v, sel) interleaves bytes of v with 0x64: fp16 1024 + byte.
  k.mul_lo = as_h2(__builtin_amdgcn_perm(0x64646464u, scp, 0x04000400u)) - k1024;
  k.add_lo = k.mul_lo * kneg1024;
  const h2_t p_hi = as_h2(__builtin_amdgcn_perm(0x64646464u, scp, 0x04010401u));
  k.mul_hi = __builtin_elementwise_fma(p_hi, h2_t{(_Float16)0.0625f, (_Float16)0.0625f}, h2_t{(_Float16)-64.0f, (_Float16)-64.0f});
  k.add_hi = k.mul_hi * kneg1024;
  // bytes 0..3 = m_{4g}..m_{4g+3} for g < 2; zero for g >= 2 (k = 8..15 unused)
  const uint32_t m03 = hd.z & 0x3F3F3F3Fu, m47 = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
  const uint32_t mb = g >= 2 ? 0u : (g == 0 ? m03 : m47);
  const h2_t k32 = {(_Float16)32.0f, (_Float16)32.0f}, kneg32768 = {(_Float16)-32768.0f, (_Float16)-32768.0f};
  const h2_t m01 = __builtin_elementwise_fma(as_h2(__builtin_amdgcn_perm(0x64646464u, mb, 0x04010400u)), k32, kneg32768);
  const h2_t m23 = __builtin_elementwise_fma(as_h2(__builtin_amdgcn_perm(0x64646464u, mb, 0x04030402u)), k32, kneg32768);
  k.bmin = h4_t{m01[0], m01[1], m23[0], m23[1]};
  return k;
}

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

// Element offset of (row, 8-element chunk c) in the GEMV fragment layout:
// fragment ((row / 16) * nb + b) * 8 + s holds, for lane 16g + (row % 16),
// elements b*256 + 64g + 32*(s/4) + 8*(s%4) + [0, 8).
__device__ __forceinline__ size_t frag_offset(int row, int c, int nb) {
  const int kk = c * 8, b = kk >> 8, e = kk & 255, g = e >> 6, sl = ((e >> 5) & 1) * 4 + ((e >> 3) & 3);
  return ((((size_t)(row >> 4) * nb + b) * 8 + sl) * 64 + (g * 16 + (row & 15))) * 8;
}

// Half index of (row, sub-block j of block b) in the min-term fragments: per
// (row tile, block), lane 16 * (j / 4) + row % 16 holds j % 4 of 4 halves --
// the A operand of v_mfma_f32_16x16x16_f16 with k = sub-block (8 of 16 used).
__device__ __forceinline__ size_t xs_offset(int row, int b, int j, int nb) {
  return (((size_t)(row >> 4) * nb + b) * 32 + 16 * (j >> 2) + (row & 15)) * 4 + (j & 3);
}

// Converts and stores one 8-element chunk; all 256 threads of the workgroup
// must call it together (the sub-block sum is reduced over 4 lanes).
template <int MODE>
__device__ __forceinline__ void stage_store(_Float16* xo, _Float16* xs, int row, int c, bool live, int m, int k, int nb, const float* v,
                                            float up) {
  h8_t hi, lo;
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float t = v[i] * up;
    hi[i] = (_Float16)t;
    lo[i] = (_Float16)(t - (float)hi[i]);
    sum += t;
  }
  if (MODE == kStageRowMajor) {
    if (live)
      *reinterpret_cast<h8_t*>(xo + (size_t)row * k + (size_t)c * 8) = hi;
    return;
  }
  if (live) {
    *reinterpret_cast<h8_t*>(xo + frag_offset(row, c, nb)) = hi;
    if (MODE == kStageFragSplit)
      *reinterpret_cast<h8_t*>(xo + frag_offset(m + row, c, nb)) = lo;
  }
  // Chunks 4q..4q+3 (lanes 4q..4q+3) form one sub-block.
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  if (live && (c & 3) == 0) {
    const float s32 = sum * 0.03125f;
    const _Float16 sh = (_Float16)s32;
    const int b = c >> 5, j = (c >> 2) & 7;
    xs[xs_offset(row, b, j, nb)] = sh;
    if (MODE == kStageFragSplit)
      xs[xs_offset(m + row, b, j, nb)] = (_Float16)(s32 - (float)sh);
  }
}

template <typename InT, int MODE>
__global__ __launch_bounds__(256) void stage_x_kernel(const InT* __restrict__ x, _Float16* __restrict__ xo, _Float16* __restrict__ xs,
                                                      float* __restrict__ rowscale, int m, int k) {
  const int row = blockIdx.x;
  const InT* xr = x + (size_t)row * k;
  const int chunks = k >> 3, nb = k >> 8;
  const bool in_regs = chunks <= 256 * kStageRegChunks;
  float v[kStageRegChunks][8] = {};
  float mx = 0.0f;
  if (in_regs) {
#pragma unroll
    for (int j = 0; j < kStageRegChunks; ++j) {
      const int c = threadIdx.x + 256 * j;
      if (c < chunks) {
        load8(xr + c * 8, v[j]);
#pragma unroll
        for (int i = 0; i < 8; ++i)
          mx = fmaxf(mx, fabsf(v[j][i]));
      }
    }
  } else {
    for (int c = threadIdx.x; c < chunks; c += 256) {
      float t[8];
      load8(xr + c * 8, t);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        mx = fmaxf(mx, fabsf(t[i]));
    }
  }
  mx = block_max_256(mx);
  // Scale the row so its largest magnitude lands in [2^14, 2^15): finite in
  // fp16 with the full 11-bit significand for every large element.
  float up = 1.0f, down = 1.0f;
  if (mx > 0.0f && mx <= FLT_MAX) {
    int e;
    frexpf(mx, &e);
    e = e < -80 ? -80 : e;
    up = ldexpf(1.0f, 15 - e);
    down = ldexpf(1.0f, e - 15);
  }
  if (threadIdx.x == 0)
    rowscale[row] = down;
  if (in_regs) {
#pragma unroll
    for (int j = 0; j < kStageRegChunks; ++j) {
      const int c = threadIdx.x + 256 * j;
      if (256 * j < chunks)  // uniform: whole groups of 4 lanes take part
        stage_store<MODE>(xo, xs, row, c, c < chunks, m, k, nb, v[j], up);
    }
  } else {
    for (int c0 = 0; c0 < chunks; c0 += 256) {
      const int c = c0 + threadIdx.x;
      float t[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (c < chunks)
        load8(xr + c * 8, t);
      stage_store<MODE>(xo, xs, row, c, c < chunks, m, k, nb, t, up);
    }
  }
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
  auto load_x = [&](h8_t (&xa)[RT][8], h4_t (&xsa)[RT], int b) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const h8_t* xp = reinterpret_cast<const h8_t*>(a.xf) + (size_t)(rt * nb + b) * 8 * 64 + lane;
#pragma unroll
      for (int s = 0; s < 8; ++s)
        xa[rt][s] = xp[s * 64];
      xsa[rt] = reinterpret_cast<const h4_t*>(a.xs)[(size_t)(rt * nb + b) * 32 + (lane & 31)];
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
          // min term: sum_j (xs_j / 32) * (32 m_j), k = sub-block
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
// Streaming GEMV (one 16-row activation tile, nb == W * BPW).
//
// Persistent workgroups (at most one per CU) loop over items of T column
// tiles.  Wave w owns blocks [w*BPW, (w+1)*BPW) of every item, so its
// activation fragments are loaded once and stay in registers.  Its weight
// tile-blocks ("units": block j, matrix mi, tile t) stream through a private
// LDS ring of D+1 slots with global_load_lds_dwordx4 (16 bytes per lane, lane
// order = slab order), D units ahead of the one being computed, so about
// D * 2.3 KB per wave is always in flight without holding VGPRs.  Every
// iteration issues exactly three loads (units past the end re-load the last
// unit, an L2 hit), so a constant vmcnt(3*D) marks the current unit complete.
// ----------------------------------------------------------------------------
// LDS-DMA loads are issued as asm: the compiler would otherwise guard every
// later LDS read with vmcnt(0) (it cannot tell the ring slots apart).  Their
// completion is covered by the explicit vmcnt waits below.  No memory
// clobber: one makes the compiler treat the asm as an outstanding store and
// wait vmcnt(0) before every later LDS read; ordering against the LDS reads
// comes from the scheduling barrier in issue() and the clobbering wait.  The
// address is a wave-uniform SGPR base plus a fixed per-lane VGPR offset, so
// issuing costs no vector ALU work.  M0 is written here; nothing else in this
// kernel uses it.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Wave-uniform values the compiler cannot prove uniform are moved to SGPRs.
__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const uint8_t*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

template <int OFFSET>
__device__ __forceinline__ void lds_dma16(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 offset:%3" ::"v"(voff), "s"(sbase), "s"(lds), "n"(OFFSET) : "m0");
}

template <int OFFSET>
__device__ __forceinline__ void lds_dma4(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1 offset:%3" ::"v"(voff), "s"(sbase), "s"(lds), "n"(OFFSET) : "m0");
}

// Register loads issued as asm for the same reason: a compiler-visible load
// makes its first use wait vmcnt(0), draining the ring.  Their results are
// released to the compiler by hold() after an explicit wait.
__device__ __forceinline__ u4_t asm_load16(const void* p) {
  u4_t r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p));
  return r;
}

__device__ __forceinline__ h4_t asm_load8(const void* p) {
  h4_t r;
  asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(r) : "v"(p));
  return r;
}

__device__ __forceinline__ float asm_load4(const void* p) {
  float r;
  asm volatile("global_load_dword %0, %1, off" : "=v"(r) : "v"(p));
  return r;
}

template <typename V>
__device__ __forceinline__ void hold(V& v) {
  asm volatile("" : "+v"(v));
}

template <int T, int NM, int W, int BPW, int D, typename OutT>
__global__ __launch_bounds__(64 * W) void q4k_gemv_stream_kernel(GemvArgs a, int items) {
  constexpr int MT = NM * T;       // (matrix, tile) pairs of an item
  constexpr int U = BPW * MT;      // units per item per wave, order (j, mi, t)
  constexpr int R = D + 1;         // ring slots per wave
  __shared__ __attribute__((aligned(16))) uint8_t ring[W][R][kTileBlockBytes];
  // Per-wave partial sums of the current item, [wave][mi*T+t][row][col]: each
  // wave accumulates its own slot in program order (deterministic), and the
  // epilogue sums the W slots in wave order.
  __shared__ float red[W][MT][16][16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, col = lane & 15;
  const int nb = a.nb, bw = wave * BPW;
  const int first = blockIdx.x, stride = gridDim.x;
  const int n_items = first < items ? (items - 1 - first) / stride + 1 : 0;
  if (n_items == 0)
    return;
  const uint32_t ring0 = lds_addr(&ring[wave][0][0]);
  const uint32_t voff16 = 16u * (uint32_t)lane, voff4 = 4u * (uint32_t)lane;
  const size_t tile_bytes = (size_t)nb * kTileBlockBytes;

  // Issue unit s of this wave's stream into ring slot `slot`; units past the
  // end re-load the last unit (an L2 hit) so every iteration issues exactly
  // three loads.
  auto issue = [&](int s, int slot) {
    __builtin_amdgcn_sched_barrier(0);
    int it = s / U;
    int q = s - it * U;
    if (it >= n_items) {
      it = n_items - 1;
      q = U - 1;
    }
    const int j = q / MT, mt = q - j * MT, mi = mt / T, t = mt - mi * T;
    const int ct = (first + it * stride) * T + t;
    const uint8_t* p = uniform_ptr((mi ? a.wu : a.w) + (size_t)ct * tile_bytes + (size_t)(bw + j) * kTileBlockBytes);
    // The immediate offset applies to both addresses: LDS = M0 + offset + lane * size.
    const uint32_t l = __builtin_amdgcn_readfirstlane(ring0 + (uint32_t)slot * kTileBlockBytes);
    lds_dma16<0>(p, voff16, l);
    lds_dma16<kSlabBytes>(p, voff16, l);
    lds_dma4<kHeaderOffset>(p, voff4, l);
  };

  // Resident activations of this wave's blocks (dead rows of the 16-row tile
  // are loaded unmasked; they only reach unread C rows) and the scales of the
  // rows this thread finishes in the epilogues (clamped: always issued), then
  // the first D units.  One wait covers the activations and unit 0.
  u4_t xw[BPW][8];
  h4_t xsa[BPW];
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
    const u4_t* xp = reinterpret_cast<const u4_t*>(a.xf) + (size_t)(bw + j) * 8 * 64 + lane;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      xw[j][s] = asm_load16(xp + s * 64);
    xsa[j] = asm_load8(reinterpret_cast<const h4_t*>(a.xs) + (size_t)(bw + j) * 32 + (lane & 31));
  }
  constexpr int EPI = 16 * T;  // outputs per row of an item
  const int r0 = tid / EPI, r1 = (tid + 64 * W) / EPI;
  float sc0 = asm_load4(a.rowscale + (r0 < a.m ? r0 : a.m - 1));
  float sc1 = asm_load4(a.rowscale + (r1 < a.m ? r1 : a.m - 1));
#pragma unroll
  for (int s = 0; s < D; ++s)
    issue(s, s);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * (D - 1)) : "memory");
  h8_t xa[BPW][8];
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      hold(xw[j][s]);
      xa[j][s] = __builtin_bit_cast(h8_t, xw[j][s]);
    }
    hold(xsa[j]);
  }
  hold(sc0);
  hold(sc1);

  OutT* y = reinterpret_cast<OutT*>(a.y);
  const OutT* aux = reinterpret_cast<const OutT*>(a.aux);
  int slot = 0;  // ring slot of the unit being computed
  int s = 0;     // stream index of the unit being computed
  for (int it = 0; it < n_items; ++it) {
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
      for (int mt = 0; mt < MT; ++mt, ++s) {
        issue(s + D, slot == 0 ? R - 1 : slot - 1);
        // Three loads per unit: vmcnt(3*D) leaves exactly the D newer units
        // outstanding.  The memory clobber keeps the LDS reads below the wait.
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * D) : "memory");
        const u4_t* sl = reinterpret_cast<const u4_t*>(&ring[wave][slot][0]);
        const u4_t q0 = sl[lane];
        const u4_t q1 = sl[kSlabBytes / 16 + lane];
        const u4_t hd = sl[kHeaderOffset / 16 + col];
        slot = slot == R - 1 ? 0 : slot + 1;
        const BlockConsts kc = block_consts(hd, g);
        // Two accumulation chains (low / high nibbles) keep the MFMA pipe busy.
        f4_t cl = f4_t{0.0f, 0.0f, 0.0f, 0.0f}, ch = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const u4_t qq = u < 2 ? q0 : q1;
          const uint32_t wa = qq[2 * (u & 1)], wb = qq[2 * (u & 1) + 1];
          const h8_t blo = quant_times_scale(wa, wb, 0x000F000Fu, 0x64006400u, kc.mul_lo, kc.add_lo);
          const h8_t bhi = quant_times_scale(wa, wb, 0x00F000F0u, 0x64006400u, kc.mul_hi, kc.add_hi);
          cl = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[j][u], blo, cl, 0, 0, 0);
          ch = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[j][4 + u], bhi, ch, 0, 0, 0);
        }
        const f4_t cm = __builtin_amdgcn_mfma_f32_16x16x16f16(xsa[j], kc.bmin, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        float* r = &red[wave][mt][4 * g][col];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float part = fmaf(kc.d, cl[v] + ch[v], -kc.dmin * cm[v]);
          r[16 * v] = j == 0 ? part : r[16 * v] + part;
        }
      }
    }

    // Item complete: sum the W partial slots and run the epilogue.
    __syncthreads();
    const int ct0 = (first + it * stride) * T;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int o = tid + k * 64 * W;
      if (o < a.m * EPI) {
        const int row = o / EPI, c = o % EPI, t = c >> 4, cc = c & 15;
        const float escale = k == 0 ? sc0 : sc1;
        float sm[NM];
#pragma unroll
        for (int mi = 0; mi < NM; ++mi) {
          float v = 0.0f;
#pragma unroll
          for (int w = 0; w < W; ++w)
            v += red[w][mi * T + t][row][cc];
          if (a.split) {
#pragma unroll
            for (int w = 0; w < W; ++w)
              v += red[w][mi * T + t][a.m + row][cc];
          }
          sm[mi] = v;
        }
        const size_t off = (size_t)row * a.n + (size_t)(ct0 + t) * 16 + cc;
        float out;
        if (NM == 2) {
          float gv = sm[0] * escale, uv = sm[NM - 1] * escale;
          if (sizeof(OutT) == 2) {
            gv = round_half(gv);
            uv = round_half(uv);
          }
          out = silu(gv) * uv;
        } else {
          float acc_v = sm[0] * escale;
          if (sizeof(OutT) == 2)
            acc_v = round_half(acc_v);
          out = a.post == 1 ? acc_v + load_elem(aux, off) : a.post == 2 ? silu(load_elem(aux, off)) * acc_v : acc_v;
        }
        store_elem(y, off, out);
      }
    }
    __syncthreads();
  }
  // Drain the trailing (re-load) units before the ring is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// ----------------------------------------------------------------------------
// GEMM (prefill).  Workgroup tile 128 x 128, 4 waves of 64 x 64, k-step 64
// (one quarter of a Q4_K block).  Per k-step: the 128x64 fp16 activation tile
// is copied to LDS; 256 threads dequantise the 128x64 weight tile to
// h(d*sc*q - dmin*m) (quant_linear.metal:43,45) into LDS; each wave then runs
// 16 v_mfma_f32_32x32x16_f16.
// ----------------------------------------------------------------------------
constexpr int kBM = 128, kBN = 128, kBK = 64, kLds = kBK + 8;

template <typename OutT>
__global__ __launch_bounds__(256) void q4k_gemm_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 As[kBM * kLds];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[kBN * kLds];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  const int nb = a.nb;

  f16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        acc[i][j][v] = 0.0f;

  // A copy: thread -> (row, 32-element half of the k-step).
  const int ar = tid >> 1, ak = (tid & 1) * 32;
  const bool a_live = m0 + ar < a.m;
  const _Float16* a_src = a.xh + (size_t)(m0 + ar) * a.k + ak;
  // B dequant: thread -> (column, slab).
  const int bc = tid >> 1, hh = tid & 1;
  const int bn = n0 + bc;
  const bool b_live = bn < a.n;
  const uint8_t* b_tile = a.w + (size_t)(bn >> 4) * nb * kTileBlockBytes;
  const int bi = bn & 15;

  for (int kb = 0; kb < nb; ++kb) {
    const uint8_t* tb = b_tile + (size_t)kb * kTileBlockBytes;
    u4_t hd = b_live ? *reinterpret_cast<const u4_t*>(tb + kHeaderOffset + 16 * bi) : u4_t{0u, 0u, 0u, 0u};
    const float d = half_bits_to_float(hd.x & 0xffffu), dmin = half_bits_to_float(hd.x >> 16);
    for (int gq = 0; gq < 4; ++gq) {
      // Stage A.
      h8_t av[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        av[j] = a_live ? *reinterpret_cast<const h8_t*>(a_src + (size_t)kb * 256 + gq * 64 + j * 8) : h8_t{};
      // Dequantise B: 16 quant bytes = 16 low-nibble + 16 high-nibble weights.
      u4_t raw = b_live ? *reinterpret_cast<const u4_t*>(tb + hh * kSlabBytes + 16 * (gq * 16 + bi)) : u4_t{0u, 0u, 0u, 0u};
      uint32_t sc0, mn0, sc1, mn1;
      scale_min_pair(hd, gq, sc0, mn0, sc1, mn1);
      const float ds0 = d * (float)sc0, dm0 = dmin * (float)mn0, ds1 = d * (float)sc1, dm1 = dmin * (float)mn1;
      h8_t lo[2], hi[2];
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        const uint32_t wv = raw[wd];
        // Stored byte order within a word is (0, 2, 1, 3) of the quant bytes.
        const uint32_t qb[4] = {wv & 0xffu, (wv >> 16) & 0xffu, (wv >> 8) & 0xffu, wv >> 24};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo[wd >> 1][(wd & 1) * 4 + e] = (_Float16)(ds0 * (float)(qb[e] & 15u) - dm0);
          hi[wd >> 1][(wd & 1) * 4 + e] = (_Float16)(ds1 * (float)(qb[e] >> 4) - dm1);
        }
      }
      __syncthreads();  // previous k-step's MFMA reads are done
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<h8_t*>(&As[ar * kLds + ak + j * 8]) = av[j];
      _Float16* bdst = &Bs[bc * kLds + 16 * hh];
      *reinterpret_cast<h8_t*>(bdst) = lo[0];
      *reinterpret_cast<h8_t*>(bdst + 8) = lo[1];
      *reinterpret_cast<h8_t*>(bdst + 32) = hi[0];
      *reinterpret_cast<h8_t*>(bdst + 40) = hi[1];
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < kBK / 16; ++kk) {
        h8_t af[2], bf[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          af[i] = *reinterpret_cast<const h8_t*>(&As[(wm * 64 + i * 32 + (lane & 31)) * kLds + kk * 16 + 8 * (lane >> 5)]);
          bf[i] = *reinterpret_cast<const h8_t*>(&Bs[(wn * 64 + i * 32 + (lane & 31)) * kLds + kk * 16 + 8 * (lane >> 5)]);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  OutT* y = reinterpret_cast<OutT*>(a.y);
  const OutT* aux = reinterpret_cast<const OutT*>(a.aux);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn * 64 + j * 32 + (lane & 31);
      if (n >= a.n)
        continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row >= a.m)
          continue;
        const size_t o = (size_t)row * a.n + n;
        float acc_v = acc[i][j][v] * a.rowscale[row];
        if (sizeof(OutT) == 2)
          acc_v = round_half(acc_v);
        const float out = a.post == 1 ? acc_v + load_elem(aux, o) : a.post == 2 ? silu(load_elem(aux, o)) * acc_v : acc_v;
        store_elem(y, o, out);
      }
    }
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
hipError_t gemv_multi_row_tile(hipStream_t s, const GemvArgs& a, int dtype, int waves) {
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
    return gemv_multi_row_tile<2, GATED>(s, a, dtype, shape.waves);
  return gemv_multi_row_tile<3, GATED>(s, a, dtype, shape.waves);
}

template <int T, int NM, int W, int BPW, int D>
hipError_t stream_launch(hipStream_t s, const GemvArgs& a, int dtype, int grid, int items) {
  if (dtype == kF32)
    (void)dispatch(q4k_gemv_stream_kernel<T, NM, W, BPW, D, float>, dim3((unsigned)grid), dim3(64 * W), s, a, items);
  else
    (void)dispatch(q4k_gemv_stream_kernel<T, NM, W, BPW, D, _Float16>, dim3((unsigned)grid), dim3(64 * W), s, a, items);
  return hipGetLastError();
}

}  // namespace

bool gemv_stream_supported(int rows, int nb, int n, bool gated) {
  (void)gated;
  static const bool enabled = env_int("Q4K_GEMV_STREAM", 1) != 0;
  return enabled && rows <= 16 && nb == 16 && n % 16 == 0;
}

hipError_t launch_gemv_stream(hipStream_t s, const GemvArgs& a, int dtype, bool gated, int cus) {
  // One row tile, K = 4096 (nb = 16): 8 waves x 2 blocks, 4 units in flight
  // per wave.  Items of T column tiles: T = 3 makes N = 12288 exactly one item
  // per CU; wide outputs take T = 4; otherwise one tile per item.
  const int ctiles = a.n / 16;
  int tiles = 1;
  if (ctiles % 3 == 0 && ctiles / 3 == cus)
    tiles = 3;
  else if (!gated && ctiles % 4 == 0 && ctiles / 4 >= 4 * cus)
    tiles = 4;
  else if (!gated && ctiles % 2 == 0 && ctiles / 2 >= 2 * cus)
    tiles = 2;
  const int items = ctiles / tiles;
  const int grid = items < cus ? items : cus;
  if (gated)
    return tiles == 3 ? stream_launch<3, 2, 8, 2, 4>(s, a, dtype, grid, items) : stream_launch<1, 2, 8, 2, 4>(s, a, dtype, grid, items);
  if (tiles == 4)
    return stream_launch<4, 1, 8, 2, 4>(s, a, dtype, grid, items);
  if (tiles == 3)
    return stream_launch<3, 1, 8, 2, 4>(s, a, dtype, grid, items);
  if (tiles == 2)
    return stream_launch<2, 1, 8, 2, 4>(s, a, dtype, grid, items);
  return stream_launch<1, 1, 8, 2, 4>(s, a, dtype, grid, items);
}

template <typename InT>
hipError_t stage_launch(hipStream_t s, const InT* x, _Float16* xo, _Float16* xs, float* rowscale, int m, int k, int mode) {
  const dim3 grid((unsigned)m), block(256);
  if (mode == kStageRowMajor)
    (void)dispatch(stage_x_kernel<InT, kStageRowMajor>, grid, block, s, x, xo, xs, rowscale, m, k);
  else if (mode == kStageFrag)
    (void)dispatch(stage_x_kernel<InT, kStageFrag>, grid, block, s, x, xo, xs, rowscale, m, k);
  else
    (void)dispatch(stage_x_kernel<InT, kStageFragSplit>, grid, block, s, x, xo, xs, rowscale, m, k);
  return hipGetLastError();
}

hipError_t launch_stage_x(hipStream_t s, const void* x, int dtype, _Float16* xo, _Float16* xs, float* rowscale, int m, int k, int mode) {
  if (m <= 0)
    return hipSuccess;
  if (dtype == kF32)
    return stage_launch(s, static_cast<const float*>(x), xo, xs, rowscale, m, k, mode);
  return stage_launch(s, static_cast<const _Float16*>(x), xo, xs, rowscale, m, k, mode);
}

GemvShape gemv_shape(int rows, int n, int nb, bool gated) {
  GemvShape sh;
  sh.row_tiles = rows <= 16 ? 1 : rows <= 32 ? 2 : 3;
  // One 16-column tile per workgroup (two for very wide outputs, one row tile,
  // no gate/up pair), and enough waves per workgroup -- each taking 1/waves
  // of K -- for about 12-16 resident waves per CU across the grid.
  const int ctiles = n / 16;
  static const int env_tiles = env_int("Q4K_GEMV_TILES", 0), env_waves = env_int("Q4K_GEMV_WAVES", 0);
  sh.tiles = (sh.row_tiles == 1 && !gated && n % 32 == 0 && ctiles >= 4096) ? 2 : 1;
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

hipError_t launch_gemm(hipStream_t s, const GemmArgs& a, int dtype) {
  const dim3 grid((unsigned)((a.n + kBN - 1) / kBN), (unsigned)((a.m + kBM - 1) / kBM)), block(256);
  if (dtype == kF32)
    (void)dispatch(q4k_gemm_kernel<float>, grid, block, s, a);
  else
    (void)dispatch(q4k_gemm_kernel<_Float16>, grid, block, s, a);
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

hipError_t launch_relayout(hipStream_t s, const uint8_t* src, uint8_t* dst, uint32_t n, uint32_t k) {
  const uint32_t nb = k / 256;
  const size_t tiles = (size_t)(n / 16) * nb;
  if (tiles == 0)
    return hipSuccess;
  (void)dispatch(relayout_kernel, dim3((unsigned)tiles), dim3(64), s, src, dst, n, nb);
  return hipGetLastError();
}

}  // namespace q4k
