// Device helpers shared by the kernel sources (q4k_kernels.hip,
// q4k_rows.hip): fp16 bit tricks, the Q4_K block constants, cross-lane
// reductions, activation fragment offsets, LDS-DMA and coherent loads and
// stores, and the cross-workgroup arrival counter.
#pragma once
#include <float.h>
#include <hip/hip_runtime.h>

#include "q4k_internal.h"

namespace q4k {
namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef float f16_t __attribute__((ext_vector_type(16)));

// g * sigmoid(g) with the hardware exponential and reciprocal (a few ulp;
// 1 + exp(-g) >= 1, so the reciprocal never sees a denormal or zero).
__device__ __forceinline__ float silu(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
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

// Scales and mins of sub-blocks 2g and 2g + 1 from the three packed words of
// a block header (quant_linear.metal:12-20, taken four bytes at a time), as
// 16-bit lanes: p0 = sc(2g) | m(2g) << 16, p1 = sc(2g + 1) | m(2g + 1) << 16.
// Bytes 0 / 1 of the selected words are gathered with one v_perm_b32 per
// word pair.
__device__ __forceinline__ void scale_min_packed(u4_t hd, int g, uint32_t& p0, uint32_t& p1) {
  const uint32_t sh = 16u * (uint32_t)(g & 1);
  const uint32_t a = hd.y >> sh, b = hd.z >> sh, c = hd.w >> sh;
  const bool low = g < 2;
  const uint32_t ysh = low ? 0u : 2u, xsh = low ? 0u : 4u;
  const uint32_t xa = low ? a : c, xb = (low ? b : c) >> xsh, ya = a >> ysh, yb = b >> ysh;
  const uint32_t x0 = __builtin_amdgcn_perm(xb, xa, 0x0C040C00u), x1 = __builtin_amdgcn_perm(xb, xa, 0x0C050C01u);
  const uint32_t y0 = __builtin_amdgcn_perm(yb, ya, 0x0C040C00u), y1 = __builtin_amdgcn_perm(yb, ya, 0x0C050C01u);
  p0 = (x0 & 0x000F000Fu) | (y0 & 0x00300030u);
  p1 = (x1 & 0x000F000Fu) | (y1 & 0x00300030u);
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
  h4_t bsc;  // 7.5 sc_j, j = 4(g - 2)..4(g - 2)+3 for g >= 2 (zero for g < 2): the mean-quant correction's B operand
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
  // k = 8..15 of the min-term MFMA: bytes 0..3 = sc_{4(g-2)}..sc_{4(g-2)+3}
  // for g >= 2, zero for g < 2; (1024 + sc) * 7.5 - 7680 = 7.5 sc exactly
  const uint32_t s03 = hd.y & 0x3F3F3F3Fu, s47 = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
  const uint32_t sb = g < 2 ? 0u : (g == 2 ? s03 : s47);
  const h2_t k75 = {(_Float16)7.5f, (_Float16)7.5f}, kneg7680 = {(_Float16)-7680.0f, (_Float16)-7680.0f};
  const h2_t s01 = __builtin_elementwise_fma(as_h2(__builtin_amdgcn_perm(0x64646464u, sb, 0x04010400u)), k75, kneg7680);
  const h2_t s23 = __builtin_elementwise_fma(as_h2(__builtin_amdgcn_perm(0x64646464u, sb, 0x04030402u)), k75, kneg7680);
  k.bsc = h4_t{s01[0], s01[1], s23[0], s23[1]};
  return k;
}

// Element offset of (row, 8-element chunk c) in the GEMV fragment layout:
// fragment ((row / 16) * nb + b) * 8 + s holds, for lane 16g + (row % 16),
// elements b*256 + 64g + 32*(s/4) + 8*(s%4) + [0, 8).
__device__ __forceinline__ size_t frag_offset(int row, int c, int nb) {
  const int kk = c * 8, b = kk >> 8, e = kk & 255, g = e >> 6, sl = ((e >> 5) & 1) * 4 + ((e >> 3) & 3);
  return ((((size_t)(row >> 4) * nb + b) * 8 + sl) * 64 + (g * 16 + (row & 15))) * 8;
}

// Element offset of (row, 8-element chunk c) in the pipelined GEMM's order:
// per (128-row block R, 256-element block b, u-step u) one contiguous 16 KB
// run of 16 fragments f = 2 * (row tile within R) + h, h = 0 for the low-
// nibble half (elements 64g + 8u + [0, 8)) and 1 for the high-nibble half
// (64g + 32 + 8u + [0, 8)); fragment lane 16g + row % 16.  One u-step of a
// workgroup's A operand is then a single contiguous read.
__device__ __forceinline__ size_t gemm_frag_offset(int row, int c, int nb) {
  const int kk = c * 8, b = kk >> 8, e = kk & 255, g = e >> 6, h = (e >> 5) & 1, u = (e >> 3) & 3;
  const int f = 2 * ((row >> 4) & 7) + h;
  return (((((size_t)(row >> 7) * nb + b) * 4 + u) * 16 + f) * 64 + (g * 16 + (row & 15))) * 8;
}

// Halves of one plane of min-term fragments (xs_offset) for `rows` staged
// rows; single fp16 staging writes a second plane, of the sub-blocks' sums of
// rounding residuals, right after the first.
__host__ __device__ inline size_t xs_plane_halves(int rows, int nb) {
  return (size_t)((rows + 15) / 16) * nb * 128;
}

// Half index of (row, sub-block j of block b) in the min-term fragments: per
// (row tile, block), lane 16 * (j / 4) + row % 16 holds j % 4 of 4 halves --
// the A operand of v_mfma_f32_16x16x16_f16 with k = sub-block (8 of 16 used).
__device__ __forceinline__ size_t xs_offset(int row, int b, int j, int nb) {
  return (((size_t)(row >> 4) * nb + b) * 32 + 16 * (j >> 2) + (row & 15)) * 4 + (j & 3);
}

// Cross-lane steps on the VALU (DPP), without the LDS crossbar's latency.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppQuadSwap1 = 0xB1;   // quad_perm(1, 0, 3, 2)
constexpr int kDppQuadSwap2 = 0x4E;   // quad_perm(2, 3, 0, 1)
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i within 8 lanes
constexpr int kDppRowMirror = 0x140;  // lane i <-> 15 - i within 16 lanes

// Sum over each aligned group of 8 lanes, in every lane of the group.
__device__ __forceinline__ float sum8_lanes(float v) {
  v += dpp_f<kDppQuadSwap1>(v);
  v += dpp_f<kDppQuadSwap2>(v);
  return v + dpp_f<kDppHalfMirror>(v);
}

// Maximum over the 64 lanes (uniform result).
__device__ __forceinline__ float max64_lanes(float v) {
  v = fmaxf(v, dpp_f<kDppQuadSwap1>(v));
  v = fmaxf(v, dpp_f<kDppQuadSwap2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppRowMirror>(v));
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)), r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)), r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// LDS-DMA loads are issued as asm: the compiler would otherwise guard every
// later LDS read with vmcnt(0) (it cannot tell the ring slots apart).  Their
// completion is covered by explicit vmcnt waits in the kernels that issue
// them.  No memory clobber: one makes the compiler treat the asm as an
// outstanding store and wait vmcnt(0) before every later LDS read; ordering
// against the LDS reads comes from a scheduling barrier at the issue point
// and the clobbering wait.  The address is a wave-uniform SGPR base plus a
// fixed per-lane VGPR offset, so issuing costs no vector ALU work.  M0 is
// written here; no other code of these kernels uses it.
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

// Stores and loads that bypass every cache level (sc0 sc1: system
// coherence), for data exchanged between workgroups on different XCDs.  The
// loads return through vmcnt like the others: wait before use.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  asm volatile("global_store_dword %0, %1, off sc0 sc1" ::"v"(p), "v"(v) : "memory");
}

__device__ __forceinline__ float load_coherent(const float* p) {
  float r;
  asm volatile("global_load_dword %0, %1, off sc0 sc1" : "=v"(r) : "v"(p));
  return r;
}

// The store reads its 16 data bytes after issue: a vector write to them must
// wait (wait states the compiler cannot insert after an asm store), hence the
// s_nop.
__device__ __forceinline__ void store_coherent4(float* p, f4_t v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1\n\ts_nop 2" ::"v"(p), "v"(v) : "memory");
}

__device__ __forceinline__ f4_t load_coherent4(const float* p) {
  f4_t r;
  asm volatile("global_load_dwordx4 %0, %1, off sc0 sc1" : "=v"(r) : "v"(p));
  return r;
}

// Pins a register value to this point of the program: an asm load's result
// is used only after the explicit wait that precedes hold().
template <typename V>
__device__ __forceinline__ void hold(V& v) {
  asm volatile("" : "+v"(v));
}

// Count of arrivals at a counter shared by workgroups on any XCD: the atomic
// is performed at system scope (past every XCD's L2).
__device__ __forceinline__ int count_arrival(int* ctr) {
  return __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ void reset_counter(int* ctr) {
  __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Power-of-two scale that puts a row's largest magnitude mx in [2^14, 2^15):
// finite in fp16 with the full 11-bit significand for every large element.
__device__ __forceinline__ void pow2_scale(float mx, float& up, float& down) {
  up = 1.0f;
  down = 1.0f;
  if (mx > 0.0f && mx <= FLT_MAX) {
    int e;
    frexpf(mx, &e);
    e = e < -80 ? -80 : e;
    up = ldexpf(1.0f, 15 - e);
    down = ldexpf(1.0f, e - 15);
  }
}

}  // namespace
}  // namespace q4k
