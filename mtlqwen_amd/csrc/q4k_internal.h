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

// ---- the other GGUF types on the same surface ------------------------------
// Per 256 elements: block_q8_0 is eight 34-byte records (d fp16, 32 int8),
// block_q5_K 176 bytes (d, dmin, the Q4_K 6-bit scale/min bytes, qh[32],
// qs[128]), block_iq4_xs 136 bytes (d, scales_h, scales_l[4], qs[128]).  Every
// tile-block keeps its type's byte count (16 rows x one block):
//   Q8_0 (4352 B): four slabs, lane l = 16g + i holding the 64 quants of its
//     elements (the Q6_K element order) as bytes q ^ 0x80, byte 2o + hf of the
//     lane for B dword o, half hf; then lane l's dword at 4096 + 4l with d of
//     records 2g, 2g + 1 of row 16c + i.
//   Q5_K (2816 B): the Q4_K tile-block of the low nibbles and headers (2304 B),
//     then lane l's two dwords at 2304 + 8l with the fifth bits: bit
//     4 (fs % 4) + t (+16 for the high half) of dword fs / 4 for B dword t of
//     MFMA fs.
//   IQ4_XS (2176 B): two slabs, lane l's dword fs (slab fs / 4, word fs % 4)
//     holding the codebook indices of MFMA fs: byte b's low nibble for value
//     b, its high nibble for value 4 + b (value h = B dword h / 2, half h % 2);
//     then the 16 rows' first 8 bytes (d, scales_h, scales_l) at 2048 + 8i.
constexpr int kQ8BlockBytes = 272;
constexpr int kQ5BlockBytes = 176;
constexpr int kIQ4BlockBytes = 136;
constexpr uint32_t kTypeQ8_0 = 8, kTypeQ4_K = 12, kTypeQ5_K = 13, kTypeQ6_K = 14, kTypeIQ4_XS = 23;

// Bytes per 256-element block of a served ggml type (0 if not served).
__host__ __device__ inline int type_block_bytes(uint32_t type) {
  switch (type) {
    case kTypeQ4_K:
      return kBlockBytes;
    case kTypeQ6_K:
      return kQ6BlockBytes;
    case kTypeQ8_0:
      return kQ8BlockBytes;
    case kTypeQ5_K:
      return kQ5BlockBytes;
    case kTypeIQ4_XS:
      return kIQ4BlockBytes;
    default:
      return 0;
  }
}

__host__ __device__ inline void put_u32(uint8_t* p, uint32_t v) {
  p[0] = (uint8_t)v;
  p[1] = (uint8_t)(v >> 8);
  p[2] = (uint8_t)(v >> 16);
  p[3] = (uint8_t)(v >> 24);
}

// Lane `lane`'s share of one tile-block `tb` of a Q6_K, Q8_0, Q5_K or IQ4_XS
// tensor, from block `blk` of row 16c + lane % 16 (lanes 0..15 also write
// their row's per-row bytes).  Shared by the host and device re-layouts.
__host__ __device__ inline void encode_lane(uint32_t type, const uint8_t* blk, uint8_t* tb, int lane) {
  const int g = lane >> 4, i = lane & 15;
  if (type == kTypeQ6_K) {
    uint32_t wd[12] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    for (int o = 0; o < 32; ++o)
      for (int hf = 0; hf < 2; ++hf)
        q6_place(wd, o, hf, q6_quant(blk, q6_elem(g, o, hf)));
    for (int j = 0; j < 12; ++j)
      put_u32(tb + (j >> 2) * 1024 + 16 * lane + 4 * (j & 3), wd[j]);
    for (int j = 0; j < 4; ++j)
      tb[kQ6ScaleOffset + 4 * lane + j] = (uint8_t)(blk[192 + 4 * g + j] ^ 0x80u);
    if (g == 0) {
      tb[kQ6DOffset + 2 * i] = blk[208];
      tb[kQ6DOffset + 2 * i + 1] = blk[209];
    }
  } else if (type == kTypeQ8_0) {
    for (int o = 0; o < 32; ++o)
      for (int hf = 0; hf < 2; ++hf) {
        const int e = q6_elem(g, o, hf), byte = 2 * o + hf;
        tb[(byte >> 4) * 1024 + 16 * lane + (byte & 15)] = (uint8_t)(blk[34 * (e >> 5) + 2 + (e & 31)] ^ 0x80u);
      }
    const uint8_t* r0 = blk + 34 * (2 * g);
    const uint8_t* r1 = blk + 34 * (2 * g + 1);
    put_u32(tb + 4096 + 4 * lane, (uint32_t)r0[0] | ((uint32_t)r0[1] << 8) | ((uint32_t)r1[0] << 16) | ((uint32_t)r1[1] << 24));
  } else if (type == kTypeQ5_K) {
    // Low nibbles and header exactly as Q4_K (its qs sit at byte 48, not 16).
    for (int h = 0; h < 2; ++h)
      for (int w = 0; w < 4; ++w) {
        const uint8_t* q = blk + 48 + 32 * g + 16 * h + 4 * w;
        uint8_t* t = tb + h * kSlabBytes + 16 * lane + 4 * w;
        t[0] = q[0];
        t[1] = q[2];
        t[2] = q[1];
        t[3] = q[3];
      }
    if (g == 0)
      for (int j = 0; j < 16; ++j)
        tb[kHeaderOffset + 16 * i + j] = blk[j];
    uint32_t hw[2] = {0u, 0u};
    for (int fs = 0; fs < 8; ++fs)
      for (int t = 0; t < 4; ++t)
        for (int hf = 0; hf < 2; ++hf) {
          const int e = q6_elem(g, 4 * fs + t, hf);
          const uint32_t bit = (blk[16 + (e & 31)] >> (2 * (e >> 6) + ((e >> 5) & 1))) & 1u;
          hw[fs >> 2] |= bit << (4 * (fs & 3) + t + 16 * hf);
        }
    put_u32(tb + 2304 + 8 * lane, hw[0]);
    put_u32(tb + 2304 + 8 * lane + 4, hw[1]);
  } else if (type == kTypeIQ4_XS) {
    for (int fs = 0; fs < 8; ++fs) {
      uint32_t w = 0;
      for (int h = 0; h < 8; ++h) {
        const int e = q6_elem(g, 4 * fs + (h >> 1), h & 1);
        const uint32_t v = (blk[8 + 16 * (e >> 5) + (e & 15)] >> (4 * ((e >> 4) & 1))) & 15u;
        w |= v << (h < 4 ? 8 * h : 8 * (h - 4) + 4);
      }
      put_u32(tb + (fs >> 2) * 1024 + 16 * lane + 4 * (fs & 3), w);
    }
    if (g == 0)
      for (int j = 0; j < 8; ++j)
        tb[2048 + 8 * i + j] = blk[j];
  }
}

__host__ __device__ inline uint32_t get_u32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

__host__ __device__ inline float half_to_float(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// The 64 weights of lane `lane` of one tile-block of a type other than Q4_K,
// in fp32 as the reference's prefill tiles compute them before their half()
// store (quant_linear.metal:54-115): w[8 fs + h] is element
// q6_elem(g, 4 fs + h / 2, h % 2) of row 16c + lane % 16.
__host__ __device__ inline void decode_lane(uint32_t type, const uint8_t* tb, int lane, float* w) {
  const int g = lane >> 4, i = lane & 15;
  if (type == kTypeQ6_K) {
    uint32_t wd[12];
    #pragma unroll
    for (int j = 0; j < 12; ++j)
      wd[j] = get_u32(tb + (j >> 2) * 1024 + 16 * lane + 4 * (j & 3));
    const float d = half_to_float(tb[kQ6DOffset + 2 * i] | (tb[kQ6DOffset + 2 * i + 1] << 8));
    #pragma unroll
    for (int o = 0; o < 32; ++o) {
      const float sc = (float)(int8_t)(tb[kQ6ScaleOffset + 4 * lane + (o >> 3)] ^ 0x80u);
      #pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        w[2 * o + hf] = d * sc * (float)((int)q6_take(wd, o, hf) - 32);
    }
  } else if (type == kTypeQ8_0) {
    const uint32_t dd = get_u32(tb + 4096 + 4 * lane);
    #pragma unroll
    for (int o = 0; o < 32; ++o)
      #pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int byte = 2 * o + hf;
        const float d = half_to_float(o < 16 ? dd & 0xffffu : dd >> 16);
        w[byte] = d * (float)(int8_t)(tb[(byte >> 4) * 1024 + 16 * lane + (byte & 15)] ^ 0x80u);
      }
  } else if (type == kTypeQ5_K) {
    const uint8_t* hd = tb + kHeaderOffset + 16 * i;
    const float d = half_to_float(hd[0] | (hd[1] << 8)), dm = half_to_float(hd[2] | (hd[3] << 8));
    const uint32_t hb[2] = {get_u32(tb + 2304 + 8 * lane), get_u32(tb + 2304 + 8 * lane + 4)};
    #pragma unroll
    for (int fs = 0; fs < 8; ++fs) {
      // sub-block 2g + fs / 4: the 6-bit scale / min of the header (quant_linear.metal:12-20)
      const int j = 2 * g + (fs >> 2);
      const uint8_t* q = hd + 4;
      const uint32_t sc = j < 4 ? q[j] & 63u : (q[j + 4] & 15u) | ((q[j - 4] >> 6) << 4);
      const uint32_t mn = j < 4 ? q[j + 4] & 63u : (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
      #pragma unroll
      for (int h = 0; h < 8; ++h) {
        const int t = h >> 1, hf = h & 1;
        const int jj = 8 * (fs & 3) + 2 * t + hf;  // quant byte 32g + jj of the row
        const int ob = jj & 3, sb = ob == 1 ? 2 : ob == 2 ? 1 : ob;  // middle bytes swapped
        const uint32_t byte = tb[(jj >> 4) * kSlabBytes + 16 * lane + (jj & 12) + sb];
        const uint32_t nib = fs < 4 ? byte & 15u : byte >> 4;
        const uint32_t bit = (hb[fs >> 2] >> (4 * (fs & 3) + t + 16 * hf)) & 1u;
        w[8 * fs + h] = d * (float)sc * (float)(nib + 16 * bit) - dm * (float)mn;
      }
    }
  } else if (type == kTypeIQ4_XS) {
    const uint8_t* hd = tb + 2048 + 8 * i;
    const float d = half_to_float(hd[0] | (hd[1] << 8));
    const uint32_t sh = hd[2] | (hd[3] << 8), sl = get_u32(hd + 4);
    // iq4nl (quant_linear.metal:5) + 128, four bytes per word.
    const uint32_t tab[4] = {0x3F2D1801u, 0x766A5D4Fu, 0xA6998D81u, 0xF1D9C5B5u};
    #pragma unroll
    for (int fs = 0; fs < 8; ++fs) {
      const int j = 2 * g + (fs >> 2);
      const int ls = (int)(((sl >> (4 * j)) & 15u) | (((sh >> (2 * j)) & 3u) << 4)) - 32;
      const uint32_t wq = get_u32(tb + (fs >> 2) * 1024 + 16 * lane + 4 * (fs & 3));
      #pragma unroll
      for (int h = 0; h < 8; ++h) {
        const uint32_t v = h < 4 ? (wq >> (8 * h)) & 15u : (wq >> (8 * (h - 4) + 4)) & 15u;
        const float cb = (float)((int)((tab[v >> 2] >> (8 * (v & 3))) & 0xFFu) - 128);
        w[8 * fs + h] = d * (float)ls * cb;
      }
    }
  }
}

// Rows of a GEMV call are padded to 16-row MFMA tiles; the GEMV handles up to
// kGemvMaxRowTiles of them (48 rows: the 8 x 5 decode rows of the reference).
constexpr int kGemvMaxRowTiles = 3;

enum Dtype : int { kF32 = 0, kF16 = 1 };

// Decode pack: the MFMA operands of x (m <= 8 rows) for the per-item and
// persistent GEMVs (layout in q4k_kernels.hip, stage_pack_kernel).
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
  DecodePack pack;        // packed operands of x (per-item and persistent GEMVs)
  void* y;
  const void* aux;
  int m, n, k, nb, post;
  int rows;  // staged fragment rows: 2m when split (rows m.. hold the low parts), else m
  int split;
  // Fused gate/up and rows GEMVs: when non-null, x is RMS-normalised first,
  // x * rsqrt(sum(x^2) / k + eps) * norm_w (native_ops.metal:6-40).
  const float* norm_w = nullptr;
  float eps = 0.0f;
  // Rows GEMV in K-slices: the slices' sums and per-group arrival counters
  // (zero before the launch; every launch leaves them zero).
  float* part = nullptr;
  int* counters = nullptr;
};

struct GemmArgs {
  const uint8_t* w;
  const uint8_t* wu = nullptr;  // the gated GEMM's up matrix (w is the gate)
  const _Float16* xh;  // staged activations in the GEMM order (gemm_frag_offset)
  const float* rowscale;
  void* y;
  const void* aux;
  int m, n, k, nb, post;
  // K-split (gemm2_split_plan): the two segments' accumulators and per-tile
  // arrival counters (zero before the launch; every launch leaves them
  // zero).  Segment 0 of a tile is blocks [0, split_b), segment 1 blocks
  // [split_b, nb).  split_q > 0: segment 0 of tile t runs on workgroup t and
  // the segments 1 split_q per workgroup on the workgroups past the tiles;
  // split_q == 0: the 2 x tiles segments are dealt round robin.
  float* part = nullptr;
  int* counters = nullptr;
  int split_b = 0, split_q = 0;
};

struct GatherIndex {
  uint32_t rows;
  uint32_t src[64];
};

// The queries of a packed batch for the token embedding: query q owns rows
// [start[q], start[q] + count[q]) and reads its tokens from row slot[q] of
// the request buffer (capacity tokens per slot), from position[q] on.
constexpr uint32_t kEmbedMaxQueries = 64;
struct EmbedQueries {
  uint32_t n, capacity;
  uint32_t start[kEmbedMaxQueries], count[kEmbedMaxQueries], position[kEmbedMaxQueries], slot[kEmbedMaxQueries];
};

// Activation staging layouts.
enum StageMode : int {
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
// norm_w != nullptr: x is RMS-normalised on the way in, x * rsqrt(sum(x^2) /
// k + eps) * norm_w (native_ops.metal:6-40), before the conversion.
hipError_t launch_stage_x(hipStream_t s, const void* x, int dtype, _Float16* xo, _Float16* xs, float* rowscale, int m, int k, int mode,
                          const float* norm_w = nullptr, float eps = 0.0f);
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
GemvShape gemv_shape(int rows, int n, int nb, bool gated, int cus);

// Fused gate/up GEMV for m <= 8 rows and K = 4096 that packs x itself (no
// staging launch); reads a.x, a.w, a.wu (and a.norm_w when set) and writes a.y.
bool gemv_gate_up_supported(int m, int nb, int n);
hipError_t launch_gemv_gate_up(hipStream_t s, const GemvArgs& a, int dtype, int cus);
// GEMV over staged x of 17..48 fragment rows: T column tiles of NM matrices
// per workgroup, 8 waves splitting K (K = 2048 .. 12288), each block of x
// read once per wave.  gemv_rows_plan returns T (0: not this kernel) and the
// K-slices (1, or 3 for K = 12288: partials and counters in the split-K
// workspace, gemv_rows_part_floats floats and n / (16 T) counters).
struct RowsPlan {
  int tiles = 0, slices = 1;
};
RowsPlan gemv_rows_plan(int rows, int nb, int n, bool gated, int cus);
size_t gemv_rows_part_floats(const RowsPlan& p, int n);
hipError_t launch_gemv_rows(hipStream_t s, const GemvArgs& a, int dtype, const RowsPlan& p, bool gated);
// The same for gate and up weights of one other type with a fused decode
// kernel in the reference (Q5_K, IQ4_XS).
bool typed_gate_up_supported(uint32_t type, int m, int nb, int n);
hipError_t launch_typed_gate_up(hipStream_t s, const GemvArgs& a, uint32_t type, int dtype, int cus);

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

// Pipelined GEMM: xh holds the activations staged in the GEMM order
// (kStageGemm) for gemm2_rows(m) rows; any N that is a multiple of 16.
bool gemm2_supported(int m, int n);
int gemm2_rows(int m);
// Whether the pipelined GEMM (plain and gated alike) of this shape runs as two
// K-halves per tile (few tiles for the CUs), and the workspace it then needs.
int gemm2_split_b(int m, int n, int nb, int cus);
void gemm2_split_workspace(int m, int n, bool gated, size_t* part_floats, size_t* counters);
hipError_t launch_gemm2(hipStream_t s, const GemmArgs& a, int dtype, int cus);
// Gate and up projections of one prefill MLP in one launch (both Q4_K, the
// same n and k, x staged once): y = SiLU(x W^T) * (x Wu^T) with the
// roundings of the two-call form (gate stored, then up with post 2 over it).
hipError_t launch_gemm2_gated(hipStream_t s, const GemmArgs& a, int dtype, int cus);

// One MFMA-ceiling launch: `blocks` workgroups of 4 waves, each wave issuing
// 32 * iters v_mfma_f32_16x16x32_f16 (16384 FLOP each); out holds blocks * 256 floats.
hipError_t launch_mfma_ceiling(hipStream_t s, float* out, int blocks, int iters);
// Streaming read of `bytes` (a multiple of 16) at p; `out` takes `blocks`
// words (almost never written).
hipError_t launch_stream_read(hipStream_t s, const void* p, size_t bytes, uint32_t* out, int blocks);

hipError_t launch_gather(hipStream_t s, const void* x, void* out, int k, int dtype, const GatherIndex& idx);

// p[0, n) = v on stream s (a kernel, so that graph capture records a kernel
// node rather than a memset).
hipError_t launch_fill_u32(hipStream_t s, uint32_t* p, uint32_t v, uint32_t n);

// Token embedding from a tiled Q4_K table (n rows of k): y[t] = row ids[t].
hipError_t launch_embedding(hipStream_t s, const uint8_t* w, const int32_t* ids, void* y, int rows, int n, int k, int dtype);
hipError_t launch_embedding_batch(hipStream_t s, const uint8_t* w, const int32_t* tokens, const EmbedQueries& qs, void* y, int rows, int n, int k,
                                  int dtype);

// RMS norm of `rows` rows of k (idx == nullptr: row r reads x row r;
// otherwise x row idx->src[r]).
hipError_t launch_rms_norm(hipStream_t s, const void* x, const float* w, void* y, int rows, int k, float eps, int dtype, const GatherIndex* idx);

// Device-side GGUF -> tiled re-layout (src and dst are device buffers).
hipError_t launch_relayout(hipStream_t s, const uint8_t* src, uint8_t* dst, uint32_t n, uint32_t k);

// Q4_K on the persistent GEMV of the other types (16 waves, x fragments in
// registers): K = 4096, at least 16 column tiles per CU (the LM head), m <= 8,
// a.pack = the decode pack of x.
bool q4k_persistent_supported(int m, int nb, int n, int cus);
hipError_t launch_q4k_persistent(hipStream_t s, const GemvArgs& a, int dtype, int cus);

// GEMV for m <= 8 rows over the decode pack of x (launch_stage_pack): a.w =
// tiled weights of ggml type `type` (Q4_K, Q6_K, Q8_0, Q5_K or IQ4_XS),
// post 0/1/2 on a.y / a.aux.
hipError_t launch_typed_gemv(hipStream_t s, const GemvArgs& a, uint32_t type, int dtype, int cus);

// Prefill GEMM for Q5_K, Q6_K, Q8_0 and IQ4_XS weights (x staged in the GEMM
// order, 128-row tiles; any n that is a multiple of 16).
bool typed_gemm_supported(uint32_t type, int m, int n);
hipError_t launch_typed_gemm(hipStream_t s, const GemmArgs& a, uint32_t type, int dtype, int cus);

// Device-side GGUF -> tiled re-layout of Q6_K, Q8_0, Q5_K or IQ4_XS weights.
hipError_t launch_typed_relayout(hipStream_t s, const uint8_t* src, uint8_t* dst, uint32_t n, uint32_t k, uint32_t type);

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
