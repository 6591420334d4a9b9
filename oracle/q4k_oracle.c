/*
 * q4k_oracle.c -- CPU restatement of MTLQwen's Q4_K linear() arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path (see q4k_oracle.h).
 * Built with -ffp-contract=off so every fp32 operation rounds exactly once,
 * in the order written.
 */
#include "q4k_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ---------------------------------------------------------------- fp16 -- */

float q4o_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: man * 2^-24, renormalise */
      int e = -1;
      do {
        ++e;
        man <<= 1;
      } while ((man & 0x400u) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t q4o_float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) /* inf / nan (quiet) */
    return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0u));
  if (ax >= 0x477ff000u) /* >= 65520 rounds to inf */
    return (uint16_t)(sign | 0x7c00u);
  if (ax < 0x38800000u) { /* below 2^-14: half subnormal, unit 2^-24 */
    uint32_t e = ax >> 23;
    if (e < 102u) /* < 2^-25 */
      return (uint16_t)sign;
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e;
    uint32_t q = mant >> shift, rem = mant & ((1u << shift) - 1u), halfway = 1u << (shift - 1u);
    if (rem > halfway || (rem == halfway && (q & 1u)))
      ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t r = ax - 0x38000000u; /* rebias 127 -> 15 */
  uint32_t q = r >> 13, rem = r & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u)))
    ++q;
  return (uint16_t)(sign | q);
}

static float h2f(const uint8_t* p) {
  return q4o_half_to_float((uint16_t)(p[0] | (p[1] << 8)));
}

static float hround(float v) {
  return q4o_half_to_float(q4o_float_to_half(v));
}

/* ---------------------------------------------------------- the format -- */

/* quant_linear.metal:12-20 */
void q4o_scale_min(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 15) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

void q4o_pack_scale_min(const uint8_t sc[8], const uint8_t m[8], uint8_t q[12]) {
  for (int j = 0; j < 4; ++j) {
    q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    q[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
    q[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
  }
}

/* Element e of a block: byte qs[(e/64)*32 + e%32], low nibble when e%64 < 32
 * (quant_linear.metal:39-45). */
static inline uint8_t nibble(const uint8_t* qs, int e) {
  uint8_t b = qs[(e >> 6) * 32 + (e & 31)];
  return (e & 32) ? (uint8_t)(b >> 4) : (uint8_t)(b & 15);
}

/* quant_linear.metal:32-48 */
void q4o_dequant_block(const uint8_t* blk, float* out) {
  float d = h2f(blk), dm = h2f(blk + 2);
  for (int t = 0; t < 4; ++t) {
    for (int lane = 0; lane < 32; ++lane) {
      uint8_t sc, mn, q = blk[16 + t * 32 + lane];
      int r = t * 64 + lane, j = t * 2;
      q4o_scale_min(j, blk + 4, &sc, &mn);
      out[r] = d * (float)sc * (float)(q & 15) - dm * (float)mn;
      q4o_scale_min(j + 1, blk + 4, &sc, &mn);
      out[r + 32] = d * (float)sc * (float)(q >> 4) - dm * (float)mn;
    }
  }
}

void q4o_dequant_block_f16(const uint8_t* blk, uint16_t* out) {
  float tmp[256];
  q4o_dequant_block(blk, tmp);
  for (int i = 0; i < 256; ++i)
    out[i] = q4o_float_to_half(tmp[i]);
}

/* quant_linear.metal:69-86 (dequant_tile<q6_k_tag>): half h = e / 128,
 * rr = e % 128, l = rr % 32; the low nibble of ql[64h + 32((rr >> 5) & 1) + l]
 * (high nibble when rr >= 64), the two bits (qh[32h + l] >> 2(rr / 32)) & 3
 * on top. */
int q6o_quant(const uint8_t* blk, int e) {
  const int h = e >> 7, rr = e & 127, l = rr & 31, s = rr >> 5;
  const uint8_t q = blk[64 * h + ((rr & 32) ? 32 : 0) + l];
  const int lo = (rr & 64) ? (q >> 4) : (q & 15);
  const int hi = (blk[128 + 32 * h + l] >> (2 * s)) & 3;
  return (hi << 4) | lo;
}

/* quant_linear.metal:82: scales[8h + rr / 16] = scales[e / 16], int8. */
int q6o_scale(const uint8_t* blk, int e) {
  return (int8_t)blk[192 + 8 * (e >> 7) + ((e & 127) >> 4)];
}

/* quant_linear.metal:79-83: (d * sc) * (q - 32) in fp32. */
void q6o_dequant_block(const uint8_t* blk, float* out) {
  const float d = h2f(blk + 208);
  for (int e = 0; e < 256; ++e)
    out[e] = d * (float)q6o_scale(blk, e) * (float)(q6o_quant(blk, e) - 32);
}

void q6o_dequant_block_f16(const uint8_t* blk, uint16_t* out) {
  float tmp[256];
  q6o_dequant_block(blk, tmp);
  for (int i = 0; i < 256; ++i)
    out[i] = q4o_float_to_half(tmp[i]);
}

/* ---- block_q8_0 (quant_linear.metal:89-100): 8 records of (d fp16, 32 int8)
 * per 256 elements; element e of record e / 32 is d * qs[e % 32]. */
void q8o_dequant_block(const uint8_t* blk, float* out) {
  for (int e = 0; e < 256; ++e) {
    const uint8_t* r = blk + 34 * (e >> 5);
    out[e] = h2f(r) * (float)(int8_t)r[2 + (e & 31)];
  }
}

/* ---- block_q5_K (quant_linear.metal:50-67): d @0, dmin @2, the Q4_K 6-bit
 * scale/min bytes @4, qh[32] @16, qs[128] @48.  Element e (t = e / 64,
 * l = e % 32, high nibble when e % 64 >= 32): the nibble of qs[32t + l] plus
 * 16 when bit 2t (+1 for the high nibble) of qh[l] is set. */
int q5o_quant(const uint8_t* blk, int e) {
  const int t = e >> 6, l = e & 31, hi = (e >> 5) & 1;
  const uint8_t q = blk[48 + 32 * t + l];
  const int lo = hi ? (q >> 4) : (q & 15);
  return lo + (((blk[16 + l] >> (2 * t + hi)) & 1) << 4);
}

void q5o_dequant_block(const uint8_t* blk, float* out) {
  const float d = h2f(blk), dm = h2f(blk + 2);
  for (int e = 0; e < 256; ++e) {
    uint8_t sc, mn;
    q4o_scale_min(e >> 5, blk + 4, &sc, &mn);
    out[e] = d * (float)sc * (float)q5o_quant(blk, e) - dm * (float)mn;
  }
}

/* ---- block_iq4_xs (quant_linear.metal:102-115): d @0, scales_h u16 @2,
 * scales_l[4] @4, qs[128] @8.  Sub-block j = e / 32 has the 6-bit scale
 * ls = (scales_l[j / 2] >> 4(j % 2)) & 15 | ((scales_h >> 2j) & 3) << 4; element e
 * is d * (ls - 32) * iq4nl[v] with v the low nibble of qs[16j + e % 16], the
 * high nibble when e % 32 >= 16. */
static const float kIq4nl[16] = {-127.0f, -104.0f, -83.0f, -65.0f, -49.0f, -35.0f, -22.0f, -10.0f,
                                 1.0f,    13.0f,   25.0f,  38.0f,  53.0f,  69.0f,  89.0f,  113.0f};

int iq4o_index(const uint8_t* blk, int e) {
  const int j = e >> 5, r = e & 31;
  const uint8_t q = blk[8 + 16 * j + (r & 15)];
  return (r & 16) ? (q >> 4) : (q & 15);
}

int iq4o_scale(const uint8_t* blk, int j) {
  const int sh = blk[2] | (blk[3] << 8);
  return (((blk[4 + j / 2] >> (4 * (j % 2))) & 15) | (((sh >> (2 * j)) & 3) << 4)) - 32;
}

float iq4o_value(int v) {
  return kIq4nl[v & 15];
}

void iq4o_dequant_block(const uint8_t* blk, float* out) {
  const float d = h2f(blk);
  for (int e = 0; e < 256; ++e)
    out[e] = d * (float)iq4o_scale(blk, e >> 5) * kIq4nl[iq4o_index(blk, e)];
}

static size_t block_bytes(int type) {
  switch (type) {
    case Q4O_TYPE_Q6_K:
      return Q6O_BLOCK_BYTES;
    case Q4O_TYPE_Q8_0:
      return Q8O_BLOCK_BYTES;
    case Q4O_TYPE_Q5_K:
      return Q5O_BLOCK_BYTES;
    case Q4O_TYPE_IQ4_XS:
      return IQ4O_BLOCK_BYTES;
    default:
      return Q4O_BLOCK_BYTES;
  }
}

/* Weight e of a 256-element block of any served type, in double (the
 * dequantize-then-dot formulation). */
static double weight64(const uint8_t* p, int type, int e) {
  switch (type) {
    case Q4O_TYPE_Q6_K:
      return (double)h2f(p + 208) * (double)q6o_scale(p, e) * (double)(q6o_quant(p, e) - 32);
    case Q4O_TYPE_Q8_0:
      return (double)h2f(p + 34 * (e >> 5)) * (double)(int8_t)p[34 * (e >> 5) + 2 + (e & 31)];
    case Q4O_TYPE_Q5_K: {
      uint8_t sc, mn;
      q4o_scale_min(e >> 5, p + 4, &sc, &mn);
      return (double)h2f(p) * (double)sc * (double)q5o_quant(p, e) - (double)h2f(p + 2) * (double)mn;
    }
    case Q4O_TYPE_IQ4_XS:
      return (double)h2f(p) * (double)iq4o_scale(p, e >> 5) * (double)kIq4nl[iq4o_index(p, e)];
    default: {
      uint8_t sc, mn;
      q4o_scale_min(e / 32, p + 4, &sc, &mn);
      return (double)h2f(p) * (double)sc * (double)nibble(p + 16, e) - (double)h2f(p + 2) * (double)mn;
    }
  }
}

/* ------------------------------------------------------- contraction -- */

/* One (row n of W) x (M rows of x) contraction in the decode algebraic form of
 * quant_linear.metal:259-303: per sub-block sum(x*q) and sum(x) in fp32, then
 * acc += d * sum_j(sc_j*sum(x*q)_j) - dmin * sum_j(m_j*sum(x)_j). */
static void contract_row(float* acc, const float* x, int M, int K, const uint8_t* wrow) {
  int nb = K / 256;
  for (int m = 0; m < M; ++m)
    acc[m] = 0.0f;
  float q[256];
  for (int b = 0; b < nb; ++b) {
    const uint8_t* blk = wrow + (size_t)b * Q4O_BLOCK_BYTES;
    float d = h2f(blk), dm = h2f(blk + 2);
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; ++j)
      q4o_scale_min(j, blk + 4, &sc[j], &mn[j]);
    for (int e = 0; e < 256; ++e)
      q[e] = (float)nibble(blk + 16, e);
    for (int m = 0; m < M; ++m) {
      const float* xb = x + (size_t)m * K + (size_t)b * 256;
      float bq = 0.0f, bm = 0.0f;
      for (int j = 0; j < 8; ++j) {
        float sq = 0.0f, sx = 0.0f;
        for (int i = 0; i < 32; ++i) {
          sq += xb[j * 32 + i] * q[j * 32 + i];
          sx += xb[j * 32 + i];
        }
        bq += (float)sc[j] * sq;
        bm += (float)mn[j] * sx;
      }
      acc[m] += d * bq - dm * bm;
    }
  }
}

/* The block_q6_K contraction in the decode form of quant_linear.metal:437-497:
 * per 16-element sub-block j, sum(x * (q - 32)) in fp32, then
 * acc += d * sum_j(sc_j * sum_j). */
/* block_q8_0 in the decode form of quant_linear.metal:525-533: per 32-element
 * record, sum(q * x) in fp32, times d. */
static void contract_row_q8(float* acc, const float* x, int M, int K, const uint8_t* wrow) {
  const int nr = K / 32;
  for (int m = 0; m < M; ++m) {
    float a = 0.0f;
    for (int r = 0; r < nr; ++r) {
      const uint8_t* rec = wrow + (size_t)r * 34;
      const float* xb = x + (size_t)m * K + (size_t)r * 32;
      float sq = 0.0f;
      for (int i = 0; i < 32; ++i)
        sq += (float)(int8_t)rec[2 + i] * xb[i];
      a += sq * h2f(rec);
    }
    acc[m] = a;
  }
}

/* block_q5_K in the decode form of quant_linear.metal:345-412: per 32-element
 * sub-block sum(x * q5) and sum(x) in fp32, then d * sum(sc * .) - dmin * sum(m * .). */
static void contract_row_q5(float* acc, const float* x, int M, int K, const uint8_t* wrow) {
  const int nb = K / 256;
  for (int m = 0; m < M; ++m)
    acc[m] = 0.0f;
  float q[256];
  for (int b = 0; b < nb; ++b) {
    const uint8_t* blk = wrow + (size_t)b * Q5O_BLOCK_BYTES;
    const float d = h2f(blk), dm = h2f(blk + 2);
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; ++j)
      q4o_scale_min(j, blk + 4, &sc[j], &mn[j]);
    for (int e = 0; e < 256; ++e)
      q[e] = (float)q5o_quant(blk, e);
    for (int m = 0; m < M; ++m) {
      const float* xb = x + (size_t)m * K + (size_t)b * 256;
      float bq = 0.0f, bm = 0.0f;
      for (int j = 0; j < 8; ++j) {
        float sq = 0.0f, sx = 0.0f;
        for (int i = 0; i < 32; ++i) {
          sq += xb[j * 32 + i] * q[j * 32 + i];
          sx += xb[j * 32 + i];
        }
        bq += (float)sc[j] * sq;
        bm += (float)mn[j] * sx;
      }
      acc[m] += d * bq - dm * bm;
    }
  }
}

/* block_iq4_xs in the decode form of fused_kernels.metal:156-178: per 32-element
 * sub-block sum(x * iq4nl[v]) in fp32, times d * (ls - 32). */
static void contract_row_iq4(float* acc, const float* x, int M, int K, const uint8_t* wrow) {
  const int nb = K / 256;
  for (int m = 0; m < M; ++m)
    acc[m] = 0.0f;
  float v[256];
  for (int b = 0; b < nb; ++b) {
    const uint8_t* blk = wrow + (size_t)b * IQ4O_BLOCK_BYTES;
    const float d = h2f(blk);
    for (int e = 0; e < 256; ++e)
      v[e] = kIq4nl[iq4o_index(blk, e)];
    for (int m = 0; m < M; ++m) {
      const float* xb = x + (size_t)m * K + (size_t)b * 256;
      for (int j = 0; j < 8; ++j) {
        float s = 0.0f;
        for (int i = 0; i < 32; ++i)
          s += xb[j * 32 + i] * v[j * 32 + i];
        acc[m] += d * (float)iq4o_scale(blk, j) * s;
      }
    }
  }
}

typedef void (*contract_fn)(float*, const float*, int, int, const uint8_t*);

static void contract_row_q6(float* acc, const float* x, int M, int K, const uint8_t* wrow);

static contract_fn contract_for(int type) {
  switch (type) {
    case Q4O_TYPE_Q6_K:
      return contract_row_q6;
    case Q4O_TYPE_Q8_0:
      return contract_row_q8;
    case Q4O_TYPE_Q5_K:
      return contract_row_q5;
    case Q4O_TYPE_IQ4_XS:
      return contract_row_iq4;
    default:
      return contract_row;
  }
}

static void contract_row_q6(float* acc, const float* x, int M, int K, const uint8_t* wrow) {
  int nb = K / 256;
  for (int m = 0; m < M; ++m)
    acc[m] = 0.0f;
  float q[256];
  for (int b = 0; b < nb; ++b) {
    const uint8_t* blk = wrow + (size_t)b * Q6O_BLOCK_BYTES;
    float d = h2f(blk + 208);
    for (int e = 0; e < 256; ++e)
      q[e] = (float)(q6o_quant(blk, e) - 32);
    for (int m = 0; m < M; ++m) {
      const float* xb = x + (size_t)m * K + (size_t)b * 256;
      float bq = 0.0f;
      for (int j = 0; j < 16; ++j) {
        float sq = 0.0f;
        for (int i = 0; i < 16; ++i)
          sq += xb[j * 16 + i] * q[j * 16 + i];
        bq += (float)q6o_scale(blk, j * 16) * sq;
      }
      acc[m] += d * bq;
    }
  }
}

static float silu(float g) {
  return g / (1.0f + expf(-g));
}

enum { KIND_F32, KIND_F16, KIND_GATE_F32, KIND_GATE_F16, KIND_F64 };

typedef struct {
  int kind, M, N, K, post, type;
  void* y;
  const float* x; /* fp32 copy of the activations */
  const double* xd;
  const uint8_t* w;
  const uint8_t* wu;
  const void* aux;
  int n0, n1;
} job_t;

static void* run_job(void* arg) {
  job_t* j = (job_t*)arg;
  int M = j->M, N = j->N, K = j->K;
  const size_t bb = block_bytes(j->type), row_bytes = (size_t)(K / 256) * bb;
  const contract_fn contract = contract_for(j->type);
  if (j->kind == KIND_F64) {
    double* y = (double*)j->y;
    for (int n = j->n0; n < j->n1; ++n) {
      for (int m = 0; m < M; ++m)
        y[(size_t)m * N + n] = 0.0;
      for (int b = 0; b < K / 256; ++b) {
        const uint8_t* p = j->w + n * row_bytes + (size_t)b * bb;
        for (int e = 0; e < 256; ++e) {
          const double wv = weight64(p, j->type, e);
          for (int m = 0; m < M; ++m)
            y[(size_t)m * N + n] += j->xd[(size_t)m * K + (size_t)b * 256 + e] * wv;
        }
      }
    }
    return NULL;
  }
  float* acc = (float*)malloc(sizeof(float) * (size_t)M);
  float* acc2 = (float*)malloc(sizeof(float) * (size_t)M);
  for (int n = j->n0; n < j->n1; ++n) {
    contract(acc, j->x, M, K, j->w + n * row_bytes);
    if (j->kind == KIND_GATE_F32 || j->kind == KIND_GATE_F16)
      contract(acc2, j->x, M, K, j->wu + n * row_bytes);
    for (int m = 0; m < M; ++m) {
      size_t o = (size_t)m * N + n;
      switch (j->kind) {
      case KIND_F32: {
        float v = acc[m];
        const float* aux = (const float*)j->aux;
        if (j->post == 1)
          v = v + aux[o];
        else if (j->post == 2)
          v = silu(aux[o]) * v;
        ((float*)j->y)[o] = v;
        break;
      }
      case KIND_F16: {
        const uint16_t* aux = (const uint16_t*)j->aux;
        float v = hround(acc[m]);
        if (j->post == 1)
          v = v + q4o_half_to_float(aux[o]);
        else if (j->post == 2)
          v = silu(q4o_half_to_float(aux[o])) * v;
        ((uint16_t*)j->y)[o] = q4o_float_to_half(v);
        break;
      }
      case KIND_GATE_F32:
        ((float*)j->y)[o] = silu(acc[m]) * acc2[m];
        break;
      case KIND_GATE_F16: {
        float gh = hround(acc[m]), uh = hround(acc2[m]);
        ((uint16_t*)j->y)[o] = q4o_float_to_half(silu(gh) * uh);
        break;
      }
      }
    }
  }
  free(acc);
  free(acc2);
  return NULL;
}

static int run(job_t proto, int threads) {
  if (threads <= 0) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    threads = n > 0 ? (int)n : 1;
  }
  if (threads > proto.N)
    threads = proto.N;
  if (threads < 1)
    threads = 1;
  job_t* jobs = (job_t*)calloc((size_t)threads, sizeof(job_t));
  pthread_t* tid = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
  for (int t = 0; t < threads; ++t) {
    jobs[t] = proto;
    jobs[t].n0 = (int)((long long)proto.N * t / threads);
    jobs[t].n1 = (int)((long long)proto.N * (t + 1) / threads);
  }
  for (int t = 1; t < threads; ++t)
    pthread_create(&tid[t], NULL, run_job, &jobs[t]);
  run_job(&jobs[0]);
  for (int t = 1; t < threads; ++t)
    pthread_join(tid[t], NULL);
  free(jobs);
  free(tid);
  return 0;
}

static int bad_shape(int M, int N, int K) {
  return M < 0 || N <= 0 || K <= 0 || (K % 256) != 0;
}

static int bad_type(int type) {
  return type != Q4O_TYPE_Q4_K && type != Q4O_TYPE_Q6_K && type != Q4O_TYPE_Q8_0 && type != Q4O_TYPE_Q5_K && type != Q4O_TYPE_IQ4_XS;
}

/* Results are written to a private buffer first so aux may alias y. */
static int linear_common(int kind, int type, void* y, size_t elem, const float* x, const uint8_t* w, const uint8_t* wu, const void* aux, int M,
                         int N, int K, int post, int threads) {
  if (bad_shape(M, N, K) || post < 0 || post > 2 || !w || (M && (!x || !y)) || (post && !aux) || bad_type(type))
    return -1;
  if (M == 0)
    return 0;
  void* out = malloc(elem * (size_t)M * N);
  job_t p;
  memset(&p, 0, sizeof(p));
  p.kind = kind;
  p.type = type;
  p.M = M;
  p.N = N;
  p.K = K;
  p.post = post;
  p.y = out;
  p.x = x;
  p.w = w;
  p.wu = wu;
  p.aux = aux;
  run(p, threads);
  memcpy(y, out, elem * (size_t)M * N);
  free(out);
  return 0;
}

int q4o_linear_typed_f32(float* y, const float* x, const uint8_t* w, int type, const float* aux, int M, int N, int K, int post, int threads) {
  return linear_common(KIND_F32, type, y, 4, x, w, NULL, aux, M, N, K, post, threads);
}

int q4o_linear_f32(float* y, const float* x, const uint8_t* w, const float* aux, int M, int N, int K, int post, int threads) {
  return q4o_linear_typed_f32(y, x, w, Q4O_TYPE_Q4_K, aux, M, N, K, post, threads);
}

static float* widen(const uint16_t* x, size_t count) {
  float* f = (float*)malloc(sizeof(float) * (count ? count : 1));
  for (size_t i = 0; i < count; ++i)
    f[i] = q4o_half_to_float(x[i]);
  return f;
}

int q4o_linear_typed_f16(uint16_t* y, const uint16_t* x, const uint8_t* w, int type, const uint16_t* aux, int M, int N, int K, int post,
                         int threads) {
  if (bad_shape(M, N, K) || (M && !x))
    return -1;
  float* xf = widen(x, (size_t)M * K);
  int rc = linear_common(KIND_F16, type, y, 2, xf, w, NULL, aux, M, N, K, post, threads);
  free(xf);
  return rc;
}

int q4o_linear_f16(uint16_t* y, const uint16_t* x, const uint8_t* w, const uint16_t* aux, int M, int N, int K, int post, int threads) {
  return q4o_linear_typed_f16(y, x, w, Q4O_TYPE_Q4_K, aux, M, N, K, post, threads);
}

int q4o_mlp_gate_up_typed_f32(float* y, const float* x, const uint8_t* wg, const uint8_t* wu, int type, int M, int N, int K, int threads) {
  if (!wu)
    return -1;
  return linear_common(KIND_GATE_F32, type, y, 4, x, wg, wu, NULL, M, N, K, 0, threads);
}

int q4o_mlp_gate_up_f32(float* y, const float* x, const uint8_t* wg, const uint8_t* wu, int M, int N, int K, int threads) {
  return q4o_mlp_gate_up_typed_f32(y, x, wg, wu, Q4O_TYPE_Q4_K, M, N, K, threads);
}

int q4o_mlp_gate_up_typed_f16(uint16_t* y, const uint16_t* x, const uint8_t* wg, const uint8_t* wu, int type, int M, int N, int K, int threads) {
  if (bad_shape(M, N, K) || !wu || (M && !x))
    return -1;
  float* xf = widen(x, (size_t)M * K);
  int rc = linear_common(KIND_GATE_F16, type, y, 2, xf, wg, wu, NULL, M, N, K, 0, threads);
  free(xf);
  return rc;
}

int q4o_mlp_gate_up_f16(uint16_t* y, const uint16_t* x, const uint8_t* wg, const uint8_t* wu, int M, int N, int K, int threads) {
  return q4o_mlp_gate_up_typed_f16(y, x, wg, wu, Q4O_TYPE_Q4_K, M, N, K, threads);
}

int q4o_linear_typed_f64(double* y, const double* x, const uint8_t* w, int type, int M, int N, int K, int threads) {
  if (bad_shape(M, N, K) || !w || (M && (!x || !y)) || bad_type(type))
    return -1;
  if (M == 0)
    return 0;
  job_t p;
  memset(&p, 0, sizeof(p));
  p.kind = KIND_F64;
  p.type = type;
  p.M = M;
  p.N = N;
  p.K = K;
  p.y = y;
  p.xd = x;
  p.w = w;
  return run(p, threads);
}

int q4o_linear_f64(double* y, const double* x, const uint8_t* w, int M, int N, int K, int threads) {
  return q4o_linear_typed_f64(y, x, w, Q4O_TYPE_Q4_K, M, N, K, threads);
}

/* ------------------------------------------------- selection, packing -- */

/* forward.cpp:52 with decode accumulated as in forward.cpp:190 */
int q4o_phase(const uint32_t* counts, int nqueries, int gated) {
  int decode = 1;
  uint64_t rows = 0;
  for (int i = 0; i < nqueries; ++i) {
    decode &= counts[i] <= 5u;
    rows += counts[i];
  }
  return decode ? (gated ? 3 : 0) : (rows <= 8 ? 2 : 1);
}

/* forward.cpp:179,186,188-189 */
uint32_t q4o_pack(const uint32_t* counts, const uint32_t* samples, int nqueries, uint32_t* start, uint32_t* logit) {
  uint32_t rows = 0, logits = 0;
  for (int i = 0; i < nqueries; ++i) {
    start[i] = rows;
    logit[i] = logits;
    logits += samples ? samples[i] : 0u;
    rows += counts[i];
  }
  return rows;
}

/* batch.hpp:25-29 (queryLogit) + native_ops.metal:13-14 */
int64_t q4o_gather_row(const uint32_t* start, const uint32_t* count, const uint32_t* samples, const uint32_t* logit, int nqueries, uint32_t r) {
  for (int i = 0; i < nqueries; ++i)
    if (samples[i] && r < logit[i] + samples[i])
      return (int64_t)start[i] + count[i] - samples[i] + (r - logit[i]);
  return -1;
}

/* quant_linear.metal:577-584 (embedding_q4_k, mode 0, a target query) with
 * queryRow (batch.hpp:19-23): row t belongs to the first query q with
 * t < start[q] + count[q]; its token is the request buffer's entry
 * tokens[slot[q] * capacity + position[q] + (t - start[q])].  Returns the
 * token, or -1 when no query owns row t. */
int64_t q4o_embedding_token(const uint32_t* start, const uint32_t* count, const uint32_t* position, const uint32_t* slot, int nqueries,
                            uint32_t capacity, const int32_t* tokens, uint32_t t) {
  for (int q = 0; q < nqueries; ++q)
    if (t < start[q] + count[q])
      return tokens[(size_t)slot[q] * capacity + position[q] + (t - start[q])];
  return -1;
}

/* ------------------------------------------------- adjacent consumers -- */

/* quant_linear.metal:572-591: element r of the row's block (col >> 8) is
 * d*sc_j*v - dmin*m_j with j = r >> 5 and v the nibble of byte
 * (r >> 6) * 32 + (r & 31) (high nibble when r & 32). */
static int embedding_common(float* yf, uint16_t* yh, const uint8_t* w, int n, int k, const int32_t* ids, int rows) {
  if ((!yf && !yh) || !w || !ids || n <= 0 || k <= 0 || k % 256 != 0 || rows < 0)
    return -1;
  const int nb = k / 256;
  float row[256];
  for (int t = 0; t < rows; ++t) {
    const int32_t id = ids[t];
    for (int b = 0; b < nb; ++b) {
      if (id >= 0 && id < n)
        q4o_dequant_block(w + ((size_t)id * nb + b) * Q4O_BLOCK_BYTES, row);
      else
        memset(row, 0, sizeof row);
      for (int e = 0; e < 256; ++e) {
        const size_t o = (size_t)t * k + (size_t)b * 256 + e;
        if (yf)
          yf[o] = row[e];
        else
          yh[o] = q4o_float_to_half(row[e]);
      }
    }
  }
  return 0;
}

int q4o_embedding_f32(float* y, const uint8_t* w, int n, int k, const int32_t* ids, int rows) {
  return embedding_common(y, NULL, w, n, k, ids, rows);
}

int q4o_embedding_f16(uint16_t* y, const uint8_t* w, int n, int k, const int32_t* ids, int rows) {
  return embedding_common(NULL, y, w, n, k, ids, rows);
}

/* native_ops.metal:6-40 (rms_norm / rms_norm_gather). */
static int rms_norm_common(float* yf, uint16_t* yh, const float* xf, const uint16_t* xh, const float* w, const int64_t* src, int rows, int k,
                           float eps) {
  if ((!yf && !yh) || (!xf && !xh) || !w || rows < 0 || k <= 0)
    return -1;
  for (int r = 0; r < rows; ++r) {
    const int64_t s = src ? src[r] : r;
    if (s < 0)
      return -1;
    double ss = 0.0;
    for (int d = 0; d < k; ++d) {
      const double v = xf ? (double)xf[(size_t)s * k + d] : (double)q4o_half_to_float(xh[(size_t)s * k + d]);
      ss += v * v;
    }
    const double scale = 1.0 / sqrt(ss / (double)k + (double)eps);
    for (int d = 0; d < k; ++d) {
      const double v = xf ? (double)xf[(size_t)s * k + d] : (double)q4o_half_to_float(xh[(size_t)s * k + d]);
      const float out = (float)(v * scale * (double)w[d]);
      if (yf)
        yf[(size_t)r * k + d] = out;
      else
        yh[(size_t)r * k + d] = q4o_float_to_half(out);
    }
  }
  return 0;
}

int q4o_rms_norm_f32(float* y, const float* x, const float* w, const int64_t* src, int rows, int k, float eps) {
  return rms_norm_common(y, NULL, x, NULL, w, src, rows, k, eps);
}

int q4o_rms_norm_f16(uint16_t* y, const uint16_t* x, const float* w, const int64_t* src, int rows, int k, float eps) {
  return rms_norm_common(NULL, y, NULL, x, w, src, rows, k, eps);
}
