/*
 * q4k_oracle.h -- CPU restatement of MTLQwen's Q4_K linear() arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library (mtlqwen_amd/) never
 * links, loads or falls back to it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the MTLQwen source tree).  Activations default to the fp32 domain of the
 * benchmark configs; the *_f16 variants apply the reference's fp16 rounding
 * points for engine-style half activations.
 */
#ifndef Q4K_ORACLE_H
#define Q4K_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q4O_BLOCK_ELEMS 256
#define Q4O_BLOCK_BYTES 144

/* IEEE binary16 <-> binary32.  half->float is exact; float->half rounds to
 * nearest-even (the conversion Metal's half(float) performs). */
float q4o_half_to_float(uint16_t h);
uint16_t q4o_float_to_half(float f);

/* 6-bit scale / min of sub-block j (0..7) from the 12 packed bytes at block+4.
 * backend/metal/kernel/quant_linear.metal:12-20 (scale_min_k4). */
void q4o_scale_min(int j, const uint8_t* q12, uint8_t* sc, uint8_t* m);

/* Inverse of q4o_scale_min: pack 8 scales and 8 mins (each < 64) into 12 bytes. */
void q4o_pack_scale_min(const uint8_t sc[8], const uint8_t m[8], uint8_t q12[12]);

/* Dequantize one 144-byte block_q4_K into 256 fp32 values d*sc*q - dmin*m.
 * quant_linear.metal:32-48 (dequant_tile<q4_k_tag>, before its half() store). */
void q4o_dequant_block(const uint8_t* blk, float* out);

/* Same value rounded to fp16, as the reference's prefill tiles store it
 * (quant_linear.metal:43,45).  Returns fp16 bit patterns. */
void q4o_dequant_block_f16(const uint8_t* blk, uint16_t* out);

/* y[M,N] = x[M,K] . W[N,K]^T with W in GGUF block_q4_K rows (N rows of K/256
 * blocks).  fp32 accumulation in the decode kernel's algebraic form
 * (quant_linear.metal:259-303): per sub-block sum(x*q) and sum(x), then
 * d*sc and dmin*m applied.
 * post 0: y = acc;  post 1: y = acc + aux;  post 2: y = silu(aux) * acc
 * (quant_linear.metal:146-147 epilogue, forward.cpp:67-68 post codes).
 * aux may alias y.  threads <= 0 means all hardware threads.
 * Returns 0, or -1 on invalid arguments. */
int q4o_linear_f32(float* y, const float* x, const uint8_t* w, const float* aux, int M, int N, int K, int post, int threads);

/* fp16 activations, reference rounding points:
 * post 0: h(acc); post 1: h(h(acc) + aux) (quant_linear.metal:237-243);
 * post 2: h(silu(aux) * h(acc)) (quant_linear.metal:146-147). */
int q4o_linear_f16(uint16_t* y, const uint16_t* x, const uint8_t* w, const uint16_t* aux, int M, int N, int K, int post, int threads);

/* Fused gate/up: y = silu(x.Wg^T) * (x.Wu^T).
 * backend/metal/kernel/fused_kernels.metal:44-78.  f16 variant rounds g and u
 * to half before the SiLU and rounds the product (fused_kernels.metal:74-75). */
int q4o_mlp_gate_up_f32(float* y, const float* x, const uint8_t* wg, const uint8_t* wu, int M, int N, int K, int threads);
int q4o_mlp_gate_up_f16(uint16_t* y, const uint16_t* x, const uint8_t* wg, const uint8_t* wu, int M, int N, int K, int threads);

/* Same contraction, double-precision dequantize-then-dot (quant_linear.metal:32-48
 * values, no fp16 rounding).  A second formulation used to cross-check the
 * fp32 decode form. */
int q4o_linear_f64(double* y, const double* x, const uint8_t* w, int M, int N, int K, int threads);

/* ---- block_q6_K (ggml type 14): ql[128] @0, qh[64] @128, int8 scales[16]
 * @192, d fp16 @208; 210 bytes per 256 weights d * sc * (q - 32). */
#define Q4O_TYPE_Q4_K 12
#define Q4O_TYPE_Q6_K 14
#define Q6O_BLOCK_BYTES 210

/* Raw 6-bit quant (0..63) and int8 scale of element e (0..255) of a block.
 * backend/metal/kernel/quant_linear.metal:69-86 (dequant_tile<q6_k_tag>). */
int q6o_quant(const uint8_t* blk, int e);
int q6o_scale(const uint8_t* blk, int e);

/* Dequantize one block_q6_K: (d * sc) * (q - 32) in fp32 (quant_linear.metal:
 * 79-83 before its half() store); the f16 variant is that store. */
void q6o_dequant_block(const uint8_t* blk, float* out);
void q6o_dequant_block_f16(const uint8_t* blk, uint16_t* out);

/* ---- block_q8_0 (type 8, 34 B per 32: d fp16, int8 qs[32]), block_q5_K
 * (type 13, 176 B per 256: d, dmin, Q4_K scale/min bytes, qh[32], qs[128]) and
 * block_iq4_xs (type 23, 136 B per 256: d, scales_h, scales_l[4], qs[128]),
 * backend/metal/kernel/quant_linear.metal:50-115 (dequant_tile). */
#define Q4O_TYPE_Q8_0 8
#define Q4O_TYPE_Q5_K 13
#define Q4O_TYPE_IQ4_XS 23
#define Q8O_BLOCK_BYTES 272 /* eight 34-byte records per 256 elements */
#define Q5O_BLOCK_BYTES 176
#define IQ4O_BLOCK_BYTES 136

void q8o_dequant_block(const uint8_t* blk, float* out);       /* 256 elements = 8 records */
int q5o_quant(const uint8_t* blk, int e);                      /* 5-bit quant 0..31 */
void q5o_dequant_block(const uint8_t* blk, float* out);       /* d * sc * q - dmin * m */
int iq4o_index(const uint8_t* blk, int e);                     /* 4-bit codebook index */
int iq4o_scale(const uint8_t* blk, int j);                     /* ls_j - 32, sub-block j of 8 */
float iq4o_value(int v);                                       /* the iq4nl codebook (quant_linear.metal:5) */
void iq4o_dequant_block(const uint8_t* blk, float* out);      /* d * (ls - 32) * iq4nl[v] */

/* q4o_linear_* / q4o_mlp_gate_up_* over weights of ggml type `type` (Q4_K,
 * Q6_K, Q8_0, Q5_K or IQ4_XS), each accumulated in the decode form of its
 * reference kernel: Q6_K per 16-element sub-block sum(x * (q - 32)), then
 * d * sum(sc * .) (quant_linear.metal:437-497); Q8_0 per 32-element record
 * sum(q * x) * d (:525-533); Q5_K as Q4_K with 5-bit quants (:345-412);
 * IQ4_XS per 32-element sub-block d * (ls - 32) * sum(x * iq4nl[v])
 * (fused_kernels.metal:156-178).  The untyped entry points above are type
 * Q4_K.  Returns -1 for another type. */
int q4o_linear_typed_f32(float* y, const float* x, const uint8_t* w, int type, const float* aux, int M, int N, int K, int post, int threads);
int q4o_linear_typed_f16(uint16_t* y, const uint16_t* x, const uint8_t* w, int type, const uint16_t* aux, int M, int N, int K, int post,
                         int threads);
int q4o_mlp_gate_up_typed_f32(float* y, const float* x, const uint8_t* wg, const uint8_t* wu, int type, int M, int N, int K, int threads);
int q4o_mlp_gate_up_typed_f16(uint16_t* y, const uint16_t* x, const uint8_t* wg, const uint8_t* wu, int type, int M, int N, int K, int threads);
int q4o_linear_typed_f64(double* y, const double* x, const uint8_t* w, int type, int M, int N, int K, int threads);

/* Kernel phase of Ops::linear: 0 decode, 1 prefill, 2 prefill_small, 3 gated
 * decode.  decode holds iff every query contributes <= 5 rows
 * (model/qwen35/forward.cpp:52,190; qwen35.hpp:22). */
int q4o_phase(const uint32_t* counts, int nqueries, int gated);

/* Ragged packing (model/qwen35/forward.cpp:171-191): start = running row count,
 * logit = running sample count.  Returns total rows. */
uint32_t q4o_pack(const uint32_t* counts, const uint32_t* samples, int nqueries, uint32_t* start, uint32_t* logit);

/* Input row read by LM-head output row r (native_ops.metal:12-15 with
 * batch.hpp:25-29 queryLogit): start + count - samples + (r - logit) of the
 * query that owns logit row r.  Returns -1 if r is not owned by any query. */
int64_t q4o_gather_row(const uint32_t* start, const uint32_t* count, const uint32_t* samples, const uint32_t* logit, int nqueries, uint32_t r);

/* Token id of row t of a packed batch for the token embedding
 * (quant_linear.metal:577-584 mode 0, batch.hpp:19-23 queryRow): the first
 * query q with t < start[q] + count[q] owns it; its token is
 * tokens[slot[q] * capacity + position[q] + (t - start[q])].  -1 when no
 * query owns row t. */
int64_t q4o_embedding_token(const uint32_t* start, const uint32_t* count, const uint32_t* position, const uint32_t* slot, int nqueries,
                            uint32_t capacity, const int32_t* tokens, uint32_t t);

/* Token-embedding gather-dequant: row t of y (k values) is row ids[t] of the
 * Q4_K table w (n rows of k/256 blocks), each element d*sc*q - dmin*m in fp32
 * ((d*sc)*q first, then the min product subtracted).
 * backend/metal/kernel/quant_linear.metal:572-591 (embedding_q4_k, the row's
 * element addressing at :585-590); the f16 variant is its half() store.  The
 * reference resolves ids from its query records and drafter proposals
 * (:577-582); here they are given.  ids outside [0, n) give a zero row.
 * Returns 0, or -1 on invalid arguments. */
int q4o_embedding_f32(float* y, const uint8_t* w, int n, int k, const int32_t* ids, int rows);
int q4o_embedding_f16(uint16_t* y, const uint8_t* w, int n, int k, const int32_t* ids, int rows);

/* RMS norm over rows of k values (native_ops.metal:6-40):
 * y[r][d] = x[s][d] * rsqrt(sum_d x[s][d]^2 / k + eps) * w[d] with s = src[r]
 * (src == NULL: s = r, rms_norm; otherwise the LM-head rows of rms_norm_gather,
 * q4o_gather_row).  The sum of squares and the scale are taken in double; the
 * f16 variant reads and writes half (x widened exactly, y rounded once).
 * Returns 0, or -1 on invalid arguments. */
int q4o_rms_norm_f32(float* y, const float* x, const float* w, const int64_t* src, int rows, int k, float eps);
int q4o_rms_norm_f16(uint16_t* y, const uint16_t* x, const float* w, const int64_t* src, int rows, int k, float eps);

#ifdef __cplusplus
}
#endif
#endif
