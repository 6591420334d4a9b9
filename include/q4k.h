/*
 * q4k.h -- C ABI of the MI355X (gfx950) Q4_K linear() path.
 *
 * Drop-in for MTLQwen's quantized linear layer: the Weight type with its
 * four-slot kernel cache, Ops::linear with its decode / prefill_small /
 * prefill / gated-decode selection, the post 0/1/2 epilogues and the fused
 * gate/up MLP, over a packed ragged batch of up to 8 sequences.
 *
 * Conventions
 *  - Every entry point returns Q4K_OK (0) or a negative Q4K_E* code; the
 *    message of the last failure on the calling thread is q4k_last_error().
 *    (Mirrors the reference's create<T> error capture, runtime/engine.cpp:236-243.)
 *  - stream is a hipStream_t passed as void* (NULL = the null stream).  Calls
 *    enqueue work and return without synchronising.
 *  - Activations are row-major: x [m, k], y and aux [m, n].  dtype selects
 *    fp32 (Q4K_DTYPE_F32) or fp16 (Q4K_DTYPE_F16) for x, y and aux together.
 *  - Calls on one device share that device's staging workspace: issue them
 *    from one submitter / one stream at a time, as the reference engine does
 *    (single worker thread, one command buffer per pass).
 *  - The workspace grows (hipMalloc) on the first call of a larger shape and
 *    is kept until the process ends.  A call made while its stream captures
 *    a HIP graph must not need growth: the launch that would need it fails
 *    with Q4K_ECAPTURE before allocating (q4k_mlp and the two-call form of
 *    q4k_mlp_gate_up may have enqueued their earlier launches by then).  One
 *    call of the same shapes before the capture avoids it.
 */
#ifndef Q4K_H
#define Q4K_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q4K_OK 0
#define Q4K_EINVAL (-1) /* null pointer, bad post code, bad dtype, bad count table */
#define Q4K_ETYPE (-2)  /* ggml type the path does not serve (not Q4_K / Q6_K / Q5_K / Q8_0 / IQ4_XS), or a type an entry point does not take (q4k_embedding: Q4_K only) */
#define Q4K_ESHAPE (-3) /* k % 256 != 0, n % 16 != 0, m out of range, byte count mismatch */
#define Q4K_EALIAS (-4) /* x overlaps y (aux may alias y) */
#define Q4K_EHIP (-5)   /* HIP runtime failure */
#define Q4K_ENOMEM (-6)
#define Q4K_EFORMAT (-7)   /* malformed or truncated GGUF file */
#define Q4K_ENOTFOUND (-8) /* missing file, tensor or metadata key */
#define Q4K_ECAPTURE (-9)  /* the call needs more workspace than the device holds, and its stream is capturing a graph */

#define Q4K_GGML_TYPE_Q4_K 12u
#define Q4K_GGML_TYPE_Q6_K 14u   /* the Q6_K LM head / mixed-type files (quant_linear.metal:69-86,437-497) */
#define Q4K_GGML_TYPE_Q8_0 8u    /* quant_linear.metal:89-100, 513-570 */
#define Q4K_GGML_TYPE_Q5_K 13u   /* quant_linear.metal:50-67, 329-435 */
#define Q4K_GGML_TYPE_IQ4_XS 23u /* quant_linear.metal:102-115; fused_kernels.metal:156-200 */

#define Q4K_DTYPE_F32 0u
#define Q4K_DTYPE_F16 1u

/* Epilogue ("post") codes: quant_linear.metal:146-147, forward.cpp:67-68. */
#define Q4K_POST_STORE 0u /* y = acc */
#define Q4K_POST_ADD 1u   /* y = acc + aux        (aux may be y: in-place residual) */
#define Q4K_POST_GATE 2u  /* y = silu(aux) * acc  (aux may be y: gate buffer overwritten) */

/* Kernel phases, the index of Weight::kernels[4] (model/qwen35/forward.cpp:52). */
#define Q4K_PHASE_DECODE 0u
#define Q4K_PHASE_PREFILL 1u
#define Q4K_PHASE_PREFILL_SMALL 2u
#define Q4K_PHASE_GATED_DECODE 3u

/* Rows per query above which a pass is not a decode pass
 * (model/qwen35/qwen35.hpp:22 maxDecodeRows). */
#define Q4K_MAX_DECODE_ROWS 5u
#define Q4K_MAX_QUERIES 8u   /* qwen35.hpp:22 maxBatchSequences */
#define Q4K_MAX_LOGIT_ROWS 64u /* qwen35.hpp:23 maxLogitRows */

typedef struct q4k_weight q4k_weight;

/* Message of the last failing call on this thread ("" if none). */
const char* q4k_last_error(void);

/* Upload one GGUF tensor of type Q4_K (n rows of k/256 block_q4_K records,
 * 144 B each), Q6_K (210 B per 256), Q5_K (176), IQ4_XS (136) or Q8_0 (eight
 * 34-byte records per 256); ggml ne[0] = k, ne[1] = n.
 * The bytes are re-laid out for the kernels during the upload; the caller's
 * buffer is not retained.  Replaces the zero-copy Weight view built by
 * loadWeights (model/qwen35/forward.cpp:12-23, qwen35.hpp:34-37), whose
 * Weight keys its kernels on the type (forward.cpp:55-57).  Every type
 * serves q4k_linear, q4k_linear_norm, q4k_mlp_gate_up and q4k_mlp in every
 * phase.  Decode passes of a gated pair run one fused gate/up kernel for
 * Q4_K pairs, and for Q5_K and IQ4_XS pairs with m <= 8 and k = 4096 (the
 * types the reference fuses, fused_kernels.metal:44-200); other gated
 * decode passes (Q6_K, Q8_0, pairs of two types) make the reference's two
 * calls.  q4k_embedding and q4k_embedding_batch take Q4_K tables only
 * (Q4K_ETYPE otherwise). */
int q4k_weight_create(const void* gguf_bytes, size_t bytes, uint32_t n, uint32_t k, uint32_t ggml_type, int device, q4k_weight** out);

/* Same, from bytes already in device memory of `device` (GGUF order). */
int q4k_weight_create_from_device(const void* gguf_device_bytes, size_t bytes, uint32_t n, uint32_t k, uint32_t ggml_type, int device,
                                  void* stream, q4k_weight** out);

int q4k_weight_destroy(q4k_weight* w);

/* n, k, device bytes held. */
int q4k_weight_info(const q4k_weight* w, uint32_t* n, uint32_t* k, uint64_t* device_bytes);

/* Name of the kernel cached in slot `phase` ("" if the slot was never
 * resolved).  Mirrors Weight::kernels[phase] (qwen35.hpp:29-37). */
int q4k_weight_kernel_name(const q4k_weight* w, uint32_t phase, char* buf, size_t buflen);

/* Resolve slot `phase` without launching anything: the engine's prepare
 * passes (runtime/engine.cpp:104-108) fill every slot ahead of the first pass. */
int q4k_weight_prepare(q4k_weight* w, uint32_t phase);

/* Ops::linear (model/qwen35/forward.cpp:51-70).
 * y[m, n] = post(x[m, k] . W^T, aux).  query_counts/nqueries describe the
 * packed ragged batch (rows per sequence, summing to m); they select the
 * phase exactly as the reference does: decode iff every query has <= 5 rows,
 * else prefill_small iff m <= 8, else prefill.  query_counts == NULL means
 * a single query of m rows.  `aux` is required for post 1 and 2 and may
 * equal y; x must not overlap y. */
int q4k_linear(void* stream, q4k_weight* w, const void* x, void* y, const void* aux, uint32_t m, const uint32_t* query_counts,
               uint32_t nqueries, uint32_t post, uint32_t dtype);

/* The projection of an RMS-normalised input: y = post(rms_norm(x, norm_w,
 * eps) . W^T, aux), rms_norm as native_ops.metal:6-40 (x * rsqrt(sum(x^2) /
 * k + eps) * norm_w, norm_w k fp32 values), the pair the decoder runs for the
 * attention input (forward.cpp:82 attn_norm, then the QKV projections
 * :86-87, :99).  The norm is folded into the activation staging of the
 * selected kernel (decode GEMV, prefill GEMM); paths that pack x inside the
 * GEMV (split-K, the wide persistent GEMV) normalise into the workspace
 * first.  Arguments otherwise as q4k_linear; aux must not be x. */
int q4k_linear_norm(void* stream, q4k_weight* w, const float* norm_w, float eps, const void* x, void* y, const void* aux, uint32_t m,
                    const uint32_t* query_counts, uint32_t nqueries, uint32_t post, uint32_t dtype);

/* q4k_linear for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference, whose kernels allocate nothing; here the
 * staging, split-K partials and counters of q4k_linear normally live in a
 * workspace that grows on demand.  Same arguments, selection, kernels and
 * results as q4k_linear, but the workspace is a fixed 120 MiB device array
 * that each GPU the library runs on holds until the process ends: 2 MiB of
 * decode pack (m <= 8, k <= 61440), 64 MiB of split-K partials (the decode
 * split-K GEMV and the prefill GEMM's two K-segments), 4096 split-K
 * counters, 65536 row scales, and about 54 MiB of staged activations (e.g.
 * m * k <= 28.1 million for prefill, rows padded to 128).  A call needing
 * more fails with Q4K_ESHAPE and a message naming the buffer.  Every weight
 * type is served, prefill included.  Calls allocate nothing (no hipMalloc,
 * hipFree or allocating library routine).  Every call on a GPU shares that
 * GPU's array and leaves
 * its contents behind: calls that overlap on one GPU (other streams or
 * threads) race; issue them in one stream order. */
int q4k_linear_noalloc(void* stream, q4k_weight* w, const void* x, void* y, const void* aux, uint32_t m, const uint32_t* query_counts,
                       uint32_t nqueries, uint32_t post, uint32_t dtype);

/* Gated MLP projection (model/qwen35/forward.cpp:115-118).
 * Decode passes: one fused gate/up kernel, y = silu(x.Wg^T) * (x.Wu^T)
 * (fused_kernels.metal:44-78).  Other passes: the result of the reference's
 * two calls, gate with post 0 into y, then up with post 2 over y in place;
 * Q4_K pairs at prefill row counts compute it in one gated GEMM launch (y
 * bit for bit as the two calls leave it), other cases make the two calls.
 * y is the gate buffer [m, n]. */
int q4k_mlp_gate_up(void* stream, q4k_weight* wg, q4k_weight* wu, const void* x, void* y, uint32_t m, const uint32_t* query_counts,
                    uint32_t nqueries, uint32_t dtype);

/* The MLP of Ops::decoder (model/qwen35/forward.cpp:114-119):
 *   xn = norm_w ? rms_norm(x, norm_w, eps) : x    (native_ops.metal:6-40)
 *   gate = silu(xn.Wg^T) * (xn.Wu^T)        [m, n]  (the gate buffer)
 *   hidden = hidden + gate.Wd^T              [m, k]  (post 1, in place)
 * with wg, wu n x k, wd k x n and norm_w k fp32 values (or NULL).  The
 * decoder passes x = hidden with the layer's ffn_norm; the norm runs inside
 * the fused gate/up GEMV (decode, m <= 8, k = 4096) or inside the activation
 * staging that the gate and up projections share (prefill GEMM, other
 * decode GEMVs); only paths that pack x inside the GEMV normalise into a
 * workspace buffer first.  The gate buffer must not overlap x or hidden; x
 * may equal hidden. */
int q4k_mlp(void* stream, q4k_weight* wg, q4k_weight* wu, q4k_weight* wd, const float* norm_w, float eps, const void* x, void* gate, void* hidden,
            uint32_t m, const uint32_t* query_counts, uint32_t nqueries, uint32_t dtype);

/* Phase Ops::linear would use for this batch (forward.cpp:52,190). */
int q4k_select_phase(const uint32_t* query_counts, uint32_t nqueries, uint32_t m, int gated, uint32_t* phase);

/* Ragged packing of forward.cpp:171-191: start[i] = rows before query i,
 * logit[i] = sampled rows before query i.  samples may be NULL (all zero).
 * Writes total rows and total sampled rows. */
int q4k_pack_queries(const uint32_t* counts, const uint32_t* samples, uint32_t nqueries, uint32_t* start, uint32_t* logit, uint32_t* rows,
                     uint32_t* logit_rows);

/* LM-head row gather (native_ops.metal:6-15 rms_norm_gather's row choice,
 * batch.hpp:25-29 queryLogit): out row r = x row
 * start + count - samples + (r - logit) of the query owning logit row r,
 * for r < sum(samples) (<= 64).  Copies k elements per row on `stream`. */
int q4k_gather_rows(void* stream, const void* x, void* out, uint32_t k, const uint32_t* counts, const uint32_t* samples, uint32_t nqueries,
                    uint32_t dtype, uint32_t* rows_out);

/* Token embedding (backend/metal/kernel/quant_linear.metal:572-591,
 * embedding_q4_k; dispatched at model/qwen35/forward.cpp:125,201-202):
 * row t of y [rows, k] is row ids[t] of the Q4_K table, dequantised as
 * d*sc*q - dmin*m in fp32 (then rounded to half for Q4K_DTYPE_F16).  ids is
 * a device array of rows int32 token ids; the reference derives them from its
 * query records and drafter proposals (quant_linear.metal:577-582), which
 * stay with the engine.  Ids outside [0, n) give a zero row.  y must not
 * overlap ids. */
int q4k_embedding(void* stream, const q4k_weight* table, const int32_t* ids, uint32_t rows, void* y, uint32_t dtype);

/* Token embedding of a packed batch, each row's token resolved in the kernel
 * as embedding_q4_k does for a target query (quant_linear.metal:577-584,
 * mode 0, with queryRow, batch.hpp:19-23; forward.cpp:125): query q owns
 * counts[q] consecutive rows, starting at the sum of the counts before it,
 * and row t of those takes token tokens[slots[q] * capacity + positions[q] +
 * (t - start_q)] of the engine's request token buffer (a device array of
 * int32, one row of `capacity` tokens per slot).  counts, positions and
 * slots are host arrays of nqueries (1..64) entries; positions[q] +
 * counts[q] must not exceed capacity.  Rows are dequantised as
 * q4k_embedding's; *rows_out (if not NULL) receives the row count, the sum
 * of counts.  The reference's drafter branches of the same kernel (DFlash
 * mask rows, MTP proposals: modes 1 and 2, and mode 0 with a drafter state)
 * stay with the engine.  y must not overlap tokens. */
int q4k_embedding_batch(void* stream, const q4k_weight* table, const int32_t* tokens, uint32_t capacity, const uint32_t* counts,
                        const uint32_t* positions, const uint32_t* slots, uint32_t nqueries, void* y, uint32_t dtype, uint32_t* rows_out);

/* RMS norm (native_ops.metal:6-40 rms_norm; forward.cpp:82,114):
 * y[r] = x[r] * rsqrt(sum(x[r]^2) / k + eps) * w for m rows of k; w is a
 * device array of k fp32 weights (the reference uses eps = 1e-6,
 * native_ops.metal:31).  y may equal x; otherwise they must not overlap. */
int q4k_rms_norm(void* stream, const void* x, const float* w, void* y, uint32_t m, uint32_t k, float eps, uint32_t dtype);

/* rms_norm_gather (native_ops.metal:6-40 with Gather, forward.cpp:72-75): the
 * LM-head rows that q4k_gather_rows selects, each RMS-normalised as above,
 * written to out [sum(samples), k]. */
int q4k_rms_norm_gather(void* stream, const void* x, const float* w, void* out, uint32_t k, const uint32_t* counts, const uint32_t* samples,
                        uint32_t nqueries, float eps, uint32_t dtype, uint32_t* rows_out);

/* ---- GGUF reader ---------------------------------------------------------
 * Replaces the reference's ggml gguf_init_from_buffer over the mapped model
 * file (model/qwen35/forward.cpp:12-23, loadWeights).  The file is mapped
 * read-only; versions 2 and 3 of the GGUF container are read, every offset
 * and length is checked against the file size, and malformed files return
 * Q4K_EFORMAT.  A handle is read-only after open and may be shared by
 * threads; close it after the last use of q4k_gguf_tensor_data pointers. */
typedef struct q4k_gguf q4k_gguf;

int q4k_gguf_open(const char* path, q4k_gguf** out);
int q4k_gguf_close(q4k_gguf* g);

/* Container version, tensor and metadata counts, start of the data section
 * (gguf_get_data_offset, forward.cpp:14) and file size. */
int q4k_gguf_info(const q4k_gguf* g, uint32_t* version, uint64_t* n_tensors, uint64_t* n_kv, uint64_t* data_offset, uint64_t* file_bytes);

/* Tensor i (gguf_get_tensor_name / _type / _ne / _offset / _size,
 * forward.cpp:18-21): name (NUL-terminated into name[name_len]), ggml type,
 * dimensions (ne[0] fastest; unused ones are 1), absolute file offset and
 * byte size (0 for ggml types whose block size the reader does not know). */
int q4k_gguf_tensor(const q4k_gguf* g, uint64_t i, char* name, size_t name_len, uint32_t* ggml_type, uint32_t* n_dims, uint64_t ne[4],
                    uint64_t* file_offset, uint64_t* bytes);

/* Index of the tensor called name; Q4K_ENOTFOUND ("missing weight", the
 * reference's lookup error, forward.cpp:37-41) if there is none. */
int q4k_gguf_find(const q4k_gguf* g, const char* name, uint64_t* index);

/* Host pointer to tensor i's bytes inside the mapping, valid until close. */
int q4k_gguf_tensor_data(const q4k_gguf* g, uint64_t i, const void** data, uint64_t* bytes);

/* Metadata value of key: any integer or bool type as int64; a string. */
int q4k_gguf_meta_int(const q4k_gguf* g, const char* key, int64_t* value);
int q4k_gguf_meta_str(const q4k_gguf* g, const char* key, char* buf, size_t len);

/* Upload the matrix called name to device as a weight with n = ne[1] rows
 * of k = ne[0] (the Weight loadWeights builds, forward.cpp:18-21), as
 * q4k_weight_create does; Q4K_ETYPE if its ggml type is not one of Q4_K,
 * Q6_K, Q5_K, Q8_0 and IQ4_XS, Q4K_ESHAPE if it is not a 2-D matrix. */
int q4k_weight_from_gguf(const q4k_gguf* g, const char* name, int device, q4k_weight** out);

/* Number of device allocations (hipMalloc) the library has made for its
 * workspaces (staging, split-K partials and counters, normalised inputs) in
 * this process, on every device.  No counterpart in the reference; it lets
 * a caller or a test show that a call allocated nothing (the count does not
 * change across it).  Weight uploads and the measurement entry points
 * (q4k_mfma_ceiling, q4k_read_ceiling) are not counted. */
int q4k_workspace_allocations(uint64_t* count);

/* Kernel families, for q4k_profile_query. */
#define Q4K_KERNEL_STAGE 0u      /* activation staging (fp16 + row scale) */
#define Q4K_KERNEL_GEMV 1u       /* MFMA GEMV, phases 0/2 and small prefill */
#define Q4K_KERNEL_GEMV_GATED 2u /* fused gate/up GEMV, phase 3 */
#define Q4K_KERNEL_GEMM 3u       /* LDS-tiled MFMA GEMM, phase 1 */
#define Q4K_KERNEL_AUX 4u        /* token embedding, RMS norm, rms_norm_gather */

/* Event timing of every kernel launch (no counterpart in the reference, whose
 * method is paired A/B timing, agents/KERNELS.md:13-21).  While enabled, each
 * kernel dispatch carries a pair of hipEvents that the runtime stamps with the
 * dispatch's own begin and end times (hipExtLaunchKernel), so durations
 * exclude host launch overhead.  Do not enable it during graph capture.
 * q4k_profile_enable(1) clears earlier records; q4k_profile_query
 * synchronises the recorded events and reports launches and summed, minimum
 * and maximum durations in milliseconds for one kernel family. */
int q4k_profile_enable(int on);
int q4k_profile_query(uint32_t kernel, uint32_t* launches, double* total_ms, double* min_ms, double* max_ms);

/* Measured fp16 MFMA ceiling of the device (no counterpart in the reference;
 * bench.py records it beside the published peak).  Runs a loop of the GEMM's
 * MFMA instruction, v_mfma_f32_16x16x32_f16, on every CU (one wave per SIMD,
 * operands in registers) for about `iters` x 32 instructions per wave, and
 * returns the achieved dense FLOP rate in TFLOP/s.  Synchronises the stream;
 * allocates and frees a small device buffer. */
int q4k_mfma_ceiling(void* stream, int device, uint32_t iters, double* tflops);

/* Measured streaming-read rate of the device (no counterpart in the
 * reference; bench.py records it beside the published HBM peak).  Reads the
 * `count` device buffers of `bytes` each (16-byte aligned, `bytes` a multiple
 * of 16) in turn, `reps` launches in all after one warm-up pass, with the
 * non-temporal 16-byte loads the GEMVs stream their weights with, and returns
 * the average rate in GB/s (launch gaps included).  Rotating buffers larger
 * than the memory-side cache together keep the reads on HBM.  Synchronises
 * the stream; allocates and frees a small device buffer. */
int q4k_read_ceiling(void* stream, int device, const void* const* buffers, uint32_t count, uint64_t bytes, uint32_t reps, double* gbs);

/* The device layout as a host transform (for tests and tooling):
 * GGUF-order block_q4_K bytes <-> the kernels' tiled order.  Both buffers are
 * n * (k / 256) * 144 bytes. */
int q4k_relayout_host(const void* gguf_bytes, void* tiled, uint32_t n, uint32_t k);
int q4k_unrelayout_host(const void* tiled, void* gguf_bytes, uint32_t n, uint32_t k);

/* Same for any served ggml type (n * (k / 256) * bytes per 256); the inverse
 * covers Q4_K and Q6_K (Q4K_ETYPE for the others). */
int q4k_relayout_host_typed(const void* gguf_bytes, void* tiled, uint32_t n, uint32_t k, uint32_t ggml_type);
int q4k_unrelayout_host_typed(const void* tiled, void* gguf_bytes, uint32_t n, uint32_t k, uint32_t ggml_type);

#ifdef __cplusplus
}
#endif
#endif
