"""MI355X-native (gfx950) Q4_K quantized linear() path of MTLQwen.

Hand-written HIP kernels behind a C ABI (include/q4k.h, libq4k.so): MFMA
GEMVs for decode-shaped batches (<= 48 packed rows), a pipelined MFMA GEMM
for prefill, the fused gate/up MLP, and the reference's phase selection over
a packed ragged batch; Q6_K (the LM head of real GGUF files), Q5_K, Q8_0 and
IQ4_XS weights on the same linear() surface; the path's neighbours in a pass (Q4_K token
embedding, RMS norm and the LM-head rms_norm_gather) and a GGUF reader that
uploads those tensors from model files.
"""
from ._lib import DTYPE_F16, DTYPE_F32, GGML_TYPE_IQ4_XS, GGML_TYPE_Q4_K, GGML_TYPE_Q5_K, GGML_TYPE_Q6_K, GGML_TYPE_Q8_0, PHASE_DECODE, PHASE_GATED_DECODE, PHASE_PREFILL, \
    PHASE_PREFILL_SMALL, POST_ADD, POST_GATE, POST_STORE, KERNEL_STAGE, KERNEL_GEMV, KERNEL_GEMV_GATED, KERNEL_GEMM, \
    KERNEL_AUX, ECAPTURE, ENOMEM, Q4KError, lib
from .gguf import GGUFFile, TensorInfo
from .linear import (PHASE_NAMES, Weight, embedding, embedding_batch, gather_rows, linear, linear_norm, mfma_ceiling, read_ceiling, mlp, mlp_gate_up, pack_queries,
                     profile_enable, profile_query, q4k_nbytes, relayout_host, rms_norm, rms_norm_gather, select_phase,
                     unrelayout_host)

__all__ = [
    "Weight", "linear", "linear_norm", "mlp_gate_up", "mlp", "select_phase", "pack_queries", "gather_rows", "relayout_host",
    "unrelayout_host", "q4k_nbytes", "Q4KError", "lib", "PHASE_NAMES", "DTYPE_F32", "DTYPE_F16", "GGML_TYPE_Q4_K",
    "GGML_TYPE_Q6_K", "GGML_TYPE_Q8_0", "GGML_TYPE_Q5_K", "GGML_TYPE_IQ4_XS",
    "POST_STORE", "POST_ADD", "POST_GATE", "PHASE_DECODE", "PHASE_PREFILL", "PHASE_PREFILL_SMALL",
    "PHASE_GATED_DECODE", "KERNEL_STAGE", "KERNEL_GEMV", "KERNEL_GEMV_GATED", "KERNEL_GEMM", "profile_enable",
    "profile_query", "mfma_ceiling", "read_ceiling", "embedding", "embedding_batch", "rms_norm", "rms_norm_gather", "KERNEL_AUX", "GGUFFile", "TensorInfo",
    "ECAPTURE", "ENOMEM"
]
