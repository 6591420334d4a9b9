"""ctypes binding of libq4k.so, the C ABI declared in include/q4k.h.

The library is loaded after torch so that both share torch's HIP runtime
(same soname, libamdhip64.so.7).  There is no fallback: if the library has
not been built this module raises ImportError.
"""
import ctypes
import os

import torch  # noqa: F401  (must be loaded first: provides the HIP runtime)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libq4k.so")

OK = 0
EINVAL = -1
ETYPE = -2
ESHAPE = -3
EALIAS = -4
EHIP = -5
ENOMEM = -6
EFORMAT = -7
ENOTFOUND = -8
ECAPTURE = -9

GGML_TYPE_Q4_K = 12
GGML_TYPE_Q6_K = 14
GGML_TYPE_Q8_0 = 8
GGML_TYPE_Q5_K = 13
GGML_TYPE_IQ4_XS = 23
# bytes per 256 weights
BLOCK_BYTES_BY_TYPE = {GGML_TYPE_Q4_K: 144, GGML_TYPE_Q6_K: 210, GGML_TYPE_Q8_0: 272, GGML_TYPE_Q5_K: 176, GGML_TYPE_IQ4_XS: 136}
DTYPE_F32 = 0
DTYPE_F16 = 1
POST_STORE, POST_ADD, POST_GATE = 0, 1, 2
PHASE_DECODE, PHASE_PREFILL, PHASE_PREFILL_SMALL, PHASE_GATED_DECODE = 0, 1, 2, 3
KERNEL_STAGE, KERNEL_GEMV, KERNEL_GEMV_GATED, KERNEL_GEMM, KERNEL_AUX = 0, 1, 2, 3, 4


class Q4KError(RuntimeError):
    """A negative status from the C ABI, with q4k_last_error()'s message."""

    def __init__(self, code, message):
        super().__init__(f"q4k error {code}: {message}")
        self.code = code
        self.message = message


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                          "(the Q4_K path has no non-HIP fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    u32, p, c_int, size_t = ctypes.c_uint32, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    pu32 = ctypes.POINTER(ctypes.c_uint32)
    pu64 = ctypes.POINTER(ctypes.c_uint64)
    sigs = {
        "q4k_last_error": (ctypes.c_char_p, []),
        "q4k_weight_create": (c_int, [p, size_t, u32, u32, u32, c_int, ctypes.POINTER(p)]),
        "q4k_weight_create_from_device": (c_int, [p, size_t, u32, u32, u32, c_int, p, ctypes.POINTER(p)]),
        "q4k_weight_destroy": (c_int, [p]),
        "q4k_weight_info": (c_int, [p, pu32, pu32, ctypes.POINTER(ctypes.c_uint64)]),
        "q4k_weight_kernel_name": (c_int, [p, u32, ctypes.c_char_p, size_t]),
        "q4k_weight_prepare": (c_int, [p, u32]),
        "q4k_linear": (c_int, [p, p, p, p, p, u32, pu32, u32, u32, u32]),
        "q4k_linear_noalloc": (c_int, [p, p, p, p, p, u32, pu32, u32, u32, u32]),
        "q4k_workspace_allocations": (c_int, [ctypes.POINTER(ctypes.c_uint64)]),
        "q4k_linear_norm": (c_int, [p, p, p, ctypes.c_float, p, p, p, u32, pu32, u32, u32, u32]),
        "q4k_mlp_gate_up": (c_int, [p, p, p, p, p, u32, pu32, u32, u32]),
        "q4k_mlp": (c_int, [p, p, p, p, p, ctypes.c_float, p, p, p, u32, pu32, u32, u32]),
        "q4k_select_phase": (c_int, [pu32, u32, u32, c_int, pu32]),
        "q4k_pack_queries": (c_int, [pu32, pu32, u32, pu32, pu32, pu32, pu32]),
        "q4k_gather_rows": (c_int, [p, p, p, u32, pu32, pu32, u32, u32, pu32]),
        "q4k_embedding": (c_int, [p, p, p, u32, p, u32]),
        "q4k_embedding_batch": (c_int, [p, p, p, u32, pu32, pu32, pu32, u32, p, u32, pu32]),
        "q4k_rms_norm": (c_int, [p, p, p, p, u32, u32, ctypes.c_float, u32]),
        "q4k_rms_norm_gather": (c_int, [p, p, p, p, u32, pu32, pu32, u32, ctypes.c_float, u32, pu32]),
        "q4k_profile_enable": (c_int, [c_int]),
        "q4k_profile_query": (c_int, [u32, pu32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                      ctypes.POINTER(ctypes.c_double)]),
        "q4k_mfma_ceiling": (c_int, [p, c_int, u32, ctypes.POINTER(ctypes.c_double)]),
        "q4k_read_ceiling": (c_int, [p, c_int, ctypes.POINTER(p), u32, ctypes.c_uint64, u32, ctypes.POINTER(ctypes.c_double)]),
        "q4k_relayout_host": (c_int, [p, p, u32, u32]),
        "q4k_gguf_open": (c_int, [ctypes.c_char_p, ctypes.POINTER(p)]),
        "q4k_gguf_close": (c_int, [p]),
        "q4k_gguf_info": (c_int, [p, pu32, pu64, pu64, pu64, pu64]),
        "q4k_gguf_tensor": (c_int, [p, ctypes.c_uint64, ctypes.c_char_p, size_t, pu32, pu32, pu64, pu64, pu64]),
        "q4k_gguf_find": (c_int, [p, ctypes.c_char_p, pu64]),
        "q4k_gguf_tensor_data": (c_int, [p, ctypes.c_uint64, ctypes.POINTER(p), pu64]),
        "q4k_gguf_meta_int": (c_int, [p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
        "q4k_gguf_meta_str": (c_int, [p, ctypes.c_char_p, ctypes.c_char_p, size_t]),
        "q4k_weight_from_gguf": (c_int, [p, ctypes.c_char_p, c_int, ctypes.POINTER(p)]),
        "q4k_unrelayout_host": (c_int, [p, p, u32, u32]),
        "q4k_relayout_host_typed": (c_int, [p, p, u32, u32, u32]),
        "q4k_unrelayout_host_typed": (c_int, [p, p, u32, u32, u32]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(rc):
    if rc != OK:
        raise Q4KError(rc, lib.q4k_last_error().decode())
    return rc


def u32_array(values):
    """(ctypes uint32 array, length) or (None, 0) for None."""
    if values is None:
        return None, 0
    values = [int(v) for v in values]
    return (ctypes.c_uint32 * len(values))(*values), len(values)
