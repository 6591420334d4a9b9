"""Python face of the Q4_K linear() path, shaped like the reference's host API.

``Weight`` mirrors ``struct Weight`` (model/qwen35/qwen35.hpp:34-37): a Q4_K
tensor of n rows by k columns plus a four-slot kernel cache indexed by phase.
``linear`` mirrors ``Ops::linear`` (model/qwen35/forward.cpp:51-70) and
``mlp`` the MLP section of ``Ops::decoder`` (forward.cpp:114-119).  All work
is done by libq4k.so through its C ABI; tensors are torch tensors on the GPU
(torch supplies device memory and the current stream, nothing else).
"""
import ctypes

import numpy as np
import torch

from ._lib import (BLOCK_BYTES_BY_TYPE, DTYPE_F16, DTYPE_F32, GGML_TYPE_Q4_K, POST_ADD, POST_GATE, POST_STORE, Q4KError,
                   check, lib, u32_array)

BLOCK_BYTES = 144
PHASE_NAMES = ("decode", "prefill", "prefill_small", "gated_decode")


def q4k_nbytes(n, k, ggml_type=GGML_TYPE_Q4_K):
    """GGUF bytes of an n x k tensor of ggml type Q4_K (144 B per 256) or Q6_K (210 B)."""
    return n * (k // 256) * BLOCK_BYTES_BY_TYPE[ggml_type]


def _dtype_code(t):
    if t.dtype == torch.float32:
        return DTYPE_F32
    if t.dtype == torch.float16:
        return DTYPE_F16
    raise TypeError(f"activations must be float32 or float16, got {t.dtype}")


def _stream(stream, device=None):
    """The stream handle to launch on: ``stream`` if given, else the current
    stream of ``device`` (the weight's device; the current device if None)."""
    if stream is None:
        dev = None if device is None else torch.device("cuda", device)
        return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    if isinstance(stream, torch.cuda.Stream):
        return ctypes.c_void_p(stream.cuda_stream)
    return ctypes.c_void_p(stream)


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("tensors passed to the Q4_K path must be on the GPU")
    if not t.is_contiguous():
        raise ValueError("tensors passed to the Q4_K path must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def _check_tensor(t, numel, what, device=None):
    """The C ABI takes raw pointers: a tensor must hold at least ``numel``
    elements (and sit on ``device``) before its address is handed over, so a
    mis-sized buffer is a ValueError here rather than an out-of-bounds access
    on the GPU."""
    if t is None:
        return
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{what} must be a GPU tensor")
    if device is not None and t.device.index != device:
        raise ValueError(f"{what} is on cuda:{t.device.index}, the weights on cuda:{device}")
    if t.numel() < numel:
        raise ValueError(f"{what} holds {t.numel()} elements, needs {numel}")


class Weight:
    """A quantized weight (Q4_K, Q6_K, Q5_K, Q8_0 or IQ4_XS) uploaded once to HBM (re-laid out for the kernels).

    ``data`` holds GGUF block_q4_K (or block_q6_K, ``ggml_type=14``) bytes for
    n rows of k/256 blocks: a host numpy/bytes buffer, or a uint8 CUDA tensor
    (re-laid out on the device).
    """

    def __init__(self, data, n, k, ggml_type=GGML_TYPE_Q4_K, device=0):
        handle = ctypes.c_void_p()
        if isinstance(data, torch.Tensor) and data.is_cuda:
            if data.dtype != torch.uint8 or not data.is_contiguous():
                raise ValueError("device weight bytes must be a contiguous uint8 tensor")
            rc = lib.q4k_weight_create_from_device(ctypes.c_void_p(data.data_ptr()), data.numel(), n, k, ggml_type,
                                                   device, _stream(None, device), ctypes.byref(handle))
        else:
            buf = np.ascontiguousarray(np.frombuffer(memoryview(data).cast("B"), dtype=np.uint8)
                                       if not isinstance(data, np.ndarray) else data.view(np.uint8).reshape(-1))
            rc = lib.q4k_weight_create(buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes, n, k, ggml_type, device,
                                       ctypes.byref(handle))
        check(rc)
        self._h = handle
        self.n, self.k, self.type, self.device = n, k, ggml_type, device

    @property
    def handle(self):
        if self._h is None:
            raise ValueError("weight has been released")
        return self._h

    @classmethod
    def _from_handle(cls, handle, n, k, ggml_type, device):
        """Wrap a handle the C ABI created (GGUF uploads)."""
        obj = cls.__new__(cls)
        obj._h = handle
        obj.n, obj.k, obj.type, obj.device = n, k, ggml_type, device
        return obj

    def kernel_name(self, phase):
        buf = ctypes.create_string_buffer(256)
        check(lib.q4k_weight_kernel_name(self.handle, phase, buf, 256))
        return buf.value.decode()

    def prepare(self, phase):
        """Resolve a kernel slot ahead of use (the engine's prepare passes)."""
        check(lib.q4k_weight_prepare(self.handle, phase))

    @property
    def nbytes(self):
        return q4k_nbytes(self.n, self.k, self.type)

    def close(self):
        if getattr(self, "_h", None) is not None:
            lib.q4k_weight_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def select_phase(query_counts, m=None, gated=False):
    """Phase of Ops::linear for a packed batch (forward.cpp:52,190)."""
    arr, nq = u32_array(query_counts)
    if m is None:
        m = sum(query_counts)
    out = ctypes.c_uint32()
    check(lib.q4k_select_phase(arr, nq, m, int(bool(gated)), ctypes.byref(out)))
    return out.value


def pack_queries(counts, samples=None):
    """Ragged packing (forward.cpp:171-191): (start, logit, rows, logit_rows)."""
    c, nq = u32_array(counts)
    s, _ = u32_array(samples)
    start = (ctypes.c_uint32 * max(nq, 1))()
    logit = (ctypes.c_uint32 * max(nq, 1))()
    rows, lrows = ctypes.c_uint32(), ctypes.c_uint32()
    check(lib.q4k_pack_queries(c, s, nq, start, logit, ctypes.byref(rows), ctypes.byref(lrows)))
    return list(start[:nq]), list(logit[:nq]), rows.value, lrows.value


def linear(x, w, count, output, auxiliary=None, gated=False, query_counts=None, stream=None):
    """Ops::linear(x, w, count, output, auxiliary, gated) (forward.cpp:51-70).

    post = 2 when gated, 1 when an auxiliary tensor is given, else 0.  With
    gated=True and a Weight as auxiliary (the decode form of forward.cpp:118),
    runs the fused gate/up projection with ``w`` as gate and ``auxiliary`` as up.
    query_counts are the rows of each packed sequence (default: one sequence).
    """
    if gated and isinstance(auxiliary, Weight):
        return mlp_gate_up(x, w, auxiliary, count, output, query_counts=query_counts, stream=stream)
    dt = _dtype_code(x)
    if output.dtype != x.dtype or (auxiliary is not None and auxiliary.dtype != x.dtype):
        raise TypeError("x, output and auxiliary must share a dtype")
    _check_tensor(x, count * w.k, "x", w.device)
    _check_tensor(output, count * w.n, "output", w.device)
    _check_tensor(auxiliary, count * w.n, "auxiliary", w.device)
    post = POST_GATE if gated else (POST_ADD if auxiliary is not None else POST_STORE)
    counts, nq = u32_array(query_counts if query_counts is not None else [count])
    check(lib.q4k_linear(_stream(stream, w.device), w.handle, _ptr(x), _ptr(output), _ptr(auxiliary), count, counts, nq, post, dt))
    return output


def linear_norm(x, w, norm_weight, count, output, auxiliary=None, gated=False, query_counts=None, stream=None, eps=1e-6):
    """linear() of rms_norm(x, norm_weight, eps) (native_ops.metal:6-40): the
    decoder's attention input, attn_norm then the QKV projection
    (forward.cpp:82, 86-87), with the norm folded into the projection's
    activation staging (q4k_linear_norm)."""
    dt = _dtype_code(x)
    if output.dtype != x.dtype or (auxiliary is not None and auxiliary.dtype != x.dtype):
        raise TypeError("x, output and auxiliary must share a dtype")
    _check_norm_weight(norm_weight, w.k)
    _check_tensor(norm_weight, w.k, "norm_weight", w.device)
    _check_tensor(x, count * w.k, "x", w.device)
    _check_tensor(output, count * w.n, "output", w.device)
    _check_tensor(auxiliary, count * w.n, "auxiliary", w.device)
    post = POST_GATE if gated else (POST_ADD if auxiliary is not None else POST_STORE)
    counts, nq = u32_array(query_counts if query_counts is not None else [count])
    check(lib.q4k_linear_norm(_stream(stream, w.device), w.handle, _ptr(norm_weight), float(eps), _ptr(x), _ptr(output), _ptr(auxiliary),
                              count, counts, nq, post, dt))
    return output


def mlp_gate_up(x, gate, up, count, output, query_counts=None, stream=None):
    """silu(x . gate^T) * (x . up^T) into ``output`` (the gate buffer)."""
    dt = _dtype_code(x)
    if output.dtype != x.dtype:
        raise TypeError("x and output must share a dtype")
    _check_tensor(x, count * gate.k, "x", gate.device)
    _check_tensor(output, count * gate.n, "output", gate.device)
    counts, nq = u32_array(query_counts if query_counts is not None else [count])
    check(lib.q4k_mlp_gate_up(_stream(stream, gate.device), gate.handle, up.handle, _ptr(x), _ptr(output), count, counts, nq, dt))
    return output


def mlp(x, gate, up, down, hidden, gate_buffer, count, query_counts=None, stream=None, norm_weight=None, eps=1e-6):
    """MLP of Ops::decoder (forward.cpp:114-119): optionally the RMS norm of
    ``x`` with ``norm_weight`` (fp32 [k]), then gate/up into gate_buffer,
    then down with the residual added in place into ``hidden`` (q4k_mlp).
    ``x`` may be ``hidden`` (the decoder passes the residual stream and
    the layer's ffn_norm)."""
    dt = _dtype_code(x)
    if gate_buffer.dtype != x.dtype or hidden.dtype != x.dtype:
        raise TypeError("x, gate_buffer and hidden must share a dtype")
    _check_tensor(x, count * gate.k, "x", gate.device)
    _check_tensor(gate_buffer, count * gate.n, "gate_buffer", gate.device)
    _check_tensor(hidden, count * down.n, "hidden", gate.device)
    counts, nq = u32_array(query_counts if query_counts is not None else [count])
    if norm_weight is not None:
        _check_norm_weight(norm_weight, gate.k)
        _check_tensor(norm_weight, gate.k, "norm_weight", gate.device)
    check(lib.q4k_mlp(_stream(stream, gate.device), gate.handle, up.handle, down.handle, _ptr(norm_weight), float(eps), _ptr(x),
                      _ptr(gate_buffer), _ptr(hidden), count, counts, nq, dt))
    return hidden


def gather_rows(x, out, counts, samples, stream=None):
    """LM-head row gather (native_ops.metal:12-15): returns the gathered row count."""
    dt = _dtype_code(x)
    if out.dtype != x.dtype:
        raise TypeError("x and out must share a dtype")
    k = x.shape[-1]
    _check_tensor(x, sum(counts) * k, "x")
    _check_tensor(out, sum(samples) * k, "out", x.device.index)
    c, nq = u32_array(counts)
    s, _ = u32_array(samples)
    rows = ctypes.c_uint32()
    check(lib.q4k_gather_rows(_stream(stream, x.device.index), _ptr(x), _ptr(out), k, c, s, nq, dt, ctypes.byref(rows)))
    return rows.value


def embedding(table, ids, y, stream=None):
    """Token embedding (embedding_q4_k, quant_linear.metal:572-591): row t of
    ``y`` is row ids[t] of the Q4_K ``table`` dequantised.  ``ids`` is an
    int32 device tensor; ids outside [0, n) give zero rows."""
    if ids.dtype != torch.int32:
        raise TypeError("ids must be an int32 tensor")
    rows = ids.numel()
    if y.shape[0] < rows or y.numel() < rows * table.k:
        raise ValueError("y must hold len(ids) rows of table.k values")
    _check_tensor(ids, rows, "ids", table.device)
    _check_tensor(y, rows * table.k, "y", table.device)
    check(lib.q4k_embedding(_stream(stream, table.device), table.handle, _ptr(ids), rows, _ptr(y), _dtype_code(y)))
    return y


def embedding_batch(table, tokens, capacity, counts, positions, slots, y, stream=None):
    """Token embedding of a packed batch with each row's token resolved in
    the kernel (embedding_q4_k mode 0 with queryRow, quant_linear.metal:577-584,
    batch.hpp:19-23): query q owns counts[q] consecutive rows, which read
    tokens[slots[q] * capacity + positions[q] + i] of the request token buffer
    ``tokens`` (int32 device tensor, ``capacity`` tokens per slot).  Returns
    the row count."""
    if tokens.dtype != torch.int32:
        raise TypeError("tokens must be an int32 tensor")
    if not (len(counts) == len(positions) == len(slots)):
        raise ValueError("counts, positions and slots must have one entry per query")
    rows = int(sum(counts))
    _check_tensor(tokens, (max(slots) + 1) * capacity if len(slots) else 0, "tokens", table.device)
    _check_tensor(y, rows * table.k, "y", table.device)
    c, nq = u32_array(counts)
    p, _ = u32_array(positions)
    sl, _ = u32_array(slots)
    out = ctypes.c_uint32()
    check(lib.q4k_embedding_batch(_stream(stream, table.device), table.handle, _ptr(tokens), capacity, c, p, sl, nq, _ptr(y), _dtype_code(y),
                                  ctypes.byref(out)))
    return out.value


def rms_norm(x, weight, y, eps=1e-6, stream=None):
    """RMS norm of every row of ``x`` (native_ops.metal:6-40) with fp32
    ``weight`` [k]; ``y`` may be ``x``."""
    _check_norm_weight(weight, x.shape[-1])
    if y.dtype != x.dtype:
        raise TypeError("x and y must share a dtype")
    m = x.numel() // x.shape[-1]
    _check_tensor(weight, x.shape[-1], "weight", x.device.index)
    _check_tensor(y, x.numel(), "y", x.device.index)
    check(lib.q4k_rms_norm(_stream(stream, x.device.index), _ptr(x), _ptr(weight), _ptr(y), m, x.shape[-1], float(eps), _dtype_code(x)))
    return y


def rms_norm_gather(x, weight, out, counts, samples, eps=1e-6, stream=None):
    """LM-head rms_norm_gather (native_ops.metal:6-40, forward.cpp:72-75):
    the rows gather_rows selects, RMS-normalised; returns their count."""
    _check_norm_weight(weight, x.shape[-1])
    if out.dtype != x.dtype:
        raise TypeError("x and out must share a dtype")
    k = x.shape[-1]
    _check_tensor(x, sum(counts) * k, "x")
    _check_tensor(weight, k, "weight", x.device.index)
    _check_tensor(out, sum(samples) * k, "out", x.device.index)
    c, nq = u32_array(counts)
    s, _ = u32_array(samples)
    rows = ctypes.c_uint32()
    check(lib.q4k_rms_norm_gather(_stream(stream, x.device.index), _ptr(x), _ptr(weight), _ptr(out), k, c, s, nq, float(eps),
                                  _dtype_code(x), ctypes.byref(rows)))
    return rows.value


def _check_norm_weight(weight, k):
    if weight.dtype != torch.float32 or weight.numel() != k:
        raise ValueError(f"norm weight must be {k} float32 values")


def profile_enable(on=True):
    """Bracket every kernel launch with hipEvents (clears earlier records)."""
    check(lib.q4k_profile_enable(int(bool(on))))


def profile_query(kernel):
    """(launches, total_ms, min_ms, max_ms) of one kernel family (KERNEL_*)."""
    n = ctypes.c_uint32()
    tot, lo, hi = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    check(lib.q4k_profile_query(kernel, ctypes.byref(n), ctypes.byref(tot), ctypes.byref(lo), ctypes.byref(hi)))
    return n.value, tot.value, lo.value, hi.value


def mfma_ceiling(device=0, iters=20000, stream=None):
    """Measured fp16 MFMA rate of the device in TFLOP/s (a loop of the GEMM's
    MFMA instruction on every CU); synchronises the stream."""
    t = ctypes.c_double()
    check(lib.q4k_mfma_ceiling(_stream(stream, int(device)), int(device), int(iters), ctypes.byref(t)))
    return t.value


def read_ceiling(buffers, reps=50, stream=None):
    """Measured streaming-read rate in GB/s over equal-sized device byte
    buffers read in turn (non-temporal 16-byte loads); synchronises the
    stream."""
    bufs = list(buffers)
    if not bufs:
        raise ValueError("read_ceiling needs at least one buffer")
    nbytes = bufs[0].numel() * bufs[0].element_size()
    dev = bufs[0].device.index
    for b in bufs:
        _ptr(b)  # a contiguous GPU tensor
        if b.numel() * b.element_size() != nbytes:
            raise ValueError("read_ceiling buffers must have equal sizes")
        if b.device.index != dev:
            raise ValueError("read_ceiling buffers must be on one GPU")
    if nbytes % 16 != 0:
        raise ValueError("read_ceiling buffer sizes must be a multiple of 16 bytes")
    arr = (ctypes.c_void_p * len(bufs))(*[b.data_ptr() for b in bufs])
    g = ctypes.c_double()
    check(lib.q4k_read_ceiling(_stream(stream, dev), dev, arr, len(bufs), nbytes, int(reps), ctypes.byref(g)))
    return g.value


def relayout_host(gguf, n, k, ggml_type=GGML_TYPE_Q4_K):
    """GGUF-order bytes of type Q4_K or Q6_K -> the kernels' tiled order."""
    src = np.ascontiguousarray(gguf, dtype=np.uint8).reshape(-1)
    dst = np.empty_like(src)
    check(lib.q4k_relayout_host_typed(src.ctypes.data_as(ctypes.c_void_p), dst.ctypes.data_as(ctypes.c_void_p), n, k,
                                      ggml_type))
    return dst


def unrelayout_host(tiled, n, k, ggml_type=GGML_TYPE_Q4_K):
    src = np.ascontiguousarray(tiled, dtype=np.uint8).reshape(-1)
    dst = np.empty_like(src)
    check(lib.q4k_unrelayout_host_typed(src.ctypes.data_as(ctypes.c_void_p), dst.ctypes.data_as(ctypes.c_void_p), n, k,
                                        ggml_type))
    return dst


__all__ = ["Weight", "linear", "linear_norm", "mlp_gate_up", "mlp", "select_phase", "pack_queries", "gather_rows", "embedding", "rms_norm",
           "rms_norm_gather", "relayout_host",
           "profile_enable", "profile_query", "mfma_ceiling", "read_ceiling",
           "unrelayout_host", "q4k_nbytes", "Q4KError", "PHASE_NAMES"]
