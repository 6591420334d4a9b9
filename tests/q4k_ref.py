"""Shared test helpers: seeded Q4_K data, the oracle's ctypes binding, and an
independent numpy formulation of the Q4_K format used to pin the oracle.

The oracle (oracle/libq4k_oracle.so) is test infrastructure: tests use it as
the checker of the HIP path, never as the thing measured.
"""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "_build", "libq4k_oracle.so")
BLOCK_BYTES = 144
Q6_BLOCK_BYTES = 210
TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0, TYPE_Q5_K, TYPE_IQ4_XS = 12, 14, 8, 13, 23
# bytes per 256 weights
TYPE_BLOCK_BYTES = {TYPE_Q4_K: BLOCK_BYTES, TYPE_Q6_K: Q6_BLOCK_BYTES, TYPE_Q8_0: 272, TYPE_Q5_K: 176, TYPE_IQ4_XS: 136}
IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float64)

# --------------------------------------------------------------------------
# Synthetic data (the benchmark's config-0 recipe).
# --------------------------------------------------------------------------


def make_q4k(rng, n, k, dmax=0.01):
    """GGUF block_q4_K bytes [n, k/256*144]: d, dmin = fp16(U(0, dmax)),
    12 uniform scale bytes (uniform 6-bit scales/mins), uniform quant bytes."""
    nb = k // 256
    w = rng.integers(0, 256, size=(n, nb, BLOCK_BYTES), dtype=np.uint8)
    d = rng.uniform(0.0, dmax, size=(n, nb, 2)).astype(np.float16)
    w[:, :, 0:4] = d.view(np.uint8).reshape(n, nb, 4)
    return w.reshape(n, nb * BLOCK_BYTES)


def make_q6k(rng, n, k, dmax=0.01):
    """GGUF block_q6_K bytes [n, k/256*210]: uniform quant and qh bytes,
    uniform int8 scales (-128..127), d = fp16(U(0, dmax))."""
    nb = k // 256
    w = rng.integers(0, 256, size=(n, nb, Q6_BLOCK_BYTES), dtype=np.uint8)
    d = rng.uniform(0.0, dmax, size=(n, nb, 1)).astype(np.float16)
    w[:, :, 208:210] = d.view(np.uint8).reshape(n, nb, 2)
    return w.reshape(n, nb * Q6_BLOCK_BYTES)


def make_q8_0(rng, n, k, dmax=0.01):
    """GGUF block_q8_0 bytes [n, k/32*34]: d = fp16(U(0, dmax)) per 32, uniform int8."""
    nr = k // 32
    w = rng.integers(0, 256, size=(n, nr, 34), dtype=np.uint8)
    w[:, :, 0:2] = rng.uniform(0.0, dmax, size=(n, nr, 1)).astype(np.float16).view(np.uint8).reshape(n, nr, 2)
    return w.reshape(n, nr * 34)


def make_q5k(rng, n, k, dmax=0.01):
    """GGUF block_q5_K bytes [n, k/256*176]: d, dmin = fp16(U(0, dmax)), uniform rest."""
    nb = k // 256
    w = rng.integers(0, 256, size=(n, nb, 176), dtype=np.uint8)
    w[:, :, 0:4] = rng.uniform(0.0, dmax, size=(n, nb, 2)).astype(np.float16).view(np.uint8).reshape(n, nb, 4)
    return w.reshape(n, nb * 176)


def make_iq4xs(rng, n, k, dmax=0.01):
    """GGUF block_iq4_xs bytes [n, k/256*136]: d = fp16(U(0, dmax)), uniform rest."""
    nb = k // 256
    w = rng.integers(0, 256, size=(n, nb, 136), dtype=np.uint8)
    w[:, :, 0:2] = rng.uniform(0.0, dmax, size=(n, nb, 1)).astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    return w.reshape(n, nb * 136)


_MAKERS = {TYPE_Q4_K: make_q4k, TYPE_Q6_K: make_q6k, TYPE_Q8_0: make_q8_0, TYPE_Q5_K: make_q5k, TYPE_IQ4_XS: make_iq4xs}


def make_weight(rng, n, k, ggml_type, dmax=0.01):
    return _MAKERS[ggml_type](rng, n, k, dmax)


def make_x(rng, m, k, scale=1.0):
    return (rng.standard_normal((m, k)) * scale).astype(np.float32)


# --------------------------------------------------------------------------
# Independent numpy formulation.
#
# Element addressing follows embedding_q4_k (quant_linear.metal:585-590):
#   j = r >> 5, qj = (r >> 6) * 32 + (r & 31), v = (r & 32) ? q >> 4 : q & 15
# and the 6-bit fields use the kmask form of quant_linear.metal:278-284
# (four fields per 16-bit word), not the per-j branches the oracle restates.
# --------------------------------------------------------------------------


def scale_min_kmask(hdr12):
    """[..., 12] uint8 -> (sc[..., 8], m[..., 8]) via the 0x3f3f/0x0f0f/0xc0c0 masks."""
    q = hdr12.astype(np.uint32)
    w = q[..., 0::2] | (q[..., 1::2] << 8)  # six little-endian 16-bit words
    k1, k2, k3 = 0x3F3F, 0x0F0F, 0xC0C0
    sc, mn = np.zeros(hdr12.shape[:-1] + (8,), np.uint32), np.zeros(hdr12.shape[:-1] + (8,), np.uint32)
    # iq = 0 team: words 0, 2, 4 give (j0, j1) scales / mins and (j4, j5)
    # iq = 1 team: words 1, 3, 5 give (j2, j3) and (j6, j7)
    for iq in range(2):
        s0, s2, s4 = w[..., iq], w[..., iq + 2], w[..., iq + 4]
        a = s0 & k1
        b = s2 & k1
        c = (s4 & k2) | ((s0 & k3) >> 2)
        d = ((s4 >> 4) & k2) | ((s2 & k3) >> 2)
        j = 2 * iq
        sc[..., j], sc[..., j + 1] = a & 0xFF, a >> 8
        mn[..., j], mn[..., j + 1] = b & 0xFF, b >> 8
        sc[..., j + 4], sc[..., j + 5] = c & 0xFF, c >> 8
        mn[..., j + 4], mn[..., j + 5] = d & 0xFF, d >> 8
    return sc, mn


def dequant_numpy(w, n, k):
    """[n, k] float64 weights from GGUF Q4_K bytes."""
    nb = k // 256
    blk = w.reshape(n, nb, BLOCK_BYTES)
    d = blk[:, :, 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    dmin = blk[:, :, 2:4].copy().view(np.float16).astype(np.float64)[..., 0]
    sc, mn = scale_min_kmask(blk[:, :, 4:16])
    r = np.arange(256)
    j = r >> 5
    qj = (r >> 6) * 32 + (r & 31)
    qb = blk[:, :, 16 + qj].astype(np.uint32)
    v = np.where((r & 32) != 0, qb >> 4, qb & 15).astype(np.float64)
    out = d[..., None] * sc[..., j].astype(np.float64) * v - dmin[..., None] * mn[..., j].astype(np.float64)
    return out.reshape(n, k)


def dequant_q6k_numpy(w, n, k):
    """[n, k] float64 weights from GGUF Q6_K bytes, in the bit-mask form of
    the reference's Q6_K decode kernel (quant_linear.metal:473-478): for half
    h and l < 32, with q1 = ql[64h + l], q2 = ql[64h + 32 + l], qh = qh[32h + l],
    elements 128h + l + 32s are (q1 & 15) | (qh & 3) << 4, (q2 & 15) | (qh & 12) << 2,
    (q1 >> 4) | (qh & 48), (q2 >> 4) | (qh & 192) >> 2, minus 32, with scales
    sc[8h + l / 16 + 2s] (:451, :481) -- not the per-element addressing of
    the oracle (quant_linear.metal:69-86)."""
    nb = k // 256
    blk = w.reshape(n, nb, Q6_BLOCK_BYTES).astype(np.int64)
    d = w.reshape(n, nb, Q6_BLOCK_BYTES)[:, :, 208:210].copy().view(np.float16).astype(np.float64)[..., 0]
    sc = w.reshape(n, nb, Q6_BLOCK_BYTES)[:, :, 192:208].copy().view(np.int8).astype(np.float64)
    out = np.zeros((n, nb, 256), np.float64)
    l = np.arange(32)
    for h in range(2):
        q1 = blk[:, :, 64 * h + l]
        q2 = blk[:, :, 64 * h + 32 + l]
        qh = blk[:, :, 128 + 32 * h + l]
        vals = [(q1 & 15) | ((qh & 3) << 4), (q2 & 15) | ((qh & 12) << 2), (q1 >> 4) | (qh & 48), (q2 >> 4) | ((qh & 192) >> 2)]
        for s_, v in enumerate(vals):
            out[:, :, 128 * h + 32 * s_ + l] = d[..., None] * sc[:, :, 8 * h + l // 16 + 2 * s_] * (v - 32)
    return out.reshape(n, k)


def dequant_q8_0_numpy(w, n, k):
    """[n, k] float64 from Q8_0 bytes: per 34-byte record d * int8 (the decode
    kernel's qs = o + 2 + 8 il, d = the record's half, quant_linear.metal:529-533)."""
    rec = w.reshape(n, k // 32, 34)
    d = rec[:, :, 0:2].copy().view(np.float16).astype(np.float64)
    q = rec[:, :, 2:].copy().view(np.int8).astype(np.float64)
    return (d * q).reshape(n, k)


def dequant_q5k_numpy(w, n, k):
    """[n, k] float64 from Q5_K bytes, in the bit-mask form of the reference's
    Q5_K decode kernel (quant_linear.metal:356-406): for iq in {0, 1, 2, 3}
    (two per 128-element half) and l < 32, low nibbles of qs[32 iq + l] with qh
    bit 2 iq, high nibbles with bit 2 iq + 1 (hm1..hm4), scales and mins from
    the kmask words -- not the per-element addressing of the oracle."""
    nb = k // 256
    blk = w.reshape(n, nb, 176)
    d = blk[:, :, 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    dmin = blk[:, :, 2:4].copy().view(np.float16).astype(np.float64)[..., 0]
    sc, mn = scale_min_kmask(blk[:, :, 4:16])
    qh = blk[:, :, 16:48].astype(np.int64)
    qs = blk[:, :, 48:176].astype(np.int64)
    out = np.zeros((n, nb, 256), np.float64)
    l = np.arange(32)
    for iq in range(4):
        q = qs[:, :, 32 * iq + l]
        lo = (q & 0x0F) + np.where(qh & (1 << (2 * iq)), 16, 0)
        hi = (q & 0xF0) / 16 + np.where(qh & (1 << (2 * iq + 1)), 16, 0)
        for j, v in ((2 * iq, lo), (2 * iq + 1, hi)):
            out[:, :, 32 * j + l] = d[..., None] * sc[:, :, j:j + 1] * v - dmin[..., None] * mn[:, :, j:j + 1]
    return out.reshape(n, k)


def dequant_iq4xs_numpy(w, n, k):
    """[n, k] float64 from IQ4_XS bytes, in the form of the reference's fused
    IQ4_XS decode (fused_kernels.metal:159-174): for sub-block part and il in
    {0, 1}, the words of qs[16 part + 8 il ..] masked with 0x0f0f0f0f give
    elements 32 part + 8 il + [0, 8) and, shifted by 4, the same + 16."""
    nb = k // 256
    blk = w.reshape(n, nb, 136)
    d = blk[:, :, 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    sh = blk[:, :, 2].astype(np.int64) | (blk[:, :, 3].astype(np.int64) << 8)
    out = np.zeros((n, nb, 256), np.float64)
    for part in range(8):
        ls = ((blk[:, :, 4 + part // 2].astype(np.int64) >> (4 * (part % 2))) & 15) | (((sh >> (2 * part)) & 3) << 4)
        for il in range(2):
            words = blk[:, :, 8 + 16 * part + 8 * il:8 + 16 * part + 8 * il + 8].copy().view(np.uint32).astype(np.int64)
            for wi in range(2):
                lo = (words[:, :, wi] & 0x0F0F0F0F)
                hi = ((words[:, :, wi] >> 4) & 0x0F0F0F0F)
                for b in range(4):
                    e = 32 * part + 8 * il + 4 * wi + b
                    out[:, :, e] = d * (ls - 32) * IQ4NL[(lo >> (8 * b)) & 15]
                    out[:, :, e + 16] = d * (ls - 32) * IQ4NL[(hi >> (8 * b)) & 15]
    return out.reshape(n, k)


_DEQUANT = {TYPE_Q4_K: dequant_numpy, TYPE_Q6_K: dequant_q6k_numpy, TYPE_Q8_0: dequant_q8_0_numpy, TYPE_Q5_K: dequant_q5k_numpy,
            TYPE_IQ4_XS: dequant_iq4xs_numpy}


def dequant_any_numpy(w, n, k, ggml_type):
    return _DEQUANT[ggml_type](w, n, k)


def silu64(g):
    return g / (1.0 + np.exp(-g))


def _to_f16(v):
    return np.asarray(v, np.float64).astype(np.float32).astype(np.float16).astype(np.float64)


def prefill_arithmetic(x, w, n, k):
    """The reference's prefill arithmetic for Q4_K, in float64: activations
    rounded once to fp16 (the engine's activation type; an fp32 row is first
    scaled by a power of two, which is exact, so that its largest magnitude
    lies in [2^14, 2^15)), weights at the prefill tile value
    h(fp32(d*sc*q - dmin*m)) (quant_linear.metal:43,45), products summed
    exactly.  Returns the [m, n] contraction."""
    x = np.asarray(x)
    if x.dtype == np.float16:
        a = x.astype(np.float64)
    else:
        x64 = x.astype(np.float64)
        mx = np.abs(x64).max(axis=1)
        ex = np.frexp(np.where(mx > 0, mx, 1.0))[1]
        s = np.ldexp(1.0, 15 - ex)
        a = _to_f16(x64 * s[:, None]) / s[:, None]
    return a @ _to_f16(dequant_numpy(w, n, k)).T


def gated_prefill_arithmetic(x, wg, wu, n, k, f16_out=False):
    """SiLU(gate) * up over prefill_arithmetic's projections, with the fp16
    rounding points of the reference's post-2 epilogue for fp16 outputs
    (h(silu(h(g)) * h(u)), quant_linear.metal:146-147)."""
    g, u = prefill_arithmetic(x, wg, n, k), prefill_arithmetic(x, wu, n, k)
    if f16_out:
        return _to_f16(silu64(_to_f16(g)) * _to_f16(u))
    return silu64(g) * u


# --------------------------------------------------------------------------
# Oracle binding.
# --------------------------------------------------------------------------


def _build_oracle():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


def load_oracle():
    if not os.path.exists(ORACLE_SO):
        _build_oracle()
    lib = ctypes.CDLL(ORACLE_SO)
    p, i, u8p = ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p
    lib.q4o_half_to_float.restype = ctypes.c_float
    lib.q4o_half_to_float.argtypes = [ctypes.c_uint16]
    lib.q4o_float_to_half.restype = ctypes.c_uint16
    lib.q4o_float_to_half.argtypes = [ctypes.c_float]
    lib.q4o_scale_min.argtypes = [i, u8p, ctypes.POINTER(ctypes.c_uint8), ctypes.POINTER(ctypes.c_uint8)]
    lib.q4o_pack_scale_min.argtypes = [u8p, u8p, u8p]
    lib.q4o_dequant_block.argtypes = [u8p, p]
    lib.q4o_dequant_block_f16.argtypes = [u8p, p]
    for name in ("q4o_linear_f32", "q4o_linear_f16"):
        getattr(lib, name).restype = i
        getattr(lib, name).argtypes = [p, p, u8p, p, i, i, i, i, i]
    for name in ("q4o_linear_typed_f32", "q4o_linear_typed_f16"):
        getattr(lib, name).restype = i
        getattr(lib, name).argtypes = [p, p, u8p, i, p, i, i, i, i, i]
    for name in ("q4o_mlp_gate_up_f32", "q4o_mlp_gate_up_f16"):
        getattr(lib, name).restype = i
        getattr(lib, name).argtypes = [p, p, u8p, u8p, i, i, i, i]
    for name in ("q4o_mlp_gate_up_typed_f32", "q4o_mlp_gate_up_typed_f16"):
        getattr(lib, name).restype = i
        getattr(lib, name).argtypes = [p, p, u8p, u8p, i, i, i, i, i]
    lib.q4o_linear_f64.restype = i
    lib.q4o_linear_f64.argtypes = [p, p, u8p, i, i, i, i]
    lib.q4o_linear_typed_f64.restype = i
    lib.q4o_linear_typed_f64.argtypes = [p, p, u8p, i, i, i, i, i]
    lib.q6o_quant.restype = i
    lib.q6o_quant.argtypes = [u8p, i]
    lib.q6o_scale.restype = i
    lib.q6o_scale.argtypes = [u8p, i]
    lib.q6o_dequant_block.argtypes = [u8p, p]
    lib.q6o_dequant_block_f16.argtypes = [u8p, p]
    for name in ("q8o_dequant_block", "q5o_dequant_block", "iq4o_dequant_block"):
        getattr(lib, name).argtypes = [u8p, p]
    lib.q5o_quant.restype = i
    lib.q5o_quant.argtypes = [u8p, i]
    lib.iq4o_index.restype = i
    lib.iq4o_index.argtypes = [u8p, i]
    lib.iq4o_scale.restype = i
    lib.iq4o_scale.argtypes = [u8p, i]
    lib.iq4o_value.restype = ctypes.c_float
    lib.iq4o_value.argtypes = [i]
    lib.q4o_phase.restype = i
    lib.q4o_phase.argtypes = [ctypes.POINTER(ctypes.c_uint32), i, i]
    lib.q4o_pack.restype = ctypes.c_uint32
    lib.q4o_pack.argtypes = [ctypes.POINTER(ctypes.c_uint32)] * 2 + [i] + [ctypes.POINTER(ctypes.c_uint32)] * 2
    lib.q4o_gather_row.restype = ctypes.c_int64
    lib.q4o_gather_row.argtypes = [ctypes.POINTER(ctypes.c_uint32)] * 4 + [i, ctypes.c_uint32]
    lib.q4o_embedding_token.restype = ctypes.c_int64
    lib.q4o_embedding_token.argtypes = [ctypes.POINTER(ctypes.c_uint32)] * 4 + [i, ctypes.c_uint32, ctypes.POINTER(ctypes.c_int32),
                                                                                ctypes.c_uint32]
    for name in ("q4o_embedding_f32", "q4o_embedding_f16"):
        getattr(lib, name).restype = i
        getattr(lib, name).argtypes = [p, u8p, i, i, p, i]
    for name in ("q4o_rms_norm_f32", "q4o_rms_norm_f16"):
        getattr(lib, name).restype = i
        getattr(lib, name).argtypes = [p, p, p, p, i, i, ctypes.c_float]
    return lib


# Host threads for the oracle: the GPU box's CPU share is 16 cores per GPU.
DEFAULT_THREADS = max(1, min(16, os.cpu_count() or 1))


class Oracle:
    """numpy-level wrappers of the C oracle."""

    def __init__(self):
        self.lib = load_oracle()

    @staticmethod
    def _p(a):
        return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None

    def linear(self, x, w, n, k, aux=None, post=0, threads=DEFAULT_THREADS, ggml_type=TYPE_Q4_K):
        x = np.ascontiguousarray(x)
        m = x.shape[0]
        w = np.ascontiguousarray(w, np.uint8)
        if x.dtype == np.float16:
            y = np.empty((m, n), np.float16)
            auxa = None if aux is None else np.ascontiguousarray(aux, np.float16)
            rc = self.lib.q4o_linear_typed_f16(self._p(y), self._p(x.view(np.uint16)), self._p(w), ggml_type, self._p(auxa),
                                               m, n, k, post, threads)
        else:
            x = x.astype(np.float32, copy=False)
            y = np.empty((m, n), np.float32)
            auxa = None if aux is None else np.ascontiguousarray(aux, np.float32)
            rc = self.lib.q4o_linear_typed_f32(self._p(y), self._p(x), self._p(w), ggml_type, self._p(auxa), m, n, k, post,
                                               threads)
        assert rc == 0
        return y

    def mlp_gate_up(self, x, wg, wu, n, k, threads=DEFAULT_THREADS, ggml_type=TYPE_Q4_K):
        x = np.ascontiguousarray(x)
        m = x.shape[0]
        if x.dtype == np.float16:
            y = np.empty((m, n), np.float16)
            rc = self.lib.q4o_mlp_gate_up_typed_f16(self._p(y), self._p(x), self._p(wg), self._p(wu), ggml_type, m, n, k,
                                                    threads)
        else:
            y = np.empty((m, n), np.float32)
            rc = self.lib.q4o_mlp_gate_up_typed_f32(self._p(y), self._p(x.astype(np.float32, copy=False)), self._p(wg),
                                                    self._p(wu), ggml_type, m, n, k, threads)
        assert rc == 0
        return y

    def linear_f64(self, x, w, n, k, threads=DEFAULT_THREADS, ggml_type=TYPE_Q4_K):
        x = np.ascontiguousarray(x, np.float64)
        y = np.empty((x.shape[0], n), np.float64)
        assert self.lib.q4o_linear_typed_f64(self._p(y), self._p(x), self._p(np.ascontiguousarray(w, np.uint8)), ggml_type,
                                             x.shape[0], n, k, threads) == 0
        return y

    def dequant_block(self, blk, ggml_type=TYPE_Q4_K):
        out = np.empty(256, np.float32)
        fn = {TYPE_Q6_K: self.lib.q6o_dequant_block, TYPE_Q8_0: self.lib.q8o_dequant_block, TYPE_Q5_K: self.lib.q5o_dequant_block,
              TYPE_IQ4_XS: self.lib.iq4o_dequant_block}.get(ggml_type, self.lib.q4o_dequant_block)
        fn(self._p(np.ascontiguousarray(blk, np.uint8)), self._p(out))
        return out

    def dequant_block_f16(self, blk, ggml_type=TYPE_Q4_K):
        """The 256 fp16 bit patterns of one block at the reference's prefill
        tile value (Q4_K and Q6_K: q4o_ / q6o_dequant_block_f16)."""
        out = np.empty(256, np.uint16)
        fn = self.lib.q6o_dequant_block_f16 if ggml_type == TYPE_Q6_K else self.lib.q4o_dequant_block_f16
        fn(self._p(np.ascontiguousarray(blk, np.uint8)), self._p(out))
        return out

    def q6_fields(self, blk):
        """(quants 0..63, int8 scales) of the 256 elements of one block_q6_K."""
        b = np.ascontiguousarray(blk, np.uint8)
        return (np.array([self.lib.q6o_quant(self._p(b), e) for e in range(256)]),
                np.array([self.lib.q6o_scale(self._p(b), e) for e in range(256)]))

    def phase(self, counts, gated=False):
        arr = (ctypes.c_uint32 * len(counts))(*counts)
        return self.lib.q4o_phase(arr, len(counts), int(gated))

    def pack(self, counts, samples):
        n = len(counts)
        c = (ctypes.c_uint32 * n)(*counts)
        s = (ctypes.c_uint32 * n)(*samples)
        start, logit = (ctypes.c_uint32 * n)(), (ctypes.c_uint32 * n)()
        rows = self.lib.q4o_pack(c, s, n, start, logit)
        return list(start), list(logit), rows

    def embedding(self, w, n, k, ids, f16=False):
        ids = np.ascontiguousarray(ids, np.int32)
        if f16:
            y = np.empty((len(ids), k), np.float16)
            rc = self.lib.q4o_embedding_f16(self._p(y), self._p(w), n, k, self._p(ids), len(ids))
        else:
            y = np.empty((len(ids), k), np.float32)
            rc = self.lib.q4o_embedding_f32(self._p(y), self._p(w), n, k, self._p(ids), len(ids))
        assert rc == 0
        return y

    def rms_norm(self, x, w, src=None, eps=1e-6):
        """RMS norm of rows src (default: every row) of x [rows, k]."""
        x = np.ascontiguousarray(x)
        k = x.shape[-1]
        w = np.ascontiguousarray(w, np.float32)
        srca = None if src is None else np.ascontiguousarray(src, np.int64)
        rows = x.shape[0] if src is None else len(srca)
        if x.dtype == np.float16:
            y = np.empty((rows, k), np.float16)
            rc = self.lib.q4o_rms_norm_f16(self._p(y), self._p(x), self._p(w), self._p(srca), rows, k, eps)
        else:
            x = x.astype(np.float32, copy=False)
            y = np.empty((rows, k), np.float32)
            rc = self.lib.q4o_rms_norm_f32(self._p(y), self._p(x), self._p(w), self._p(srca), rows, k, eps)
        assert rc == 0
        return y

    def logit_sources(self, counts, samples):
        """Input row of every LM-head output row (q4o_gather_row over the pack)."""
        start, logit, _ = self.pack(counts, samples)
        return [self.gather_row(start, counts, samples, logit, r) for r in range(sum(samples))]

    def embedding_tokens(self, counts, positions, slots, capacity, tokens):
        """Token id of every row of a packed batch (q4o_embedding_token;
        starts are the prefix sums of counts)."""
        n = len(counts)
        start = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.uint32)
        arrs = [(ctypes.c_uint32 * n)(*[int(v) for v in a]) for a in (start, counts, positions, slots)]
        tok = np.ascontiguousarray(tokens, np.int32)
        tp = tok.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
        return [self.lib.q4o_embedding_token(*arrs, n, capacity, tp, t) for t in range(int(sum(counts)) + 1)]

    def gather_row(self, start, count, samples, logit, r):
        n = len(start)
        arrs = [(ctypes.c_uint32 * n)(*v) for v in (start, count, samples, logit)]
        return self.lib.q4o_gather_row(*arrs, n, r)


def row_rel_err(y, ref):
    """Max over rows of ||y - ref|| / ||ref|| (the tolerance metric of the parity bar)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    num = np.linalg.norm(y - ref, axis=-1)
    den = np.linalg.norm(ref, axis=-1)
    den = np.where(den == 0, 1.0, den)
    return float(np.max(num / den)) if num.size else 0.0
