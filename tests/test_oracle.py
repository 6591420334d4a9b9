"""Pins the CPU oracle before it is trusted as the checker of the HIP path.

The reference ships no golden vectors for the Q4_K linear (its tests are
end-to-end token checks that need a 9B GGUF and a Metal GPU), so each oracle
function is pinned by checks a plausible mistake cannot pass:
  - fp16 conversions against numpy's independent implementation (exhaustive);
  - the 6-bit scale/min unpack against the kmask form of quant_linear.metal:278-284
    and an exhaustive pack/unpack round trip;
  - the element -> nibble map by one-hot activations against the
    embedding_q4_k addressing of quant_linear.metal:585-590 (tests/q4k_ref.py);
  - closed forms (constant quants, zero quants, zero blocks);
  - the fp32 decode-form contraction against a float64 dequantize-then-dot and
    against brute-force Python loops;
  - epilogues and the fused MLP against numpy compositions (numpy's own fp16);
  - phase selection and ragged packing against tables from forward.cpp.
"""
import itertools

import numpy as np
import pytest

from q4k_ref import dequant_numpy, make_q4k, make_x, row_rel_err, scale_min_kmask, silu64


def test_half_to_float_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.lib.q4o_half_to_float(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_float_to_half_matches_numpy(oracle):
    rng = np.random.default_rng(1)
    vals = [0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, 1e9, -1e9, 2.0**-24, 2.0**-25, 2.0**-25 * 1.0000001,
            3 * 2.0**-26, 2.0**-14, 2.0**-14 * (1 - 2.0**-11), 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, np.inf, -np.inf]
    # Random bit patterns over the whole float range plus values near fp16 ties.
    raw = rng.integers(0, 2**32, size=20000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    ties = (rng.integers(0, 2**11, size=5000) + 0.5) * 2.0**rng.integers(-24, 5, size=5000)
    allv = np.concatenate([np.array(vals, np.float32), raw[np.isfinite(raw)], ties.astype(np.float32)])
    with np.errstate(over="ignore"):
        ref = allv.astype(np.float16).view(np.uint16)
    got = np.array([oracle.lib.q4o_float_to_half(float(v)) for v in allv], np.uint16)
    assert np.array_equal(got, ref)


def test_scale_min_roundtrip_exhaustive(oracle):
    """Every (scale, min) pair at every sub-block position survives pack -> unpack."""
    import ctypes
    rng = np.random.default_rng(2)
    sc_out, m_out = ctypes.c_uint8(), ctypes.c_uint8()
    for j in range(8):
        for s in range(64):
            ms = np.arange(64, dtype=np.uint8)
            for mv in ms[:: 7 if s % 5 else 1]:
                sc = rng.integers(0, 64, 8, dtype=np.uint8)
                mn = rng.integers(0, 64, 8, dtype=np.uint8)
                sc[j], mn[j] = s, mv
                q = np.zeros(12, np.uint8)
                oracle.lib.q4o_pack_scale_min(sc.ctypes.data, mn.ctypes.data, q.ctypes.data)
                for jj in range(8):
                    oracle.lib.q4o_scale_min(jj, q.ctypes.data, ctypes.byref(sc_out), ctypes.byref(m_out))
                    assert (sc_out.value, m_out.value) == (sc[jj], mn[jj])


def test_scale_min_matches_kmask_form(oracle):
    import ctypes
    rng = np.random.default_rng(3)
    hdr = rng.integers(0, 256, size=(2000, 12), dtype=np.uint8)
    sc_ref, m_ref = scale_min_kmask(hdr)
    sc_out, m_out = ctypes.c_uint8(), ctypes.c_uint8()
    for r in range(hdr.shape[0]):
        row = np.ascontiguousarray(hdr[r])
        for j in range(8):
            oracle.lib.q4o_scale_min(j, row.ctypes.data, ctypes.byref(sc_out), ctypes.byref(m_out))
            assert sc_out.value == sc_ref[r, j] and m_out.value == m_ref[r, j]
    # Uniform random bytes give (near) uniform 6-bit fields over [0, 63].
    assert sc_ref.min() == 0 and sc_ref.max() == 63 and m_ref.max() == 63


def test_dequant_matches_embedding_addressing(oracle):
    rng = np.random.default_rng(4)
    w = make_q4k(rng, 16, 1024)
    ref = dequant_numpy(w, 16, 1024)
    blocks = w.reshape(-1, 144)
    got = np.stack([oracle.dequant_block(b) for b in blocks]).reshape(16, 1024)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-7)


def test_dequant_block_f16_tile_value(oracle):
    """q4o_dequant_block_f16 stores the reference's prefill tile value
    half(fp32(d * sc * q - dmin * m)) (quant_linear.metal:43,45): the kmask
    form in float64 (its two products are exact) rounded to fp32, then to
    fp16, bit for bit, over random blocks and blocks whose d and dmin push
    values into fp16 denormals and past the fp16 range."""
    rng = np.random.default_rng(41)
    for dmax in (0.01, 1e-7, 100.0):
        w = make_q4k(rng, 64, 256, dmax=dmax)
        ref = dequant_numpy(w, 64, 256)
        with np.errstate(over="ignore"):
            want = ref.astype(np.float32).astype(np.float16).view(np.uint16)
        got = np.stack([oracle.dequant_block_f16(b) for b in w.reshape(64, 144)])
        np.testing.assert_array_equal(got, want)


def test_one_hot_element_map(oracle):
    """x = e_k gives y[n] = W[n, k]: pins every (element -> byte, nibble, sub-block) position."""
    rng = np.random.default_rng(5)
    n, k = 8, 512
    w = make_q4k(rng, n, k)
    ref = dequant_numpy(w, n, k)
    x = np.eye(k, dtype=np.float32)
    y = oracle.linear(x, w, n, k)
    np.testing.assert_allclose(y, ref.T, rtol=2e-6, atol=1e-7)


def _block(d=1.0, dmin=0.0, sc=None, mn=None, q=None, oracle=None):
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([d], np.float16).view(np.uint8)
    blk[2:4] = np.array([dmin], np.float16).view(np.uint8)
    sc = np.zeros(8, np.uint8) if sc is None else np.asarray(sc, np.uint8)
    mn = np.zeros(8, np.uint8) if mn is None else np.asarray(mn, np.uint8)
    hdr = np.zeros(12, np.uint8)
    oracle.lib.q4o_pack_scale_min(sc.ctypes.data, mn.ctypes.data, hdr.ctypes.data)
    blk[4:16] = hdr
    if q is not None:
        blk[16:] = q
    return blk


def test_closed_forms(oracle):
    rng = np.random.default_rng(6)
    x = make_x(rng, 3, 256)
    sx = x.astype(np.float64).sum(axis=1)
    for c in (0, 1, 7, 15):
        for s in (1, 13, 63):
            blk = _block(d=1.0, sc=[s] * 8, q=np.full(128, c | (c << 4), np.uint8), oracle=oracle)
            y = oracle.linear(x, blk.reshape(1, 144), 1, 256)[:, 0]
            np.testing.assert_allclose(y, s * c * sx, rtol=1e-5, atol=1e-4)
    # Zero quants: only the min term remains.
    for m in (1, 40, 63):
        blk = _block(d=0.5, dmin=0.25, sc=[9] * 8, mn=[m] * 8, q=np.zeros(128, np.uint8), oracle=oracle)
        y = oracle.linear(x, blk.reshape(1, 144), 1, 256)[:, 0]
        np.testing.assert_allclose(y, -0.25 * m * sx, rtol=1e-5, atol=1e-4)
    zero = np.zeros((1, 144), np.uint8)
    assert np.all(oracle.linear(x, zero, 1, 256) == 0)


def test_decode_form_matches_float64_dot(oracle):
    rng = np.random.default_rng(7)
    n, k, m = 64, 2048, 5
    w = make_q4k(rng, n, k)
    x = make_x(rng, m, k)
    ref = x.astype(np.float64) @ dequant_numpy(w, n, k).T
    y32 = oracle.linear(x, w, n, k)
    y64 = oracle.linear_f64(x, w, n, k)
    np.testing.assert_allclose(y64, ref, rtol=1e-12, atol=1e-10)
    assert row_rel_err(y32, ref) < 1e-6


def test_brute_force_tiny(oracle):
    rng = np.random.default_rng(8)
    n, k, m = 3, 256, 2
    w = make_q4k(rng, n, k)
    x = make_x(rng, m, k)
    wb = w.reshape(n, 144)
    y = oracle.linear(x, w, n, k)
    for r, c in itertools.product(range(m), range(n)):
        b = wb[c]
        d = float(np.frombuffer(bytes(b[0:2]), np.float16)[0])
        dm = float(np.frombuffer(bytes(b[2:4]), np.float16)[0])
        acc = 0.0
        for e in range(256):
            j = e // 32
            if j < 4:
                sc, mn = b[4 + j] & 63, b[8 + j] & 63
            else:
                sc = (b[8 + j] & 15) | ((b[j] >> 6) << 4)
                mn = (b[8 + j] >> 4) | ((b[4 + j] >> 6) << 4)
            byte = b[16 + 32 * (e // 64) + (e % 32)]
            q = (byte >> 4) if (e % 64) >= 32 else (byte & 15)
            acc += float(x[r, e]) * (d * sc * q - dm * mn)
        assert abs(y[r, c] - acc) <= 1e-5 * max(1.0, abs(acc))


def test_epilogues_f32(oracle):
    rng = np.random.default_rng(9)
    n, k, m = 48, 512, 4
    w = make_q4k(rng, n, k)
    x = make_x(rng, m, k)
    aux = make_x(rng, m, n, 3.0)
    acc = oracle.linear(x, w, n, k).astype(np.float64)
    np.testing.assert_allclose(oracle.linear(x, w, n, k, aux=aux, post=1), acc + aux, rtol=1e-6, atol=1e-5)
    np.testing.assert_allclose(oracle.linear(x, w, n, k, aux=aux, post=2), silu64(aux.astype(np.float64)) * acc,
                               rtol=1e-5, atol=1e-5)


def test_epilogues_f16_rounding_points(oracle):
    rng = np.random.default_rng(10)
    n, k, m = 32, 512, 3
    w = make_q4k(rng, n, k)
    x = make_x(rng, m, k, 0.2).astype(np.float16)
    aux = make_x(rng, m, n, 2.0).astype(np.float16)
    acc = oracle.linear(x.astype(np.float32), w, n, k)
    h = acc.astype(np.float16)
    assert np.array_equal(oracle.linear(x, w, n, k), h)
    # post 1: h(h(acc) + r) -- numpy adds float16 operands with one rounding.
    assert np.array_equal(oracle.linear(x, w, n, k, aux=aux, post=1), (h + aux).astype(np.float16))
    g = aux.astype(np.float32)
    want = ((g / (1 + np.exp(-g))) * h.astype(np.float32)).astype(np.float16)
    got = oracle.linear(x, w, n, k, aux=aux, post=2)
    assert np.max(np.abs(got.astype(np.float32) - want.astype(np.float32)) /
                  np.maximum(np.abs(want.astype(np.float32)), 1e-3)) <= 2.0**-10


def test_mlp_gate_up(oracle):
    rng = np.random.default_rng(11)
    n, k, m = 64, 512, 3
    wg, wu = make_q4k(rng, n, k), make_q4k(rng, n, k)
    x = make_x(rng, m, k, 0.5)
    g = x.astype(np.float64) @ dequant_numpy(wg, n, k).T
    u = x.astype(np.float64) @ dequant_numpy(wu, n, k).T
    assert row_rel_err(oracle.mlp_gate_up(x, wg, wu, n, k), silu64(g) * u) < 1e-5
    # f16 form: h(silu(h(g)) * h(u))
    xh = x.astype(np.float16)
    g16 = oracle.linear(xh, wg, n, k).astype(np.float32)
    u16 = oracle.linear(xh, wu, n, k).astype(np.float32)
    want = (g16 / (1 + np.exp(-g16)) * u16).astype(np.float16).astype(np.float32)
    got = oracle.mlp_gate_up(xh, wg, wu, n, k).astype(np.float32)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-2)) <= 2.0**-10


# Phase table: (per-query row counts, gated) -> phase, from forward.cpp:52,190
# (decode iff every query has <= maxDecodeRows = 5 rows; small iff rows <= 8).
PHASE_CASES = [
    ([1], False, 0), ([1] * 8, False, 0), ([5] * 8, False, 0), ([1] * 8, True, 3), ([5] * 8, True, 3),
    ([6], False, 2), ([8], False, 2), ([6], True, 2), ([2, 6], False, 2), ([9], False, 1), ([6, 5], False, 1),
    ([512, 37, 1, 1, 200, 5, 1, 64], False, 1), ([512, 37, 1, 1, 200, 5, 1, 64], True, 1), ([2048], False, 1),
]


@pytest.mark.parametrize("counts,gated,phase", PHASE_CASES)
def test_phase_table(oracle, counts, gated, phase):
    assert oracle.phase(counts, gated) == phase


def test_pack_and_gather_config3(oracle):
    lengths = [512, 37, 1, 1, 200, 5, 1, 64]
    start, logit, rows = oracle.pack(lengths, [1] * 8)
    assert rows == 821
    assert start == [0, 512, 549, 550, 551, 751, 756, 757]
    assert logit == list(range(8))
    last = [oracle.gather_row(start, lengths, [1] * 8, logit, r) for r in range(8)]
    assert last == [s + c - 1 for s, c in zip(start, lengths)]
    assert oracle.gather_row(start, lengths, [1] * 8, logit, 8) == -1
    # Speculative verify (config 2): 8 x (1 + 4) rows, every row sampled.
    start, logit, rows = oracle.pack([5] * 8, [5] * 8)
    assert rows == 40 and start == list(range(0, 40, 5)) and logit == list(range(0, 40, 5))
    assert [oracle.gather_row(start, [5] * 8, [5] * 8, logit, r) for r in range(40)] == list(range(40))
    # Queries without samples are skipped (intermediate prompt chunks).
    start, logit, _ = oracle.pack([3, 4, 2], [0, 1, 2])
    assert [oracle.gather_row(start, [3, 4, 2], [0, 1, 2], logit, r) for r in range(3)] == [6, 7, 8]
