"""Pins the oracle's Q8_0, Q5_K and IQ4_XS restatements (the rest of the
linear() surface's GGUF types) without the reference: the element map of
each against an independent numpy formulation taken from the reference's
decode kernels' bit-mask forms, closed forms, the cross-formulation
invariant (decode form in fp32 vs dequantize-then-dot in fp64) and brute
force.  The reference holds no golden vectors for these types."""
import ctypes

import numpy as np
import pytest

from q4k_ref import (IQ4NL, TYPE_IQ4_XS, TYPE_Q5_K, TYPE_Q8_0, TYPE_BLOCK_BYTES, Oracle, dequant_any_numpy, make_weight, make_x,
                     row_rel_err, silu64)

TYPES = [TYPE_Q8_0, TYPE_Q5_K, TYPE_IQ4_XS]


@pytest.fixture(scope="module")
def oracle():
    return Oracle()


@pytest.mark.parametrize("t", TYPES)
def test_dequant_block_matches_numpy_form(oracle, t):
    rng = np.random.default_rng(20 + t)
    w = make_weight(rng, 4, 256, t)
    for r in range(4):
        got = oracle.dequant_block(w[r], ggml_type=t)
        np.testing.assert_allclose(got, dequant_any_numpy(w[r], 1, 256, t)[0], rtol=1e-6, atol=0)


@pytest.mark.parametrize("t", TYPES)
def test_one_hot_element_map(oracle, t):
    rng = np.random.default_rng(30 + t)
    n, k = 16, 256
    w = make_weight(rng, n, k, t)
    y = oracle.linear(np.eye(k, dtype=np.float32), w, n, k, ggml_type=t)
    np.testing.assert_allclose(y.T, dequant_any_numpy(w, n, k, t), rtol=1e-6, atol=0)


@pytest.mark.parametrize("t", TYPES)
def test_decode_form_matches_f64_and_brute_force(oracle, t):
    rng = np.random.default_rng(40 + t)
    n, k, m = 48, 1024, 5
    w = make_weight(rng, n, k, t)
    x = make_x(rng, m, k)
    y32 = oracle.linear(x, w, n, k, ggml_type=t)
    y64 = oracle.linear_f64(x, w, n, k, ggml_type=t)
    assert row_rel_err(y32, y64) < 1e-5
    ref = x.astype(np.float64) @ dequant_any_numpy(w, n, k, t).T
    np.testing.assert_allclose(y64, ref, rtol=1e-11, atol=1e-11)


@pytest.mark.parametrize("t", TYPES)
def test_posts_and_gate_up(oracle, t):
    rng = np.random.default_rng(50 + t)
    n, k, m = 32, 512, 3
    wg, wu = make_weight(rng, n, k, t), make_weight(rng, n, k, t)
    x = make_x(rng, m, k)
    g = oracle.linear(x, wg, n, k, ggml_type=t).astype(np.float64)
    u = oracle.linear(x, wu, n, k, ggml_type=t).astype(np.float64)
    aux = make_x(rng, m, n)
    np.testing.assert_allclose(oracle.linear(x, wu, n, k, aux=aux, post=1, ggml_type=t), u + aux, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(oracle.linear(x, wu, n, k, aux=g.astype(np.float32), post=2, ggml_type=t), silu64(g) * u,
                               rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(oracle.mlp_gate_up(x, wg, wu, n, k, ggml_type=t), silu64(g) * u, rtol=1e-5, atol=1e-6)


def test_q8_0_closed_form(oracle):
    """Every record d = 0.5, q = -3: y = -1.5 * sum(x)."""
    rec = np.zeros(34, np.uint8)
    rec[0:2] = np.array([0.5], np.float16).view(np.uint8)
    rec[2:] = np.array([-3] * 32, np.int8).view(np.uint8)
    w = np.tile(rec, (16, 16))  # 16 rows, K = 512
    x = make_x(np.random.default_rng(60), 2, 512)
    y = oracle.linear(x, w, 16, 512, ggml_type=TYPE_Q8_0)
    np.testing.assert_allclose(y, np.repeat(-1.5 * x.astype(np.float64).sum(1)[:, None], 16, 1), rtol=1e-5, atol=1e-4)


def _q5_block(q5, sc, mn, d=1.0, dmin=1.0):
    from q4k_ref import load_oracle
    lib = load_oracle()
    blk = np.zeros(176, np.uint8)
    blk[0:2] = np.array([d], np.float16).view(np.uint8)
    blk[2:4] = np.array([dmin], np.float16).view(np.uint8)
    q12 = np.zeros(12, np.uint8)
    lib.q4o_pack_scale_min(np.ascontiguousarray(sc, np.uint8).ctypes.data_as(ctypes.c_void_p),
                           np.ascontiguousarray(mn, np.uint8).ctypes.data_as(ctypes.c_void_p), q12.ctypes.data_as(ctypes.c_void_p))
    blk[4:16] = q12
    for e in range(256):
        t, l, hi = e // 64, e % 32, (e // 32) % 2
        blk[48 + 32 * t + l] |= (q5[e] & 15) << (4 * hi)
        blk[16 + l] |= ((q5[e] >> 4) & 1) << (2 * t + hi)
    return blk


def test_q5_k_fields_and_closed_form(oracle):
    rng = np.random.default_rng(61)
    q5 = rng.integers(0, 32, 256)
    blk = _q5_block(q5, rng.integers(0, 64, 8), rng.integers(0, 64, 8))
    got = np.array([oracle.lib.q5o_quant(blk.ctypes.data_as(ctypes.c_void_p), e) for e in range(256)])
    np.testing.assert_array_equal(got, q5)
    # All q = 31, sc = 2, m = 3, d = dmin = 1: y = (2 * 31 - 3) * sum(x).
    blk = _q5_block(np.full(256, 31), np.full(8, 2), np.full(8, 3))
    w = np.tile(blk, (16, 1))
    x = make_x(rng, 2, 256)
    y = oracle.linear(x, w, 16, 256, ggml_type=TYPE_Q5_K)
    np.testing.assert_allclose(y, np.repeat(59.0 * x.astype(np.float64).sum(1)[:, None], 16, 1), rtol=1e-5, atol=1e-4)


def test_iq4_xs_codebook_scales_and_closed_form(oracle):
    np.testing.assert_array_equal([oracle.lib.iq4o_value(v) for v in range(16)], IQ4NL)
    rng = np.random.default_rng(62)
    ls = rng.integers(0, 64, 8)
    blk = make_weight(rng, 1, 256, TYPE_IQ4_XS)[0]
    blk[2:4] = np.array([sum(int(ls[j] >> 4) << (2 * j) for j in range(8))], np.uint16).view(np.uint8)
    blk[4:8] = [(ls[2 * i] & 15) | ((ls[2 * i + 1] & 15) << 4) for i in range(4)]
    p = blk.ctypes.data_as(ctypes.c_void_p)
    np.testing.assert_array_equal([oracle.lib.iq4o_scale(p, j) for j in range(8)], ls - 32)
    # Every index v and scale ls = 33 (ls - 32 = 1), d = 2: y = 2 * iq4nl[v] * sum(x).
    for v in (0, 7, 8, 15):
        blk = np.zeros(136, np.uint8)
        blk[0:2] = np.array([2.0], np.float16).view(np.uint8)
        blk[2:4] = np.array([sum(2 << (2 * j) for j in range(8))], np.uint16).view(np.uint8)  # high bits 2 -> 32
        blk[4:8] = 0x11  # low bits 1
        blk[8:] = v | (v << 4)
        w = np.tile(blk, (16, 1))
        x = make_x(rng, 2, 256)
        y = oracle.linear(x, w, 16, 256, ggml_type=TYPE_IQ4_XS)
        np.testing.assert_allclose(y, np.repeat(2.0 * IQ4NL[v] * x.astype(np.float64).sum(1)[:, None], 16, 1), rtol=1e-5, atol=1e-3)


@pytest.mark.parametrize("t", TYPES)
def test_block_bytes(t):
    assert make_weight(np.random.default_rng(0), 2, 512, t).shape == (2, 2 * TYPE_BLOCK_BYTES[t])
