"""Pins the oracle's block_q6_K restatement (the Q6_K row of the linear()
surface) without the reference: the element map against an independent
bit-mask formulation, closed forms, the cross-formulation invariant
(decode form in fp32 vs dequantize-then-dot in fp64) and brute force.

The reference holds no Q6_K golden vectors (its tests are end-to-end token
checks); these checks are chosen so that a swapped nibble, a wrong qh shift,
a wrong scale index or a dropped -32 fails at least one of them.
"""
import numpy as np
import pytest

from q4k_ref import (Q6_BLOCK_BYTES, TYPE_Q6_K, Oracle, dequant_q6k_numpy, make_q6k, make_x, row_rel_err, silu64)


@pytest.fixture(scope="module")
def oracle():
    return Oracle()


def q6_block(quants, scales, d=1.0):
    """Encode 256 quants (0..63) and 16 int8 scales as one block_q6_K
    (the GGUF layout: ql low/high nibbles, qh 2-bit fields, scales, d)."""
    q = np.asarray(quants, np.int64)
    blk = np.zeros(Q6_BLOCK_BYTES, np.uint8)
    for e in range(256):
        h, rr = divmod(e, 128)
        l, s = rr % 32, rr // 32
        qi = 64 * h + (32 if rr & 32 else 0) + l
        if rr & 64:
            blk[qi] |= (q[e] & 15) << 4
        else:
            blk[qi] |= q[e] & 15
        blk[128 + 32 * h + l] |= ((q[e] >> 4) & 3) << (2 * s)
    blk[192:208] = np.asarray(scales, np.int8).view(np.uint8)
    blk[208:210] = np.array([d], np.float16).view(np.uint8)
    return blk


def test_fields_match_bitmask_form(oracle):
    rng = np.random.default_rng(3)
    blk = make_q6k(rng, 1, 256)[0]
    quants, scales = oracle.q6_fields(blk)
    d = float(blk[208:210].view(np.float16)[0])
    ref = dequant_q6k_numpy(blk, 1, 256)[0]
    np.testing.assert_allclose(d * scales * (quants - 32), ref, rtol=0, atol=0)
    assert quants.min() >= 0 and quants.max() <= 63
    assert scales.min() >= -128 and scales.max() <= 127


def test_encode_decode_roundtrip(oracle):
    rng = np.random.default_rng(4)
    quants = rng.integers(0, 64, 256)
    scales = rng.integers(-128, 128, 16)
    blk = q6_block(quants, scales)
    got_q, got_s = oracle.q6_fields(blk)
    np.testing.assert_array_equal(got_q, quants)
    np.testing.assert_array_equal(got_s, np.repeat(scales, 16))


def test_one_hot_element_map(oracle):
    """x = e_k for every k of a K=256 row gives y[n] = W[n][k]: the full
    element -> (ql byte, nibble, qh bits, scale) map of all 16 rows."""
    rng = np.random.default_rng(5)
    n, k = 16, 256
    w = make_q6k(rng, n, k)
    x = np.eye(k, dtype=np.float32)
    y = oracle.linear(x, w, n, k, ggml_type=TYPE_Q6_K)
    np.testing.assert_allclose(y.T, dequant_q6k_numpy(w, n, k), rtol=1e-6, atol=0)


@pytest.mark.parametrize("c,s", [(0, 1), (63, 1), (32, 127), (5, -128), (40, -7)])
def test_closed_form_constant_block(oracle, c, s):
    """All quants c, all scales s, d = 1: y = s * (c - 32) * sum(x)."""
    blk = q6_block(np.full(256, c), np.full(16, s))
    w = np.tile(blk, (16, 2))  # 16 rows, K = 512
    x = make_x(np.random.default_rng(6), 3, 512)
    y = oracle.linear(x, w, 16, 512, ggml_type=TYPE_Q6_K)
    expect = s * (c - 32) * x.astype(np.float64).sum(axis=1)
    np.testing.assert_allclose(y, np.repeat(expect[:, None], 16, axis=1), rtol=1e-5, atol=1e-4)


def test_subblock_scales_index(oracle):
    """Scale j multiplies exactly elements 16j..16j+15: with quants 33
    (q - 32 = 1) and scale j = j + 1, x = ones gives sum_j 16 (j + 1)."""
    blk = q6_block(np.full(256, 33), np.arange(1, 17))
    w = np.tile(blk, (16, 1))
    for j in range(16):
        x = np.zeros((1, 256), np.float32)
        x[0, 16 * j:16 * j + 16] = 1.0
        y = oracle.linear(x, w, 16, 256, ggml_type=TYPE_Q6_K)
        np.testing.assert_array_equal(y, np.full((1, 16), 16.0 * (j + 1), np.float32))


def test_decode_form_matches_f64_dequant_dot(oracle):
    rng = np.random.default_rng(7)
    n, k, m = 64, 1024, 5
    w = make_q6k(rng, n, k)
    x = make_x(rng, m, k)
    y32 = oracle.linear(x, w, n, k, ggml_type=TYPE_Q6_K)
    y64 = oracle.linear_f64(x, w, n, k, ggml_type=TYPE_Q6_K)
    assert row_rel_err(y32, y64) < 1e-5


def test_brute_force_numpy(oracle):
    rng = np.random.default_rng(8)
    n, k, m = 8, 256, 3
    w = make_q6k(rng, n, k)
    x = make_x(rng, m, k).astype(np.float64)
    ref = x @ dequant_q6k_numpy(w, n, k).T
    np.testing.assert_allclose(oracle.linear_f64(x, w, n, k, ggml_type=TYPE_Q6_K), ref, rtol=1e-12, atol=1e-12)


def test_dequant_block_f32(oracle):
    rng = np.random.default_rng(9)
    blk = make_q6k(rng, 1, 256)[0]
    f32 = oracle.dequant_block(blk, ggml_type=TYPE_Q6_K)
    np.testing.assert_allclose(f32, dequant_q6k_numpy(blk, 1, 256)[0], rtol=1e-6, atol=0)


def test_dequant_block_f16_tile_value(oracle):
    """q6o_dequant_block_f16 stores the reference's prefill tile value
    half(fp32(d * sc * (q - 32))) (quant_linear.metal:83): the bit-mask form
    in float64 (its products are exact) rounded to fp32, then to fp16, bit
    for bit, over random blocks and blocks whose d pushes values into fp16
    denormals and past the fp16 range."""
    rng = np.random.default_rng(91)
    for dmax in (0.01, 1e-7, 40.0):
        w = make_q6k(rng, 64, 256, dmax=dmax)
        ref = dequant_q6k_numpy(w, 64, 256)
        with np.errstate(over="ignore"):
            want = ref.astype(np.float32).astype(np.float16).view(np.uint16)
        got = np.stack([oracle.dequant_block_f16(b, ggml_type=TYPE_Q6_K) for b in w.reshape(64, Q6_BLOCK_BYTES)])
        np.testing.assert_array_equal(got, want)


def test_posts_and_gate_up(oracle):
    rng = np.random.default_rng(10)
    n, k, m = 32, 512, 4
    wg, wu = make_q6k(rng, n, k), make_q6k(rng, n, k)
    x = make_x(rng, m, k)
    g = oracle.linear(x, wg, n, k, ggml_type=TYPE_Q6_K)
    u = oracle.linear(x, wu, n, k, ggml_type=TYPE_Q6_K)
    aux = make_x(rng, m, n)
    np.testing.assert_allclose(oracle.linear(x, wu, n, k, aux=aux, post=1, ggml_type=TYPE_Q6_K), u + aux, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(oracle.linear(x, wu, n, k, aux=g, post=2, ggml_type=TYPE_Q6_K),
                               silu64(g.astype(np.float64)) * u, rtol=1e-5, atol=1e-6)
    gu = oracle.mlp_gate_up(x, wg, wu, n, k, ggml_type=TYPE_Q6_K)
    np.testing.assert_allclose(gu, silu64(g.astype(np.float64)) * u, rtol=1e-5, atol=1e-6)


def test_unknown_type_rejected(oracle):
    import ctypes
    y = np.zeros((1, 16), np.float32)
    x = np.zeros((1, 256), np.float32)
    w = np.zeros(16 * 256, np.uint8)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    assert oracle.lib.q4o_linear_typed_f32(p(y), p(x), p(w), 10, None, 1, 16, 256, 0, 1) == -1
