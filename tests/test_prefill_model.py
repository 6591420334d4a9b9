"""Pins the float64 model of the reference's prefill arithmetic
(q4k_ref.prefill_arithmetic), which the gated-GEMM tests use to tell the
GEMM's own error from the ill-conditioning of SiLU(gate) * up.

  - with fp16 activations and weights whose tile values are exact in fp16,
    the model is the exact contraction (no rounding is invented);
  - fp32 activations are rounded once: the model stays within 2^-11 of the
    exact contraction per row norm and differs from it (rounding happens);
  - weights whose value is not an fp16 number are rounded to nearest;
  - a row's power-of-two scale does not change the result (it is exact).
"""
import numpy as np

from q4k_ref import BLOCK_BYTES, dequant_numpy, gated_prefill_arithmetic, make_q4k, make_x, prefill_arithmetic, row_rel_err, silu64


def _exact_block_weights(rng, n, k):
    """Q4_K bytes with d = 1, dmin = 0.5: every weight sc*q - m/2 is a small
    multiple of 1/2, exact in fp16."""
    w = make_q4k(rng, n, k).reshape(n, k // 256, BLOCK_BYTES)
    w[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    w[:, :, 2:4] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    return w.reshape(n, -1)


def test_exact_inputs_give_the_exact_contraction():
    rng = np.random.default_rng(91)
    n, k, m = 24, 512, 5
    w = _exact_block_weights(rng, n, k)
    x = make_x(rng, m, k).astype(np.float16)
    want = x.astype(np.float64) @ dequant_numpy(w, n, k).T
    assert np.array_equal(prefill_arithmetic(x, w, n, k), want)
    # fp32 activations that are fp16 numbers: the same
    assert np.array_equal(prefill_arithmetic(x.astype(np.float32), w, n, k), want)


def test_fp32_activations_are_rounded_once():
    rng = np.random.default_rng(92)
    n, k, m = 24, 512, 6
    w = _exact_block_weights(rng, n, k)
    x = make_x(rng, m, k)
    exact = x.astype(np.float64) @ dequant_numpy(w, n, k).T
    got = prefill_arithmetic(x, w, n, k)
    err = row_rel_err(got, exact)
    assert 0.0 < err <= 2.0 ** -11
    # A power-of-two scale of a row changes nothing but the scale.
    x2 = x.copy()
    x2[0] *= 2.0 ** 20
    got2 = prefill_arithmetic(x2, w, n, k)
    assert np.array_equal(got2[0], got[0] * 2.0 ** 20) and np.array_equal(got2[1:], got[1:])


def test_weights_round_to_nearest_fp16():
    rng = np.random.default_rng(93)
    n, k = 16, 256
    w = make_q4k(rng, n, k)
    wd = dequant_numpy(w, n, k)
    # one-hot fp16 activations read single tile values
    x = np.eye(k, dtype=np.float16)[::17]
    got = prefill_arithmetic(x, w, n, k)
    cols = wd[:, ::17].T
    err = np.abs(got - cols)
    # within half an fp16 ulp of the exact weight, and not all exact
    ulp = np.spacing(np.abs(cols).astype(np.float16)).astype(np.float64)
    assert np.all(err <= 0.5 * ulp + 1e-12) and np.any(err > 0)


def test_gated_model_composes_the_projections():
    rng = np.random.default_rng(94)
    n, k, m = 32, 512, 4
    wg, wu = make_q4k(rng, n, k), make_q4k(rng, n, k)
    x = make_x(rng, m, k, 0.5)
    g, u = prefill_arithmetic(x, wg, n, k), prefill_arithmetic(x, wu, n, k)
    assert np.array_equal(gated_prefill_arithmetic(x, wg, wu, n, k), silu64(g) * u)
    h = gated_prefill_arithmetic(x, wg, wu, n, k, f16_out=True)
    assert np.array_equal(h, h.astype(np.float16).astype(np.float64))
