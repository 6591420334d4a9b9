"""Pins the oracle's restatement of the path's neighbours in a pass: the
Q4_K token embedding (embedding_q4_k, quant_linear.metal:572-591) and the RMS
norm / LM-head rms_norm_gather (native_ops.metal:6-40).

  - embedding rows against the independent numpy formulation of the format
    (kmask unpacking, embedding_q4_k addressing) in float64, and bit for bit
    against the same products taken in float32 numpy;
  - embedding rows against the pinned linear() oracle on one-hot activations
    (a second contraction that reads every element position);
  - RMS norm closed forms: constant rows, a 3-4-5 row, zero rows, exact
    power-of-two scale invariance, eps;
  - rms_norm_gather as rms_norm composed with the LM-head row table, whose
    config-3 rows are written out by hand.
"""
import numpy as np
import pytest

from q4k_ref import dequant_numpy, make_q4k, scale_min_kmask


def test_embedding_matches_numpy_format(oracle):
    rng = np.random.default_rng(70)
    n, k = 48, 1024
    w = make_q4k(rng, n, k)
    ids = [0, 47, 16, 15, 3, 3]
    got = oracle.embedding(w, n, k, ids)
    ref = dequant_numpy(w, n, k)[ids]
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-9)
    # float32 products in the kernel's order: (d * sc) * q - dmin * m.
    blk = w.reshape(n, k // 256, 144)[ids]
    d = blk[..., 0:2].copy().view(np.float16).astype(np.float32)[..., 0]
    dmin = blk[..., 2:4].copy().view(np.float16).astype(np.float32)[..., 0]
    sc, mn = scale_min_kmask(blk[..., 4:16])
    r = np.arange(256)
    qb = blk[..., 16 + (r >> 6) * 32 + (r & 31)].astype(np.uint32)
    q = np.where((r & 32) != 0, qb >> 4, qb & 15).astype(np.float32)
    f32 = (d[..., None] * sc[..., r >> 5].astype(np.float32)) * q - dmin[..., None] * mn[..., r >> 5].astype(np.float32)
    assert np.array_equal(got.view(np.uint32), f32.reshape(len(ids), k).astype(np.float32).view(np.uint32))


def test_embedding_equals_one_hot_linear(oracle):
    rng = np.random.default_rng(71)
    n, k = 32, 256
    w = make_q4k(rng, n, k)
    cols = oracle.linear(np.eye(k, dtype=np.float32), w, n, k)  # [k, n]: cols[e][row] = W[row][e]
    ids = list(range(n))
    emb = oracle.embedding(w, n, k, ids)
    assert np.allclose(emb, cols.T, rtol=1e-6, atol=1e-8)


def test_embedding_out_of_range_rows_are_zero(oracle):
    rng = np.random.default_rng(72)
    n, k = 16, 512
    w = make_q4k(rng, n, k)
    got = oracle.embedding(w, n, k, [-1, 16, 1 << 30, 5])
    assert np.all(got[:3] == 0)
    assert np.any(got[3] != 0)


def test_embedding_f16_is_the_rounded_f32(oracle):
    rng = np.random.default_rng(73)
    n, k = 16, 512
    w = make_q4k(rng, n, k, dmax=4.0)
    ids = [1, 9, 15]
    assert np.array_equal(oracle.embedding(w, n, k, ids, f16=True), oracle.embedding(w, n, k, ids).astype(np.float16))


def test_rms_norm_closed_forms(oracle):
    k = 64
    w = np.linspace(-2, 2, k).astype(np.float32)
    # constant row c: rms = |c|, so y = sign(c) * w (eps = 0)
    x = np.full((2, k), 3.0, np.float32)
    x[1] = -0.25
    y = oracle.rms_norm(x, w, eps=0.0)
    assert np.allclose(y[0], w, rtol=1e-7) and np.allclose(y[1], -w, rtol=1e-7)
    # 3-4-5: mean square 25 / 4, rms 2.5
    x4 = np.array([[3.0, 4.0, 0.0, 0.0]], np.float32)
    w4 = np.array([1.0, 1.0, 1.0, 2.0], np.float32)
    assert np.allclose(oracle.rms_norm(x4, w4, eps=0.0), [[1.2, 1.6, 0.0, 0.0]], rtol=1e-7)
    # zero row with eps > 0 stays zero
    assert np.all(oracle.rms_norm(np.zeros((1, k), np.float32), w) == 0)
    # eps enters under the root: mean square 1, eps 3 -> scale 1/2
    assert np.allclose(oracle.rms_norm(np.ones((1, 4), np.float32), np.ones(4, np.float32), eps=3.0), 0.5, rtol=1e-7)


def test_rms_norm_power_of_two_scale_invariance(oracle):
    rng = np.random.default_rng(74)
    x = rng.standard_normal((4, 4096)).astype(np.float32)
    w = rng.standard_normal(4096).astype(np.float32)
    a = oracle.rms_norm(x, w, eps=0.0)
    for e in (-20, 10, 40):
        assert np.array_equal(oracle.rms_norm(x * np.float32(2.0**e), w, eps=0.0), a)


def test_rms_norm_f16_reads_and_rounds_half(oracle):
    rng = np.random.default_rng(75)
    x = (rng.standard_normal((3, 256)) * 8).astype(np.float16)
    w = rng.standard_normal(256).astype(np.float32)
    ref = oracle.rms_norm(x.astype(np.float32), w)
    got = oracle.rms_norm(x, w)
    assert got.dtype == np.float16
    assert np.array_equal(got, ref.astype(np.float16))


def test_rms_norm_gather_is_rms_norm_of_the_lm_head_rows(oracle):
    lengths = [512, 37, 1, 1, 200, 5, 1, 64]
    # each sequence's last prompt row: exclusive prefix sum + length - 1
    assert oracle.logit_sources(lengths, [1] * 8) == [511, 548, 549, 550, 750, 755, 756, 820]
    rng = np.random.default_rng(76)
    x = rng.standard_normal((821, 128)).astype(np.float32)
    w = rng.standard_normal(128).astype(np.float32)
    src = oracle.logit_sources(lengths, [1] * 8)
    assert np.array_equal(oracle.rms_norm(x, w, src=src), oracle.rms_norm(x, w)[src])
    # speculative verify rows: every row of 8 queries of 5 (forward.cpp:180-183)
    assert oracle.logit_sources([5] * 8, [5] * 8) == list(range(40))


def test_embedding_tokens_closed_form(oracle):
    """Rows of a packed batch to request-buffer tokens (quant_linear.metal:577-584
    mode 0 with queryRow, batch.hpp:19-23), worked by hand: queries of 3, 1 and
    2 rows at positions 5, 0, 7 of slots 2, 0, 1 of a 3 x 10 token buffer."""
    tokens = np.arange(30, dtype=np.int32) * 7 + 1
    got = oracle.embedding_tokens([3, 1, 2], [5, 0, 7], [2, 0, 1], 10, tokens)
    assert got == [176, 183, 190, 1, 120, 127, -1]


def test_embedding_tokens_are_the_slot_slices_in_query_order(oracle):
    """Every batch: the row tokens are the queries' slices
    buffer[slot, position:position + count] concatenated in query order."""
    rng = np.random.default_rng(77)
    for _ in range(40):
        nq, slots_n, capacity = int(rng.integers(1, 9)), 9, 64
        counts = rng.integers(1, 20, nq)
        positions = np.array([rng.integers(0, capacity - c + 1) for c in counts])
        slots = rng.permutation(slots_n)[:nq]
        tokens = rng.integers(0, 248320, slots_n * capacity).astype(np.int32)
        got = oracle.embedding_tokens(counts, positions, slots, capacity, tokens)
        buf = tokens.reshape(slots_n, capacity)
        want = np.concatenate([buf[s, p:p + c] for s, p, c in zip(slots, positions, counts)])
        assert got[:-1] == want.tolist() and got[-1] == -1
