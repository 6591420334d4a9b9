"""The GEMV for decode-shaped batches of 9..48 activation rows (x staged
once per call into fp16 MFMA fragments with per-(row, block) power-of-two
scales; one 16-column tile per workgroup, K split over its waves) against
the CPU oracle: several block counts (K = 768 .. 12288, odd ones
included), partial and single column tiles, hi/lo rows (m <= 24) and single
fp16 rows (25..48), gated pairs, fp16 activations, post 1 / 2; back-to-back
calls of one shape give identical results.  Gated pairs at least 48 columns
per CU wide (N = 12288), and plain projections with K = 12288, take the rows
GEMV (several column tiles per workgroup, 8 waves splitting K, each block of
staged x read once per wave).
Bar: max row-relative error 1e-3."""
import numpy as np
import pytest
import torch

from q4k_ref import make_q4k, make_x, row_rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
# Single fp16 rows (25..48) of fp32 activations, in the rows GEMV and the
# staged GEMV: the mean-quant correction of the rounding (each sub-block's sum of residuals times 7.5 sc) removes the
# part of the error common to every column; measured 1.5e-4 .. 3.0e-4 (plain
# and gated), against 4.6e-4 .. 9.7e-4 without it.
CORRECTED_TOL = 5e-4

# (m, n, k, counts): decode phase (counts <= 5 per query) unless noted
SHAPES = [
    (40, 4096, 12288, [5] * 8),   # down projection of config 2: several K-slices
    (40, 12288, 4096, [5] * 8),   # wide N
    (24, 2048, 4096, [3] * 8),    # hi/lo rows, three row tiles
    (9, 1040, 1024, [5, 4]),      # partial last column group
    (13, 48, 768, [5, 5, 3]),     # fewer tiles than one group
    (48, 4096, 2048, [48]),       # prefill batch of 48 rows (GEMV side)
    (30, 272, 3328, [30]),        # odd block count (13)
]


@pytest.mark.parametrize("m,n,k,counts", SHAPES)
def test_rows_store(q4k, oracle, gpu, m, n, k, counts):
    rng = np.random.default_rng(1500 + m + n % 97)
    w = make_q4k(rng, n, k)
    W = q4k.Weight(w, n, k)
    x = make_x(rng, m, k)
    y = torch.full((m, n), float("nan"), device=gpu)
    xt = torch.from_numpy(x).to(gpu)
    q4k.linear(xt, W, m, y, query_counts=counts)
    # A second call of the same shape must give the same result.
    y2 = torch.full((m, n), float("nan"), device=gpu)
    q4k.linear(xt, W, m, y2, query_counts=counts)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert torch.equal(y, y2)
    err = row_rel_err(got, oracle.linear(x, w, n, k))
    print(f"rows store m={m} n={n} k={k}: max row error {err:.3e}")
    assert err <= (CORRECTED_TOL if m > 24 else TOL)


@pytest.mark.parametrize("m,post,dtype", [(40, 1, torch.float32), (17, 2, torch.float32), (33, 1, torch.float16),
                                          (6, 0, torch.float16)])
def test_rows_epilogues(q4k, oracle, gpu, m, post, dtype):
    n, k = 1024, 4096
    rng = np.random.default_rng(1550 + m)
    w = make_q4k(rng, n, k)
    W = q4k.Weight(w, n, k)
    npdt = np.float16 if dtype == torch.float16 else np.float32
    x = make_x(rng, m, k, 0.25).astype(npdt)
    aux = make_x(rng, m, n, 2.0).astype(npdt) if post else None
    y = torch.from_numpy(aux).to(gpu) if post else torch.empty((m, n), device=gpu, dtype=dtype)
    q4k.linear(torch.from_numpy(x).to(gpu), W, m, y, auxiliary=y if post else None, gated=(post == 2), query_counts=[5] * (m // 5) + ([m % 5] if m % 5 else []))
    torch.cuda.synchronize()
    ref = oracle.linear(x, w, n, k, aux=aux, post=post)
    assert row_rel_err(y.float().cpu().numpy(), ref.astype(np.float32)) <= TOL


@pytest.mark.parametrize("m", [9, 24, 40])
def test_rows_gated(q4k, oracle, gpu, m):
    n, k = 3072, 4096
    rng = np.random.default_rng(1560 + m)
    wg, wu = make_q4k(rng, n, k), make_q4k(rng, n, k)
    G, U = q4k.Weight(wg, n, k), q4k.Weight(wu, n, k)
    x = make_x(rng, m, k, 0.5)
    y = torch.empty((m, n), device=gpu)
    counts = [5] * (m // 5) + ([m % 5] if m % 5 else [])
    q4k.mlp_gate_up(torch.from_numpy(x).to(gpu), G, U, m, y, query_counts=counts)
    torch.cuda.synchronize()
    assert row_rel_err(y.cpu().numpy(), oracle.mlp_gate_up(x, wg, wu, n, k)) <= TOL


@pytest.mark.parametrize("m,dtype", [(9, torch.float32), (24, torch.float32), (33, torch.float16), (40, torch.float32),
                                     (40, torch.float16)])
def test_rows_gated_wide(q4k, oracle, gpu, m, dtype):
    """The config-2 MLP width: one gated launch (the rows gate/up GEMV) after
    the staging, every row against the oracle, identical on a second call."""
    n, k = 12288, 4096
    rng = np.random.default_rng(1570 + m)
    wg, wu = make_q4k(rng, n, k), make_q4k(rng, n, k)
    G, U = q4k.Weight(wg, n, k), q4k.Weight(wu, n, k)
    npdt = np.float16 if dtype == torch.float16 else np.float32
    x = make_x(rng, m, k, 0.5).astype(npdt)
    xt = torch.from_numpy(x).to(gpu)
    counts = [5] * (m // 5) + ([m % 5] if m % 5 else [])
    y = torch.full((m, n), float("nan"), device=gpu, dtype=dtype)
    q4k.profile_enable(True)
    q4k.mlp_gate_up(xt, G, U, m, y, query_counts=counts)
    torch.cuda.synchronize()
    gated = q4k.profile_query(q4k.KERNEL_GEMV_GATED)[0]
    q4k.profile_enable(False)
    assert gated == 1
    y2 = torch.full((m, n), float("nan"), device=gpu, dtype=dtype)
    q4k.mlp_gate_up(xt, G, U, m, y2, query_counts=counts)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    got = y.float().cpu().numpy()
    assert np.all(np.isfinite(got))
    err = row_rel_err(got, oracle.mlp_gate_up(x, wg, wu, n, k))
    print(f"gated rows m={m} {dtype}: max row error {err:.3e}")
    assert err <= (CORRECTED_TOL if m > 24 and dtype == torch.float32 else TOL)


@pytest.mark.parametrize("m,n,post,dtype", [(40, 4096, 1, torch.float32), (17, 8192, 2, torch.float32), (33, 4096, 1, torch.float16),
                                            (24, 12288, 0, torch.float32), (24, 4096, 1, torch.float32)])
def test_rows_k12288(q4k, oracle, gpu, m, n, post, dtype):
    """Plain projections with K = 12288 (the config-2 down projection and
    wider ones) on the rows GEMV: epilogues, fp16, hi/lo rows (at N = 4096
    also in K-slices)."""
    k = 12288
    rng = np.random.default_rng(1580 + m + n % 89)
    w = make_q4k(rng, n, k)
    W = q4k.Weight(w, n, k)
    npdt = np.float16 if dtype == torch.float16 else np.float32
    x = make_x(rng, m, k, 0.25).astype(npdt)
    aux = make_x(rng, m, n, 2.0).astype(npdt) if post else None
    y = torch.from_numpy(aux).to(gpu) if post else torch.full((m, n), float("nan"), device=gpu, dtype=dtype)
    counts = [5] * (m // 5) + ([m % 5] if m % 5 else [])
    q4k.linear(torch.from_numpy(x).to(gpu), W, m, y, auxiliary=y if post else None, gated=(post == 2), query_counts=counts)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    assert np.all(np.isfinite(got))
    ref = oracle.linear(x, w, n, k, aux=aux, post=post)
    err = row_rel_err(got, ref.astype(np.float32))
    print(f"rows K=12288 m={m} n={n} post={post} {dtype}: max row error {err:.3e}")
    assert err <= (CORRECTED_TOL if m > 24 and dtype == torch.float32 else TOL)
