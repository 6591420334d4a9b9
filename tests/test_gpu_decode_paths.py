"""The decode kernels for m <= 8 rows (fused gate/up GEMV packing x in
registers, split-K GEMV packing its K-slice in LDS, decode pack + streaming
GEMV) against the CPU oracle, over the row counts, dtypes and epilogues of a
decode pass.  Shapes are chosen to reach each kernel:

  gated, K=4096, N=12288   fused gate/up GEMV, 3 column tiles per workgroup
  gated, K=4096, N=512     fused gate/up GEMV, 1 column tile per workgroup
  plain, K=12288, N=1024   split-K GEMV (8 tiles x 8 K-slices of 6 blocks)
  plain, K=4096, N=65536   decode pack + persistent GEMV (16 waves, x in registers)

Bar: max row-relative error 1e-3 against the fp32-accumulated oracle.
"""
import numpy as np
import pytest
import torch

from q4k_ref import make_q4k, make_x, row_rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _t(a, dev, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dtype)


@pytest.mark.parametrize("m", [1, 3, 8])
@pytest.mark.parametrize("n", [12288, 512])
def test_gated_stream(q4k, oracle, gpu, m, n):
    k = 4096
    rng = np.random.default_rng(1000 + m + n)
    wg, wu = make_q4k(rng, n, k), make_q4k(rng, n, k)
    x = make_x(rng, m, k, 0.5)
    G, U = q4k.Weight(wg, n, k), q4k.Weight(wu, n, k)
    y = torch.full((m, n), float("nan"), device=gpu)
    q4k.mlp_gate_up(_t(x, gpu), G, U, m, y, query_counts=[1] * m)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert row_rel_err(got, oracle.mlp_gate_up(x, wg, wu, n, k)) <= TOL


def test_gated_stream_f16(q4k, oracle, gpu):
    m, n, k = 8, 12288, 4096
    rng = np.random.default_rng(1100)
    wg, wu = make_q4k(rng, n, k), make_q4k(rng, n, k)
    x = make_x(rng, m, k, 0.5).astype(np.float16)
    G, U = q4k.Weight(wg, n, k), q4k.Weight(wu, n, k)
    y = torch.empty((m, n), device=gpu, dtype=torch.float16)
    q4k.mlp_gate_up(_t(x, gpu, torch.float16), G, U, m, y, query_counts=[1] * m)
    torch.cuda.synchronize()
    assert row_rel_err(y.float().cpu().numpy(), oracle.mlp_gate_up(x, wg, wu, n, k)) <= TOL


@pytest.mark.parametrize("m,n", [(1, 12288), (5, 12288), (5, 256), (7, 48)])
def test_gated_register_pack_f16(q4k, oracle, gpu, m, n):
    """fp16 activations through both column-tile widths of the fused gate/up
    GEMV, with row counts that leave dead rows in the register pack."""
    k = 4096
    rng = np.random.default_rng(1150 + m + n)
    wg, wu = make_q4k(rng, n, k), make_q4k(rng, n, k)
    x = make_x(rng, m, k, 0.5).astype(np.float16)
    G, U = q4k.Weight(wg, n, k), q4k.Weight(wu, n, k)
    y = torch.full((m, n), float("nan"), device=gpu, dtype=torch.float16)
    q4k.mlp_gate_up(_t(x, gpu, torch.float16), G, U, m, y, query_counts=[1] * m)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    assert np.all(np.isfinite(got))
    assert row_rel_err(got, oracle.mlp_gate_up(x, wg, wu, n, k)) <= TOL


@pytest.mark.parametrize("m", [1, 5, 8])
@pytest.mark.parametrize("post", [0, 1, 2])
def test_splitk(q4k, oracle, gpu, m, post):
    n, k = 1024, 12288
    rng = np.random.default_rng(1200 + 10 * m + post)
    w = make_q4k(rng, n, k)
    x = make_x(rng, m, k, 0.5)
    aux = make_x(rng, m, n, 2.0)
    W = q4k.Weight(w, n, k)
    y = _t(aux, gpu) if post else torch.full((m, n), float("nan"), device=gpu)
    q4k.linear(_t(x, gpu), W, m, y, auxiliary=y if post else None, gated=(post == 2), query_counts=[1] * m)
    torch.cuda.synchronize()
    ref = oracle.linear(x, w, n, k, aux=aux if post else None, post=post)
    assert row_rel_err(y.cpu().numpy(), ref) <= TOL


def test_splitk_f16_and_repeat(q4k, oracle, gpu):
    """fp16 activations; then the same call again (the group counters must
    have been left at zero by the first launch)."""
    m, n, k = 8, 2048, 12288
    rng = np.random.default_rng(1300)
    w = make_q4k(rng, n, k)
    x = make_x(rng, m, k, 0.5).astype(np.float16)
    W = q4k.Weight(w, n, k)
    ref = oracle.linear(x, w, n, k)
    for _ in range(3):
        y = torch.empty((m, n), device=gpu, dtype=torch.float16)
        q4k.linear(_t(x, gpu, torch.float16), W, m, y, query_counts=[1] * m)
        torch.cuda.synchronize()
        assert row_rel_err(y.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("m,n,post,dtype", [(3, 65536, 0, torch.float32), (8, 16 * 4401, 1, torch.float32),
                                             (1, 16 * 4401, 2, torch.float32), (8, 65536, 1, torch.float16)])
def test_wide_persistent(q4k, oracle, gpu, m, n, post, dtype):
    """Wide plain projections (the LM head's shape class): the persistent
    GEMV, 2 column tiles per item (16 * 4401 columns: one tile in the last)."""
    k = 4096
    rng = np.random.default_rng(1400 + m + post)
    w = make_q4k(rng, n, k)
    npdt = np.float16 if dtype == torch.float16 else np.float32
    x = make_x(rng, m, k).astype(npdt)
    aux = make_x(rng, m, n, 2.0).astype(npdt) if post else None
    W = q4k.Weight(w, n, k)
    y = torch.full((m, n), float("nan"), device=gpu, dtype=dtype)
    if post:
        y.copy_(_t(aux, gpu).to(dtype))
    q4k.linear(_t(x, gpu).to(dtype), W, m, y, auxiliary=y if post else None, gated=post == 2, query_counts=[1] * m)
    torch.cuda.synchronize()
    assert row_rel_err(y.float().cpu().numpy(), oracle.linear(x, w, n, k, aux=aux, post=post)) <= TOL


def test_decode_rows_of_extreme_magnitude(q4k, oracle, gpu):
    """Rows far outside fp16 range (and a zero row) through both decode
    kernels: the per-(row, block) power-of-two scales keep them exact to
    the same relative precision."""
    rng = np.random.default_rng(1500)
    for n, k, gated in [(12288, 4096, True), (1024, 12288, False)]:
        m = 4
        x = make_x(rng, m, k)
        x[0] *= 1e6
        x[1] *= 1e-6
        x[2] = 0.0
        w = make_q4k(rng, n, k)
        W = q4k.Weight(w, n, k)
        y = torch.empty((m, n), device=gpu)
        if gated:
            wu = make_q4k(rng, n, k)
            U = q4k.Weight(wu, n, k)
            # Scale the gate/up inputs down so that SiLU stays in range.
            x *= 1e-3
            q4k.mlp_gate_up(_t(x, gpu), W, U, m, y, query_counts=[1] * m)
            ref = oracle.mlp_gate_up(x, w, wu, n, k)
        else:
            q4k.linear(_t(x, gpu), W, m, y, query_counts=[1] * m)
            ref = oracle.linear(x, w, n, k)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.all(got[2] == 0)
        assert row_rel_err(got, ref) <= TOL


def test_shard_shapes(q4k, oracle, gpu):
    """One GPU's share of the config-1 MLP sharded 8 ways: gate/up N = 1536
    (column-parallel), down K = 1536 (row-parallel, partial sums)."""
    m, k, n = 8, 4096, 1536
    rng = np.random.default_rng(1600)
    wg, wu, wd = make_q4k(rng, n, k), make_q4k(rng, n, k), make_q4k(rng, k, n)
    x = make_x(rng, m, k, 0.5)
    G, U, D = q4k.Weight(wg, n, k), q4k.Weight(wu, n, k), q4k.Weight(wd, k, n)
    g = torch.empty((m, n), device=gpu)
    q4k.mlp_gate_up(_t(x, gpu), G, U, m, g, query_counts=[1] * m)
    y = torch.empty((m, k), device=gpu)
    q4k.linear(g, D, m, y, query_counts=[1] * m)
    torch.cuda.synchronize()
    gn = g.cpu().numpy()
    assert row_rel_err(gn, oracle.mlp_gate_up(x, wg, wu, n, k)) <= TOL
    assert row_rel_err(y.cpu().numpy(), oracle.linear(gn, wd, k, n)) <= TOL
