"""The gated prefill GEMM: the gate and up projections of one Q4_K MLP in a
single launch (q4k_mlp_gate_up / q4k_mlp at prefill row counts), against the
reference's two-call form (forward.cpp:116-118: gate stored with post 0, then
up with post 2 over it in place) run through linear(): the same buffer bit for
bit, one GEMM launch instead of two, and the oracle on the first and last row
of every 128-row block.  Cases: ragged row blocks and column blocks (a
workgroup with one live output tile), one block of K, fp16 activations, the
config-4 shape, long K with few tiles (two K-halves per tile, summed by the
second half to finish), and the ffn_norm folded into the shared staging.
Bar for the oracle: max row-relative error 1e-3."""
import numpy as np
import pytest
import torch

from q4k_ref import make_q4k, make_x, row_rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _edge_rows(m):
    rows = set()
    for r0 in range(0, m, 128):
        rows.update((r0, min(r0 + 127, m - 1)))
    return np.array(sorted(rows))


def _gemm_launches(q4k, fn):
    q4k.profile_enable(True)
    fn()
    torch.cuda.synchronize()
    n = q4k.profile_query(q4k.KERNEL_GEMM)[0]
    q4k.profile_enable(False)
    return n


# (m, n, k, dtype): n = 1296 and 272 leave the last 128-column workgroup one
# live output tile; k = 256 is one block; k = 8192 and 12288 with few tiles
# run as two K-halves per tile in both forms.
SHAPES = [(300, 512, 1024, torch.float32), (257, 1296, 2048, torch.float32), (129, 272, 1024, torch.float32),
          (130, 512, 256, torch.float16), (2048, 12288, 4096, torch.float32),
          (200, 1024, 8192, torch.float32), (130, 512, 12288, torch.float16)]


@pytest.mark.parametrize("m,n,k,dtype", SHAPES)
def test_gated_gemm_matches_two_calls(q4k, oracle, gpu, m, n, k, dtype):
    rng = np.random.default_rng(6100 + m + n)
    wg, wu = make_q4k(rng, n, k), make_q4k(rng, n, k)
    npdt = np.float16 if dtype == torch.float16 else np.float32
    x = make_x(rng, m, k, 0.05 if dtype == torch.float16 else 0.5).astype(npdt)
    G, U = q4k.Weight(wg, n, k), q4k.Weight(wu, n, k)
    xt = torch.from_numpy(x).to(gpu)
    y1 = torch.full((m, n), float("nan"), device=gpu, dtype=dtype)
    q4k.linear(xt, G, m, y1, query_counts=[m])
    q4k.linear(xt, U, m, y1, auxiliary=y1, gated=True, query_counts=[m])
    y2 = torch.full((m, n), float("nan"), device=gpu, dtype=dtype)
    assert _gemm_launches(q4k, lambda: q4k.mlp_gate_up(xt, G, U, m, y2, query_counts=[m])) == 1
    torch.cuda.synchronize()
    assert torch.isfinite(y2).all()
    diff = (y1 != y2).nonzero()
    assert diff.numel() == 0, f"{diff.shape[0]} outputs differ from the two-call form, first {diff[:4].tolist()}"
    rows = _edge_rows(m)
    ref = oracle.mlp_gate_up(x[rows], wg, wu, n, k)
    assert row_rel_err(y2.float().cpu().numpy()[rows], ref.astype(np.float32)) <= TOL


def test_gated_gemm_with_ffn_norm(q4k, gpu):
    """q4k_mlp with a norm weight: the gated GEMM over x normalised in its
    staging gives the gate buffer of linear_norm's two calls."""
    m, n, k = 300, 1024, 2048
    rng = np.random.default_rng(6200)
    wg, wu, wd = make_q4k(rng, n, k), make_q4k(rng, n, k), make_q4k(rng, k, n)
    G, U, D = q4k.Weight(wg, n, k), q4k.Weight(wu, n, k), q4k.Weight(wd, k, n)
    h0 = make_x(rng, m, k)
    nw = torch.from_numpy((1.0 + 0.2 * rng.standard_normal(k)).astype(np.float32)).to(gpu)
    ht = torch.from_numpy(h0).to(gpu)
    y1 = torch.empty((m, n), device=gpu)
    q4k.linear_norm(ht, G, nw, m, y1, query_counts=[m])
    q4k.linear_norm(ht, U, nw, m, y1, auxiliary=y1, gated=True, query_counts=[m])
    gate = torch.empty((m, n), device=gpu)
    hidden = ht.clone()
    q4k.mlp(hidden, G, U, D, hidden, gate, m, query_counts=[m], norm_weight=nw)
    torch.cuda.synchronize()
    assert torch.equal(gate, y1)
