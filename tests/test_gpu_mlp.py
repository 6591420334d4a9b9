"""The MLP entry point (q4k_mlp: the MLP section of Ops::decoder,
forward.cpp:114-119 -- fused gate/up into the gate buffer, then the down
projection with the residual added in place) against the CPU oracle at the
config-1 shapes: decode row counts, back-to-back calls (the split-K
counters must return to zero), a HIP graph replayed with eager work between
replays, agreement with the explicit two-call sequence, and a prefill-phase
pass.  Bar: max row-relative error 1e-3 for the gate buffer and the output."""
import numpy as np
import pytest
import torch

from q4k_ref import make_q4k, make_x, row_rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
K, N = 4096, 12288


@pytest.fixture(scope="module")
def mlp_weights(q4k):
    rng = np.random.default_rng(0x51A70100)
    wg, wu, wd = make_q4k(rng, N, K), make_q4k(rng, N, K), make_q4k(rng, K, N)
    return (wg, wu, wd), (q4k.Weight(wg, N, K), q4k.Weight(wu, N, K), q4k.Weight(wd, K, N))


def _check(oracle, x, h0, gate, hidden, w):
    wg, wu, wd = w
    g_gpu = gate.cpu().numpy()
    assert row_rel_err(g_gpu, oracle.mlp_gate_up(x, wg, wu, N, K)) <= TOL
    ref = oracle.linear(g_gpu, wd, K, N, aux=h0, post=1)
    assert row_rel_err(hidden.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("m", [8, 1, 3, 5])
def test_decode_mlp_matches_oracle(q4k, oracle, gpu, mlp_weights, m):
    w, (G, U, D) = mlp_weights
    rng = np.random.default_rng(500 + m)
    x, h0 = make_x(rng, m, K, 0.5), make_x(rng, m, K)
    gate = torch.full((m, N), float("nan"), device=gpu)
    hidden = torch.from_numpy(h0).to(gpu)
    q4k.mlp(torch.from_numpy(x).to(gpu), G, U, D, hidden, gate, m, query_counts=[1] * m)
    torch.cuda.synchronize()
    _check(oracle, x, h0, gate, hidden, w)


def test_back_to_back_calls(q4k, oracle, gpu, mlp_weights):
    w, (G, U, D) = mlp_weights
    m = 8
    rng = np.random.default_rng(600)
    cases = [(make_x(rng, m, K, 0.5), make_x(rng, m, K)) for _ in range(10)]
    outs = []
    for x, h0 in cases:
        gate = torch.empty((m, N), device=gpu)
        hidden = torch.from_numpy(h0).to(gpu)
        q4k.mlp(torch.from_numpy(x).to(gpu), G, U, D, hidden, gate, m, query_counts=[1] * m)
        outs.append((gate, hidden))
    torch.cuda.synchronize()
    for (x, h0), (gate, hidden) in zip(cases[::3], outs[::3]):
        _check(oracle, x, h0, gate, hidden, w)


def test_graph_replays(q4k, gpu, mlp_weights):
    """A captured MLP replayed five times with eager calls between the
    replays: every replay equals the eager result bit for bit."""
    _, (G, U, D) = mlp_weights
    m = 8
    rng = np.random.default_rng(700)
    x = torch.from_numpy(make_x(rng, m, K, 0.5)).to(gpu)
    h0 = torch.from_numpy(make_x(rng, m, K)).to(gpu)
    gate, hidden = torch.empty((m, N), device=gpu), h0.clone()
    q4k.mlp(x, G, U, D, hidden, gate, m, query_counts=[1] * m)
    torch.cuda.synchronize()
    eager_gate, eager_hidden = gate.clone(), hidden.clone()
    g_gate, g_hidden = torch.empty_like(gate), torch.empty_like(hidden)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_hidden.copy_(h0)
        q4k.mlp(x, G, U, D, g_hidden, g_gate, m, query_counts=[1] * m)
    for i in range(5):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(g_gate, eager_gate), i
        assert torch.equal(g_hidden, eager_hidden), i
        scratch_gate, scratch_hidden = torch.empty_like(gate), h0.clone()
        q4k.mlp(x, G, U, D, scratch_hidden, scratch_gate, m, query_counts=[1] * m)  # eager work between replays
        torch.cuda.synchronize()


def test_matches_the_two_calls(q4k, gpu, mlp_weights):
    _, (G, U, D) = mlp_weights
    m = 8
    rng = np.random.default_rng(800)
    x = torch.from_numpy(make_x(rng, m, K, 0.5)).to(gpu)
    h0 = make_x(rng, m, K)
    gate1, hidden1 = torch.empty((m, N), device=gpu), torch.from_numpy(h0).to(gpu)
    q4k.mlp(x, G, U, D, hidden1, gate1, m, query_counts=[1] * m)
    gate2, hidden2 = torch.empty((m, N), device=gpu), torch.from_numpy(h0).to(gpu)
    q4k.mlp_gate_up(x, G, U, m, gate2, query_counts=[1] * m)
    q4k.linear(gate2, D, m, hidden2, auxiliary=hidden2, query_counts=[1] * m)
    torch.cuda.synchronize()
    assert torch.equal(gate1, gate2) and torch.equal(hidden1, hidden2)


def test_prefill_phase_pass(q4k, oracle, gpu, mlp_weights):
    """A pass with a sequence of more than 5 rows is not a decode pass: the
    reference's prefill MLP sequence runs (forward.cpp:116-119)."""
    w, (G, U, D) = mlp_weights
    m = 12
    rng = np.random.default_rng(900)
    x, h0 = make_x(rng, m, K, 0.5), make_x(rng, m, K)
    gate, hidden = torch.empty((m, N), device=gpu), torch.from_numpy(h0).to(gpu)
    q4k.mlp(torch.from_numpy(x).to(gpu), G, U, D, hidden, gate, m, query_counts=[6, 6])
    torch.cuda.synchronize()
    _check(oracle, x, h0, gate, hidden, w)


@pytest.mark.parametrize("m,counts,dtype", [(8, [1] * 8, torch.float32), (3, [1, 1, 1], torch.float32),
                                            (12, [6, 6], torch.float32), (4, [1] * 4, torch.float16)])
def test_mlp_block_with_ffn_norm(q4k, oracle, gpu, mlp_weights, m, counts, dtype):
    """The decoder's MLP block as the reference runs it (forward.cpp:114-119):
    x = hidden, the layer's ffn_norm applied first -- inside the fused
    gate/up GEMV for decode passes, as a separate RMS norm otherwise."""
    (wg, wu, wd), (G, U, D) = mlp_weights
    rng = np.random.default_rng(1000 + m)
    h0 = make_x(rng, m, K, 3.0)
    h0[0] *= 50.0
    # ffn_norm weights of a size that keeps SiLU(gate) * up and the down
    # projection's outputs within fp16 range for these synthetic weights.
    scale = 0.005 if dtype == torch.float16 else 0.05
    norm = (scale * (1.0 + 0.2 * rng.standard_normal(K))).astype(np.float32)
    if dtype == torch.float16:
        h0 = h0.astype(np.float16)
    hidden = torch.from_numpy(h0).to(gpu)
    gate = torch.empty((m, N), device=gpu, dtype=dtype)
    q4k.mlp(hidden, G, U, D, hidden, gate, m, query_counts=counts, norm_weight=torch.from_numpy(norm).to(gpu))
    torch.cuda.synchronize()
    xn = oracle.rms_norm(h0, norm)
    g_ref = oracle.mlp_gate_up(xn, wg, wu, N, K)
    g_gpu = gate.cpu().numpy()
    assert row_rel_err(g_gpu.astype(np.float32), g_ref.astype(np.float32)) <= TOL
    ref = oracle.linear(g_gpu, wd, K, N, aux=h0, post=1)
    assert row_rel_err(hidden.cpu().numpy().astype(np.float32), ref.astype(np.float32)) <= TOL
