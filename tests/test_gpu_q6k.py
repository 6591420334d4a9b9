"""Q6_K weights on the linear() surface (the LM head of real GGUF files and the
down projections of mixed-type files) against the CPU oracle on identical
seeded inputs.  Bar: max row-relative error 1e-3 (the products (q - 32) * sc
are exact in fp16 up to 2048 and rounded once above; activations are the
decode pack's hi/lo fp16, so the expected error is ~1e-6).

Covers decode and small-prefill row counts, ragged column tails (the last
workgroup's tiles past N), blocks per wave from 1 to 6 (K = 256 .. 12288),
post 1 / 2 in place, fp16 activations, prefill batches (the GEMV per group of
8 rows), the device-side upload, the gated projection with Q6_K weights,
mixed Q4_K / Q6_K MLPs as mixed-type GGUF files have them, graph replays, a
Q6_K tensor read from a GGUF file, and the full Qwen3.5 LM head
(K = 4096 -> N = 248,320) checked on a sample of its columns.
"""
import numpy as np
import pytest
import torch

from gguf_writer import GGML_Q6_K, write_gguf
from q4k_ref import TYPE_Q6_K, make_q4k, make_q6k, make_x, row_rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _t(a, dev, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dtype)


def _linear(q4k, oracle, gpu, seed, m, n, k, post=0, dtype=torch.float32, counts=None, device_upload=False):
    rng = np.random.default_rng(seed)
    w = make_q6k(rng, n, k)
    x = make_x(rng, m, k)
    npdt = np.float16 if dtype == torch.float16 else np.float32
    xq = x.astype(npdt)
    aux = make_x(rng, m, n, 2.0).astype(npdt) if post else None
    W = q4k.Weight(torch.from_numpy(w).to(gpu) if device_upload else w, n, k, ggml_type=TYPE_Q6_K)
    y = torch.full((m, n), float("nan"), device=gpu, dtype=dtype)
    auxt = None
    if post:
        y.copy_(_t(aux, gpu, dtype))
        auxt = y
    q4k.linear(_t(xq, gpu, dtype), W, m, y, auxiliary=auxt, gated=(post == 2), query_counts=counts)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    ref = oracle.linear(xq, w, n, k, aux=aux, post=post, ggml_type=TYPE_Q6_K)
    assert np.all(np.isfinite(got))
    err = row_rel_err(got, ref)
    assert err <= TOL, f"m={m} n={n} k={k} post={post} {dtype}: rel err {err:.3g}"
    return W, got, err


# (m, n, k): K = 256 (waves 1..7 idle), 2304 (waves with 2 and 1 blocks),
# 4096, 12288 (6 blocks per wave); N = 16 * 2049 (4 tiles per workgroup, one
# in the last) and 16 * 1025 (2 per workgroup, one in the last); N = 16 * 4401
# at K = 4096 takes the persistent form (2201 items of 2 tiles, one in the last).
SHAPES = [(1, 16, 256), (8, 16, 256), (3, 48, 768), (2, 80, 2304), (5, 4096, 4096), (8, 1024, 12288),
          (2, 16 * 2049, 512), (1, 16 * 1025, 256), (4, 592, 1024), (3, 16 * 4401, 4096)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_q6k_linear_store(q4k, oracle, gpu, m, n, k):
    _linear(q4k, oracle, gpu, 700 + m + k, m, n, k, counts=[1] * m)


@pytest.mark.parametrize("post", [1, 2])
@pytest.mark.parametrize("m,counts", [(8, [1] * 8), (20, [20])])
def test_q6k_epilogues_in_place(q4k, oracle, gpu, post, m, counts):
    _linear(q4k, oracle, gpu, 710 + post + m, m, 1024, 4096, post=post, counts=counts)


@pytest.mark.parametrize("m,post", [(8, 0), (5, 1), (13, 2)])
def test_q6k_fp16(q4k, oracle, gpu, m, post):
    _linear(q4k, oracle, gpu, 720 + m, m, 2048, 4096, post=post, dtype=torch.float16, counts=[m])


def test_q6k_prefill_groups_and_kernel_names(q4k, oracle, gpu):
    W, _, _ = _linear(q4k, oracle, gpu, 730, 64, 512, 2048, counts=None)
    assert W.kernel_name(1) == "linear_q6_k_k2048_n512_prefill_mfma16x16x32"
    W2, _, _ = _linear(q4k, oracle, gpu, 731, 8, 512, 2048, counts=[4, 4])
    assert W2.kernel_name(0) == "linear_q6_k_k2048_n512_decode_mfma16x16x32"
    _linear(q4k, oracle, gpu, 732, 21, 256, 1024, counts=[7, 14])  # prefill: groups of 8, 8, 5


def test_q6k_device_upload_is_bit_identical(q4k, oracle, gpu):
    _, a, _ = _linear(q4k, oracle, gpu, 740, 8, 4096, 4096, counts=[1] * 8)
    _, b, _ = _linear(q4k, oracle, gpu, 740, 8, 4096, 4096, counts=[1] * 8, device_upload=True)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("m,counts", [(8, [1] * 8), (12, [12])])
def test_q6k_gate_up(q4k, oracle, gpu, m, counts):
    n, k = 1536, 4096
    rng = np.random.default_rng(750 + m)
    wg, wu = make_q6k(rng, n, k), make_q6k(rng, n, k)
    x = make_x(rng, m, k, 0.5)
    G, U = q4k.Weight(wg, n, k, ggml_type=TYPE_Q6_K), q4k.Weight(wu, n, k, ggml_type=TYPE_Q6_K)
    gate = torch.full((m, n), float("nan"), device=gpu)
    q4k.mlp_gate_up(_t(x, gpu), G, U, m, gate, query_counts=counts)
    torch.cuda.synchronize()
    assert row_rel_err(gate.cpu().numpy(), oracle.mlp_gate_up(x, wg, wu, n, k, ggml_type=TYPE_Q6_K)) <= TOL


@pytest.mark.parametrize("m,counts,norm", [(8, [1] * 8, False), (8, [1] * 8, True), (20, [20], True)])
def test_mixed_type_mlp(q4k, oracle, gpu, m, counts, norm):
    """Q4_K gate/up with a Q6_K down projection (the mix of UD-Q4_K_XL files)."""
    k, n = 4096, 12288
    rng = np.random.default_rng(760 + m + norm)
    wg, wu, wd = make_q4k(rng, n, k), make_q4k(rng, n, k), make_q6k(rng, k, n)
    G, U = q4k.Weight(wg, n, k), q4k.Weight(wu, n, k)
    D = q4k.Weight(wd, k, n, ggml_type=TYPE_Q6_K)
    x, h0 = make_x(rng, m, k, 0.5), make_x(rng, m, k)
    nw = (0.05 * (1.0 + 0.1 * rng.standard_normal(k))).astype(np.float32) if norm else None
    hidden = _t(h0, gpu)
    gate = torch.full((m, n), float("nan"), device=gpu)
    q4k.mlp(_t(x, gpu), G, U, D, hidden, gate, m, query_counts=counts,
            norm_weight=None if nw is None else _t(nw, gpu), eps=1e-6)
    torch.cuda.synchronize()
    xin = oracle.rms_norm(x, nw) if norm else x
    g_gpu = gate.cpu().numpy()
    assert row_rel_err(g_gpu, oracle.mlp_gate_up(xin, wg, wu, n, k)) <= TOL
    ref = oracle.linear(g_gpu, wd, k, n, aux=h0, post=1, ggml_type=TYPE_Q6_K)
    assert row_rel_err(hidden.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("gate_q6", [True, False])
def test_mixed_type_gate_up_prefill(q4k, oracle, gpu, gate_q6):
    """Gate and up of different types in a prefill pass: the Q4_K projection
    must not reuse activations staged for a Q6_K one."""
    n, k, m = 512, 2048, 20
    rng = np.random.default_rng(770 + gate_q6)
    wq4, wq6 = make_q4k(rng, n, k), make_q6k(rng, n, k)
    A, B = q4k.Weight(wq4, n, k), q4k.Weight(wq6, n, k, ggml_type=TYPE_Q6_K)
    x = make_x(rng, m, k, 0.5)
    (G, wg, tg), (U, wu, tu) = ((B, wq6, TYPE_Q6_K), (A, wq4, 12)) if gate_q6 else ((A, wq4, 12), (B, wq6, TYPE_Q6_K))
    gate = torch.full((m, n), float("nan"), device=gpu)
    q4k.mlp_gate_up(_t(x, gpu), G, U, m, gate, query_counts=[m])
    torch.cuda.synchronize()
    g = oracle.linear(x, wg, n, k, ggml_type=tg).astype(np.float64)
    u = oracle.linear(x, wu, n, k, ggml_type=tu).astype(np.float64)
    assert row_rel_err(gate.cpu().numpy(), g / (1.0 + np.exp(-g)) * u) <= TOL


def test_q6k_graph_replays(q4k, oracle, gpu):
    n, k, m = 4096, 4096, 8
    rng = np.random.default_rng(780)
    w = make_q6k(rng, n, k)
    W = q4k.Weight(w, n, k, ggml_type=TYPE_Q6_K)
    x = _t(make_x(rng, m, k), gpu)
    y = torch.zeros((m, n), device=gpu)
    s = torch.cuda.Stream()
    q4k.linear(x, W, m, y, query_counts=[1] * m)  # sizes the workspace
    torch.cuda.synchronize()
    eager = y.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        q4k.linear(x, W, m, y, query_counts=[1] * m)
    for i in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {i}"
        q4k.linear(x, W, m, torch.empty_like(y), query_counts=[1] * m)  # eager work between replays
        torch.cuda.synchronize()
    ref = oracle.linear(x.cpu().numpy(), w, n, k, ggml_type=TYPE_Q6_K)
    assert row_rel_err(eager.cpu().numpy(), ref) <= TOL


def test_q6k_tensor_from_gguf(q4k, oracle, gpu, tmp_path):
    n, k, m = 1024, 4096, 8
    rng = np.random.default_rng(790)
    w = make_q6k(rng, n, k)
    path = tmp_path / "head.gguf"
    write_gguf(path, [("output.weight", GGML_Q6_K, (k, n), w.tobytes())])
    with q4k.GGUFFile(path) as f:
        W = f.weight("output.weight")
    assert (W.n, W.k, W.type) == (n, k, TYPE_Q6_K)
    x = make_x(rng, m, k)
    y = torch.empty((m, n), device=gpu)
    q4k.linear(_t(x, gpu), W, m, y, query_counts=[m])
    torch.cuda.synchronize()
    assert row_rel_err(y.cpu().numpy(), oracle.linear(x, w, n, k, ggml_type=TYPE_Q6_K)) <= TOL


def test_q6k_lm_head_full_size(q4k, oracle, gpu):
    """The Qwen3.5 LM head at its real shape, 8 gathered rows (config 3's
    prefill_small pass), uploaded through the device re-layout; every output
    is finite and a sample of 2048 columns matches the oracle."""
    n, k, m = 248320, 4096, 8
    rng = np.random.default_rng(800)
    w = make_q6k(rng, n, k)
    W = q4k.Weight(torch.from_numpy(w).to(gpu), n, k, ggml_type=TYPE_Q6_K)
    x = make_x(rng, m, k)
    y = torch.empty((m, n), device=gpu)
    q4k.linear(_t(x, gpu), W, m, y, query_counts=[1] * m)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.all(np.isfinite(got))
    cols = np.sort(np.concatenate([rng.choice(n, 2032, replace=False), np.arange(n - 16, n)]))
    ref = oracle.linear(x, np.ascontiguousarray(w[cols]), len(cols), k, ggml_type=TYPE_Q6_K)
    assert row_rel_err(got[:, cols], ref) <= TOL
