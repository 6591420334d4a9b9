"""RMS norm folded into the projections (forward.cpp:82 attn_norm before the
QKV projections, :114 ffn_norm before the MLP): q4k_linear_norm and q4k_mlp
with a norm weight against the oracle's rms_norm composed with its linear,
on every kernel family; the paths that stage x run no separate norm launch.
Bar: max row-relative error 1e-3."""
import numpy as np
import pytest
import torch

from q4k_ref import TYPE_IQ4_XS, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, make_q4k, make_weight, make_x, row_rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _norm_weight(rng, k, scale=1.0):
    return (scale * (1.0 + 0.2 * rng.standard_normal(k))).astype(np.float32)


def _aux_launches(q4k):
    return q4k.profile_query(q4k.KERNEL_AUX)[0]


# (label, m, counts, n, k, post, fused): fused = the norm rides in the staging
CASES = [
    ("decode QKV, staged GEMV", 8, [1] * 8, 6144, 4096, 0, True),
    ("decode, 40 rows", 40, [5] * 8, 1024, 4096, 1, True),
    ("prefill GEMM", 300, [300], 4096, 4096, 0, True),
    ("prefill GEMM, eight-row staging", 2050, [2050], 256, 4096, 2, True),
    ("prefill GEMM, K=12288 staging through LDS", 300, [300], 256, 12288, 1, True),
    ("split-K (K=12288)", 8, [1] * 8, 4096, 12288, 1, False),
    ("narrow prefill (GEMV groups)", 100, [100], 128, 1024, 0, False),
]


@pytest.mark.parametrize("label,m,counts,n,k,post,fused", CASES, ids=[c[0] for c in CASES])
def test_linear_norm(q4k, oracle, gpu, label, m, counts, n, k, post, fused):
    rng = np.random.default_rng(1400 + m + n % 101)
    w = make_q4k(rng, n, k)
    W = q4k.Weight(w, n, k)
    x = make_x(rng, m, k, 3.0)
    x[0] *= 40.0  # a row far from the others' scale
    nw = _norm_weight(rng, k)
    aux = make_x(rng, m, n, 2.0) if post else None
    y = torch.from_numpy(aux).to(gpu) if post else torch.full((m, n), float("nan"), device=gpu)
    xt = torch.from_numpy(x).to(gpu)
    nwt = torch.from_numpy(nw).to(gpu)
    torch.cuda.synchronize()
    q4k.profile_enable(True)
    q4k.linear_norm(xt, W, nwt, m, y, auxiliary=y if post else None, gated=(post == 2), query_counts=counts)
    torch.cuda.synchronize()
    aux_n = _aux_launches(q4k)
    q4k.profile_enable(False)
    xn = oracle.rms_norm(x, nw)
    ref = oracle.linear(xn, w, n, k, aux=aux, post=post)
    got = y.cpu().numpy()
    assert np.all(np.isfinite(got))
    err = row_rel_err(got, ref)
    assert err <= TOL, f"{label}: {err:.3g}"
    assert aux_n == (0 if fused else 1), f"{label}: {aux_n} separate norm launches"


@pytest.mark.parametrize("t,m,n,k,post", [(TYPE_Q6_K, 300, 1024, 4096, 0), (TYPE_Q5_K, 130, 592, 2048, 1), (TYPE_Q8_0, 64, 512, 1024, 2),
                                          (TYPE_IQ4_XS, 200, 768, 2048, 0)])
def test_linear_norm_typed_prefill(q4k, oracle, gpu, t, m, n, k, post):
    """The other types' prefill GEMM with attn_norm folded into its staging
    (no separate norm launch)."""
    rng = np.random.default_rng(1470 + t + m)
    w = make_weight(rng, n, k, t)
    W = q4k.Weight(w, n, k, ggml_type=t)
    x = make_x(rng, m, k, 3.0)
    x[1] *= 25.0
    nw = _norm_weight(rng, k)
    aux = make_x(rng, m, n, 2.0) if post else None
    y = torch.from_numpy(aux).to(gpu) if post else torch.full((m, n), float("nan"), device=gpu)
    torch.cuda.synchronize()
    q4k.profile_enable(True)
    q4k.linear_norm(torch.from_numpy(x).to(gpu), W, torch.from_numpy(nw).to(gpu), m, y, auxiliary=y if post else None, gated=(post == 2),
                    query_counts=[m])
    torch.cuda.synchronize()
    aux_n = _aux_launches(q4k)
    q4k.profile_enable(False)
    ref = oracle.linear(oracle.rms_norm(x, nw), w, n, k, aux=aux, post=post, ggml_type=t)
    got = y.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert row_rel_err(got, ref) <= TOL
    assert aux_n == 0


def test_linear_norm_f16(q4k, oracle, gpu):
    rng = np.random.default_rng(1450)
    m, n, k = 130, 512, 2048
    w = make_q4k(rng, n, k)
    W = q4k.Weight(w, n, k)
    x = make_x(rng, m, k, 2.0).astype(np.float16)
    nw = _norm_weight(rng, k, 0.01)
    y = torch.empty((m, n), device=gpu, dtype=torch.float16)
    q4k.linear_norm(torch.from_numpy(x).to(gpu), W, torch.from_numpy(nw).to(gpu), m, y, query_counts=[m])
    torch.cuda.synchronize()
    ref = oracle.linear(oracle.rms_norm(x, nw).astype(np.float32), w, n, k)
    assert row_rel_err(y.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("m,counts", [(300, [300]), (40, [5] * 8), (12, [6, 6])])
def test_mlp_ffn_norm_in_staging(q4k, oracle, gpu, m, counts):
    """q4k_mlp with the layer's ffn_norm outside the fused decode GEMV: the
    gate and up projections share one staging of x that applies the norm;
    no separate norm launch runs."""
    k, n = 1024, 2048
    rng = np.random.default_rng(1460 + m)
    wg, wu, wd = make_q4k(rng, n, k), make_q4k(rng, n, k), make_q4k(rng, k, n)
    G, U, D = q4k.Weight(wg, n, k), q4k.Weight(wu, n, k), q4k.Weight(wd, k, n)
    h0 = make_x(rng, m, k, 3.0)
    nw = _norm_weight(rng, k, 0.05)
    hidden = torch.from_numpy(h0).to(gpu)
    gate = torch.empty((m, n), device=gpu)
    torch.cuda.synchronize()
    q4k.profile_enable(True)
    q4k.mlp(hidden, G, U, D, hidden, gate, m, query_counts=counts, norm_weight=torch.from_numpy(nw).to(gpu))
    torch.cuda.synchronize()
    aux_n = _aux_launches(q4k)
    q4k.profile_enable(False)
    g_gpu = gate.cpu().numpy()
    assert row_rel_err(g_gpu, oracle.mlp_gate_up(oracle.rms_norm(h0, nw), wg, wu, n, k)) <= TOL
    assert row_rel_err(hidden.cpu().numpy(), oracle.linear(g_gpu, wd, k, n, aux=h0, post=1)) <= TOL
    assert aux_n == 0
