"""Q8_0, Q5_K and IQ4_XS weights on the linear() surface against the CPU
oracle on identical seeded inputs (the Q6_K cases are in test_gpu_q6k.py).
Bar: max row-relative error 1e-3.  Q5_K products q * sc are exact in fp16;
Q8_0 rounds q * d and IQ4_XS rounds products above 2048 once to fp16 (as the
reference's prefill tiles round every dequantised weight), so their expected
errors are ~1e-4 and ~1e-6.

Per type: decode and small-prefill row counts; K from one block (waves 1..7
idle) to 48 blocks (six per wave) and 9 blocks (ragged per wave); ragged
column tails of the 4- and 2-tile workgroups; the persistent form at K = 4096
(16 * 4401 columns, one tile in the last item); post 1 / 2 in place in
decode and prefill (per-8-row groups); fp16 activations; the device-side
upload (bit-identical to the host one); the gated projection (one fused
launch for Q5_K and IQ4_XS in the decode phase, with and without the
ffn_norm); a GGUF file;
and, for every non-Q4_K type, prefill batches of 64 rows and more (the
typed MFMA GEMM): M = 2048, ragged row and column tails (a workgroup with
one live column tile, waves with none), one block of K, post 0 / 1 / 2 and
fp16 activations, and one-hot rows that read single dequantised weights
out, which must equal the oracle's fp32 value rounded to fp16 exactly.
"""
import numpy as np
import pytest
import torch

from gguf_writer import write_gguf
from q4k_ref import TYPE_IQ4_XS, TYPE_Q5_K, TYPE_Q8_0, make_weight, make_x, row_rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
TYPES = [TYPE_Q8_0, TYPE_Q5_K, TYPE_IQ4_XS]


def _t(a, dev, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dtype)


def _linear(q4k, oracle, gpu, t, seed, m, n, k, post=0, dtype=torch.float32, counts=None, device_upload=False):
    rng = np.random.default_rng(seed)
    w = make_weight(rng, n, k, t)
    x = make_x(rng, m, k)
    npdt = np.float16 if dtype == torch.float16 else np.float32
    xq = x.astype(npdt)
    aux = make_x(rng, m, n, 2.0).astype(npdt) if post else None
    W = q4k.Weight(torch.from_numpy(w).to(gpu) if device_upload else w, n, k, ggml_type=t)
    y = torch.full((m, n), float("nan"), device=gpu, dtype=dtype)
    auxt = None
    if post:
        y.copy_(_t(aux, gpu, dtype))
        auxt = y
    q4k.linear(_t(xq, gpu, dtype), W, m, y, auxiliary=auxt, gated=(post == 2), query_counts=counts)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    ref = oracle.linear(xq, w, n, k, aux=aux, post=post, ggml_type=t)
    assert np.all(np.isfinite(got))
    err = row_rel_err(got, ref)
    assert err <= TOL, f"type={t} m={m} n={n} k={k} post={post} {dtype}: rel err {err:.3g}"
    return W, got


SHAPES = [(1, 16, 256), (8, 48, 768), (2, 80, 2304), (5, 4096, 4096), (8, 1024, 12288), (2, 16 * 2049, 512),
          (1, 16 * 1025, 256), (3, 16 * 4401, 4096)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("t", TYPES)
def test_linear_store(q4k, oracle, gpu, t, m, n, k):
    _linear(q4k, oracle, gpu, t, 900 + m + k + t, m, n, k, counts=[1] * m)


@pytest.mark.parametrize("post", [1, 2])
@pytest.mark.parametrize("m,counts", [(8, [1] * 8), (20, [20])])
@pytest.mark.parametrize("t", TYPES)
def test_epilogues_in_place(q4k, oracle, gpu, t, post, m, counts):
    _linear(q4k, oracle, gpu, t, 910 + post + m + t, m, 1024, 4096, post=post, counts=counts)


@pytest.mark.parametrize("t", TYPES)
def test_fp16_and_kernel_names(q4k, oracle, gpu, t):
    W, _ = _linear(q4k, oracle, gpu, t, 920 + t, 8, 2048, 4096, post=1, dtype=torch.float16, counts=[8])
    name = {TYPE_Q8_0: "q8_0", TYPE_Q5_K: "q5_k", TYPE_IQ4_XS: "iq4_xs"}[t]
    assert W.kernel_name(2) == f"linear_{name}_k4096_n2048_prefill_small_mfma16x16x32"


@pytest.mark.parametrize("t", TYPES)
def test_device_upload_is_bit_identical(q4k, oracle, gpu, t):
    _, a = _linear(q4k, oracle, gpu, t, 930 + t, 8, 4096, 4096, counts=[1] * 8)
    _, b = _linear(q4k, oracle, gpu, t, 930 + t, 8, 4096, 4096, counts=[1] * 8, device_upload=True)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("m,counts", [(8, [1] * 8), (12, [12])])
@pytest.mark.parametrize("t", TYPES)
def test_gate_up(q4k, oracle, gpu, t, m, counts):
    n, k = 1536, 4096
    rng = np.random.default_rng(940 + m + t)
    wg, wu = make_weight(rng, n, k, t), make_weight(rng, n, k, t)
    x = make_x(rng, m, k, 0.5)
    G, U = q4k.Weight(wg, n, k, ggml_type=t), q4k.Weight(wu, n, k, ggml_type=t)
    gate = torch.full((m, n), float("nan"), device=gpu)
    q4k.mlp_gate_up(_t(x, gpu), G, U, m, gate, query_counts=counts)
    torch.cuda.synchronize()
    assert row_rel_err(gate.cpu().numpy(), oracle.mlp_gate_up(x, wg, wu, n, k, ggml_type=t)) <= TOL


FUSED_GATE_UP = [TYPE_Q5_K, TYPE_IQ4_XS]


@pytest.mark.parametrize("m,n,dtype", [(8, 12288, torch.float32), (1, 512, torch.float32), (3, 1536, torch.float16)])
@pytest.mark.parametrize("t", FUSED_GATE_UP)
def test_gate_up_fused_decode(q4k, oracle, gpu, t, m, n, dtype):
    """Q5_K / IQ4_XS gate and up in the decode phase run as one fused launch
    (fused_kernels.metal:80-200): three column tiles per workgroup at
    N = 12288, one at N = 512 and 1536; fp32 and fp16 activations."""
    k = 4096
    rng = np.random.default_rng(980 + m + t)
    wg, wu = make_weight(rng, n, k, t), make_weight(rng, n, k, t)
    # fp16: small enough that SiLU(gate) * up stays inside the fp16 range.
    x = make_x(rng, m, k, 0.01 if dtype == torch.float16 else 0.5)
    npdt = np.float16 if dtype == torch.float16 else np.float32
    xq = x.astype(npdt)
    G, U = q4k.Weight(wg, n, k, ggml_type=t), q4k.Weight(wu, n, k, ggml_type=t)
    gate = torch.full((m, n), float("nan"), device=gpu, dtype=dtype)
    xt = _t(xq, gpu, dtype)
    torch.cuda.synchronize()
    q4k.profile_enable(True)
    q4k.mlp_gate_up(xt, G, U, m, gate, query_counts=[1] * m)
    torch.cuda.synchronize()
    launches = [q4k.profile_query(kind)[0] for kind in (q4k.KERNEL_STAGE, q4k.KERNEL_GEMV, q4k.KERNEL_GEMV_GATED, q4k.KERNEL_AUX)]
    q4k.profile_enable(False)
    assert launches == [0, 0, 1, 0], launches
    assert G.kernel_name(q4k.PHASE_GATED_DECODE).startswith("mlp_")
    ref = oracle.mlp_gate_up(xq, wg, wu, n, k, ggml_type=t)
    assert row_rel_err(gate.float().cpu().numpy(), ref.astype(np.float32)) <= TOL


@pytest.mark.parametrize("t", FUSED_GATE_UP)
def test_gate_up_fused_with_ffn_norm(q4k, oracle, gpu, t):
    """q4k_mlp with the layer's ffn_norm over Q5_K / IQ4_XS gate and up in the
    decode phase: the norm runs inside the fused launch (no separate norm
    launch), then the down projection adds the residual in place."""
    m, n, k = 8, 1536, 4096
    rng = np.random.default_rng(990 + t)
    wg, wu, wd = make_weight(rng, n, k, t), make_weight(rng, n, k, t), make_weight(rng, k, n, t)
    h0 = make_x(rng, m, k, 3.0)
    nw = (1.0 + 0.2 * rng.standard_normal(k)).astype(np.float32)
    G, U, D = (q4k.Weight(w, r, c, ggml_type=t) for w, r, c in ((wg, n, k), (wu, n, k), (wd, k, n)))
    hidden = _t(h0, gpu)
    gate = torch.empty((m, n), device=gpu)
    torch.cuda.synchronize()
    q4k.profile_enable(True)
    q4k.mlp(hidden, G, U, D, hidden, gate, m, query_counts=[1] * m, norm_weight=_t(nw, gpu))
    torch.cuda.synchronize()
    gated, aux = q4k.profile_query(q4k.KERNEL_GEMV_GATED)[0], q4k.profile_query(q4k.KERNEL_AUX)[0]
    q4k.profile_enable(False)
    assert (gated, aux) == (1, 0), (gated, aux)
    g_gpu = gate.cpu().numpy()
    assert row_rel_err(g_gpu, oracle.mlp_gate_up(oracle.rms_norm(h0, nw), wg, wu, n, k, ggml_type=t)) <= TOL
    assert row_rel_err(hidden.cpu().numpy(), oracle.linear(g_gpu, wd, k, n, aux=h0, post=1, ggml_type=t)) <= TOL


@pytest.mark.parametrize("t", TYPES)
def test_tensor_from_gguf(q4k, oracle, gpu, tmp_path, t):
    n, k, m = 512, 4096, 8
    rng = np.random.default_rng(950 + t)
    w = make_weight(rng, n, k, t)
    path = tmp_path / "w.gguf"
    write_gguf(path, [("blk.0.ffn_down.weight", t, (k, n), w.tobytes())])
    with q4k.GGUFFile(path) as f:
        W = f.weight("blk.0.ffn_down.weight")
    assert (W.n, W.k, W.type) == (n, k, t)
    x = make_x(rng, m, k)
    y = torch.empty((m, n), device=gpu)
    q4k.linear(_t(x, gpu), W, m, y, query_counts=[m])
    torch.cuda.synchronize()
    assert row_rel_err(y.cpu().numpy(), oracle.linear(x, w, n, k, ggml_type=t)) <= TOL


# Prefill-sized batches (m >= 64) of the other types: x staged in the GEMM
# order (fp16, power-of-two row scales), the type's MFMA GEMM dequantising
# each weight to the reference's prefill tile value (fp16) in registers.  Like
# the Q4_K GEMM, activations and weights are single fp16 (expected row errors
# ~4e-4).  592 = 16 * 37 columns: the last workgroup has 5 live column tiles
# (one wave with a single tile, Q8_0's 2-tile waves: one with one) and
# waves with none.
ALL_TYPES = TYPES + [14]


@pytest.mark.parametrize("m,n,k", [(64, 1024, 4096), (97, 2048, 2304), (200, 4096, 12288), (2048, 768, 2048), (130, 592, 256),
                                   (300, 592, 1280)])
@pytest.mark.parametrize("t", ALL_TYPES)
def test_prefill_gemm(q4k, oracle, gpu, t, m, n, k):
    W, _ = _linear(q4k, oracle, gpu, t, 960 + m + t, m, n, k, counts=[m])
    assert W.kernel_name(1).endswith("_prefill_mfma16x16x32")


@pytest.mark.parametrize("m,n,k,post,dtype", [(2048, 4096, 512, 0, torch.float32), (2000, 4016, 768, 1, torch.float16)])
def test_prefill_gemm_q8_0_four_tiles(q4k, oracle, gpu, m, n, k, post, dtype):
    """Q8_0 grids where the four-column-tile form (B in half tile-blocks)
    takes fewer rounds than the three- and two-tile forms: 256 workgroups of
    256 columns; 4016 = 16 * 251 columns leave the last column block 11 live
    tiles (waves with 4, 4, 3 and none) and 2000 rows a partial row block."""
    _linear(q4k, oracle, gpu, 8, 995 + m, m, n, k, post=post, dtype=dtype, counts=[m])


@pytest.mark.parametrize("m,n,k,post,dtype", [(2048, 6144, 512, 0, torch.float32), (2000, 6128, 768, 1, torch.float16)])
@pytest.mark.parametrize("t", [12, 23])
def test_prefill_gemm_six_tiles(q4k, oracle, gpu, t, m, n, k, post, dtype):
    """Q4_K and IQ4_XS grids where six column tiles per wave (384 columns per
    workgroup) take fewer rounds than four: 256 workgroups against 384;
    6128 = 16 * 383 columns leave the last column block 23 live tiles (waves
    with 6, 6, 6 and 5) and 2000 rows a partial row block."""
    _linear(q4k, oracle, gpu, t, 985 + m + t, m, n, k, post=post, dtype=dtype, counts=[m])


@pytest.mark.parametrize("post,dtype", [(1, torch.float32), (2, torch.float32), (0, torch.float16), (1, torch.float16)])
@pytest.mark.parametrize("t", ALL_TYPES)
def test_prefill_gemm_epilogues(q4k, oracle, gpu, t, post, dtype):
    _linear(q4k, oracle, gpu, t, 970 + post + t, 128, 1024, 4096, post=post, dtype=dtype, counts=[100, 28])


@pytest.mark.parametrize("t", ALL_TYPES + [12])
def test_prefill_gemm_dequant_bit_exact(q4k, oracle, gpu, t):
    """Row r of x is one-hot at element r of block r % nb, so y[r, j] is the
    fp16 weight the GEMM formed for (j, that element) times 1: every element
    position of a block, over all blocks, in 592 columns (512 for Q4_K, whose
    pipelined GEMM takes N in multiples of 256)."""
    m, n, k = 256, 512 if t == 12 else 592, 2048
    nb = k // 256
    rng = np.random.default_rng(990 + t)
    w = make_weight(rng, n, k, t)
    cols = np.arange(m) + 256 * (np.arange(m) % nb)
    x = np.zeros((m, k), np.float32)
    x[np.arange(m), cols] = 1.0
    W = q4k.Weight(w, n, k, ggml_type=t)
    y = torch.full((m, n), float("nan"), device=gpu)
    q4k.linear(_t(x, gpu), W, m, y, query_counts=[m])
    torch.cuda.synchronize()
    bb = w.shape[1] // nb
    blocks = w.reshape(n, nb, bb)
    expect = np.empty((m, n), np.float32)
    for j in range(n):
        deq = np.concatenate([oracle.dequant_block(blocks[j, b], t) for b in range(nb)])
        expect[:, j] = deq[cols].astype(np.float16).astype(np.float32)
    got = y.cpu().numpy()
    assert np.all(np.isfinite(got))
    bad = np.argwhere(got != expect)  # exact (a zero weight may carry either sign)
    assert bad.size == 0, f"type={t}: {len(bad)} weights differ, first (row, col) {bad[:4].tolist()}"
