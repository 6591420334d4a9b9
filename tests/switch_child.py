"""One routing switch of the library, exercised in a process of its own.

The library reads each switch (an environment variable) once, on first use,
into a static, so a switch can only be exercised in a fresh process: the
parent test (test_gpu_switches.py) sets the variable and runs
``python switch_child.py CASE``.  The case runs the shapes whose routing the
switch changes, compares every output with the CPU oracle to the per-row bar,
checks the launch counts that show the non-default route ran where the route
is observable from the kernel families, and prints one line with the largest
error.  Exit status 0 means every check passed.
"""
import os
import sys

import numpy as np
import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import mtlqwen_amd as q4k  # noqa: E402
from q4k_ref import TYPE_IQ4_XS, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, Oracle, gated_prefill_arithmetic, make_weight, make_x, row_rel_err  # noqa: E402

TOL = 1e-3
dev = torch.device("cuda:0")
oracle = Oracle()
worst = []


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def launches(fn, family):
    q4k.profile_enable(True)
    fn()
    torch.cuda.synchronize()
    n = q4k.profile_query(family)[0]
    q4k.profile_enable(False)
    return n


def check_linear(m, n, k, t=TYPE_Q4_K, post=0, seed=0, family=None, expect=None):
    rng = np.random.default_rng(seed)
    w = make_weight(rng, n, k, t)
    x = make_x(rng, m, k)
    aux = make_x(rng, m, n) if post else None
    W = q4k.Weight(w, n, k, ggml_type=t)
    y = _t(aux) if post == 1 else torch.full((m, n), float("nan"), device=dev)
    run = lambda: q4k.linear(_t(x), W, m, y, auxiliary=y if post == 1 else None, query_counts=[1] * m if m <= 8 else [m])
    if family is None:
        run()
        torch.cuda.synchronize()
    else:
        got = launches(run, family)
        assert expect(got), f"{m}x{k}->{n}: {got} launches of family {family}"
    err = row_rel_err(y.cpu().numpy(), oracle.linear(x, w, n, k, aux=aux, post=post, ggml_type=t))
    worst.append(err)
    assert err <= TOL, (m, n, k, t, post, err)


def check_gate_up(m, n, k, t=TYPE_Q4_K, seed=0, family=None, expect=None):
    """Decode passes (m <= 8) to the per-row bar; prefill passes as the gated
    GEMM tests judge them: within 2e-4 of the float64 model of the
    reference's prefill arithmetic, and within the bar or no further from the
    oracle than that arithmetic is (rows where SiLU(gate) * up is
    ill-conditioned)."""
    rng = np.random.default_rng(seed)
    wg, wu = make_weight(rng, n, k, t), make_weight(rng, n, k, t)
    x = make_x(rng, m, k, 0.5)
    G, U = q4k.Weight(wg, n, k, ggml_type=t), q4k.Weight(wu, n, k, ggml_type=t)
    y = torch.full((m, n), float("nan"), device=dev)
    counts = [1] * m if m <= 8 else [m] if m > 48 else [5] * (m // 5) + ([m % 5] if m % 5 else [])
    run = lambda: q4k.mlp_gate_up(_t(x), G, U, m, y, query_counts=counts)
    if family is None:
        run()
        torch.cuda.synchronize()
    else:
        got = launches(run, family)
        assert expect(got), f"gate/up {m}x{k}->{n}: {got} launches of family {family}"
    out = y.cpu().numpy()
    ref = oracle.mlp_gate_up(x, wg, wu, n, k, ggml_type=t)
    err = row_rel_err(out, ref)
    worst.append(err)
    if m <= 8 or counts != [m]:
        assert err <= TOL, (m, n, k, t, err)
    else:
        assert t == TYPE_Q4_K
        model = gated_prefill_arithmetic(x, wg, wu, n, k)
        assert row_rel_err(out, model) <= 2e-4, (m, n, k, row_rel_err(out, model))
        assert err <= max(TOL, 1.05 * row_rel_err(model, ref)), (m, n, k, err)


def case_splitk_off():
    # K = 12288 decode without the split-K GEMV: the staged GEMV reads x staged
    # by a staging launch (the split-K GEMV packs x itself: no staging launch).
    for m in (1, 8):
        check_linear(m, 1024, 12288, post=1, seed=10 + m, family=q4k.KERNEL_STAGE, expect=lambda c: c >= 1)


def case_gate_up_off():
    # Decode gate/up without the fused kernels that pack x in registers: Q4_K
    # pairs take the staged gated GEMV (x staged by a staging launch), Q5_K
    # pairs the reference's two calls (no gated launch).
    check_gate_up(8, 1536, 4096, t=TYPE_Q4_K, seed=20, family=q4k.KERNEL_STAGE, expect=lambda c: c >= 1)
    check_gate_up(8, 1536, 4096, t=TYPE_Q5_K, seed=21, family=q4k.KERNEL_GEMV_GATED, expect=lambda c: c == 0)
    for t in (TYPE_Q4_K, TYPE_Q5_K):
        check_gate_up(3, 512, 4096, t=t, seed=30 + t)


def case_rows():
    # Decode passes of 17..48 fragment rows: gated pairs at N = 12288 and
    # plain projections (K = 4096 and 12288) with the rows GEMV off, forced
    # to a number of column tiles, or with its K-slices off or forced.
    for m in (40, 24):
        check_gate_up(m, 12288, 4096, seed=35 + m)
    # K = 12288 at N = 4096 takes three K-slices of four column tiles by
    # default; N = 8192 (128 column groups, 384 workgroups) only when forced.
    for m, n, k in ((40, 6144, 4096), (40, 4096, 12288), (24, 8192, 12288)):
        rng = np.random.default_rng(37 + k % 97 + n % 89)
        w = make_weight(rng, n, k, TYPE_Q4_K)
        x = make_x(rng, m, k)
        aux = make_x(rng, m, n)
        W = q4k.Weight(w, n, k)
        y = _t(aux)
        q4k.linear(_t(x), W, m, y, auxiliary=y, query_counts=[5] * (m // 5) + ([m % 5] if m % 5 else []))
        torch.cuda.synchronize()
        err = row_rel_err(y.cpu().numpy(), oracle.linear(x, w, n, k, aux=aux, post=1))
        worst.append(err)
        assert err <= TOL, (m, n, k, err)


def case_gemv_generic():
    # One-row-tile GEMVs with the run-time block count per wave.
    for m, n, k in ((1, 4096, 4096), (8, 2048, 2048), (5, 256, 1536)):
        check_linear(m, n, k, post=1, seed=40 + m)


def case_gemv_shape():
    # Forced GEMV shapes (waves per workgroup, column tiles per workgroup).
    for m, n, k in ((1, 4096, 4096), (8, 1024, 2048), (40, 2048, 4096), (24, 512, 1024)):
        check_linear(m, n, k, post=1, seed=50 + m)


def case_gemm():
    # Prefill GEMMs under the switch: plain (few tiles, and more tiles than
    # CUs), long K with few tiles (two K-segments by default; a forced split
    # point gives segments of 3 and nb - 3 blocks here), gated, and the
    # typed GEMM (Q6_K).
    check_linear(200, 1024, 4096, post=1, seed=60)
    check_linear(2048, 6144, 1024, post=1, seed=61)
    check_linear(200, 4096, 12288, seed=62)
    check_gate_up(160, 1024, 2048, seed=63)
    check_linear(64, 1024, 4096, t=TYPE_Q6_K, seed=64)


def case_gated_six():
    # The gated prefill GEMM with six B column tiles per wave (three gate and
    # three up tiles) forced, or never taken: last column blocks with 9 and 5
    # live output tiles (1296 = 16 * 81, 272 = 16 * 17: waves with 3, 3, 3,
    # none and 3, 2, none, none), K of one block, and a grid where the default
    # routing takes six tiles.
    check_gate_up(257, 1296, 2048, seed=94)
    check_gate_up(130, 272, 256, seed=95)
    check_gate_up(821, 6144, 1024, seed=96)


def case_six():
    # Plain GEMMs with six column tiles per wave forced, or never taken:
    # Q4_K with a last 384-column block of 17 live tiles (1040 = 16 * 65:
    # waves with 6, 6, 5, none) and one block of K, IQ4_XS with the residual
    # epilogue and a last block of 13 live tiles (592 = 16 * 37).
    check_linear(129, 1040, 256, seed=97)
    check_linear(300, 592, 1280, t=TYPE_IQ4_XS, post=1, seed=98)
    check_linear(200, 1536, 2048, post=1, seed=99)


def case_typed_gemm():
    # Q8_0 prefill GEMMs with two, three or four column tiles per wave:
    # ragged rows, a last column block with one live column tile (n = 592 is
    # 37 column tiles), with and without the residual epilogue, and K of one
    # block (the half tile-block ring's prologue and clamped loads).
    check_linear(300, 592, 1024, t=TYPE_Q8_0, post=1, seed=90)
    check_linear(129, 3072, 2048, t=TYPE_Q8_0, seed=91)
    check_linear(200, 1536, 512, t=TYPE_Q8_0, post=1, seed=92)
    check_linear(70, 512, 256, t=TYPE_Q8_0, seed=93)


def case_typed_gemv():
    # Q6_K decode GEMV forms (persistent or not, column tiles per workgroup).
    for m, n, k in ((8, 4096, 4096), (3, 1024, 2048), (1, 8192, 4096)):
        check_linear(m, n, k, t=TYPE_Q6_K, post=1, seed=70 + m)


def case_q4k_persistent_off():
    # The Q4_K LM-head shape (K = 4096, >= 16 column tiles per CU) without the
    # persistent GEMV.
    check_linear(8, 65536, 4096, seed=80)
    check_linear(2, 65536, 4096, post=1, seed=81)


CASES = {
    "splitk_off": case_splitk_off,
    "gate_up_off": case_gate_up_off,
    "rows": case_rows,
    "gemv_generic": case_gemv_generic,
    "gemv_shape": case_gemv_shape,
    "gemm": case_gemm,
    "typed_gemm": case_typed_gemm,
    "gated_six": case_gated_six,
    "six": case_six,
    "typed_gemv": case_typed_gemv,
    "q4k_persistent_off": case_q4k_persistent_off,
}

if __name__ == "__main__":
    name = sys.argv[1]
    env = {k: v for k, v in os.environ.items() if k.startswith(("Q4K_", "Q6K_"))}
    print(f"case {name} {env}", flush=True)
    CASES[name]()
    print(f"case {name}: {len(worst)} checks, max row error {max(worst):.3e}", flush=True)
