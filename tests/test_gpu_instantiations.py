"""Every (K, N) pair of the reference's Q4_K instantiation table
(quant_linear.metal:593-618) through the phase it is instantiated for,
against the CPU oracle: decode (8 one-token queries; the +add pairs with the
residual epilogue, post 1), prefill_small (one query of 8 rows) and prefill
(one query of 96 rows).  K = 32768 has no split-K plan and takes the decode
pack plus the per-type GEMV in decode.  Bar: max row-relative error 1e-3."""
import numpy as np
import pytest
import torch

from q4k_ref import make_q4k, make_x, row_rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3

DECODE = [(4096, 1024, 0), (4096, 4096, 1), (12288, 4096, 1), (32768, 4096, 1), (4096, 8192, 0), (4096, 12288, 0)]
PREFILL = [(4096, 1024), (4096, 4096), (12288, 4096), (32768, 4096), (4096, 8192), (4096, 12288)]

_WEIGHTS = {}


def _weight(q4k, k, n):
    if (k, n) not in _WEIGHTS:
        rng = np.random.default_rng(1800 + k // 256 + n // 16)
        w = make_q4k(rng, n, k)
        _WEIGHTS[(k, n)] = (w, q4k.Weight(w, n, k))
    return _WEIGHTS[(k, n)]


def _check(q4k, oracle, gpu, k, n, m, counts, post, phase):
    w, W = _weight(q4k, k, n)
    rng = np.random.default_rng(1900 + m + k // 256 + n // 16)
    x = make_x(rng, m, k, 0.5)
    aux = make_x(rng, m, n, 2.0) if post else None
    y = torch.from_numpy(aux).to(gpu) if post else torch.full((m, n), float("nan"), device=gpu)
    q4k.linear(torch.from_numpy(x).to(gpu), W, m, y, auxiliary=y if post else None, query_counts=counts)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert row_rel_err(got, oracle.linear(x, w, n, k, aux=aux, post=post)) <= TOL
    assert phase in W.kernel_name(q4k.PHASE_NAMES.index(phase))


@pytest.mark.parametrize("k,n,post", DECODE, ids=[f"k{k}_n{n}{'_add' if p else ''}" for k, n, p in DECODE])
def test_decode(q4k, oracle, gpu, k, n, post):
    _check(q4k, oracle, gpu, k, n, 8, [1] * 8, post, "decode")


@pytest.mark.parametrize("k,n", PREFILL, ids=[f"k{k}_n{n}" for k, n in PREFILL])
def test_prefill_small(q4k, oracle, gpu, k, n):
    _check(q4k, oracle, gpu, k, n, 8, [8], 0, "prefill_small")


@pytest.mark.parametrize("k,n", PREFILL, ids=[f"k{k}_n{n}" for k, n in PREFILL])
def test_prefill(q4k, oracle, gpu, k, n):
    _check(q4k, oracle, gpu, k, n, 96, [96], 0, "prefill")
