"""q4k_linear_noalloc (the entry point that allocates nothing) against
q4k_linear through the C ABI: the same kernels on the same inputs, so the
outputs must be identical, on two calls in a row (the second smaller) for
every kernel family the entry point reaches, Q4_K and the other weight
types' prefill GEMM; the library's workspace allocation count
(q4k_workspace_allocations) unchanged across every no-allocation call; a
capture of the entry point on shapes q4k_linear was never called with,
replayed several times; and its refusals."""
import ctypes

import numpy as np
import pytest
import torch

from q4k_ref import make_q4k, make_weight, make_x, TYPE_IQ4_XS, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0

pytestmark = pytest.mark.gpu


def _noalloc(q4k, x, w, m, y, aux=None, post=0, counts=None):
    counts = counts if counts is not None else [m]
    arr = (ctypes.c_uint32 * len(counts))(*counts)
    dt = q4k.DTYPE_F16 if x.dtype == torch.float16 else q4k.DTYPE_F32
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return q4k.lib.q4k_linear_noalloc(stream, w.handle, ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()),
                                      None if aux is None else ctypes.c_void_p(aux.data_ptr()), m, arr, len(counts), post, dt)


def _allocations(q4k):
    c = ctypes.c_uint64()
    assert q4k.lib.q4k_workspace_allocations(ctypes.byref(c)) == 0
    return c.value


# (label, n, k, first (m, counts), second (m, counts), post, dtype)
CASES = [
    ("split-K down (K=12288)", 4096, 12288, (8, [1] * 8), (3, [1] * 3), 1, torch.float32),
    ("persistent GEMV (wide N)", 65536, 4096, (8, [1] * 8), (2, [1] * 2), 0, torch.float32),
    ("staged GEMV (40 rows)", 4096, 4096, (40, [5] * 8), (20, [5] * 4), 0, torch.float32),
    ("rows GEMV in K-slices (K=12288)", 4096, 12288, (40, [5] * 8), (24, [4] * 6), 1, torch.float32),
    ("prefill GEMM", 4096, 4096, (300, [300]), (129, [129]), 2, torch.float32),
    ("prefill GEMM in two K-halves", 1024, 8192, (300, [300]), (129, [129]), 1, torch.float32),
    ("narrow prefill (GEMV groups)", 128, 1024, (100, [100]), (30, [30]), 0, torch.float32),
    ("fp16 prefill GEMM", 512, 2048, (200, [200]), (70, [70]), 1, torch.float16),
    ("fp16 decode GEMV", 1024, 2048, (8, [1] * 8), (5, [1] * 5), 0, torch.float16),
]


# The other weight types' prefill GEMM (and their per-8-row group GEMV below 64 rows).
TYPED_CASES = [
    ("Q6_K prefill GEMM", 1024, 4096, (300, [300]), (129, [129]), 1, torch.float32, TYPE_Q6_K),
    ("Q8_0 prefill GEMM", 592, 2048, (200, [200]), (64, [64]), 0, torch.float16, TYPE_Q8_0),
    ("Q5_K prefill GEMM then groups", 512, 2048, (130, [130]), (20, [20]), 2, torch.float32, TYPE_Q5_K),
    ("IQ4_XS prefill GEMM", 768, 1024, (256, [256]), (65, [65]), 0, torch.float32, TYPE_IQ4_XS),
]


@pytest.mark.parametrize("label,n,k,first,second,post,dtype,t", [c + (TYPE_Q4_K,) for c in CASES] + TYPED_CASES,
                         ids=[c[0] for c in CASES + TYPED_CASES])
def test_noalloc_matches_linear(q4k, gpu, label, n, k, first, second, post, dtype, t):
    rng = np.random.default_rng(1300 + n % 97 + k % 89)
    W = q4k.Weight(make_weight(rng, n, k, t), n, k, ggml_type=t)
    for m, counts in (first, second):
        x = torch.from_numpy(make_x(rng, m, k, 0.25)).to(gpu).to(dtype)
        aux0 = torch.from_numpy(make_x(rng, m, n, 0.5)).to(gpu).to(dtype) if post else None
        y_ref = aux0.clone() if post else torch.empty((m, n), device=gpu, dtype=dtype)
        q4k.linear(x, W, m, y_ref, auxiliary=y_ref if post else None, gated=(post == 2), query_counts=counts)
        y = aux0.clone() if post else torch.full((m, n), float("nan"), device=gpu, dtype=dtype)
        torch.cuda.synchronize()
        before = _allocations(q4k)
        rc = _noalloc(q4k, x, W, m, y, aux=y if post else None, post=post, counts=counts)
        assert rc == 0, q4k.lib.q4k_last_error().decode()
        torch.cuda.synchronize()
        assert _allocations(q4k) == before, f"{label} m={m}: the call allocated device memory"
        assert torch.equal(y, y_ref), f"{label} m={m}"


def test_noalloc_captures_on_fresh_shapes(q4k, gpu):
    """Captured in a HIP graph on shapes this process never passed to
    q4k_linear (whose workspace would have to grow, which the capture
    forbids): the capture succeeds, allocates nothing, and every replay --
    with eager work and a synchronisation between replays -- gives the
    output of q4k_linear called eagerly after the capture.  The split-K
    GEMV, the GEMM's K-segments and the rows GEMV's K-slices clear their
    counters with a fill kernel inside the graph."""
    rng = np.random.default_rng(1320)
    # The split-K GEMV (K = 12288), the GEMM in two K-segments and the staged
    # GEMV at K = 16640, a K no other test of this suite uses, and the rows
    # GEMV in three K-slices at N = 2048.
    cases = [(8192, 12288, 8, [1] * 8, 1), (1024, 16640, 200, [200], 1), (1536, 16640, 40, [5] * 8, 0), (2048, 12288, 40, [5] * 8, 1)]
    for n, k, m, counts, post in cases:
        W = q4k.Weight(make_q4k(rng, n, k), n, k)
        x = torch.from_numpy(make_x(rng, m, k, 0.25)).to(gpu)
        aux0 = torch.from_numpy(make_x(rng, m, n, 0.5)).to(gpu)
        y = aux0.clone()
        s = torch.cuda.Stream()
        torch.cuda.synchronize()
        before = _allocations(q4k)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            rc = _noalloc(q4k, x, W, m, y, aux=y if post else None, post=post, counts=counts)
        assert rc == 0, q4k.lib.q4k_last_error().decode()
        assert _allocations(q4k) == before
        y_ref = aux0.clone()
        q4k.linear(x, W, m, y_ref, auxiliary=y_ref if post else None, query_counts=counts)
        torch.cuda.synchronize()
        for rep in range(3):
            y.copy_(aux0)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, y_ref), f"n={n} k={k} m={m}: replay {rep}"
            _ = (aux0 * 2.0).sum().item()  # eager work between replays
        assert _allocations(q4k) >= before


def test_noalloc_refusals(q4k, gpu):
    rng = np.random.default_rng(1310)
    # Staging 8192 x 8192 activations exceeds the scratch.
    n, k, m = 256, 8192, 8192
    W = q4k.Weight(make_q4k(rng, n, k), n, k)
    x = torch.zeros((m, k), device=gpu)
    y = torch.zeros((m, n), device=gpu)
    rc = _noalloc(q4k, x, W, m, y)
    assert rc == -3
    assert "no-allocation scratch" in q4k.lib.q4k_last_error().decode()
    # The same for the other types' prefill GEMM.
    W6 = q4k.Weight(make_weight(rng, n, k, TYPE_Q6_K), n, k, ggml_type=TYPE_Q6_K)
    rc = _noalloc(q4k, x, W6, m, y)
    assert rc == -3 and "no-allocation scratch" in q4k.lib.q4k_last_error().decode()
    torch.cuda.synchronize()
