"""The path's neighbours in a pass on the GPU against the CPU oracle: the
Q4_K token embedding (embedding_q4_k, quant_linear.metal:572-591) and the RMS
norm / LM-head rms_norm_gather (native_ops.metal:6-40).

Bars: the embedding is bit-exact (fp32 products in the oracle's order, then
the same fp16 rounding); RMS norm within 1e-5 relative per element in fp32
(the sum of squares is reduced in a different order) and one fp16 ulp in
fp16.  The full-vocabulary case reads rows at the end of a 248,320-row table.
"""
import numpy as np
import pytest
import torch

from q4k_ref import make_q4k

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.to(dtype) if dtype is not None else t


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_embedding_bit_exact(q4k, oracle, gpu, dtype):
    n, k = 1008, 4096
    rng = np.random.default_rng(80)
    w = make_q4k(rng, n, k, dmax=2.0)
    T = q4k.Weight(w, n, k)
    ids = np.array([0, 1, 15, 16, 17, 511, 1007, 3, 3, -1, 1008, 999], np.int32)
    y = torch.full((len(ids), k), float("nan"), device=gpu, dtype=dtype)
    q4k.embedding(T, _t(ids, gpu), y)
    torch.cuda.synchronize()
    ref = oracle.embedding(w, n, k, ids, f16=dtype == torch.float16)
    got = y.cpu().numpy()
    assert np.array_equal(got.view(np.uint16 if dtype == torch.float16 else np.uint32),
                          ref.view(np.uint16 if dtype == torch.float16 else np.uint32))
    assert np.all(got[9:11] == 0)


def test_embedding_full_vocabulary(q4k, oracle, gpu):
    """A 248,320-row table (572 MB) built on the device; rows at both ends and
    in the middle against the oracle on those rows' bytes."""
    n, k = 248320, 4096
    rb = k // 256 * 144
    g = torch.Generator(device=gpu).manual_seed(81)
    raw = torch.randint(0, 256, (n, rb), dtype=torch.uint8, device=gpu, generator=g)
    # d, dmin = fp16 in [0, 0.01): overwrite the first 4 bytes of every block
    dd = (torch.rand((n, k // 256, 2), device=gpu, generator=g) * 0.01).half().view(torch.uint8)
    raw.view(n, k // 256, 144)[:, :, 0:4] = dd.view(n, k // 256, 4)
    T = q4k.Weight(raw.reshape(-1), n, k)
    ids = np.array([0, 248319, 124160, 248304, 77777, 15, 16, 248318], np.int32)
    y = torch.empty((len(ids), k), device=gpu)
    q4k.embedding(T, _t(ids, gpu), y)
    torch.cuda.synchronize()
    rows = raw[torch.from_numpy(ids.astype(np.int64)).to(gpu)].cpu().numpy()
    ref = oracle.embedding(rows.reshape(-1), len(ids), k, np.arange(len(ids), dtype=np.int32))
    assert np.array_equal(y.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_embedding_batch_resolves_rows_in_kernel(q4k, oracle, gpu, dtype):
    """A packed batch with config 3's lengths {512, 37, 1, 1, 200, 5, 1, 64}
    (821 rows) at random positions of random slots of a 9 x 1024 request
    token buffer: each row's token is found in the kernel (queryRow); the
    result equals the oracle's embedding of the oracle's row tokens bit for
    bit.  Then the entry point's shape checks."""
    n, k, capacity, nslots = 1008, 4096, 1024, 9
    rng = np.random.default_rng(82)
    w = make_q4k(rng, n, k, dmax=2.0)
    T = q4k.Weight(w, n, k)
    counts = [512, 37, 1, 1, 200, 5, 1, 64]
    positions = [int(rng.integers(0, capacity - c + 1)) for c in counts]
    slots = [int(s) for s in rng.permutation(nslots)[:len(counts)]]
    tokens = rng.integers(0, n, nslots * capacity).astype(np.int32)
    y = torch.full((sum(counts), k), float("nan"), device=gpu, dtype=dtype)
    rows = q4k.embedding_batch(T, _t(tokens, gpu), capacity, counts, positions, slots, y)
    torch.cuda.synchronize()
    assert rows == 821
    ids = np.array(oracle.embedding_tokens(counts, positions, slots, capacity, tokens)[:-1], np.int32)
    ref = oracle.embedding(w, n, k, ids, f16=dtype == torch.float16)
    got = y.cpu().numpy()
    view = np.uint16 if dtype == torch.float16 else np.uint32
    assert np.array_equal(got.view(view), ref.view(view))
    # A query running past the capacity, and no queries: refused before any launch.
    with pytest.raises(RuntimeError):
        q4k.embedding_batch(T, _t(tokens, gpu), capacity, [5], [capacity - 4], [0], y)
    with pytest.raises(RuntimeError):
        q4k.embedding_batch(T, _t(tokens, gpu), capacity, [], [], [], y)


def _norm_close(got, ref, f16):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    if f16:
        # one fp16 ulp of the reference value (subnormal floor 2^-24)
        ulp = np.maximum(np.abs(ref), 2.0**-14) * 2.0**-10
        return bool(np.all(np.abs(got - ref) <= ulp))
    return bool(np.all(np.abs(got - ref) <= 1e-5 * np.abs(ref) + 1e-30))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("m,k", [(8, 4096), (3, 1000), (40, 4096)])
def test_rms_norm(q4k, oracle, gpu, dtype, m, k):
    rng = np.random.default_rng(82 + m + k)
    x = (rng.standard_normal((m, k)) * 3).astype(np.float32)
    x[0] *= 1e3 if dtype == torch.float32 else 10
    w = rng.standard_normal(k).astype(np.float32)
    xh = x.astype(np.float16) if dtype == torch.float16 else x
    xt = _t(xh, gpu)
    y = torch.empty_like(xt)
    q4k.rms_norm(xt, _t(w, gpu), y)
    torch.cuda.synchronize()
    ref = oracle.rms_norm(xh, w)
    assert _norm_close(y.cpu().numpy(), ref, dtype == torch.float16)


def test_rms_norm_in_place_and_zero_row(q4k, oracle, gpu):
    rng = np.random.default_rng(83)
    x = rng.standard_normal((4, 4096)).astype(np.float32)
    x[2] = 0.0
    w = rng.standard_normal(4096).astype(np.float32)
    xt = _t(x, gpu)
    q4k.rms_norm(xt, _t(w, gpu), xt)
    torch.cuda.synchronize()
    got = xt.cpu().numpy()
    assert np.all(got[2] == 0)
    assert _norm_close(got, oracle.rms_norm(x, w), False)


@pytest.mark.parametrize("counts,samples", [
    ([512, 37, 1, 1, 200, 5, 1, 64], [1] * 8),        # config 3: each sequence's last prompt row
    ([5] * 8, [5] * 8),                              # config 2: every verify row
    ([3, 1, 4, 1], [0, 1, 2, 0]),                    # an intermediate chunk and a partial sample
])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_rms_norm_gather(q4k, oracle, gpu, counts, samples, dtype):
    k = 4096
    m = sum(counts)
    rng = np.random.default_rng(84 + m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal(k).astype(np.float32)
    xh = x.astype(np.float16) if dtype == torch.float16 else x
    out = torch.empty((sum(samples), k), device=gpu, dtype=dtype)
    rows = q4k.rms_norm_gather(_t(xh, gpu), _t(w, gpu), out, counts, samples)
    torch.cuda.synchronize()
    assert rows == sum(samples)
    ref = oracle.rms_norm(xh, w, src=oracle.logit_sources(counts, samples))
    assert _norm_close(out.cpu().numpy(), ref, dtype == torch.float16)
