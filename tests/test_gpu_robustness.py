"""Host-side guards of the C ABI on the GPU: graph capture that would need
workspace growth, and mis-sized tensors handed to the Python wrappers."""
import ctypes

import numpy as np
import pytest
import torch

from q4k_ref import make_q4k, make_x, row_rel_err

pytestmark = pytest.mark.gpu


def test_capture_needing_workspace_growth(q4k, oracle, gpu):
    """A call whose workspace must grow is refused inside a stream capture
    (Q4K_ECAPTURE, nothing enqueued); after one eager call of the shape the
    same call captures, and every replay matches the eager result."""
    rng = np.random.default_rng(1200)
    # Staging for 8192 x 8192 activations (128 MiB of fp16) exceeds what any
    # other test of this suite grows the workspace to.
    m, n, k = 8192, 256, 8192
    w = make_q4k(rng, n, k)
    W = q4k.Weight(w, n, k)
    x = torch.from_numpy(make_x(rng, m, k)).to(gpu)
    y = torch.empty((m, n), device=gpu)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(q4k.Q4KError) as e:
        with torch.cuda.graph(g, stream=s):
            q4k.linear(x, W, m, y, query_counts=[m])
    assert e.value.code == q4k.ECAPTURE and "capturing" in e.value.message
    torch.cuda.synchronize()
    # Eager call of the shape grows the workspace; the capture then succeeds.
    q4k.linear(x, W, m, y, query_counts=[m])
    torch.cuda.synchronize()
    eager = y.clone()
    rows = np.arange(0, m, 97)
    assert row_rel_err(eager.cpu().numpy()[rows], oracle.linear(x.cpu().numpy()[rows], w, n, k)) <= 1e-3
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=s):
        q4k.linear(x, W, m, y, query_counts=[m])
    for _ in range(3):
        y.fill_(float("nan"))
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)


def test_wrapper_size_checks(q4k, gpu):
    """The wrappers check element counts and devices before handing raw
    pointers to the library."""
    n, k = 256, 256
    W = q4k.Weight(make_q4k(np.random.default_rng(1210), n, k), n, k)
    G, U = q4k.Weight(make_q4k(np.random.default_rng(1211), n, k), n, k), q4k.Weight(make_q4k(np.random.default_rng(1212), n, k), n, k)
    D = q4k.Weight(make_q4k(np.random.default_rng(1213), k, n), k, n)
    x = torch.randn(4, k, device=gpu)
    with pytest.raises(ValueError):
        q4k.linear(x, W, 4, torch.empty(3, n, device=gpu))
    with pytest.raises(ValueError):
        q4k.linear(x[:3], W, 4, torch.empty(4, n, device=gpu))
    with pytest.raises(ValueError):
        q4k.linear(x, W, 4, torch.empty(4, n, device=gpu), auxiliary=torch.empty(2, n, device=gpu))
    with pytest.raises(ValueError):
        q4k.mlp_gate_up(x, G, U, 4, torch.empty(4, n - 1, device=gpu))
    with pytest.raises(ValueError):
        q4k.mlp(x, G, U, D, torch.empty(3, k, device=gpu), torch.empty(4, n, device=gpu), 4)
    with pytest.raises(ValueError):
        q4k.gather_rows(x, torch.empty(1, k, device=gpu), [2, 2], [1, 1])
    with pytest.raises(ValueError):
        q4k.linear(x.cpu(), W, 4, torch.empty(4, n, device=gpu))
    # Correctly sized calls still go through.
    y = torch.empty(4, n, device=gpu)
    q4k.linear(x, W, 4, y)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()


def test_embedding_batch_slot_index_wrap_refused(q4k, gpu):
    """A slot whose (slot + 1) * capacity does not fit the token buffer's
    32-bit index (here slot 0xFFFFFFFF, where slot + 1 wraps to 0 in 32-bit
    arithmetic) is refused with Q4K_ESHAPE before any launch; a valid slot
    in the same call shape goes through."""
    W = q4k.Weight(make_q4k(np.random.default_rng(1214), 64, 256), 64, 256)
    tokens = torch.zeros(16, dtype=torch.int32, device=gpu)
    y = torch.zeros((1, 256), device=gpu)
    u32 = ctypes.c_uint32
    one, zero = (u32 * 1)(1), (u32 * 1)(0)
    for slot, cap in ((0xFFFFFFFF, 8), (0x7FFFFFFF, 2), (0x10000000, 8)):
        rc = q4k.lib.q4k_embedding_batch(None, W.handle, ctypes.c_void_p(tokens.data_ptr()), cap, one, zero, (u32 * 1)(slot), 1,
                                         ctypes.c_void_p(y.data_ptr()), 0, None)
        assert rc == -3, (slot, cap, rc)
        assert "32-bit" in q4k.lib.q4k_last_error().decode()
    rows = q4k.embedding_batch(W, tokens, 8, [1], [0], [1], y)
    torch.cuda.synchronize()
    assert rows == 1 and torch.isfinite(y).all()
