"""Tensors uploaded from a GGUF file through the path, end to end: the token
embedding, the MLP's RMS norm and the fused gate/up + down projections of a
Qwen3.5-9B-shaped block (K = 4096, N = 12288) read from one model file, run
as the reference's decoder runs them for a decode pass of 8 sequences
(forward.cpp:114-119 after the embedding of :125), against the CPU oracle on
the same bytes.  Weights uploaded from the file and from host bytes give
bit-identical outputs."""
import numpy as np
import pytest
import torch

from gguf_writer import GGML_F32, GGML_Q4_K, STRING, U32, write_gguf
from q4k_ref import make_q4k, row_rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


def test_decode_block_from_gguf(q4k, oracle, gpu, tmp_path):
    k, n, vocab, m = 4096, 12288, 1024, 8
    rng = np.random.default_rng(96)
    emb = make_q4k(rng, vocab, k, dmax=0.05)
    wg, wu, wd = make_q4k(rng, n, k), make_q4k(rng, n, k), make_q4k(rng, k, n)
    norm = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    path = tmp_path / "block.gguf"
    write_gguf(path, [("token_embd.weight", GGML_Q4_K, (k, vocab), emb.tobytes()),
                      ("blk.0.ffn_norm.weight", GGML_F32, (k,), norm.tobytes()),
                      ("blk.0.ffn_gate.weight", GGML_Q4_K, (k, n), wg.tobytes()),
                      ("blk.0.ffn_up.weight", GGML_Q4_K, (k, n), wu.tobytes()),
                      ("blk.0.ffn_down.weight", GGML_Q4_K, (n, k), wd.tobytes())],
               [("general.architecture", STRING, "qwen35"), ("qwen35.embedding_length", U32, k)])
    ids = np.array([5, 1023, 0, 77, 5, 512, 300, 16], np.int32)
    with q4k.GGUFFile(path) as g:
        assert g.meta_int("qwen35.embedding_length") == k
        T = g.weight("token_embd.weight")
        G, U, D = (g.weight(f"blk.0.ffn_{p}.weight") for p in ("gate", "up", "down"))
        assert (T.n, T.k, G.n, G.k, D.n, D.k) == (vocab, k, n, k, k, n)
        w_norm = torch.from_numpy(g.data("blk.0.ffn_norm.weight").copy().view(np.float32)).to(gpu)
    hidden = torch.empty((m, k), device=gpu)
    q4k.embedding(T, torch.from_numpy(ids).to(gpu), hidden)
    x = torch.empty_like(hidden)
    q4k.rms_norm(hidden, w_norm, x)
    gate = torch.empty((m, n), device=gpu)
    q4k.mlp(x, G, U, D, hidden, gate, m, query_counts=[1] * m)
    torch.cuda.synchronize()

    h0 = oracle.embedding(emb, vocab, k, ids)
    x_ref = oracle.rms_norm(h0, norm)
    g_ref = oracle.mlp_gate_up(x.cpu().numpy(), wg, wu, n, k)
    assert row_rel_err(x.cpu().numpy(), x_ref) <= 1e-6
    assert row_rel_err(gate.cpu().numpy(), g_ref) <= TOL
    out_ref = oracle.linear(gate.cpu().numpy(), wd, k, n, aux=h0, post=1)
    assert row_rel_err(hidden.cpu().numpy(), out_ref) <= TOL

    # The same projection from host bytes: bit-identical.
    G2 = q4k.Weight(wg, n, k)
    U2 = q4k.Weight(wu, n, k)
    gate2 = torch.empty_like(gate)
    q4k.mlp_gate_up(x, G2, U2, m, gate2, query_counts=[1] * m)
    torch.cuda.synchronize()
    assert torch.equal(gate, gate2)
