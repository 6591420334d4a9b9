"""The C-ABI library without a GPU: it loads, exports every symbol include/q4k.h
declares, validates arguments before touching HIP, and its host helpers (layout,
phase selection, ragged packing) match the oracle and the reference tables."""
import ctypes
import os
import re

import numpy as np
import pytest

from q4k_ref import ROOT, make_q4k
from test_oracle import PHASE_CASES

HEADER = os.path.join(ROOT, "include", "q4k.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(q4k_\w+)\s*\(", text, re.M)))


def test_exports_every_declared_symbol(q4k):
    names = declared_symbols()
    assert len(names) >= 14
    raw = ctypes.CDLL(q4k.lib._name)
    for name in names:
        assert hasattr(raw, name), name


def test_header_compiles_as_c():
    import subprocess
    src = '#include "q4k.h"\nint main(void){return Q4K_OK;}\n'
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-I", os.path.join(ROOT, "include"),
                        "-x", "c", "-"], input=src, text=True, capture_output=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.parametrize("counts,gated,phase", PHASE_CASES)
def test_select_phase_matches_reference_table(q4k, counts, gated, phase):
    assert q4k.select_phase(counts, gated=gated) == phase


def test_select_phase_rejects_bad_tables(q4k):
    with pytest.raises(q4k.Q4KError) as e:
        q4k.select_phase([1, 2], m=4)
    assert e.value.code == -1
    with pytest.raises(q4k.Q4KError):
        q4k.select_phase([1] * 9)


def test_pack_queries_matches_oracle(q4k, oracle):
    rng = np.random.default_rng(0)
    for _ in range(50):
        nq = int(rng.integers(1, 9))
        counts = [int(c) for c in rng.integers(1, 600, nq)]
        samples = [int(min(c, s)) for c, s in zip(counts, rng.integers(0, 3, nq))]
        start, logit, rows, lrows = q4k.pack_queries(counts, samples)
        ostart, ologit, orows = oracle.pack(counts, samples)
        assert (start, logit, rows) == (ostart, ologit, orows)
        assert lrows == sum(samples)


def test_relayout_is_a_byte_permutation(q4k):
    rng = np.random.default_rng(1)
    n, k = 48, 768
    w = make_q4k(rng, n, k)
    t = q4k.relayout_host(w, n, k)
    assert np.array_equal(np.sort(t), np.sort(w.reshape(-1)))
    assert np.array_equal(q4k.unrelayout_host(t, n, k), w.reshape(-1))


def test_relayout_positions(q4k):
    """Spot-check the documented tile-block layout (q4k_internal.h)."""
    n, k = 32, 512
    nb = k // 256
    w = np.zeros((n, nb, 144), np.uint8)
    # Tag every byte with (row, block, offset) through a hash we can invert per position.
    rng = np.random.default_rng(2)
    w[:] = rng.integers(0, 256, w.shape, dtype=np.uint8)
    t = q4k.relayout_host(w, n, k).reshape(n // 16, nb, 2304)
    for c in range(n // 16):
        for b in range(nb):
            for i in range(16):
                row = 16 * c + i
                assert np.array_equal(t[c, b, 2048 + 16 * i: 2048 + 16 * i + 16], w[row, b, :16])
                for g in range(4):
                    for h in range(2):
                        lane = 16 * g + i
                        got = t[c, b, h * 1024 + 16 * lane: h * 1024 + 16 * lane + 16]
                        src = w[row, b, 16 + 32 * g + 16 * h: 16 + 32 * g + 16 * h + 16]
                        assert np.array_equal(got, src[[0, 2, 1, 3, 4, 6, 5, 7, 8, 10, 9, 11, 12, 14, 13, 15]])


def test_weight_validation_before_hip(q4k):
    w = np.zeros(16 * 144, np.uint8)
    with pytest.raises(q4k.Q4KError) as e:
        q4k.Weight(w, 16, 256, ggml_type=10)  # Q2_K: not served
    assert e.value.code == -2
    with pytest.raises(q4k.Q4KError) as e:
        q4k.Weight(w, 16, 256, ggml_type=14)  # Q6_K needs 210 bytes per block
    assert e.value.code == -3
    with pytest.raises(q4k.Q4KError) as e:
        q4k.Weight(w, 16, 255)
    assert e.value.code == -3
    with pytest.raises(q4k.Q4KError) as e:
        q4k.Weight(w[:100], 16, 256)
    assert e.value.code == -3
    with pytest.raises(q4k.Q4KError) as e:
        q4k.Weight(np.zeros(8 * 144, np.uint8), 8, 256)
    assert e.value.code == -3


def test_linear_validation_before_hip(q4k):
    lib = q4k.lib
    assert lib.q4k_linear(None, None, None, None, None, 1, None, 0, 0, 0) == -1
    assert b"weight" in lib.q4k_last_error()
    assert lib.q4k_mlp_gate_up(None, None, None, None, None, 1, None, 0, 0) == -1
    assert lib.q4k_weight_destroy(None) == 0


def test_neighbour_entry_points_validate_before_hip(q4k):
    """Argument errors of the embedding / RMS-norm entry points are reported
    before any HIP call (no GPU needed)."""
    lib = q4k.lib
    fake = ctypes.c_void_p(0x1000)
    u32 = ctypes.c_uint32
    assert lib.q4k_embedding(None, None, fake, 1, fake, 0) == -1
    one = (u32 * 1)(1)
    assert lib.q4k_embedding_batch(None, None, fake, 8, one, one, one, 1, fake, 0, None) == -1
    assert lib.q4k_rms_norm(None, None, fake, fake, 1, 16, ctypes.c_float(1e-6), 0) == -1
    assert lib.q4k_rms_norm(None, fake, fake, fake, 1, 16, ctypes.c_float(-1.0), 0) == -1
    assert lib.q4k_rms_norm(None, fake, fake, fake, 1, 0, ctypes.c_float(1e-6), 0) == -3
    assert lib.q4k_rms_norm(None, fake, fake, fake, 1, 16, ctypes.c_float(1e-6), 7) == -1
    # y partially overlapping x
    assert lib.q4k_rms_norm(None, ctypes.c_void_p(0x1000), fake, ctypes.c_void_p(0x1004), 2, 16, ctypes.c_float(1e-6), 0) == -4
    counts = (u32 * 2)(40, 40)
    samples = (u32 * 2)(40, 40)  # 80 sampled rows > 64
    assert lib.q4k_rms_norm_gather(None, fake, fake, ctypes.c_void_p(0x100000), 16, counts, samples, 2,
                                   ctypes.c_float(1e-6), 0, None) == -1
    assert "exceed" in lib.q4k_last_error().decode()


def test_ceiling_entry_points_validate_before_hip(q4k):
    """The measurement entry points refuse bad arguments before any HIP call."""
    lib = q4k.lib
    out = ctypes.c_double()
    assert lib.q4k_mfma_ceiling(None, 0, 0, ctypes.byref(out)) == -1
    assert lib.q4k_mfma_ceiling(None, 0, 10, None) == -1
    bufs = (ctypes.c_void_p * 2)(0x1000, 0x2008)  # the second is not 16-byte aligned
    assert lib.q4k_read_ceiling(None, 0, None, 1, 4096, 1, ctypes.byref(out)) == -1
    assert lib.q4k_read_ceiling(None, 0, bufs, 1, 4100, 1, ctypes.byref(out)) == -1  # not a multiple of 16
    assert lib.q4k_read_ceiling(None, 0, bufs, 1, 4096, 0, ctypes.byref(out)) == -1
    assert lib.q4k_read_ceiling(None, 0, bufs, 2, 4096, 1, ctypes.byref(out)) == -1
    assert "aligned" in lib.q4k_last_error().decode()
