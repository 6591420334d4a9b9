"""The GGUF reader of the C ABI (include/q4k.h q4k_gguf_*) without a GPU.

The reference reads model files through ggml's gguf_init_from_buffer
(model/qwen35/forward.cpp:12-23); ggml is not vendored and no other GGUF
implementation is installed here, so the reader is checked against files
written from the published format by tests/gguf_writer.py: round trips of
every metadata type, tensor table and data bytes, custom alignment, both
container versions, every truncation length of a small file, and targeted
corruptions (each must fail with Q4K_EFORMAT, never read out of range).
"""
import ctypes
import struct

import numpy as np
import pytest

from gguf_writer import (ARRAY, BOOL, F32, F64, GGML_F16, GGML_F32, GGML_Q4_K, GGML_Q6_K, I8, I16, I32, I64, STRING, U8, U16,
                         U32, U64, gguf_bytes, tensor_nbytes, write_gguf)
from q4k_ref import make_q4k

EFORMAT, ENOTFOUND, ETYPE, ESHAPE, EINVAL = -7, -8, -2, -3, -1


def _sample(rng):
    w = make_q4k(rng, 32, 512).reshape(-1)
    norm = rng.standard_normal(512).astype(np.float32)
    q6 = rng.integers(0, 256, tensor_nbytes(GGML_Q6_K, (256, 4)), dtype=np.uint8)
    f16 = rng.standard_normal(15).astype(np.float16)
    tensors = [("blk.0.ffn_gate.weight", GGML_Q4_K, (512, 32), w.tobytes()),
               ("blk.0.ffn_norm.weight", GGML_F32, (512,), norm.tobytes()),
               ("output.weight", GGML_Q6_K, (256, 4), q6.tobytes()),
               ("tiny.f16", GGML_F16, (5, 3), f16.tobytes())]
    meta = [("general.architecture", STRING, "qwen35"), ("qwen35.block_count", U32, 32), ("u8", U8, 200), ("i8", I8, -5),
            ("u16", U16, 65535), ("i16", I16, -300), ("i32", I32, -70000), ("u64", U64, 2**40), ("i64", I64, -(2**40)),
            ("f32", F32, 1.5), ("f64", F64, 2.5), ("flag", BOOL, True),
            ("tokens", ARRAY, (STRING, ["a", "bb", "ccc"])), ("ids", ARRAY, (U32, [1, 2, 3])),
            ("nested", ARRAY, (ARRAY, [(U16, [1, 2]), (U8, [7])]))]
    return tensors, meta


def test_round_trip(q4k, tmp_path):
    rng = np.random.default_rng(90)
    tensors, meta = _sample(rng)
    path = tmp_path / "m.gguf"
    write_gguf(path, tensors, meta)
    with q4k.GGUFFile(path) as g:
        assert (g.version, g.n_tensors, g.n_kv) == (3, 4, len(meta))
        assert g.data_offset % 32 == 0 and g.file_bytes == path.stat().st_size
        infos = g.tensors()
        for (name, gt, ne, payload), info in zip(tensors, infos):
            assert (info.name, info.ggml_type, info.shape) == (name, gt, ne)
            assert info.nbytes == len(payload) and info.file_offset % 32 == 0
            assert bytes(g.data(name)) == payload
            assert path.read_bytes()[info.file_offset:info.file_offset + info.nbytes] == payload
        assert g.find("output.weight") == 2
        assert g.meta_str("general.architecture") == "qwen35"
        for key, val in [("qwen35.block_count", 32), ("u8", 200), ("i8", -5), ("u16", 65535), ("i16", -300), ("i32", -70000),
                         ("u64", 2**40), ("i64", -(2**40)), ("flag", 1)]:
            assert g.meta_int(key) == val, key
        with pytest.raises(q4k.Q4KError) as e:
            g.find("blk.9.missing")
        assert e.value.code == ENOTFOUND and "missing weight" in e.value.message
        with pytest.raises(q4k.Q4KError) as e:
            g.meta_int("general.architecture")
        assert e.value.code == EINVAL
        with pytest.raises(q4k.Q4KError) as e:
            g.meta_str("nope")
        assert e.value.code == ENOTFOUND


@pytest.mark.parametrize("alignment", [64, 256])
def test_custom_alignment_and_version_2(q4k, tmp_path, alignment):
    rng = np.random.default_rng(91)
    tensors, meta = _sample(rng)
    path = tmp_path / "a.gguf"
    write_gguf(path, tensors, meta, version=2, alignment=alignment)
    with q4k.GGUFFile(path) as g:
        assert g.version == 2 and g.data_offset % alignment == 0
        for (name, _, _, payload), info in zip(tensors, g.tensors()):
            assert info.file_offset % alignment == 0 and bytes(g.data(name)) == payload


def test_unknown_ggml_type_is_listed_without_size(q4k, tmp_path):
    path = tmp_path / "u.gguf"
    write_gguf(path, [("odd", 99, (7,), b"\1" * 7), ("n", GGML_F32, (2,), struct.pack("<2f", 1, 2))])
    with q4k.GGUFFile(path) as g:
        odd, n = g.tensors()
        assert odd.ggml_type == 99 and odd.nbytes == 0 and n.nbytes == 8


def _open_rc(lib, path):
    h = ctypes.c_void_p()
    rc = lib.q4k_gguf_open(str(path).encode(), ctypes.byref(h))
    if rc == 0:
        lib.q4k_gguf_close(h)
    return rc


def test_every_truncation_fails_cleanly(q4k, tmp_path):
    rng = np.random.default_rng(92)
    tensors, meta = _sample(rng)
    blob = gguf_bytes(tensors, meta)
    path = tmp_path / "t.gguf"
    for n in list(range(0, 1200)) + list(range(1200, len(blob) - 1, 97)) + [len(blob) - 1]:
        path.write_bytes(blob[:n])
        rc = _open_rc(q4k.lib, path)
        assert rc == EFORMAT, (n, rc)
    path.write_bytes(blob)
    assert _open_rc(q4k.lib, path) == 0


def _patched(blob, at, fmt, value):
    b = bytearray(blob)
    struct.pack_into(fmt, b, at, value)
    return bytes(b)


def test_corruptions(q4k, tmp_path):
    ok = [("w", GGML_Q4_K, (256, 16), bytes(16 * 144))]
    blob = gguf_bytes(ok)
    path = tmp_path / "c.gguf"
    name_at = 24  # header: magic, version, two counts
    # (file, words of the expected message)
    cases = {
        "magic": (b"GGUX" + blob[4:], "magic"),
        "version 1": (_patched(blob, 4, "<I", 1), "version"),
        "tensor count": (_patched(blob, 8, "<Q", 2**62), "counts"),
        "metadata count": (_patched(blob, 16, "<Q", 2**40), "counts"),
        "name length": (_patched(blob, name_at, "<Q", 2**63), "truncated tensor info"),
        "zero dims": (_patched(blob, name_at + 9, "<I", 0), "dimensions"),
        "five dims": (_patched(blob, name_at + 9, "<I", 5), "dimensions"),
        "zero extent": (_patched(blob, name_at + 13, "<Q", 0), "bad dimension"),
        "partial block": (_patched(blob, name_at + 13, "<Q", 100), "whole blocks"),
        "misaligned offset": (_patched(blob, name_at + 13 + 16 + 4, "<Q", 8), "not aligned"),
        "past the end": (_patched(blob, name_at + 13 + 16 + 4, "<Q", 1 << 20), "past the end"),
        "bad alignment": (gguf_bytes(ok, [("general.alignment", U32, 48)]), "power of two"),
        "bad value type": (_bad_type(ok), "metadata value"),
        "duplicate name": (gguf_bytes(ok + ok), "duplicate"),
        "huge array": (_huge_array(ok), "metadata value"),
    }
    for what, (data, words) in cases.items():
        path.write_bytes(data)
        assert _open_rc(q4k.lib, path) == EFORMAT, what
        assert words in q4k.lib.q4k_last_error().decode(), (what, q4k.lib.q4k_last_error())
    assert _open_rc(q4k.lib, tmp_path / "absent.gguf") == ENOTFOUND


def _bad_type(tensors):
    blob = bytearray(gguf_bytes(tensors, [("k", U8, 1)]))
    at = 24 + 8 + 1  # after the key "k": its value type
    struct.pack_into("<I", blob, at, 13)
    return bytes(blob)


def _huge_array(tensors):
    blob = bytearray(gguf_bytes(tensors, [("a", ARRAY, (U32, [1]))]))
    at = 24 + 8 + 1 + 4 + 4  # key "a", value type, element type: the count
    struct.pack_into("<Q", blob, at, 2**61)
    return bytes(blob)


def test_weight_from_gguf_rejects_before_upload(q4k, tmp_path):
    rng = np.random.default_rng(93)
    tensors, meta = _sample(rng)
    tensors.append(("vec.q4k", GGML_Q4_K, (512,), bytes(2 * 144)))
    path = tmp_path / "w.gguf"
    write_gguf(path, tensors, meta)
    with q4k.GGUFFile(path) as g:
        # output.weight is Q6_K (served) but 4 rows: not a whole 16-row tile.
        for name, code in [("blk.0.ffn_norm.weight", ETYPE), ("tiny.f16", ETYPE), ("output.weight", ESHAPE),
                           ("vec.q4k", ESHAPE), ("nope", ENOTFOUND)]:
            with pytest.raises(q4k.Q4KError) as e:
                g.weight(name)
            assert e.value.code == code, name
