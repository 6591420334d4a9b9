"""Writes GGUF files for the reader's tests (test infrastructure), following
the published GGUF container format: "GGUF", u32 version, u64 tensor count,
u64 metadata count, metadata (string key, u32 type, value), tensor infos
(string name, u32 n_dims, u64 ne[], u32 ggml type, u64 data offset), padding
to general.alignment (default 32), the data section."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q", I64: "<q",
           F64: "<d"}

GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K, GGML_IQ4_XS = 0, 1, 8, 12, 13, 14, 23
BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_Q8_0: (32, 34), GGML_Q4_K: (256, 144), GGML_Q5_K: (256, 176),
         GGML_Q6_K: (256, 210), GGML_IQ4_XS: (256, 136)}


def _str(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_value(et, x) for x in items)
    return struct.pack(_SCALAR[t], v)


def tensor_nbytes(ggml_type, ne):
    be, bb = BLOCK[ggml_type]
    n = int(np.prod(ne))
    return n // be * bb


def gguf_bytes(tensors, meta=(), version=3, alignment=None, offsets=None):
    """tensors: [(name, ggml_type, ne (ne[0] fastest), data bytes)];
    meta: [(key, type, value)].  offsets overrides the data offsets."""
    meta = list(meta)
    if alignment is not None:
        meta.append(("general.alignment", U32, alignment))
    align = alignment or 32
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    for key, t, v in meta:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    data = b""
    infos = b""
    for i, (name, gt, ne, payload) in enumerate(tensors):
        if len(data) % align:
            data += b"\0" * (align - len(data) % align)
        off = len(data) if offsets is None else offsets[i]
        infos += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        infos += struct.pack("<IQ", gt, off)
        data += bytes(payload)
    body = head + infos
    pad = (-len(body)) % align
    return body + b"\0" * pad + data


def write_gguf(path, tensors, meta=(), version=3, alignment=None, offsets=None):
    blob = gguf_bytes(tensors, meta, version, alignment, offsets)
    with open(path, "wb") as f:
        f.write(blob)
    return blob
