"""GGUF model files for the Q4_K path, over the C ABI's reader.

``GGUFFile`` mirrors what the reference takes from ggml's gguf context in
``loadWeights`` (model/qwen35/forward.cpp:12-23): the tensor table (name,
ggml type, shape with ne[0] fastest, byte range) over a read-only mapping of
the file.  ``GGUFFile.weight(name)`` uploads a Q4_K matrix as a ``Weight``
(n = ne[1] rows of k = ne[0]), the Weight loadWeights builds for the path.
"""
import ctypes
from collections import namedtuple

import numpy as np

from ._lib import check, lib

TensorInfo = namedtuple("TensorInfo", "name ggml_type shape file_offset nbytes")


class GGUFFile:
    """A GGUF file mapped read-only (close() or use as a context manager)."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        check(lib.q4k_gguf_open(str(path).encode(), ctypes.byref(h)))
        self._h = h
        ver, nt, nkv, off, size = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        check(lib.q4k_gguf_info(h, ctypes.byref(ver), ctypes.byref(nt), ctypes.byref(nkv), ctypes.byref(off), ctypes.byref(size)))
        self.version, self.n_tensors, self.n_kv = ver.value, nt.value, nkv.value
        self.data_offset, self.file_bytes = off.value, size.value

    @property
    def handle(self):
        if self._h is None:
            raise ValueError("GGUF file has been closed")
        return self._h

    def tensor(self, i):
        name = ctypes.create_string_buffer(1024)
        t, nd = ctypes.c_uint32(), ctypes.c_uint32()
        ne = (ctypes.c_uint64 * 4)()
        off, nbytes = ctypes.c_uint64(), ctypes.c_uint64()
        check(lib.q4k_gguf_tensor(self.handle, i, name, len(name), ctypes.byref(t), ctypes.byref(nd), ne, ctypes.byref(off),
                                  ctypes.byref(nbytes)))
        return TensorInfo(name.value.decode(), t.value, tuple(ne[:nd.value]), off.value, nbytes.value)

    def tensors(self):
        return [self.tensor(i) for i in range(self.n_tensors)]

    def find(self, name):
        i = ctypes.c_uint64()
        check(lib.q4k_gguf_find(self.handle, name.encode(), ctypes.byref(i)))
        return i.value

    def data(self, name):
        """The tensor's bytes as a read-only numpy uint8 view into the mapping
        (valid while the file is open)."""
        i = self.find(name)
        ptr, nbytes = ctypes.c_void_p(), ctypes.c_uint64()
        check(lib.q4k_gguf_tensor_data(self.handle, i, ctypes.byref(ptr), ctypes.byref(nbytes)))
        if nbytes.value == 0:
            return np.empty(0, np.uint8)
        buf = (ctypes.c_uint8 * nbytes.value).from_address(ptr.value)
        arr = np.frombuffer(buf, dtype=np.uint8)
        arr.flags.writeable = False
        return arr

    def meta_int(self, key):
        v = ctypes.c_int64()
        check(lib.q4k_gguf_meta_int(self.handle, key.encode(), ctypes.byref(v)))
        return v.value

    def meta_str(self, key, maxlen=1 << 16):
        buf = ctypes.create_string_buffer(maxlen)
        check(lib.q4k_gguf_meta_str(self.handle, key.encode(), buf, maxlen))
        return buf.value.decode()

    def weight(self, name, device=0):
        """Upload the Q4_K or Q6_K matrix ``name`` as a Weight (forward.cpp:18-21)."""
        from .linear import Weight
        h = ctypes.c_void_p()
        check(lib.q4k_weight_from_gguf(self.handle, name.encode(), int(device), ctypes.byref(h)))
        info = self.tensor(self.find(name))
        return Weight._from_handle(h, info.shape[1], info.shape[0], info.ggml_type, device)

    def close(self):
        if self._h is not None:
            check(lib.q4k_gguf_close(self._h))
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
