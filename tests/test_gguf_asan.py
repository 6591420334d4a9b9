"""The GGUF reader's parser built on its own with AddressSanitizer (host code
only, g++) and run over every truncation of a sample file and a set of byte
corruptions: any out-of-range read aborts the harness."""
import os
import shutil
import subprocess

import numpy as np
import pytest

from gguf_writer import gguf_bytes
from q4k_ref import ROOT
from test_gguf import _sample

HARNESS = r'''
#include <cstdio>
#include <cstdint>
#include "q4k.h"
int q4k_internal_fail(int code, const char*) { return code; }
extern "C" int q4k_weight_create(const void*, size_t, uint32_t, uint32_t, uint32_t, int, q4k_weight**) { return -5; }
int main(int argc, char** argv) {
  int opened = 0;
  for (int i = 1; i < argc; ++i) {
    q4k_gguf* g = nullptr;
    if (q4k_gguf_open(argv[i], &g) == 0) {
      ++opened;
      uint64_t n = 0;
      q4k_gguf_info(g, nullptr, &n, nullptr, nullptr, nullptr);
      for (uint64_t t = 0; t < n; ++t) {
        char name[256];
        uint64_t ne[4], off, bytes;
        uint32_t type, nd;
        const void* data;
        if (q4k_gguf_tensor(g, t, name, sizeof name, &type, &nd, ne, &off, &bytes) == 0 && q4k_gguf_tensor_data(g, t, &data, &bytes) == 0 &&
            bytes)
          (void)((const volatile uint8_t*)data)[bytes - 1];
      }
      q4k_gguf_close(g);
    }
  }
  printf("opened %d of %d\n", opened, argc - 1);
  return 0;
}
'''


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_parser_under_asan(tmp_path):
    src = tmp_path / "h.cpp"
    src.write_text(HARNESS)
    exe = tmp_path / "h"
    r = subprocess.run(["g++", "-std=c++17", "-g", "-O1", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                        "-I", os.path.join(ROOT, "include"), str(src), os.path.join(ROOT, "mtlqwen_amd", "csrc", "q4k_gguf.cpp"),
                        "-o", str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    tensors, meta = _sample(np.random.default_rng(94))
    blob = gguf_bytes(tensors, meta)
    files = []
    for n in range(0, 1300, 3):
        p = tmp_path / f"t{n}.gguf"
        p.write_bytes(blob[:n])
        files.append(str(p))
    rng = np.random.default_rng(95)
    for i in range(300):
        b = bytearray(blob[:1300])
        for _ in range(4):
            b[int(rng.integers(0, len(b)))] = int(rng.integers(0, 256))
        p = tmp_path / f"c{i}.gguf"
        p.write_bytes(bytes(b))
        files.append(str(p))
    full = tmp_path / "full.gguf"
    full.write_bytes(blob)
    files.append(str(full))
    r = subprocess.run([str(exe), *files], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    assert r.stdout.startswith("opened")
