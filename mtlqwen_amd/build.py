"""Compiles the HIP sources of the Q4_K path into mtlqwen_amd/libq4k.so (gfx950).

hipcc is driven directly, one object per source in parallel, then one link.
The library is built in-tree so it travels with the repository snapshot.
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libq4k.so")
SOURCES = ["q4k_kernels.hip", "q4k_api.hip", "q4k_gguf.cpp"]
ARCH = os.environ.get("Q4K_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: no v_pk_*_f32 in device code (the host pass warns that it
# does not know the feature; that warning is harmless).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc():
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found; the Q4_K HIP library cannot be built")
    return exe


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build(verbose=False):
    """Compile every HIP source and link libq4k.so.  Always rebuilds."""
    os.makedirs(BUILD, exist_ok=True)
    hipcc = _hipcc()
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=len(cmds)) as pool:
        list(pool.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_oracle(verbose=False):
    """Build the CPU oracle (test infrastructure) with its own Makefile."""
    root = os.path.dirname(HERE)
    _run(["make", "-s", "-B", "-C", os.path.join(root, "oracle")], verbose)
    return os.path.join(root, "oracle", "_build", "libq4k_oracle.so")


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
