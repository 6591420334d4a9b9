"""Every gfx950 kernel of the library keeps its working set in registers and
LDS: compiled with the backend's resource remarks, no kernel reports private
(scratch) memory or spilled vector registers (scalar spills go to VGPR lanes,
not memory, and are allowed).  A private array the compiler fails to
promote lands in scratch (or silently in LDS) and slows the GEMVs several-fold
without changing their results, so parity tests cannot see it.  Runs on the
CPU (hipcc cross-compiles); skipped where hipcc is absent."""
import os
import re
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _remarks(tmp_path):
    sys.path.insert(0, os.path.join(ROOT, "mtlqwen_amd"))
    import build  # the package's own build recipe (flags)
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    out = {}
    for src in ("q4k_kernels.hip", "q4k_api.hip"):
        cmd = [hipcc, *build.HIPCC_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c",
               os.path.join(ROOT, "mtlqwen_amd", "csrc", src), "-o", str(tmp_path / (src + ".o"))]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        name = None
        for line in r.stderr.splitlines():
            m = re.search(r"Function Name: (\S+)", line)
            if m:
                name = m.group(1)
                out[name] = {}
                continue
            m = re.search(r"remark: +(ScratchSize \[bytes/lane\]|VGPRs Spill|SGPRs Spill): (\d+)", line)
            if m and name:
                out[name][m.group(1)] = int(m.group(2))
    return out


def test_no_kernel_uses_scratch_or_spills(tmp_path):
    res = _remarks(tmp_path)
    assert len(res) > 20
    bad = {k: v for k, v in res.items() if any(v.get(f, 0) for f in ("ScratchSize [bytes/lane]", "VGPRs Spill"))}
    assert not bad, bad
