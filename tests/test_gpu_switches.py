"""The library's routing switches, each in a process of its own.

Every routing rule of the library is a measured choice, and a few
environment variables switch a kernel family off or force a shape for
comparisons (split-K GEMV, fused gate/up, the GEMV shape and K-slices, the
GEMM tiling, the GEMM's K-segments and 192-column tiling, persistent grids
and tile order, the Q8_0 GEMM tiling, the typed GEMV forms).  The
library reads each once per process, so the default routing is all that the
rest of the suite reaches.  Here each setting runs tests/switch_child.py in a
child process with the variable set: the shapes whose routing the setting
changes are compared with the CPU oracle to the per-row bar, and where the
route shows in the kernel families' launch counts (a staging launch for the
staged GEMV, no fused launch for the two-call gate/up) that is checked too.
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))

SETTINGS = [
    ({"Q4K_GEMV_SPLITK": "-2"}, "splitk_off"),
    ({"Q4K_GEMV_GATE_UP": "0"}, "gate_up_off"),
    ({"Q4K_GEMV_ROWS": "0"}, "rows"),
    ({"Q4K_GEMV_ROWS": "2"}, "rows"),
    ({"Q4K_GEMV_ROWS_SLICES": "1"}, "rows"),
    ({"Q4K_GEMV_ROWS_SLICES": "3"}, "rows"),
    ({"Q4K_GEMV_GENERIC": "1"}, "gemv_generic"),
    ({"Q4K_GEMV_WAVES": "4", "Q4K_GEMV_TILES": "1"}, "gemv_shape"),
    ({"Q4K_GEMV_WAVES": "16", "Q4K_GEMV_TILES": "2"}, "gemv_shape"),
    ({"Q4K_GEMM_NARROW": "1"}, "gemm"),
    ({"Q4K_GEMM_NARROW": "0", "Q4K_GEMM2_SPLIT": "0", "Q4K_GEMM2_PERSIST": "0"}, "gemm"),
    ({"Q4K_GEMM_XCD_ROWS": "0"}, "gemm"),
    ({"Q4K_GEMM2_SPLIT_B": "3"}, "gemm"),
    ({"Q4K_GEMM_MID": "1"}, "gemm"),
    ({"Q4K_GEMM_MID": "0"}, "gemm"),
    ({"Q4K_TYPED_MID": "1"}, "typed_gemm"),
    ({"Q4K_TYPED_MID": "0"}, "typed_gemm"),
    ({"Q4K_TYPED_Q8W": "1"}, "typed_gemm"),
    ({"Q4K_TYPED_Q8W": "0"}, "typed_gemm"),
    ({"Q4K_GEMM_GATED_SIX": "1"}, "gated_six"),
    ({"Q4K_GEMM_GATED_SIX": "0"}, "gated_six"),
    ({"Q4K_GEMM_SIX": "1"}, "six"),
    ({"Q4K_GEMM_SIX": "0"}, "six"),
    ({"Q6K_GEMV_PERSISTENT": "1"}, "typed_gemv"),
    ({"Q6K_GEMV_PERSISTENT": "0", "Q6K_GEMV_TILES": "4"}, "typed_gemv"),
    ({"Q6K_GEMV_TILES": "2"}, "typed_gemv"),
    ({"Q4K_GEMV_PERSISTENT": "0"}, "q4k_persistent_off"),
]


@pytest.mark.parametrize("env,case", SETTINGS, ids=[",".join(f"{k}={v}" for k, v in e.items()) for e, _ in SETTINGS])
def test_switch(env, case, gpu):
    full = {k: v for k, v in os.environ.items() if not k.startswith(("Q4K_", "Q6K_"))}
    full.update(env)
    r = subprocess.run([sys.executable, "-u", os.path.join(HERE, "switch_child.py"), case], env=full, capture_output=True, text=True,
                       timeout=110)
    print(r.stdout[-2000:])
    assert r.returncode == 0, f"{env} {case}: exit {r.returncode}\n{r.stdout[-2000:]}\n{r.stderr[-3000:]}"
