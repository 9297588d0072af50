"""CPU check of the compiled kernels (gfx950 assembly from hipcc, no GPU).

No kernel may contain a loop that holds a barrier and leaves through an
exec-mask exit: the lanes of a wave could then run different iterations
around one barrier instance (tests/asm_barrier_scan.py).  This is the shape
that hung the persistent layer kernel before its ticket and plan values were
made scalar; the check runs on every kernel source of the library.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from tests.asm_barrier_scan import scan

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "altxs_amd", "csrc")


def _asm(src: str, tmp_path) -> str:
    from altxs_amd.build import common_flags, hipcc

    out = os.path.join(str(tmp_path), os.path.basename(src) + ".s")
    cmd = [hipcc(), *common_flags(), "--cuda-device-only", "-S", os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return open(out).read()


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not installed")
@pytest.mark.parametrize("src", ["persist.hip", "step.hip", "attn.hip", "qgemm.hip", "cdf.hip"])
def test_no_divergent_loop_around_barriers(src, tmp_path):
    rep = scan(_asm(src, tmp_path))
    assert rep, f"no kernels found in {src}"
    bad = {k: v for k, v in rep.items() if v}
    assert not bad, f"divergent loops holding barriers: {bad}"
    if src == "persist.hip":
        assert sum("roles_kernel" in k for k in rep) == 36  # every (act, G, KS_o, KS_d) variant
