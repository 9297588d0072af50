"""CPU check of the compiled kernels (gfx950 assembly from hipcc, no GPU).

No kernel may contain a loop that holds a barrier and leaves through an
exec-mask exit: the lanes of a wave could then run different iterations
around one barrier instance (tests/asm_barrier_scan.py).  This is the shape
that hung the persistent layer kernel before its ticket and plan values were
made scalar; the check runs on every kernel source of the library.

Every L2 write-back of a release (buffer_wbl2) is waited for (s_waitcnt
vmcnt(0)) before the next atomic publishes the stores it covers: without that
wait a consumer on another XCD can see the counter before the data.  The
compiler's own release sequence in the persistent kernel lacked the wait.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from tests.asm_barrier_scan import scan

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "altxs_amd", "csrc")


_ASM: dict[str, str] = {}


def _asm(src: str, tmp_path) -> str:
    """gfx950 assembly of one source (compiled once per test session)."""
    from altxs_amd.build import common_flags, hipcc

    if src in _ASM:
        return _ASM[src]
    out = os.path.join(str(tmp_path), os.path.basename(src) + ".s")
    cmd = [hipcc(), *common_flags(), "--cuda-device-only", "-S", os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    _ASM[src] = open(out).read()
    return _ASM[src]


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


def _wbl2_unwaited(asm: str) -> list[int]:
    """Lines of buffer_wbl2 instructions not followed by s_waitcnt vmcnt(0)
    before the next atomic or the end of the block."""
    lines = asm.splitlines()
    bad = []
    for i, ln in enumerate(lines):
        if "buffer_wbl2" not in ln:
            continue
        ok = False
        for nxt in lines[i + 1:]:
            t = nxt.strip()
            if t.startswith("s_waitcnt") and "vmcnt(0)" in t:
                ok = True
                break
            if "atomic" in t or t.startswith(".LBB") or t.startswith("s_endpgm") or t.startswith("s_branch"):
                break
        if not ok:
            bad.append(i + 1)
    return bad


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not installed")
def test_release_write_back_is_waited_for(tmp_path):
    asm = _asm("persist.hip", tmp_path)
    assert asm.count("buffer_wbl2") >= 36  # one release per roles_kernel variant
    assert not _wbl2_unwaited(asm)
