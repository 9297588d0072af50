"""altxs_step_noalloc (workspace in the library's static device scratch)
against altxs_step (caller workspace), through the C-ABI.

Two calls in a row, the second with a smaller input (fewer segments and a
narrower window), each compared bit for bit with altxs_step on its own state
built the same way: logits, probabilities, integer CDFs, the KV cache the
step wrote, and the committed positions.  A step too large for the scratch is
rejected on the host before anything is enqueued.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(int(torch.cuda.current_stream().cuda_stream))


def _run(model, st, toks, noalloc: bool) -> None:
    from altxs_amd import _lib

    L = _lib.load()
    for t in range(toks.shape[1] // st.win):
        st.token.copy_(torch.from_numpy(toks[:, t * st.win:(t + 1) * st.win].astype(np.int32)))
        d = st._desc(_lib.F_COMMIT)
        if noalloc:
            rc = L.altxs_step_noalloc(ctypes.byref(d), _stream())
            _lib.check(rc, "altxs_step_noalloc")
        else:
            rc = L.altxs_step(ctypes.byref(d), _stream())
            _lib.check(rc, "altxs_step")


def _compare(profile: str, act: str, batch: int, win: int, steps: int, seed: int) -> None:
    from altxs_amd import synth
    from altxs_amd.config import make_config
    from altxs_amd.model import StepModel

    cfg = make_config(profile)
    model = StepModel(synth.make_model(cfg, std=0.02, softcap=(30.0, 24.0)), act=act)
    toks = synth.zipf_tokens(cfg.vocab_size, (batch, win * steps), seed=seed)
    ref = model.make_static_state(256, win=win, batch=batch)
    got = model.make_static_state(256, win=win, batch=batch)
    got.logits.fill_(float("nan"))
    _run(model, ref, toks, noalloc=False)
    _run(model, got, toks, noalloc=True)
    torch.cuda.synchronize()
    ref.check_errors()
    got.check_errors()
    for name in ("logits", "probs", "cum", "kv", "pos", "prev_raw"):
        a, b = getattr(ref, name), getattr(got, name)
        assert torch.equal(a.view(torch.uint8) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.uint8) if b.dtype == torch.bfloat16 else b), name


def test_noalloc_matches_step_two_calls_second_smaller():
    from altxs_amd import _lib

    assert "altxs_step_noalloc" in _lib.EXPORTS
    _log("noalloc: cfg3 bf16 B=16 W=4 x 3 windows")
    _compare("cfg3", "bf16", batch=16, win=4, steps=3, seed=11)
    _log("noalloc: cfg3 bf16 B=2 W=1 x 5 rows (smaller input, same scratch)")
    _compare("cfg3", "bf16", batch=2, win=1, steps=5, seed=12)
    _log("noalloc: cfg1 fp32 B=3 W=2 x 2 windows")
    _compare("cfg1", "fp32", batch=3, win=2, steps=2, seed=13)


def test_noalloc_rejects_oversized_and_persistent_on_host():
    from altxs_amd import _lib, synth
    from altxs_amd.config import make_config
    from altxs_amd.model import StepModel

    _log("noalloc: host-side rejections")
    L = _lib.load()
    cfg = make_config("cfg1")
    model = StepModel(synth.make_model(cfg, std=0.02), act="bf16")
    st = model.make_static_state(256, win=1, batch=2)
    d = _lib.StepDesc.from_buffer_copy(st._desc(0))
    d.W = 4096  # 8192 rows: far more workspace than the scratch holds (never enqueued)
    need = L.altxs_step_workspace_bytes(ctypes.byref(d))
    assert need > _lib.STEP_SCRATCH_BYTES
    rc = L.altxs_step_noalloc(ctypes.byref(d), _stream())
    assert rc == -1 and b"static scratch" in L.altxs_last_error()
    d = _lib.StepDesc.from_buffer_copy(st._desc(0))
    d.plan_dev = ctypes.c_void_p(16)  # any non-NULL plan is refused before use
    rc = L.altxs_step_noalloc(ctypes.byref(d), _stream())
    assert rc == -1 and b"persistent" in L.altxs_last_error()
