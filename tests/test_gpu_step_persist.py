"""GPU: the persistent layer kernel (every slot of the step in one launch,
tasks taken in dependency order) against the per-stage launches.

Each task runs the same tile computation as the per-stage kernels, so logits
and integer CDFs must be bit-identical -- for decode rows and encode windows,
ragged batches (row tiles that are partly empty), positions that differ per
segment, both activation modes, and graph replays.  A descriptor that no
longer matches its plan is rejected with ALTXS_ERR_ARG.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

_MODELS: dict = {}


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def _synth(profile):
    if profile not in _MODELS:
        from altxs_amd import synth
        from altxs_amd.config import make_config

        std, cap = {"tiny": (0.08, (2.0, 1.5)), "cfg1": (0.02, (30.0, 24.0)),
                    "cfg3": (0.02, (30.0, 24.0)), "tiny_lora": (0.08, (2.0, 1.5))}[profile]
        cfg = (make_config("tiny", lora_rank=8, lora_alpha=12.0) if profile == "tiny_lora"
               else make_config(profile))
        _MODELS[profile] = synth.make_model(cfg, std=std, softcap=cap)
    return _MODELS[profile]


def _run_steps(sm, act, W, toks, persistent, max_len=256):
    from altxs_amd.model import StepModel

    B, T = toks.shape
    model = StepModel(sm, act=act, kv="bf16")
    st = model.make_static_state(max_len, win=W, batch=B, persistent=persistent)
    lg, cm = [], []
    for w0 in range(0, T, W):
        st.token.copy_(torch.from_numpy(toks[:, w0:w0 + W].astype(np.int32)))
        model.step(st, commit=True)
        lg.append(st.logits.cpu().clone())
        cm.append(st.cum.cpu().clone())
    torch.cuda.synchronize()
    st.check_errors()
    return torch.stack(lg), torch.stack(cm), st.pos.cpu().clone()


@pytest.mark.parametrize("profile,act,W,B,T", [
    ("tiny", "bf16", 1, 3, 10),
    ("tiny", "bf16", 4, 3, 12),
    ("tiny", "fp32", 1, 3, 8),
    ("cfg1", "bf16", 1, 2, 12),
    ("cfg1", "bf16", 2, 5, 8),
    ("tiny_lora", "bf16", 1, 3, 8),
    ("tiny_lora", "fp32", 2, 3, 8),
])
def test_persistent_bit_identical(profile, act, W, B, T):
    from altxs_amd import synth

    _log(f"persistent vs per-stage {profile} act={act} W={W} B={B}")
    sm = _synth(profile)
    toks = synth.zipf_tokens(sm.cfg.vocab_size, (B, T), seed=7)
    a = _run_steps(sm, act, W, toks, persistent=False)
    b = _run_steps(sm, act, W, toks, persistent=True)
    assert torch.equal(a[0], b[0])
    assert torch.equal(a[1], b[1])
    assert torch.equal(a[2], b[2])


@pytest.mark.parametrize("B", [40, 64])
def test_persistent_long_context_ragged(B):
    """cfg3 shapes: B rows (40: last row tile half empty), random bf16 cache,
    every segment at its own position (up to ~1000 keys)."""
    from altxs_amd import synth
    from altxs_amd.model import StepModel

    _log(f"persistent cfg3 B={B} long context")
    sm = _synth("cfg3")
    toks = synth.zipf_tokens(sm.cfg.vocab_size, (B, 1), seed=3).astype(np.int32)
    pos = torch.from_numpy((np.arange(B) * 37 + 5) % 1000).to(torch.int32)
    outs = []
    for persistent in (False, True):
        model = StepModel(sm, act="bf16", kv="bf16")
        st = model.make_static_state(1024, win=1, batch=B, persistent=persistent)
        g = torch.Generator(device="cuda").manual_seed(11)
        st.kv.normal_(generator=g)
        st.pos.copy_(pos)
        st.token.copy_(torch.from_numpy(toks))
        model.step(st)
        torch.cuda.synchronize()
        st.check_errors()
        outs.append((st.logits.cpu().clone(), st.cum.cpu().clone(), st.kv.cpu().clone()))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[0][2], outs[1][2])  # the K/V rows written at pos


def test_persistent_graph_replay():
    """The persistent step captures into a graph (counters are cleared by a
    kernel, not a memset); every replay matches the eager step."""
    from altxs_amd import synth
    from altxs_amd.model import StepModel

    _log("persistent graph replay")
    sm = _synth("cfg1")
    B = 6
    model = StepModel(sm, act="bf16", kv="bf16")
    st = model.make_static_state(256, win=1, batch=B, persistent=True)
    st.token.copy_(torch.from_numpy(synth.zipf_tokens(sm.cfg.vocab_size, (B, 1), seed=5).astype(np.int32)))
    st.pos.fill_(9)
    model.step(st)
    torch.cuda.synchronize()
    want = st.cum.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        model.step(st)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(g):
        model.step(st)
    for _ in range(3):
        st.cum.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(st.cum, want)
        model.step(st)  # eager work between replays
        torch.cuda.synchronize()
    st.check_errors()


def test_persistent_stale_plan_rejected():
    from altxs_amd import _lib
    from altxs_amd.model import StepModel

    _log("persistent stale plan")
    sm = _synth("tiny")
    model = StepModel(sm, act="bf16", kv="bf16")
    st = model.make_static_state(256, win=1, batch=2, persistent=True)
    d = _lib.StepDesc.from_buffer_copy(st._desc(0))
    other = torch.zeros_like(st.pos)
    d.pos = other.data_ptr()  # positions live in the plan
    rc = model.lib.altxs_step(ctypes.byref(d), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == -1  # ALTXS_ERR_ARG
    assert b"rebuild" in model.lib.altxs_last_error()
