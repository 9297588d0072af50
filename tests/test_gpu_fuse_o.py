"""The decode step's out-projection inside the attention launch (opt-in).

With ALTXS_F_FUSE_O (StepModel.fuse_o), in decode steps (W = 1) with bf16
activations on the tiled bf16 cache, the attention launch forms each head's
MFMA terms of the out-projection, and the group scales, the K-slice sum and
the attention scale (and residual) are applied where the result is read --
the MLP-up prologue of a sequential slot (ProOutNorm), the MLP-down epilogue
of a parallel one (OutFin) -- so the out-projection has no launch of its own.
These tests step the same tokens with the separate launch (the default) and
with the fused form and require the same bits: logits, probabilities, CDF
tables and positions over several committed steps (each step's K/V feed the
next).  Covered: every packed width of the out-projection (2, 3, 4, 6 bits),
D = 256 (one K-slice) and 512 (two), batch 1 (the small launch with prefetch
workgroups), ragged 16-row tiles, the 64-row placement (8-row tiles, one XCD
per row tile), sequential and parallel slots.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

CASES = {
    # name: (profile, config overrides, out-projection widths, batch, steps)
    "cfg1_b1": ("cfg1", {}, {}, 1, 6),
    "cfg1_b5": ("cfg1", {}, {"l0.o": 2, "l1.o": 6}, 5, 6),
    "cfg1_par_b3": ("cfg1", dict(parallel_start_layer=1), {"l1.o": 2}, 3, 6),
    "cfg1_b19_w4": ("cfg1", {}, {"l0.o": 4, "l1.o": 4}, 19, 4),
    "cfg3_b64": ("cfg3", {}, {"l0.o": 2, "l1.o": 4, "l2.o": 6}, 64, 3),
    "cfg3_mixed_b40": ("cfg3", dict(parallel_start_layer=2, num_layers=4, xsa_last_n=4),
                       {"l2.o": 6, "l3.o": 2}, 40, 4),
}


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def _run(sm, toks, fuse: bool):
    from altxs_amd import _lib
    from altxs_amd.model import StepModel

    B, T = toks.shape
    model = StepModel(sm, act="bf16")
    model.fuse_o = fuse
    st = model.make_static_state(256, win=1, batch=B)
    fused = [model.fuses_out_proj(st, s) for s in range(model.n_slots)]
    par = [sl["kind"] == _lib.SLOT_PAR for sl in model.slots]
    out = []
    for t in range(T):
        st.token.copy_(torch.from_numpy(toks[:, t:t + 1].astype(np.int32)))
        model.step(st, commit=True)
        out.append((st.logits.cpu().clone(), st.probs.cpu().clone(), st.cum.cpu().clone()))
    torch.cuda.synchronize()
    st.check_errors()
    return out, st.pos.cpu().clone(), fused, par


@pytest.mark.parametrize("case", sorted(CASES))
def test_fused_out_projection_bit_identical(case):
    from altxs_amd import synth
    from altxs_amd.config import make_config

    prof, over, widths, B, T = CASES[case]
    _log(f"fused out-projection {case}: B={B} T={T} widths={widths}")
    cfg = make_config(prof, **over)
    sm = synth.make_model(cfg, std=0.02, softcap=(30.0, 24.0), bits=widths)
    toks = synth.zipf_tokens(cfg.vocab_size, (B, T), seed=7)
    sep, pos_s, fused_s, _ = _run(sm, toks, fuse=False)
    fus, pos_f, fused_f, par = _run(sm, toks, fuse=True)
    assert not any(fused_s)
    assert all(fused_f), "the fused path must be the one under test"
    assert any(par) == ("par" in case or "mixed" in case)
    for t, (a, b) in enumerate(zip(sep, fus)):
        for name, x, y in zip(("logits", "probs", "cum"), a, b):
            assert torch.equal(x, y), f"{case}: step {t} {name} differ"
    assert torch.equal(pos_s, pos_f)


def test_fusion_conditions():
    """The fused form is taken only where it is asked for and built: the
    default, fp32 activations, GQA (tiny) and windows (W > 1) keep the
    separate launch."""
    from altxs_amd import synth
    from altxs_amd.config import make_config
    from altxs_amd.model import StepModel

    _log("fused out-projection: conditions")
    sm1 = synth.make_model(make_config("cfg1"), std=0.02, softcap=(30.0, 24.0))
    m = StepModel(sm1, act="bf16")
    assert not m.fuses_out_proj(m.make_static_state(256, win=1, batch=2))
    m.fuse_o = True
    assert m.fuses_out_proj(m.make_static_state(256, win=1, batch=2))
    assert not m.fuses_out_proj(m.make_static_state(256, win=4, batch=2))
    m32 = StepModel(sm1, act="fp32", kv="bf16")
    m32.fuse_o = True
    assert not m32.fuses_out_proj(m32.make_static_state(256, win=1, batch=2))
    smt = synth.make_model(make_config("tiny"), std=0.08, softcap=(2.0, 1.5))
    mt = StepModel(smt, act="bf16")
    mt.fuse_o = True
    assert not mt.fuses_out_proj(mt.make_static_state(256, win=1, batch=2))
    with pytest.raises(ValueError):
        m.fuses_out_proj(m.make_static_state(256, win=1, batch=2), slot=99)
