"""The stress and chunk-scoring configurations at their full shapes.

* cfg5 model (the cfg3 architecture with rank-16 q/v LoRA on every slot):
  130 decode steps from the stream start against the fp32 oracle (2e-3, and
  2e-4 for the fp32-faithful mode), so rows cross three 64-key tiles; the
  bf16 mode codes those symbols within 0.1% of the oracle's bits.
* cfg5 at full shape: 256 segments with 4095 cached positions each (ctx 4096,
  21.5 GB of bf16 KV): one decode step whose tables are exactly the count
  rule of its probabilities, and whose rows for four segments equal, bit for
  bit, the same four segments stepped alone on a copy of their caches.
* cfg4 at full shape: 64 segments x 2048 tokens scored from position 0 in
  one launch (131,072 tables; the large-tile GEMMs): segment 0's rows equal
  the rows of segment 0 scored alone, its first 130 rows equal 130 decode
  rows (16-row GEMMs) bit for bit, and its 2047 symbols code within 0.1% of
  the bits of the fp32 oracle's forward logits.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-3


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def _bits(cum: np.ndarray, syms: np.ndarray) -> float:
    """Ideal code length (bits) of syms[i] under table cum[i]."""
    idx = np.arange(len(syms))
    f = cum[idx, syms + 1] - cum[idx, syms]
    return float(-np.log2(f / cum[idx, -1]).sum())


def _model(profile: str):
    from altxs_amd import synth
    from altxs_amd.config import make_config

    cfg = make_config(profile)
    return synth.make_model(cfg, std=0.02, softcap=(30.0, 24.0))


def test_cfg5_lora_decode_matches_oracle():
    from altxs_amd import synth
    from altxs_amd.model import StepModel
    from oracle import coder
    from oracle.model_ref import OracleModel, softmax_probs

    B, T = 2, 130
    _log(f"cfg5 model: {B} x {T} decode rows vs the fp32 oracle")
    sm = _model("cfg5")
    V = sm.cfg.vocab_size
    toks = synth.zipf_tokens(V, (B, T), seed=505)
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    om = OracleModel(sm.cfg, sm.state_dict(), max_len=256)
    want = np.stack([om.decode_rows(t).numpy() for t in toks])
    for act in ("fp32", "bf16"):
        model = StepModel(sm, act=act)
        st = model.make_static_state(256, win=1, batch=B)
        lg = np.empty((B, T, V), np.float32)
        cm = np.empty((B, T, V + 1), np.int64)
        dev = torch.from_numpy(toks.astype(np.int32)).cuda()
        for t in range(T):
            st.token.copy_(dev[:, t:t + 1])
            model.step(st, commit=True)
            lg[:, t] = st.logits.cpu().numpy()
            cm[:, t] = st.cum.cpu().numpy()
        st.check_errors()
        err = np.abs(lg - want).max()
        if act == "fp32":
            _log(f"fp32: max |dlogit| {err:.3e}")
            assert err < 2e-4, err
        else:
            uni = coder.scale_cum(np.full((1, V), 1.0 / V, np.float32))[0]
            got = ref = 0.0
            for b in range(B):
                rows_r = coder.scale_cum(softmax_probs(torch.from_numpy(want[b, :-1])))
                got += _bits(np.concatenate([uni[None], cm[b, :-1]]), toks[b])
                ref += _bits(np.concatenate([uni[None], rows_r]), toks[b])
            _log(f"bf16: max |dlogit| {err:.3e}; {got / toks.size:.5f} vs {ref / toks.size:.5f} bits/symbol")
            assert abs(got - ref) / ref < 1e-3


def test_cfg5_full_shape_step():
    from altxs_amd import synth
    from altxs_amd.model import StepModel
    from oracle import coder

    B, ctx = 256, 4096
    _log(f"cfg5 full shape: {B} segments, ctx {ctx}")
    sm = _model("cfg5")
    V = sm.cfg.vocab_size
    model = StepModel(sm, act="bf16")
    st = model.make_static_state(ctx, win=1, batch=B, want_probs=True)
    g = torch.Generator(device="cuda").manual_seed(55)
    st.kv.normal_(generator=g)
    st.pos.fill_(ctx - 1)
    st.prev_raw.normal_(generator=g)
    toks = torch.from_numpy(synth.zipf_tokens(V, (B, 1), seed=56).astype(np.int32)).cuda()
    st.token.copy_(toks)
    model.step(st)
    torch.cuda.synchronize()
    st.check_errors()
    rows = [0, 17, 100, 255]
    lg, pr = st.logits[rows].cpu(), st.probs[rows].cpu()
    assert (pr - torch.softmax(lg.double(), -1).float()).abs().max().item() < 1e-6
    assert np.array_equal(st.cum[rows].cpu().numpy().astype(np.int64), coder.scale_cum(pr.numpy()))
    # the same four segments alone, on a copy of their caches
    small = model.make_static_state(ctx, win=1, batch=len(rows), want_probs=True)
    idx = torch.tensor(rows, device="cuda")
    small.kv.copy_(st.kv.index_select(1, idx))
    small.pos.fill_(ctx - 1)
    small.prev_raw.copy_(st.prev_raw.index_select(0, idx))
    small.token.copy_(toks.index_select(0, idx))
    model.step(small)
    torch.cuda.synchronize()
    small.check_errors()
    assert torch.equal(small.logits.cpu(), lg)
    assert torch.equal(small.cum.cpu(), st.cum[rows].cpu())


def test_cfg4_full_shape_pass():
    from altxs_amd import synth
    from altxs_amd.model import StepModel
    from oracle import coder
    from oracle.model_ref import OracleModel, softmax_probs

    B, T = 64, 2048
    _log(f"cfg4 full shape: {B} x {T} from position 0")
    sm = _model("cfg4")
    V = sm.cfg.vocab_size
    toks = synth.zipf_tokens(V, (B, T), seed=404)
    model = StepModel(sm, act="bf16")
    st = model.make_static_state(T, win=T, batch=B, want_probs=False)
    st.token.copy_(torch.from_numpy(toks.astype(np.int32)))
    model.step(st)
    torch.cuda.synchronize()
    st.check_errors()
    lg0 = st.logits[:T].cpu()
    cum0 = st.cum[:T].cpu().numpy().view(np.uint32).astype(np.int64)
    del st
    torch.cuda.empty_cache()
    # segment 0 scored alone
    one = model.make_static_state(T, win=T, batch=1, want_probs=False)
    one.token.copy_(torch.from_numpy(toks[:1].astype(np.int32)))
    model.step(one)
    torch.cuda.synchronize()
    one.check_errors()
    assert torch.equal(one.logits.cpu(), lg0)
    del one
    # its first 130 positions as decode rows (16-row GEMMs, decode attention)
    dec = model.make_static_state(256, win=1, batch=1)
    dt = torch.from_numpy(toks[:1].astype(np.int32)).cuda()
    for t in range(130):
        dec.token.copy_(dt[:, t:t + 1])
        model.step(dec, commit=True)
        assert torch.equal(dec.logits.cpu()[0], lg0[t]), t
    dec.check_errors()
    # bits/symbol of the 2047 coded symbols against the fp32 oracle's forward
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    want = OracleModel(sm.cfg, sm.state_dict(), max_len=T).forward_logits(toks[0]).numpy()
    ref_cum = coder.scale_cum(softmax_probs(torch.from_numpy(want[:-1])))
    got, ref = _bits(cum0[:-1], toks[0, 1:]), _bits(ref_cum, toks[0, 1:])
    _log(f"segment 0: max |dlogit| vs fp32 {np.abs(lg0.numpy() - want).max():.3e}; "
         f"{got / (T - 1):.5f} vs {ref / (T - 1):.5f} bits/symbol")
    assert abs(got - ref) / ref < 1e-3
