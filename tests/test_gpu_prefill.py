"""Prefill / chunk scoring (a window that starts at position 0) against the
reference's full causal forward (src/xsa_ttt/model.py:1375-1500, 1821-1947).

* fp32 windows from position 0 against logits the reference GPT itself wrote
  for its ``forward_logits`` (tests/golden/model_*.npz "full": tiny, cfg1,
  cfg1 over 136 tokens, the cfg3 benchmark model), within 2e-3 absolute and
  2e-4 in practice, log-sum-exp included;
* the cfg4 chunk-scoring model (the cfg3 architecture) with 4 segments x 256
  tokens = 1024 rows: fp32 windows against the CPU oracle's forward_logits
  within 2e-3; the bf16 windows of the same launch, which take the
  large-tile GEMM path (>= 1024 rows: gemm_big_kernel, norm_rows_kernel and
  the row CDF kernel forming its own tile statistics), code the 1024 symbols
  within 0.1% of the bits the fp32 oracle's tables give.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-3
FIXTURES = {"tiny": "tiny", "cfg1": "cfg1", "cfg1_long": "cfg1", "cfg3": "cfg3"}


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def _window(model, toks: np.ndarray, max_len: int):
    """One step of width T from position 0 for each row of toks [B, T]."""
    B, T = toks.shape
    st = model.make_static_state(max_len, win=T, batch=B, want_probs=True)
    st.token.copy_(torch.from_numpy(toks.astype(np.int32)))
    model.step(st)
    torch.cuda.synchronize()
    st.check_errors()
    V = model.cfg.vocab_size
    return (st.logits.view(B, T, V).cpu().numpy(), st.cum.view(B, T, V + 1).cpu().numpy().astype(np.int64))


@pytest.mark.parametrize("fixture", list(FIXTURES))
def test_window_from_zero_matches_reference_forward(golden_dir, fixture):
    from altxs_amd import synth
    from altxs_amd.config import make_config
    from altxs_amd.model import StepModel

    _log(f"prefill window vs reference forward_logits ({fixture})")
    g = np.load(os.path.join(golden_dir, f"model_{fixture}.npz"))
    cfg = make_config(FIXTURES[fixture])
    sm = synth.make_model(cfg, std=float(g["std"]), softcap=tuple(g["softcap"].tolist()))
    toks = g["tokens"].astype(np.int64)[None]
    lg, _ = _window(StepModel(sm, act="fp32"), toks, int(g["max_len"]))  # the fixture's RoPE length
    lg = lg[0]
    k = g["full"].shape[1]
    err = np.abs(lg[:, :k] - g["full"]).max()
    x = lg.astype(np.float64)
    m = x.max(1, keepdims=True)
    lse = m[:, 0] + np.log(np.exp(x - m).sum(1))
    _log(f"max |dlogit| {err:.3e}, max |dlse| {np.abs(lse - g['full_lse']).max():.3e}")
    assert err < LOGIT_TOL and np.abs(lse - g["full_lse"]).max() < LOGIT_TOL
    assert err < 2e-4


def test_cfg4_model_prefill_1024_rows():
    from altxs_amd import synth
    from altxs_amd.config import make_config
    from altxs_amd.model import StepModel
    from oracle import coder
    from oracle.model_ref import OracleModel, softmax_probs

    B, T = 4, 256
    _log(f"cfg4 model prefill {B} x {T}")
    cfg = make_config("cfg4")
    sm = synth.make_model(cfg, std=0.02, softcap=(30.0, 24.0))
    toks = synth.zipf_tokens(cfg.vocab_size, (B, T), seed=404).astype(np.int64)
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    om = OracleModel(cfg, sm.state_dict(), max_len=256)
    want = np.stack([om.forward_logits(t).numpy() for t in toks])
    lg32, _ = _window(StepModel(sm, act="fp32"), toks, 256)
    err = np.abs(lg32 - want).max()
    _log(f"fp32 window: max |dlogit| {err:.3e}")
    assert err < LOGIT_TOL, err
    lg16, cm16 = _window(StepModel(sm, act="bf16"), toks, 256)
    d16 = np.abs(lg16 - want)
    V = cfg.vocab_size
    got_bits = ref_bits = 0.0
    for b in range(B):
        # row t predicts token t+1; the last row has no next token here
        ref_cum = coder.scale_cum(softmax_probs(torch.from_numpy(want[b, :-1])))
        idx = np.arange(T - 1)
        nxt = toks[b, 1:]
        f = cm16[b, idx, nxt + 1] - cm16[b, idx, nxt]
        got_bits += float(-np.log2(f / cm16[b, idx, V]).sum())
        fr = ref_cum[idx, nxt + 1] - ref_cum[idx, nxt]
        ref_bits += float(-np.log2(fr / ref_cum[idx, V]).sum())
    n = B * (T - 1)
    _log(f"bf16 window (large-tile path): max |dlogit| {d16.max():.3e}, mean {d16.mean():.2e}; "
         f"{got_bits / n:.5f} vs oracle {ref_bits / n:.5f} bits/symbol")
    assert abs(got_bits - ref_bits) / ref_bits < 1e-3
