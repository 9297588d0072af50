"""Parity at the benchmark's own shape (bench.py's cfg3 decode step).

* The benchmark step itself: the cfg3 model (10 layers, d=512, V=16384,
  3.16 bpw group-64 weights, bf16 activations, bf16 KV) on 64 segments whose
  caches are filled to ctx 2048, every segment at position 2047 (so each row
  reads 2048 keys, 32 key tiles): probabilities = softmax(logits) within 1e-6
  (fp64 softmax), tables = _scale_cum_np(probabilities) exactly, and four of
  the segments stepped alone on copies of their caches give the same logits
  and tables bit for bit.
* The benchmark's attention at 2048 keys (the MFMA kernel on the tiled bf16
  cache, one row per (segment, kv head) workgroup, bf16 q and softmax weights
  as the step runs it) against an fp64 reference on the same cache values:
  within 2^-8 * max|v| (the bf16 rounding of the unnormalised weights; see
  tests/test_gpu_kernels.py), and the fp32-faithful form within 2e-5.
* One cfg3 segment decoded for 1040 positions from the stream start (rows
  cross 17 key tiles) against the fp32 oracle: within 2e-4 with fp32
  activations and KV, within the north-star 2e-3 with the bf16 KV cache.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

_CACHE: dict = {}


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def _cfg3(std=None):
    from altxs_amd import synth
    from altxs_amd.config import make_config

    cfg = make_config("cfg3")
    return synth.make_model(cfg) if std is None else synth.make_model(cfg, std=std, softcap=(30.0, 24.0))


def test_benchmark_step_64_segments_ctx2048():
    from altxs_amd import synth
    from altxs_amd.model import StepModel
    from oracle import coder

    B, ctx = 64, 2048
    _log(f"cfg3 benchmark step: {B} segments at position {ctx - 1}")
    sm = _cfg3()  # bench.py's model (make_model defaults)
    V = sm.cfg.vocab_size
    model = StepModel(sm, act="bf16", kv="bf16")
    st = model.make_static_state(ctx, win=1, batch=B, want_probs=True)
    g = torch.Generator(device="cuda").manual_seed(0)
    st.kv.normal_(generator=g)
    st.pos.fill_(ctx - 1)
    st.prev_raw.normal_(generator=g)
    toks = torch.from_numpy(synth.zipf_tokens(V, (B, 1)).astype(np.int32)).cuda()
    st.token.copy_(toks)
    model.step(st)
    torch.cuda.synchronize()
    st.check_errors()
    lg, pr = st.logits.cpu(), st.probs.cpu()
    assert torch.isfinite(lg).all()
    dp = (pr - torch.softmax(lg.double(), -1).float()).abs().max().item()
    _log(f"max |probs - softmax(logits)| = {dp:.2e}")
    assert dp < 1e-6
    assert np.array_equal(st.cum.cpu().numpy().astype(np.int64), coder.scale_cum(pr.numpy()))
    rows = [0, 9, 31, 63]
    small = model.make_static_state(ctx, win=1, batch=len(rows), want_probs=True)
    idx = torch.tensor(rows, device="cuda")
    small.kv.copy_(st.kv.index_select(1, idx))
    small.pos.fill_(ctx - 1)
    small.prev_raw.copy_(st.prev_raw.index_select(0, idx))
    small.token.copy_(toks.index_select(0, idx))
    model.step(small)
    torch.cuda.synchronize()
    small.check_errors()
    assert torch.equal(small.logits.cpu(), lg[rows])
    assert torch.equal(small.cum.cpu(), st.cum[rows].cpu())


def _attn_ref(q, k, v, p):
    """fp64 attention of one query row per head over keys [0, p]. q [H, 64];
    k, v [H, L, 64] (the cache values)."""
    H = q.shape[0]
    out = torch.zeros(H, 64, dtype=torch.float64)
    for h in range(H):
        s = (k[h, :p + 1].double() @ q[h].double()) / 8.0
        out[h] = torch.softmax(s, 0) @ v[h, :p + 1].double()
    return out


def test_benchmark_attention_2048_keys_against_fp64():
    from altxs_amd import ops

    _log("attention at 2048 keys (bf16 tiled cache) vs fp64")
    B, H, L = 3, 8, 2048
    gen = torch.Generator().manual_seed(2048)
    pos = torch.tensor([2047, 2047, 1500], dtype=torch.int32)
    k = torch.randn(B, H, L, 64, generator=gen).to(torch.bfloat16)
    v = torch.randn(B, H, L, 64, generator=gen).to(torch.bfloat16)
    q = torch.randn(B, H, 64, generator=gen) * 3
    args = (q.to("cuda"), k.to("cuda"), v.to("cuda"), pos.to("cuda"))
    y16 = ops.decode_attn(*args, ops_bf16=True).cpu().double().view(B, H, 64)
    y32 = ops.decode_attn(*args).cpu().double().view(B, H, 64)
    qr = (q * 0.125).to(torch.bfloat16).float() * 8.0  # the bf16 q operand the MFMAs see
    vmax = v.float().abs().max().item()
    for b in range(B):
        p = int(pos[b])
        e16 = (y16[b] - _attn_ref(qr[b], k[b].float(), v[b].float(), p)).abs().max().item()
        e32 = (y32[b] - _attn_ref(q[b], k[b].float(), v[b].float(), p)).abs().max().item()
        _log(f"segment {b} (p={p}): bf16 operands {e16:.2e} (bound {vmax * 2.0 ** -8:.2e}), fp32 {e32:.2e}")
        assert e16 <= vmax * 2.0 ** -8
        assert e32 < 2e-5


@pytest.mark.parametrize("kv,tol", [("fp32", 2e-4), ("bf16", 2e-3)])
def test_cfg3_segment_1040_positions_against_oracle(kv, tol):
    from altxs_amd import synth
    from altxs_amd.model import StepModel
    from oracle.model_ref import OracleModel

    T, L = 1040, 1280
    _log(f"cfg3 one segment, {T} positions, fp32 activations, kv={kv}")
    sm = _cfg3(std=0.02)
    toks = synth.zipf_tokens(sm.cfg.vocab_size, (T,), seed=1040)
    model = StepModel(sm, act="fp32", kv=kv)
    st = model.make_static_state(L, win=1, batch=1)
    dev_toks = torch.from_numpy(toks.astype(np.int32)).cuda()
    got = torch.empty(T, sm.cfg.vocab_size)
    for t in range(T):
        st.token.copy_(dev_toks[t:t + 1].view(1, 1))
        model.step(st, commit=True)
        got[t] = st.logits[0].cpu()
    st.check_errors()
    if "oracle" not in _CACHE:  # the same rows serve both parametrisations
        torch.set_num_threads(min(16, os.cpu_count() or 1))
        _CACHE["oracle"] = OracleModel(sm.cfg, sm.state_dict(), max_len=L).decode_rows(toks)
    want = _CACHE["oracle"]
    err = (got - want).abs()
    per_tile = [float(err[64 * i:64 * (i + 1)].max()) for i in range((T + 63) // 64)]
    _log(f"max |dlogit| per 64-position tile: {['%.1e' % e for e in per_tile]}")
    assert err.max().item() < tol, per_tile
