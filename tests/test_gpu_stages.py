"""Stage-level drop-ins (dropin.ffn_stage_rows, dropin.run_split_attn) against
oracle/stages_ref.py.

ffn_stage_rows (ac_gemv.py:455-550) on the GPU equals the oracle's three
stages:
* bf16 workspaces (bf16 weights): every output element equal except where an
  fp32 sum rounded in the MFMA order lands on the other side of a bf16
  rounding boundary than the exact sum -- at most 2% of the elements, by at
  most 4 bf16 steps (of the element or of its row's RMS, whichever is
  larger) after the rounding chain;
* fp32 workspaces: within 2e-5 of the output's scale with fp32 weights (fp32
  sums in another order; the bits-32 planes and the fp32 row's bf16 split are
  exact to ~2^-24); 2.5e-4 with bf16 weights, whose up-projection takes the
  normalised row rounded to bf16 -- where the device rsqrt and the oracle's
  differ in the last fp32 place, that rounding of an element can go the other
  way (2^-8 of it);
* sequential and parallel slots, a skip write, 1 to 37 rows, the benchmark
  shapes (d 512, MLP 2048) and a small one; inputs it must not write stay
  unchanged.

run_split_attn (split_attn.py:341-425), bf16 packed caches, against the oracle
with q rounded to bf16 for every key (the kernel's operands): within 2^-8
max|v| (the bf16 rounding of the softmax weights, as the decode kernel's own
test) plus the bf16 rounding of y; against the reference's rounding (fp32 q
for the current key) within that plus the current score's rounding effect
2 max|v| |q - bf16(q)| . |k| / 8.  fp32 packed caches against the fp32
restatement within 2e-5.  Decode (one row, the tail row max_len - 1),
encode windows (rows at pos + r), several rows sharing the tail row, MHA and
GQA, XSA and the gate.
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import stages_ref as sr

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def _ffn_inputs(seed, win, d, mlp, dt, wdt):
    g = torch.Generator().manual_seed(seed)
    t = lambda *s, sc=1.0: torch.randn(*s, generator=g) * sc
    c = dict(y=t(win, d), a_sc=t(d, sc=0.5), xin=t(win, d), ln=torch.tensor([0.7071]),
             m_sc=t(d, sc=0.5), lane0=t(win, d), lane1=t(win, d), pr=t(2, sc=0.5) + 1.0,
             pp=t(4, sc=0.5), skips=t(3, win, d), attn_s=t(win, d), hid=t(win, d),
             scr=t(win, mlp), x=t(win, d))
    w = dict(out_w=t(d, d, sc=0.05), up_w=t(mlp, d, sc=0.05), down_w=t(d, mlp, sc=0.03))
    c = {k: v.to(dt) for k, v in c.items()}
    w = {k: v.to(wdt) for k, v in w.items()}
    return c, w


def _steps(got, want):
    """(share of differing elements, max difference in bf16 steps of the
    larger of the element and its row's RMS: an element that comes out small
    by cancellation carries the absolute error of its row's terms)."""
    diff = got != want
    w2 = want.reshape(-1, want.shape[-1])
    rms = np.sqrt((w2.astype(np.float64) ** 2).mean(axis=1, keepdims=True)).reshape(want.shape[:-1] + (1,))
    step = np.maximum(np.maximum(np.abs(want), rms), 1e-30) * 2.0 ** -7
    return float(diff.mean()), float((np.abs(got - want) / step).max())


@pytest.mark.parametrize("dt,wdt", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
                                    (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("win,d,mlp", [(1, 512, 2048), (37, 512, 2048), (16, 256, 512)])
@pytest.mark.parametrize("par", [False, True])
def test_ffn_stage_rows_against_oracle(dt, wdt, win, d, mlp, par):
    from altxs_amd import dropin

    _log(f"ffn_stage_rows dt={dt} w={wdt} win={win} d={d} mlp={mlp} par={par}")
    c, w = _ffn_inputs(win * 7 + d + par, win, d, mlp, dt, wdt)
    dev = {k: v.to(DEV) for k, v in {**c, **w}.items()}
    before = {k: v.clone() for k, v in dev.items()}
    skip_dst = -1 if par else 1
    dropin.ffn_stage_rows(y=dev["y"], out_w=dev["out_w"], hid=dev["hid"], a_sc=dev["a_sc"],
                          xin=dev["xin"], attn_s=dev["attn_s"], src=dev["lane1"] if par else dev["xin"],
                          up_w=dev["up_w"], ln=dev["ln"], scr=dev["scr"], down_w=dev["down_w"],
                          m_sc=dev["m_sc"], x=dev["x"], lane0=dev["lane0"], lane1=dev["lane1"],
                          pr=dev["pr"], pp=dev["pp"], skips=dev["skips"], skip_dst=skip_dst, par=par)
    torch.cuda.synchronize()
    n = {k: v.float().numpy() for k, v in {**c, **w}.items()}
    want = sr.ffn_stage_rows(y=n["y"], out_w=n["out_w"], a_sc=n["a_sc"], xin=n["xin"],
                             src="lane1" if par else "xin", up_w=n["up_w"], ln=float(n["ln"][0]),
                             down_w=n["down_w"], m_sc=n["m_sc"], lane0=n["lane0"], lane1=n["lane1"],
                             pr=n["pr"], pp=n["pp"], skips=n["skips"], skip_dst=skip_dst, par=par,
                             bf16=dt == torch.bfloat16, w_bf16=wdt == torch.bfloat16)
    outs = ("hid", "scr", "attn_s", "lane0", "lane1") if par else ("hid", "scr", "xin", "x", "skips")
    for k in outs:
        got = dev[k].float().cpu().numpy()
        if dt == torch.bfloat16:
            share, steps = _steps(got, want[k])
            _log(f"{k}: differing share {share:.4f}, max {steps:.2f} bf16 steps")
            assert share <= 0.02 and steps <= 4.0, (k, share, steps)
        else:
            scale = np.abs(want[k]).max()
            err = np.abs(got - want[k]).max() / scale
            _log(f"{k}: max relative error {err:.2e}")
            assert err <= (2e-5 if wdt == torch.float32 else 2.5e-4), (k, err)
    untouched = ("xin", "x", "skips") if par else ("attn_s", "lane0", "lane1")
    for k in untouched + ("y", "a_sc", "m_sc", "ln", "pr", "pp", "out_w", "up_w", "down_w"):
        assert torch.equal(dev[k], before[k]), k


def _ws(seed, rows, H, n_kv, L, dt, slots=3, d=512, gate_n=12, layers=4):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(slots, n_kv, L, 64, generator=g).to(dt)
    v = torch.randn(slots, n_kv, L, 64, generator=g).to(dt)
    q = (torch.randn(rows, H, 64, generator=g) * 2).to(dt)
    attn_in = torch.randn(rows, d, generator=g).to(dt)
    gate_w = (torch.randn(layers, H, gate_n, generator=g) * 0.3).to(dt)
    ws = SimpleNamespace(q=q.to(DEV), k_pack=k.to(DEV), v_pack=v.to(DEV),
                         y=torch.zeros(rows, H * 64, dtype=dt, device=DEV), attn_in=attn_in.to(DEV),
                         gate_w=gate_w.to(DEV), n_heads=H, n_kv=n_kv, hd=64, max_len=L, d=d,
                         gate_n=gate_n, attn_splits=8)
    return ws


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,tail_at_pos,pos", [(1, False, 0), (1, False, 700), (37, True, 100),
                                                  (3, False, 250), (1, True, 63)])
@pytest.mark.parametrize("H,n_kv", [(8, 8), (8, 4)])
def test_run_split_attn_against_oracle(dt, rows, tail_at_pos, pos, H, n_kv):
    from altxs_amd import dropin

    _log(f"run_split_attn dt={dt} rows={rows} tail_at_pos={tail_at_pos} pos={pos} H={H} n_kv={n_kv}")
    L, slot, layer = 768, 2, 3
    ws = _ws(rows * 31 + pos + H + n_kv, rows, H, n_kv, L, dt)
    posd = torch.tensor([pos], dtype=torch.int64, device=DEV)
    # the current value rows, as the reference's call sites fill v_cur
    cur = [pos + r if tail_at_pos else L - 1 for r in range(rows)]
    v_cur = ws.v_pack[slot][:, cur].transpose(0, 1).reshape(rows, n_kv * 64).contiguous()
    ok = dropin.run_split_attn(ws=ws, pos=posd, slot=slot, rows=rows, layer=layer, use_xsa=1, use_gate=1,
                               v_cur=v_cur, v_cur_row_stride=n_kv * 64,
                               tail_at_pos=tail_at_pos, norm_eps=1e-12, block_l=256)
    assert ok
    torch.cuda.synchronize()
    got = ws.y.float().cpu().numpy().astype(np.float64)
    kp, vp = ws.k_pack.float().cpu().numpy(), ws.v_pack.float().cpu().numpy()
    q = ws.q.float().cpu().numpy()
    kw = dict(q=q, k_pack=kp, v_pack=vp, pos=pos, slot=slot, rows=rows, use_xsa=True, use_gate=True,
              attn_in=ws.attn_in.float().cpu().numpy(), gate_w=ws.gate_w.float().cpu().numpy(),
              layer=layer, tail_at_pos=tail_at_pos)
    vmax = float(np.abs(vp[slot]).max())
    if dt == torch.bfloat16:
        want = sr.split_attn(q_bf16_prefix=True, q_bf16_tail=True, **kw)
        bound = vmax * 2.0 ** -8 + np.abs(want) * 2.0 ** -8
        err = np.abs(got - want)
        _log(f"max err {err.max():.2e}, max err/bound {(err / bound).max():.3f}")
        assert (err <= bound).all()
        ref = sr.split_attn(q_bf16_prefix=True, q_bf16_tail=False, **kw)
        # the current key's score from bf16(q) instead of q
        g = H // n_kv
        extra = np.zeros((rows, H))
        for r in range(rows):
            t = pos + r if tail_at_pos else L - 1
            for h in range(H):
                dq = np.abs(q[r, h] - sr.round_bf16(q[r, h]))
                extra[r, h] = 2 * vmax * float(dq @ np.abs(kp[slot, h // g, t])) / 8.0
        bound2 = bound + np.repeat(extra, 64, axis=1)
        assert (np.abs(got - ref) <= bound2).all()
    else:
        want = sr.split_attn(q_bf16_prefix=False, q_bf16_tail=False, **kw)
        err = np.abs(got - want).max()
        _log(f"max err {err:.2e}")
        assert err <= 2e-5
