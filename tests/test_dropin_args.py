"""Argument checks of the stage-level drop-ins (CPU only: they raise before
any library call).

The messages the reference raises are kept where it has them:
``ffn_stage_rows`` -- "ln must be the per-layer scalar ln_scale_factor, got N
values" and "stage-fused FFN hidden shape mismatch" (ac_gemv.py:484-490).
The checks added here refuse what would read or write outside the given
buffers (a q buffer with too few rows, an attention input with too few
features, lanes or skips of the wrong shape, attn_s aliasing y).
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from altxs_amd import dropin


def _ffn_kwargs(win=3, d=256, mlp=512, par=False):
    z = lambda *s: torch.zeros(*s)
    return dict(y=z(win, d), out_w=z(d, d), hid=z(win, d), a_sc=z(d), xin=z(win, d), attn_s=z(win, d),
                src=z(win, d), up_w=z(mlp, d), ln=z(1), scr=z(win, mlp), down_w=z(d, mlp), m_sc=z(d),
                x=z(win, d), lane0=z(win, d), lane1=z(win, d), pr=z(2), pp=z(4), skips=z(2, win, d),
                skip_dst=-1, par=par)


def test_ffn_stage_rows_reference_messages():
    kw = _ffn_kwargs()
    kw["ln"] = torch.zeros(4)
    with pytest.raises(ValueError, match="ln must be the per-layer scalar ln_scale_factor, got 4 values"):
        dropin.ffn_stage_rows(**kw)
    kw = _ffn_kwargs()
    kw["hid"] = torch.zeros(2, 256)
    with pytest.raises(ValueError, match="stage-fused FFN hidden shape mismatch"):
        dropin.ffn_stage_rows(**kw)


@pytest.mark.parametrize("change,match", [
    (dict(skip_dst=2), "skip_dst=2"),
    (dict(skip_dst=0, skips=torch.zeros(2, 3, 128)), "skip_dst=0"),
    (dict(x=torch.zeros(3, 128)), "x must be"),
    (dict(a_sc=torch.zeros(128)), "a_sc has shape"),
    (dict(src=torch.zeros(2, 256)), "src has shape"),
    (dict(ln=torch.zeros(1, dtype=torch.bfloat16)), "ln must be a contiguous"),
])
def test_ffn_stage_rows_refuses_mismatched_buffers(change, match):
    kw = _ffn_kwargs()
    kw.update(change)
    with pytest.raises(ValueError, match=match):
        dropin.ffn_stage_rows(**kw)


def test_ffn_stage_rows_parallel_checks():
    kw = _ffn_kwargs(par=True)
    kw["pp"] = torch.zeros(3)
    with pytest.raises(ValueError, match="pp 4 values"):
        dropin.ffn_stage_rows(**kw)
    kw = _ffn_kwargs(par=True)
    kw["lane1"] = torch.zeros(2, 256)
    with pytest.raises(ValueError, match="lane1 must be"):
        dropin.ffn_stage_rows(**kw)
    kw = _ffn_kwargs(par=True)
    kw["attn_s"] = kw["y"]
    with pytest.raises(ValueError, match="must not alias y"):
        dropin.ffn_stage_rows(**kw)


def _ws(rows=2, H=8, n_kv=8, L=256, gate_n=12):
    return SimpleNamespace(q=torch.zeros(rows, H * 64), k_pack=torch.zeros(2, n_kv, L, 64, dtype=torch.bfloat16),
                           v_pack=torch.zeros(2, n_kv, L, 64, dtype=torch.bfloat16),
                           y=torch.zeros(rows, H * 64), attn_in=torch.zeros(rows, 512),
                           gate_w=torch.zeros(3, H, gate_n), n_heads=H, n_kv=n_kv, hd=64, max_len=L,
                           d=512, gate_n=gate_n, attn_splits=8)


def _split_kwargs(ws, **over):
    kw = dict(ws=ws, pos=torch.tensor([5]), slot=1, rows=2, layer=0, use_xsa=1, use_gate=1,
              v_cur=torch.zeros(2, 512), v_cur_row_stride=512, tail_at_pos=True, norm_eps=1e-12, block_l=256)
    kw.update(over)
    return kw


@pytest.mark.parametrize("over,match", [
    (dict(norm_eps=1e-6), "norm_eps"),
    (dict(slot=2), "slot 2"),
    (dict(rows=3), "ws.q holds 2 rows"),
    (dict(rows=0), "rows=0"),
    (dict(use_xsa=1, v_cur=None), "use_xsa needs v_cur"),
])
def test_run_split_attn_refuses_bad_arguments(over, match):
    with pytest.raises(ValueError, match=match):
        dropin.run_split_attn(**_split_kwargs(_ws(), **over))


def test_run_split_attn_checks_the_workspace():
    ws = _ws()
    ws.n_kv = 4
    with pytest.raises(ValueError, match="disagree with k_pack"):
        dropin.run_split_attn(**_split_kwargs(ws))
    ws = _ws()
    ws.k_pack = ws.k_pack.half()
    ws.v_pack = ws.v_pack.half()
    with pytest.raises(ValueError, match="bf16 or fp32"):
        dropin.run_split_attn(**_split_kwargs(ws))
