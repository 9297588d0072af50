"""Pins of oracle/stages_ref.py (CPU only).

* round_bf16 equals torch's fp32 -> bf16 conversion (ties, denormals,
  overflow to inf, NaN).
* ffn_stage_rows in fp32 equals the reference model's block formulas
  (Block.forward, src/xsa_ttt/model.py:932-979; _parallel_block 1293-1355),
  written here with torch.nn.functional: the out-projection residual, RMS,
  the leaky-square MLP and the parallel lambdas (pp[0][0] with the attention
  term of lane 0, pp[1][0] with its MLP term, ...).
* ffn_stage_rows in bf16 equals the reference's eager form of the same slot
  (persistent_step.py:777-811) run in torch bf16 arithmetic, whose tensor
  dtypes fix every rounding point; only sums rounded from a different fp32
  order may differ, by one bf16 step, in a few elements.  The same oracle
  with the roundings left out misses that match in a large share of them.
* split_attn against torch's scaled_dot_product_attention over the same
  key set (prefix rows and the current-key row), and the invariants of XSA
  (the output is orthogonal to the current value) and of the gate (a zero
  gate weight halves the output); rows between pos and the tail row are not
  read.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import stages_ref as sr


def test_round_bf16_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(4096).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 4096),
        np.array([0.0, -0.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 3.4e38, -3.4e38, 1e-40, -1e-41,
                  np.inf, -np.inf, np.nan], dtype=np.float32)]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = sr.round_bf16(x)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    m = ~np.isnan(want)
    assert np.array_equal(got[m].view(np.uint32), want[m].view(np.uint32))


def _case(seed, win=7, d=256, mlp=512):
    g = torch.Generator().manual_seed(seed)
    t = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc)
    return dict(y=t(win, d), out_w=t(d, d, sc=0.05), a_sc=t(d, sc=0.5), xin=t(win, d),
                up_w=t(mlp, d, sc=0.05), ln=torch.tensor(0.7071), down_w=t(d, mlp, sc=0.05),
                m_sc=t(d, sc=0.5), lane0=t(win, d), lane1=t(win, d), pr=t(2, sc=0.5) + 1.0,
                pp=t(2, 2, sc=0.5), skips=torch.zeros(3, win, d))


def _np(c):
    return {k: v.numpy().astype(np.float32) for k, v in c.items()}


def _rms(x, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def _mlp(n, up, down):
    return F.linear(F.leaky_relu(F.linear(n, up), negative_slope=0.5).square(), down)


def test_ffn_stages_fp32_equal_model_block():
    eps = 1e-6
    for par in (False, True):
        c = _case(1 + par)
        n = _np(c)
        got = sr.ffn_stage_rows(y=n["y"], out_w=n["out_w"], a_sc=n["a_sc"], xin=n["xin"],
                                src="lane1" if par else "xin", up_w=n["up_w"], ln=float(c["ln"]),
                                down_w=n["down_w"], m_sc=n["m_sc"], lane0=n["lane0"], lane1=n["lane1"],
                                pr=n["pr"], pp=n["pp"], skips=n["skips"], skip_dst=-1 if par else 1,
                                par=par, bf16=False, w_bf16=False, eps=eps)
        a = c["a_sc"] * F.linear(c["y"], c["out_w"])
        if par:  # _parallel_block: lanes from the attention and MLP terms
            m = c["m_sc"] * _mlp(_rms(c["lane1"], eps) * c["ln"], c["up_w"], c["down_w"])
            pr, pp = c["pr"], c["pp"]
            want0 = pr[0] * c["lane0"] + pp[0][0] * a + pp[1][0] * m
            want1 = pr[1] * c["lane1"] + pp[0][1] * a + pp[1][1] * m
            np.testing.assert_allclose(got["lane0"], want0.numpy(), rtol=1e-5, atol=1e-5)
            np.testing.assert_allclose(got["lane1"], want1.numpy(), rtol=1e-5, atol=1e-5)
            np.testing.assert_allclose(got["attn_s"], a.numpy(), rtol=1e-5, atol=1e-6)
        else:  # Block.forward: x_out = x_in + attn_scale*attn; + mlp_scale*mlp(norm(x_out))
            x_out = c["xin"] + a
            want = x_out + c["m_sc"] * _mlp(_rms(x_out, eps) * c["ln"], c["up_w"], c["down_w"])
            np.testing.assert_allclose(got["xin"], x_out.numpy(), rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(got["x"], want.numpy(), rtol=1e-5, atol=1e-5)
            assert np.array_equal(got["skips"][1], got["x"]) and not got["skips"][0].any()


def _eager_bf16(c, par, skip_dst, eps):
    """persistent_step.py:777-811 (gemv_rows writes its fp32 sums into bf16
    outputs) in torch bf16 tensor arithmetic."""
    b = {k: v.to(torch.bfloat16) for k, v in c.items()}
    gemv = lambda x, w: (x.float() @ w.float().T).to(torch.bfloat16)
    hid = gemv(b["y"], b["out_w"])
    xin, lane0, lane1 = b["xin"].clone(), b["lane0"].clone(), b["lane1"].clone()
    if par:
        attn_s = hid * b["a_sc"]
        src = lane1
    else:
        xin = xin + b["a_sc"] * hid
        src = xin
        attn_s = None
    rows = [r * torch.rsqrt(r.float().pow(2).mean() + eps).to(r.dtype) for r in src]
    attn_in = torch.stack(rows) * b["ln"]
    scr = gemv(attn_in, b["up_w"])
    scr = torch.where(scr >= 0, scr, scr * 0.5).square()
    hid = gemv(scr, b["down_w"])
    out = {"scr": scr, "hid": hid}
    if par:
        mlp_s = hid * b["m_sc"]
        pr, pp = b["pr"], b["pp"].reshape(4)
        out["lane0"] = pr[0] * lane0 + pp[0] * attn_s + pp[2] * mlp_s
        out["lane1"] = pr[1] * lane1 + pp[1] * attn_s + pp[3] * mlp_s
    else:
        out["x"] = xin + b["m_sc"] * hid
        out["xin"] = xin
    return {k: v.float().numpy() for k, v in out.items()}


def _mismatch(got, want):
    """(share of differing elements, max difference in units of bf16 steps)."""
    diff = got != want
    step = np.maximum(np.abs(want), 1e-30) * 2.0 ** -7
    return float(diff.mean()), float((np.abs(got - want) / step).max())


def test_ffn_stages_bf16_rounding_points_equal_reference_eager_form():
    eps = 1e-6
    for par in (False, True):
        c = _case(10 + par, win=9)
        c = {k: v.to(torch.bfloat16).float() for k, v in c.items()}  # bf16 values
        n = _np(c)
        kw = dict(y=n["y"], out_w=n["out_w"], a_sc=n["a_sc"], xin=n["xin"], src="lane1" if par else "xin",
                  up_w=n["up_w"], ln=float(c["ln"]), down_w=n["down_w"], m_sc=n["m_sc"],
                  lane0=n["lane0"], lane1=n["lane1"], pr=n["pr"], pp=n["pp"], skips=n["skips"],
                  skip_dst=-1, par=par, w_bf16=True, eps=eps)
        got = sr.ffn_stage_rows(bf16=True, **kw)
        want = _eager_bf16(c, par, -1, eps)
        keys = ("scr", "hid", "lane0", "lane1") if par else ("scr", "hid", "xin", "x")
        for k in keys:
            share, steps = _mismatch(got[k], want[k])
            assert share <= 0.01 and steps <= 2.0, (par, k, share, steps)
        # with the roundings left out (fp32 arithmetic on the same bf16 inputs)
        # the outputs miss the eager bf16 form broadly
        loose = sr.ffn_stage_rows(bf16=False, **kw)
        out_key = "lane0" if par else "x"
        share, _ = _mismatch(loose[out_key], want[out_key])
        assert share > 0.5, share


def _attn_case(seed, rows, dt=np.float32):
    rng = np.random.default_rng(seed)
    slots, n_kv, L, hd, H = 2, 2, 128, 64, 4
    k = rng.standard_normal((slots, n_kv, L, hd)).astype(dt)
    v = rng.standard_normal((slots, n_kv, L, hd)).astype(dt)
    q = sr.round_bf16(rng.standard_normal((rows, H, hd)).astype(np.float32) * 2)
    attn_in = rng.standard_normal((rows, 32)).astype(np.float32)
    gate_w = rng.standard_normal((3, H, 12)).astype(np.float32) * 0.3
    return q, k, v, attn_in, gate_w


def test_split_attn_against_sdpa_and_invariants():
    rows, pos, slot = 3, 40, 1
    q, k, v, attn_in, gate_w = _attn_case(0, rows)
    L = k.shape[2]
    for tail_at_pos in (False, True):
        y = sr.split_attn(q=q, k_pack=k, v_pack=v, pos=pos, slot=slot, rows=rows, use_xsa=False,
                          use_gate=False, tail_at_pos=tail_at_pos)
        for r in range(rows):
            p = pos + r
            idx = list(range(p)) + [p if tail_at_pos else L - 1]
            kk = torch.from_numpy(k[slot][:, idx]).double()  # [n_kv, n, hd]
            vv = torch.from_numpy(v[slot][:, idx]).double()
            qq = torch.from_numpy(q[r]).double().reshape(2, 2, 1, 64)  # [n_kv, group, 1, hd]
            want = F.scaled_dot_product_attention(qq, kk[:, None].expand(2, 2, -1, 64),
                                                  vv[:, None].expand(2, 2, -1, 64))
            np.testing.assert_allclose(y[r], want.reshape(-1).numpy(), rtol=0, atol=1e-12)
        # XSA leaves no component along the current value
        yx = sr.split_attn(q=q, k_pack=k, v_pack=v, pos=pos, slot=slot, rows=rows, use_xsa=True,
                           use_gate=False, tail_at_pos=tail_at_pos).reshape(rows, 4, 64)
        for r in range(rows):
            t = pos + r if tail_at_pos else L - 1
            for h in range(4):
                vc = v[slot, h // 2, t].astype(np.float64)
                assert abs(float(yx[r, h] @ vc)) < 1e-10 * np.linalg.norm(vc) * (1 + np.abs(yx[r, h]).sum())
        # a zero gate weight: sigmoid(0) = 1/2
        yg = sr.split_attn(q=q, k_pack=k, v_pack=v, pos=pos, slot=slot, rows=rows, use_xsa=False,
                           use_gate=True, attn_in=attn_in, gate_w=np.zeros_like(gate_w), layer=2,
                           tail_at_pos=tail_at_pos)
        assert np.array_equal(yg, 0.5 * y)
    # the shared tail: rows in [pos + rows, max_len - 1) are never read
    k2, v2 = k.copy(), v.copy()
    k2[slot, :, pos + rows:L - 1] = 1e3
    v2[slot, :, pos + rows:L - 1] = -1e3
    a = sr.split_attn(q=q, k_pack=k, v_pack=v, pos=pos, slot=slot, rows=rows, use_xsa=True,
                      use_gate=True, attn_in=attn_in, gate_w=gate_w, layer=1, tail_at_pos=False)
    b = sr.split_attn(q=q, k_pack=k2, v_pack=v2, pos=pos, slot=slot, rows=rows, use_xsa=True,
                      use_gate=True, attn_in=attn_in, gate_w=gate_w, layer=1, tail_at_pos=False)
    assert np.array_equal(a, b)
