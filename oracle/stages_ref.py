"""Stage-level restatements, numpy -- TEST INFRASTRUCTURE ONLY.

* :func:`ffn_stage_rows` restates the three stage kernels ``ffn_stage_rows``
  launches (src/xsa_ttt/ac_gemv.py:455-550): ``_ffn_out_residual_rows``
  (89-146), ``_ffn_up_activation_rows`` (148-200) and
  ``_ffn_down_commit_rows`` (202-310), with every rounding to the workspace
  dtype those kernels make (``.to(T.dtype.element_ty)`` and bf16 tensor
  arithmetic).  The GEMV sums are exact (float64) and then rounded to fp32.
  Pinned by tests/test_oracle_stages.py: in fp32 against the reference
  model's own block formulas (Block.forward, model.py:932-979, and
  _parallel_block 1293-1355, written with torch.nn.functional); in bf16
  against the reference's eager form of the same slot
  (persistent_step.py:786-811) run in torch bf16 arithmetic on the CPU, which
  fixes every rounding point by tensor dtype; the bf16 rounding itself
  against torch's conversion.
* :func:`split_attn` restates ``run_split_attn``'s result
  (src/xsa_ttt/split_attn.py:53-303): row r attends to cache keys [0, pos + r)
  and then to the current key (row max_len - 1, or pos + r with
  ``tail_at_pos``), softmax in float64 here (the reference merges fp32
  partials of its key splits in a fixed order), the prefix scores from the
  bf16-rounded q (its tl.dot operands), the current key's from the fp32 q,
  then XSA against the current value and the sparse gate
  sigmoid(attn_in[r, :gate_n] . gate_w[layer, h]).  Pinned against
  torch's scaled_dot_product_attention on the same keys, and by the
  invariants XSA and the gate fix (y . v = 0 after XSA; a zero gate weight
  halves y).
"""

from __future__ import annotations

import numpy as np


def round_bf16(a) -> np.ndarray:
    """fp32 -> nearest bf16 (ties to even), returned as fp32 values; NaN kept."""
    f = np.ascontiguousarray(a, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(f), f, out).astype(np.float32)


def _rnd(a, bf16: bool) -> np.ndarray:
    a = np.asarray(a, dtype=np.float32)
    return round_bf16(a) if bf16 else a


def _gemv(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """acc[r, n] = sum_k w[n, k] x[r, k], exact then rounded to fp32."""
    return (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)


def ffn_stage_rows(*, y, out_w, a_sc, xin, src, up_w, ln, down_w, m_sc, lane0, lane1, pr, pp,
                   skips, skip_dst: int, par: bool, bf16: bool, w_bf16: bool,
                   eps: float = 1e-6) -> dict:
    """Outputs of ffn_stage_rows for inputs given as fp32 arrays (bf16 values
    when ``bf16``; weights hold bf16 values when ``w_bf16``): hid, xin,
    attn_s, scr, x, lane0, lane1, skips.

    ``src`` names the stage-2 input: "xin" (sequential slots, the updated
    xin) or "lane1" (parallel slots), as ffn_slot_rows passes it
    (persistent_step.py:766).
    """
    f32 = np.float32
    xin = np.array(xin, dtype=f32, copy=True)
    lane0 = None if lane0 is None else np.array(lane0, dtype=f32, copy=True)
    lane1 = None if lane1 is None else np.array(lane1, dtype=f32, copy=True)
    skips = None if skips is None else np.array(skips, dtype=f32, copy=True)
    a_sc, m_sc = np.asarray(a_sc, f32), np.asarray(m_sc, f32)
    win, d = y.shape
    # stage 1 (ac_gemv.py:120-146)
    attn = _rnd(_gemv(y, out_w), bf16)
    hid = attn.copy()
    scaled = _rnd(attn * a_sc[None, :], bf16)
    attn_s = None
    if par:
        attn_s = scaled
    else:
        xin = _rnd(xin + scaled, bf16)
    # stage 2 (ac_gemv.py:162-200)
    s = xin if src == "xin" else lane1
    ss = (s.astype(f32) * s.astype(f32)).sum(axis=1, dtype=f32)
    scale = _rnd(f32(1.0) / np.sqrt(ss / f32(d) + f32(eps)), bf16)
    norm = _rnd(_rnd(s * scale[:, None], bf16) * f32(ln), bf16)
    if w_bf16:  # the row enters the product in the weight's dtype (ac_gemv.py:182)
        norm = round_bf16(norm)
    raw = _rnd(_gemv(norm, up_w), bf16)
    neg = _rnd(raw * f32(0.5), bf16)
    leaky = np.where(raw >= 0, raw, neg)
    scr = _rnd(leaky * leaky, bf16)
    # stage 3 (ac_gemv.py:244-310)
    mlp = _rnd(_gemv(scr, down_w), bf16)
    hid = mlp
    mlp_s = _rnd(mlp * m_sc[None, :], bf16)
    x = None
    if par:
        pr, pp = np.asarray(pr, f32).reshape(-1), np.asarray(pp, f32).reshape(-1)
        n0 = _rnd(_rnd(pr[0] * lane0, bf16) + _rnd(pp[0] * attn_s, bf16), bf16)
        n0 = _rnd(n0 + _rnd(pp[2] * mlp_s, bf16), bf16)
        n1 = _rnd(_rnd(pr[1] * lane1, bf16) + _rnd(pp[1] * attn_s, bf16), bf16)
        n1 = _rnd(n1 + _rnd(pp[3] * mlp_s, bf16), bf16)
        lane0, lane1 = n0, n1
    else:
        x = _rnd(xin + mlp_s, bf16)
        if skip_dst >= 0:
            skips[skip_dst] = x
    return {"hid": hid, "xin": xin, "attn_s": attn_s, "scr": scr, "x": x, "lane0": lane0,
            "lane1": lane1, "skips": skips}


def split_attn(*, q, k_pack, v_pack, pos: int, slot: int, rows: int, use_xsa: bool, use_gate: bool,
               attn_in=None, gate_w=None, layer: int = 0, tail_at_pos: bool,
               q_bf16_prefix: bool = True, q_bf16_tail: bool = False) -> np.ndarray:
    """y [rows, H*hd] (float64) of run_split_attn.  q [rows, H, hd]; k_pack /
    v_pack [slots, n_kv, max_len, hd]; gate_w [layers, H, gate_n].

    ``q_bf16_prefix`` / ``q_bf16_tail``: whether the prefix / current-key
    scores use the bf16-rounded q (the reference: prefix yes, current key no).
    """
    q = np.asarray(q, dtype=np.float32)
    rows_, H, hd = q.shape
    assert rows_ == rows
    n_kv, max_len = k_pack.shape[1], k_pack.shape[2]
    g = H // n_kv
    qb = round_bf16(q)
    out = np.zeros((rows, H, hd), dtype=np.float64)
    scale = 1.0 / np.sqrt(float(hd))
    for r in range(rows):
        p = int(pos) + r
        tail = p if tail_at_pos else max_len - 1
        for h in range(H):
            kh = k_pack[slot, h // g].astype(np.float64)
            vh = v_pack[slot, h // g].astype(np.float64)
            qp = (qb if q_bf16_prefix else q)[r, h].astype(np.float64)
            qt = (qb if q_bf16_tail else q)[r, h].astype(np.float64)
            s = np.concatenate([kh[:p] @ qp, [kh[tail] @ qt]]) * scale
            vals = np.concatenate([vh[:p], vh[tail][None]], 0)
            e = np.exp(s - s.max())
            yv = (e @ vals) / e.sum()
            if use_xsa:
                vc = vh[tail]
                vn = vc / max(np.sqrt((vc * vc).sum()), 1e-12)
                yv = yv - (yv @ vn) * vn
            if use_gate:
                gn = gate_w.shape[-1]
                z = float(np.asarray(attn_in, np.float64)[r, :gn] @ np.asarray(gate_w, np.float64)[layer, h])
                yv = yv * (1.0 / (1.0 + np.exp(-z)))
            out[r, h] = yv
    return out.reshape(rows, H * hd)
