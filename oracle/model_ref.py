"""fp32 eager restatement of the reference step -- TEST INFRASTRUCTURE ONLY.

Restates, op for op with the same torch calls, the CPU path the reference
tests run (XSA_AC_FUSED=0): ``GPT.static_extend`` (src/xsa_ttt/model.py:
1617-1633, body 1649-1781) and the full causal forward ``forward_logits``
(1433-1500), for one segment (B=1) at a time:

* embedding + SmearGate: _embed_tokens_window 1559-1579, _embed_tokens
  1515-1541, _smear_gate_values 1260-1273;
* slot itinerary with depth loops: GPT.__init__ 1063-1077;
* Block.forward 932-979 / _parallel_block 1293-1355 / _apply_decoder_skip
  1275-1291 / _final_parallel_hidden 1357-1362;
* CausalSelfAttention.forward 770-871 (QK-RMSNorm, RoPE 130-206 incl. YaRN,
  q_gain, _static_window_attention 550-585, XSA 760-768, sparse gate 854-862);
* MLP 874-882; _project_logits + _apply_asym_softcap 1463-1500;
* unmerged q/v LoRA per slot, when the config has a LoRA rank: LinearLoRA
  (src/xsa_ttt/ttt_lora.py:22-55) as _block_with_lora adds it (143-151).

Pinning: against logits written by the reference GPT itself on the same
weights and tokens (tests/golden/model_*.npz from tests/golden/make_golden.py:
"tiny", cfg1, cfg1 over 136 steps, and the cfg3 benchmark model);
against its own full causal forward (incremental rows == teacher-forced rows);
and, with every motif switch off, against a textbook pre-norm GPT written
with F.scaled_dot_product_attention (tests/test_oracle_model.py).

``segment_rows_tf`` restates the probability engine's row semantics
(``_segment_rows_tf`` / ``reset_segment``, src/xsa_ttt/incremental.py:858-897,
1238-1271, with ``_softmax_np``, compress.py:64-85); pinned by rows the
reference's ``StaticACEngine`` wrote (tests/golden/engine_rows.npz).

The model computes in fp32 throughout, the reference's arithmetic.  The
GPU's bf16 mode is not emulated here: its gate is an fp32-anchored bound
(logits and coded bits/symbol against this fp32 model).
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F


def iter_indices(cfg) -> tuple[list[int], list[int]]:
    """model.py:1063-1077 (looping active, as build_model sets it)."""
    n = cfg.num_layers
    if cfg.num_loops > 0:
        seg = list(range(cfg.loop_start, cfg.loop_end + 1))
        idx = list(range(cfg.loop_start))
        for _ in range(cfg.num_loops + 1):
            idx.extend(seg)
        idx.extend(range(cfg.loop_end + 1, n))
        ne = len(idx) // 2
        return idx[:ne], idx[ne:]
    ne = n // 2
    return list(range(ne)), list(range(ne, n))


def rotary_table(cfg, seq_len: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotary.forward (model.py:147-192) at ``seq_len``: cos/sin [seq_len, rd/2]."""
    rd = cfg.rope_dims if cfg.rope_dims > 0 else cfg.model_dim // cfg.num_heads
    if cfg.rope_yarn and seq_len > cfg.block_size:
        scale = seq_len / cfg.block_size
        new_base = cfg.rope_base * scale ** (rd / (rd - 2))
        inv_freq = 1.0 / new_base ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd)
    else:
        inv_freq = 1.0 / cfg.rope_base ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd)
    t = torch.arange(seq_len, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return freqs.cos(), freqs.sin()


def apply_rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, rd: int) -> torch.Tensor:
    """apply_rotary_emb (model.py:195-206); x [..., T, H, hd], cos/sin [T, rd/2]."""
    cos = cos[:, None, :]
    sin = sin[:, None, :]
    if 0 < rd < x.size(-1):
        xr, xp = x[..., :rd], x[..., rd:]
        h = rd // 2
        x1, x2 = xr[..., :h], xr[..., h:]
        return torch.cat((torch.cat((x1 * cos + x2 * sin, x1 * -sin + x2 * cos), -1), xp), -1)
    h = x.size(-1) // 2
    x1, x2 = x[..., :h], x[..., h:]
    return torch.cat((x1 * cos + x2 * sin, x1 * -sin + x2 * cos), -1)


def _rms(x: torch.Tensor) -> torch.Tensor:
    return F.rms_norm(x, (x.size(-1),))


class OracleState:
    """One segment's static-KV state (StaticState, model.py:358-461)."""

    def __init__(self, n_slots: int, max_len: int, n_kv: int, hd: int, d: int):
        self.k = [torch.zeros(max_len, n_kv, hd) for _ in range(n_slots)]
        self.v = [torch.zeros(max_len, n_kv, hd) for _ in range(n_slots)]
        self.pos = 0
        self.prev_raw = torch.zeros(d)
        self.cand_raw = torch.zeros(d)
        self.max_len = max_len


class OracleModel:
    def __init__(self, cfg, sd: dict, *, max_len: int = 2048):
        self.cfg = cfg
        self.sd = {k: torch.as_tensor(np.asarray(v), dtype=torch.float32) for k, v in sd.items()}
        self.L = cfg.num_layers
        self.D = cfg.model_dim
        self.H = cfg.num_heads
        self.Hkv = cfg.num_kv_heads
        self.hd = self.D // self.H
        self.rd = cfg.rope_dims if cfg.rope_dims > 0 else self.hd
        self.enc, self.dec = iter_indices(cfg)
        self.n_slots = len(self.enc) + len(self.dec)
        self.n_skip = min(len(self.enc), len(self.dec))
        self.max_len = int(max_len)
        self.cos, self.sin = rotary_table(cfg, self.max_len)
        # unmerged q/v LoRA per slot (ttt_lora.py:22-55, 143-151): scale alpha/rank
        self.lora_rank = int(getattr(cfg, "lora_rank", 0) or 0)
        self.lora_scale = float(cfg.lora_alpha) / self.lora_rank if self.lora_rank else 0.0

    # ---- helpers ----------------------------------------------------------
    def _bank(self, i: int):
        n, sd = self.L, self.sd
        return (sd["qo_bank"][i], sd["kv_bank"][i], sd["kv_bank"][n + i], sd["qo_bank"][n + i],
                sd["mlp_up_bank"][i], sd["mlp_down_bank"][i])

    def _ln(self, i: int) -> float:
        return 1.0 / math.sqrt(i + 1) if self.cfg.ln_scale else 1.0

    def _mlp(self, i: int, n: torch.Tensor) -> torch.Tensor:
        _, _, _, _, up, down = self._bank(i)
        h = F.leaky_relu(F.linear(n, up), negative_slope=0.5).square()
        return F.linear(h, down)

    def _skip(self, j: int, dest: torch.Tensor, skips: list) -> torch.Tensor:
        """_apply_decoder_skip (model.py:1275-1291)."""
        if j >= self.n_skip or not skips:
            return dest
        s = skips.pop()
        scaled = self.sd["skip_weights"][j] * s
        if "skip_gates" not in self.sd or not self.cfg.skip_gates_enabled:
            return dest + scaled
        g = torch.sigmoid(self.sd["skip_gates"][j])
        return torch.lerp(scaled, dest, g)

    def _final_hidden(self, lane0, lane1, x):
        if lane0 is None:
            return x
        mode = self.cfg.parallel_final_lane.lower()
        if mode == "mlp":
            return lane1
        if mode == "attn":
            return lane0
        return 0.5 * (lane0 + lane1)

    def _logits(self, x: torch.Tensor) -> torch.Tensor:
        h = _rms(x)
        lg = F.linear(h, self.sd["tok_emb.weight"])
        if self.cfg.asym_logit_rescale:
            sp, sn = self.sd["softcap_pos"], self.sd["softcap_neg"]
            return torch.where(lg >= 0, sp * torch.tanh(lg / sp), sn * torch.tanh(lg / sn))
        c = self.cfg.logit_softcap
        return c * torch.tanh(lg / c)

    # ---- attention ----------------------------------------------------------
    def _lora(self, kind: str, slot: int, x: torch.Tensor) -> torch.Tensor:
        """LinearLoRA.forward (ttt_lora.py:53-55): (x @ A.T @ B.T) * scale."""
        a, b = self.sd[f"{kind}_loras.{slot}.A"], self.sd[f"{kind}_loras.{slot}.B"]
        return (x @ a.T @ b.T) * self.lora_scale

    def _qkv(self, i: int, n: torch.Tensor, positions: torch.Tensor, slot: int = -1):
        """Projections (+ the slot's q/v LoRA, _block_with_lora ttt_lora.py:143-151)
        + QK-RMSNorm + RoPE + q_gain (model.py:783-812). n [T, D]."""
        q_w, k_w, v_w, _, _, _ = self._bank(i)
        T = n.shape[0]
        q = F.linear(n, q_w)
        v = F.linear(n, v_w)
        if self.lora_rank and slot >= 0:
            q = q + self._lora("q", slot, n)
            v = v + self._lora("v", slot, n)
        q = q.reshape(T, self.H, self.hd)
        k = F.linear(n, k_w).reshape(T, self.Hkv, self.hd)
        v = v.reshape(T, self.Hkv, self.hd)
        q = _rms(q)
        k = _rms(k)
        cos, sin = self.cos[positions], self.sin[positions]
        q = apply_rotary(q, cos, sin, self.rd)
        k = apply_rotary(k, cos, sin, self.rd)
        q = q * self.sd[f"blocks.{i}.attn.q_gain"][None, :, None]
        return q, k, v

    def _post_attn(self, i: int, y: torch.Tensor, v_cur: torch.Tensor, n: torch.Tensor):
        """XSA + sparse gate + out-projection. y [T, H, hd], v_cur [T, Hkv, hd]."""
        T = y.shape[0]
        if i >= self.L - self.cfg.xsa_last_n:  # use_xsa (model.py:1058-1060)
            g = self.H // self.Hkv
            yg = y.reshape(T, self.Hkv, g, self.hd)
            vn = F.normalize(v_cur, dim=-1).unsqueeze(-2)
            y = (yg - (yg * vn).sum(dim=-1, keepdim=True) * vn).reshape(T, self.H, self.hd)
        if self.cfg.sparse_attn_gate_enabled:
            gw = self.sd[f"blocks.{i}.attn.attn_gate_w"]
            gate = torch.sigmoid(self.cfg.sparse_attn_gate_scale *
                                 F.linear(n[:, : self.cfg.gate_window], gw))
            y = y * gate[..., None]
        _, _, _, o_w, _, _ = self._bank(i)
        return F.linear(y.reshape(T, self.D), o_w)

    def _attend(self, q, k_all, v_all, n_vis: torch.Tensor):
        """Row t attends keys [0, n_vis[t]) (model.py:550-585 semantics)."""
        T = q.shape[0]
        L = k_all.shape[0]
        g = self.H // self.Hkv
        qg = q.reshape(T, self.Hkv, g, self.hd).permute(1, 2, 0, 3)  # [Hkv, g, T, hd]
        kt = k_all.permute(1, 2, 0).unsqueeze(1)  # [Hkv, 1, hd, L]
        att = torch.matmul(qg, kt) * (1.0 / math.sqrt(self.hd))
        mask = torch.arange(L)[None, :] < n_vis[:, None]  # [T, L]
        att = att.masked_fill(~mask[None, None], float("-inf"))
        att = torch.softmax(att, dim=-1)
        vt = v_all.permute(1, 0, 2).unsqueeze(1)  # [Hkv, 1, L, hd]
        y = torch.matmul(att, vt)  # [Hkv, g, T, hd]
        return y.permute(2, 0, 1, 3).reshape(T, self.H, self.hd)

    def _attn_static(self, i: int, slot: int, st: OracleState, n: torch.Tensor):
        T = n.shape[0]
        pos = torch.arange(st.pos, st.pos + T)
        q, k, v = self._qkv(i, n, pos, slot)
        st.k[slot][st.pos:st.pos + T] = k
        st.v[slot][st.pos:st.pos + T] = v
        Lv = st.pos + T
        y = self._attend(q, st.k[slot][:Lv], st.v[slot][:Lv], pos + 1)
        return self._post_attn(i, y, v, n)

    # ---- one static window step (GPT.static_extend) ---------------------------
    def new_state(self, max_len: int | None = None) -> OracleState:
        return OracleState(self.n_slots, max_len or self.max_len, self.Hkv, self.hd, self.D)

    def embed_window(self, tokens: torch.Tensor, prev_raw: torch.Tensor):
        """_embed_tokens_window (model.py:1559-1579)."""
        raw = self.sd["tok_emb.weight"][tokens]  # [T, D]
        if not self.cfg.smear_gate_enabled:
            return _rms(raw), raw[-1]
        prev = torch.cat([prev_raw[None], raw[:-1]], 0)
        gate_in = raw[:, : self.cfg.gate_window]
        g = self.sd["smear_lambda"] * torch.sigmoid(F.linear(gate_in, self.sd["smear_gate.weight"]))
        return _rms(raw + g * prev), raw[-1]

    @torch.no_grad()
    def step(self, st: OracleState, tokens) -> torch.Tensor:
        """W-token window at st.pos; returns logits [W, V]. Does not advance."""
        tokens = torch.as_tensor(np.asarray(tokens, dtype=np.int64).reshape(-1))
        x, last_raw = self.embed_window(tokens, st.prev_raw)
        st.cand_raw = last_raw.clone()
        x0 = x
        skips: list = []
        slot = 0
        for i in self.enc:
            x = self._block(i, slot, st, x, x0)
            slot += 1
            skips.append(x)
        psl = self.cfg.parallel_start_layer
        lane0 = lane1 = None
        for j, i in enumerate(self.dec):
            if i >= psl and psl > 0:
                if lane0 is None:
                    lane0 = lane1 = x
                lane0 = self._skip(j, lane0, skips)
                lane0, lane1 = self._par_block(i, slot, st, lane0, lane1, x0)
            else:
                x = self._skip(j, x, skips)
                x = self._block(i, slot, st, x, x0)
            slot += 1
        return self._logits(self._final_hidden(lane0, lane1, x)).float()

    def advance(self, st: OracleState, w: int) -> None:
        st.pos += int(w)
        st.prev_raw = st.cand_raw.clone()

    def _block(self, i, slot, st, x, x0):
        mix = self.sd[f"blocks.{i}.resid_mix"]
        x_in = mix[0] * x + mix[1] * x0
        n = _rms(x_in) * self._ln(i)
        a = self._attn_static(i, slot, st, n)
        x_out = x_in + self.sd[f"blocks.{i}.attn_scale"] * a
        return x_out + self.sd[f"blocks.{i}.mlp_scale"] * self._mlp(i, _rms(x_out) * self._ln(i))

    def _par_block(self, i, slot, st, lane0, lane1, x0):
        mix = self.sd[f"blocks.{i}.resid_mix"]
        attn_read = mix[0] * lane0 + mix[1] * x0
        a = self.sd[f"blocks.{i}.attn_scale"] * self._attn_static(i, slot, st, _rms(attn_read) * self._ln(i))
        m = self.sd[f"blocks.{i}.mlp_scale"] * self._mlp(i, _rms(lane1) * self._ln(i))
        pr, pp = self.sd["parallel_resid_lambdas"][i], self.sd["parallel_post_lambdas"][i]
        new0 = pr[0] * lane0 + pp[0][0] * a + pp[1][0] * m
        new1 = pr[1] * lane1 + pp[0][1] * a + pp[1][1] * m
        return new0, new1

    # ---- full causal forward (forward_logits) ---------------------------------
    @torch.no_grad()
    def forward_logits(self, ids) -> torch.Tensor:
        """Teacher-forced logits [T, V] for one sequence (model.py:1375-1500).

        Position 0 is not smeared (_apply_smear 1364-1373); attention is causal
        over the sequence, computed here as an explicit masked fp32 softmax.
        """
        ids = torch.as_tensor(np.asarray(ids, dtype=np.int64).reshape(-1))
        T = ids.numel()
        raw = self.sd["tok_emb.weight"][ids]
        if self.cfg.smear_gate_enabled and T > 1:
            gate_in = raw[1:, : self.cfg.gate_window]
            g = self.sd["smear_lambda"] * torch.sigmoid(F.linear(gate_in, self.sd["smear_gate.weight"]))
            raw = torch.cat([raw[:1], raw[1:] + g * raw[:-1]], 0)
        x = _rms(raw)
        x0 = x
        pos = torch.arange(T)

        slot_ctr = [0]

        def attn(i, n):
            q, k, v = self._qkv(i, n, pos, slot_ctr[0])
            slot_ctr[0] += 1
            y = self._attend(q, k, v, pos + 1)
            return self._post_attn(i, y, v, n)

        def block(i, x):
            mix = self.sd[f"blocks.{i}.resid_mix"]
            x_in = mix[0] * x + mix[1] * x0
            x_out = x_in + self.sd[f"blocks.{i}.attn_scale"] * attn(i, _rms(x_in) * self._ln(i))
            return x_out + self.sd[f"blocks.{i}.mlp_scale"] * self._mlp(i, _rms(x_out) * self._ln(i))

        skips: list = []
        for i in self.enc:
            x = block(i, x)
            skips.append(x)
        psl = self.cfg.parallel_start_layer
        lane0 = lane1 = None
        for j, i in enumerate(self.dec):
            if i >= psl and psl > 0:
                if lane0 is None:
                    lane0 = lane1 = x
                lane0 = self._skip(j, lane0, skips)
                mix = self.sd[f"blocks.{i}.resid_mix"]
                a = self.sd[f"blocks.{i}.attn_scale"] * attn(i, _rms(mix[0] * lane0 + mix[1] * x0) * self._ln(i))
                m = self.sd[f"blocks.{i}.mlp_scale"] * self._mlp(i, _rms(lane1) * self._ln(i))
                pr, pp = self.sd["parallel_resid_lambdas"][i], self.sd["parallel_post_lambdas"][i]
                lane0, lane1 = (pr[0] * lane0 + pp[0][0] * a + pp[1][0] * m,
                                pr[1] * lane1 + pp[0][1] * a + pp[1][1] * m)
            else:
                x = self._skip(j, x, skips)
                x = block(i, x)
        return self._logits(self._final_hidden(lane0, lane1, x)).float()

    # ---- segment helpers --------------------------------------------------------
    @torch.no_grad()
    def decode_rows(self, tokens, st: OracleState | None = None) -> torch.Tensor:
        """W=1 steps over ``tokens`` from ``st`` (fresh if None): logits [T, V]."""
        st = st or self.new_state()
        out = []
        for t in np.asarray(tokens).reshape(-1):
            out.append(self.step(st, [int(t)])[0])
            self.advance(st, 1)
        return torch.stack(out)


def softmax_probs(logits: torch.Tensor) -> np.ndarray:
    """Probabilities as the engine computes them: fp32 torch.softmax (incremental.py:603-605)."""
    return torch.softmax(logits.float(), dim=-1).numpy().astype(np.float32)


# ---- probability-engine row semantics ---------------------------------------------

def softmax_np(logits: torch.Tensor) -> np.ndarray:
    """``_softmax_np`` (src/xsa_ttt/compress.py:64-85) for one row: fp32
    torch.softmax, then ``p /= float(p.sum())`` in numpy float32 (a non-finite
    or non-positive sum gives the uniform row)."""
    p = torch.softmax(logits.detach().float().reshape(-1), dim=-1).numpy().astype(np.float32)
    s = float(p.sum())
    if s <= 0 or not math.isfinite(s):
        return np.full(p.size, 1.0 / p.size, dtype=np.float32)
    p /= s
    return p


def chunk_ctx_start(start: int, block: int) -> tuple[int, int]:
    """``_chunk_ctx_start`` (compress.py:122-125)."""
    p0 = 1 if int(start) == 0 else int(start)
    return p0, max(0, p0 - int(block))


def engine_max_len(block: int, every: int, win: int) -> int:
    """Static-state length of ``StaticACEngine`` (incremental.py:239-241): the
    RoPE table is warmed at this length (warm_rotary, 106-113), which sets the
    YaRN scale."""
    return int(block) + (max(1, int(every)) + int(win) - 1) // int(win) * int(win)


@torch.no_grad()
def segment_rows_tf(om: OracleModel, arr, seg, start: int, block: int, win: int) -> np.ndarray:
    """Teacher-forced probability rows of one segment, as ``_segment_rows_tf``
    (incremental.py:1238-1271) with ``reset_segment`` (858-897): rows[0] is
    the carry -- ``_softmax_np`` of the logits after the context window
    ``arr[ctx_start:start]`` (uniform 1/V at the stream start) -- and
    rows[i + 1] = torch.softmax of the logits after seg[:i + 1].  The context
    is run as committed windows (the reference prefills it with one causal
    forward; incremental and teacher-forced logits agree to fp32 rounding).
    ``om`` must be built with ``max_len = engine_max_len(...)``."""
    V = om.cfg.vocab_size
    _, c0 = chunk_ctx_start(start, block)
    ctx = np.asarray(arr[c0:int(start)], dtype=np.int64)
    seg = np.asarray(seg, dtype=np.int64)
    st = om.new_state()
    if ctx.size:
        last = None
        for w0 in range(0, ctx.size, win):
            w = ctx[w0:w0 + win]
            last = om.step(st, w)[-1]
            om.advance(st, w.size)
        carry = softmax_np(last)
    else:
        carry = np.full(V, 1.0 / V, dtype=np.float32)
    n = seg.size
    rows = np.empty((n, V), dtype=np.float32)
    w0 = 0
    while w0 < n:
        w = min(win, n - w0)
        probs = torch.softmax(om.step(st, seg[w0:w0 + w]).float(), dim=-1).numpy()
        rows[w0] = carry
        if w > 1:
            rows[w0 + 1:w0 + w] = probs[:w - 1]
        carry = probs[w - 1]
        om.advance(st, w)
        w0 += w
    return rows
