"""Reference-shaped stand-ins for the drop-in tests (test infrastructure).

The reference cannot be imported on the GPU box, so the drop-in tests drive
``altxs_amd.dropin`` through objects with the reference's attributes and
semantics, restated here:

* :class:`RefStaticKV` / :class:`RefStaticState` -- ``StaticKV`` and
  ``StaticState`` (src/xsa_ttt/model.py:259-461): per-slot K/V buffers
  ``[1, max_len, Hkv, hd]``, the window's K/V in the last W rows,
  ``commit_window(dest)`` copying them into the prefix; built like
  ``GPT.make_static_state`` (model.py:1581-1615).
* :class:`RefModel` -- what the drop-in reads of a reference ``GPT``: ``cfg``
  with the reference's field names, ``state_dict()`` with its parameter names,
  ``_ac_compute_dtype``; ``static_extend_fused`` dispatches like
  ``_static_extend_body(fused=True)`` (model.py:1649-1661): W > 1 tries
  ``try_mega_encode`` first, then ``try_persistent_extend``.
* :class:`RefEngine` -- the parts of ``StaticACEngine`` (src/xsa_ttt/
  incremental.py) that touch the slots: ``reset_segment`` (858-897) with its
  eager prefill into ``st.slots``, ``_rebind_packed_kv`` (899-929),
  ``_sync_row_from_prefix`` (931-954), ``run_window`` / ``advance_window``
  (1017-1052), ``run_decode_row`` (1054-1081), ``_segment_rows_tf`` /
  ``_segment_rows_one_row`` (1221-1271).  The prefill (``prefill_cache``,
  model.py:1821-1947) writes the CPU oracle's K/V rows and takes the carry
  from its last logits (``_softmax_np``, compress.py:64-85).
"""

from __future__ import annotations

import os
import types

import numpy as np
import torch

from oracle.model_ref import OracleModel, chunk_ctx_start, engine_max_len, softmax_np


BF16_BANKS = ("tok_emb.weight", "qo_bank", "kv_bank", "mlp_up_bank", "mlp_down_bank")


def bf16_banks(sd: dict) -> dict:
    """The weight matrices rounded to bf16 values (engine_rows_bf16w.npz's weights)."""
    return {k: (torch.as_tensor(np.asarray(v)).to(torch.bfloat16).float().numpy() if k in BF16_BANKS
                else v) for k, v in sd.items()}


SHIPPED_STEM = os.path.join("shipped", "mixed_da_bpw3.15_upb1.8")


def student_state_dict(golden_dir: str, *, round_banks: bool = False):
    """(cfg, meta, reference-named fp32 state) of the shipped student: the
    restated Init(seed) plus the delta the oracle's codec decodes from the
    copy of the asset in tests/golden/shipped/ (``load_codec``,
    mixed_bit_delta.py:232-312); ``round_banks``: the banks rounded to bf16
    values (the reference's bf16 runtime banks, model.py:1183-1245)."""
    import json

    from safetensors.numpy import load_file

    from altxs_amd.init_seed import reference_init_state
    from altxs_amd.shipped import MODELED, config_from_meta
    from oracle import codec_ref

    meta = json.load(open(os.path.join(golden_dir, SHIPPED_STEM + ".json"), encoding="utf8"))
    cfg = config_from_meta(meta)
    state = load_file(os.path.join(golden_dir, SHIPPED_STEM + ".safetensors"))
    sd = {k: v.numpy() for k, v in reference_init_state(cfg, int(meta["seed"])).items()}
    L, width = int(meta["n_layers"]), cfg.model_dim
    for name in MODELED:
        key = lambda kind, *rest: "/".join((kind, name) + rest)  # noqa: E731
        bits = state[key("bits")]
        packed = {b: state[key("packed", f"b{b}")] for b in (2, 3, 4)}
        books = {b: state[key("codebook", f"b{b}")] for b in (2, 3, 4) if key("codebook", f"b{b}") in state}
        scales = {b: state[key("scale", f"b{b}")] for b in (2, 3, 4) if key("scale", f"b{b}") in state}
        ch = codec_ref.dequantize_channels(bits, books, packed, channel_width=width,
                                           mode=str(meta["codebook_mode"]), scales=scales or None)
        sd[name] = sd[name] + codec_ref.from_channels(name, ch, meta["layouts"][name]["shape"], L)
    for n in meta["small_params"]:
        sd[n] = state["small/" + n]
    if round_banks:
        sd = bf16_banks(sd)
    return cfg, meta, sd


class RefStaticKV:
    """model.py:259-356 (the parts the step and the engine use)."""

    def __init__(self, max_len: int, win: int):
        self.max_len, self.win = int(max_len), int(win)
        self.k: torch.Tensor | None = None
        self.v: torch.Tensor | None = None
        self.step_mode = False
        self.draft_pool = self.draft_local = 0

    def ensure(self, like: torch.Tensor) -> None:
        """Keep a full-length buffer of ``like``'s shape; else allocate zeros."""
        if (self.k is not None and self.v is not None and self.k.shape[0] == like.shape[0]
                and self.k.shape[1] == self.max_len and self.k.shape[2:] == like.shape[2:]
                and self.k.device == like.device):
            return
        b, _, h, d = like.shape
        self.k = torch.zeros(b, self.max_len, h, d, dtype=like.dtype, device=like.device)
        self.v = torch.zeros_like(self.k)


class RefStaticState:
    """model.py:358-461."""

    def __init__(self, cfg, max_len: int, win: int, device, emb_dtype, n_slots: int):
        self.max_len, self.win = int(max_len), int(win)
        self.token = torch.zeros(1, win, dtype=torch.long, device=device)
        self.prev_raw = torch.zeros(1, 1, cfg.model_dim, dtype=emb_dtype, device=device)
        self.cand_prev_raw = torch.zeros(1, 1, cfg.model_dim, dtype=emb_dtype, device=device)
        self.pos = torch.zeros(1, dtype=torch.long, device=device)
        self.logits = torch.zeros(1, win, cfg.vocab_size, dtype=torch.float32, device=device)
        self.slots = [RefStaticKV(max_len, win) for _ in range(n_slots)]

    def set_step_mode(self, on: bool) -> None:
        for sk in self.slots:
            sk.step_mode = bool(on)

    def commit_window(self, dest: int) -> None:
        w = self.win
        for sk in self.slots:
            if sk.k is None:
                continue
            sk.k[:, dest:dest + w].copy_(sk.k[:, -w:])
            sk.v[:, dest:dest + w].copy_(sk.v[:, -w:])


class RefModel:
    """The reference GPT as the drop-in sees it."""

    def __init__(self, cfg, state: dict, *, bf16: bool, device="cuda"):
        self.cfg = types.SimpleNamespace(**{f: getattr(cfg, f) for f in cfg.__dataclass_fields__})
        self._sd = {k: torch.as_tensor(np.asarray(v, np.float32)).to(device) for k, v in state.items()}
        self._ac_compute_dtype = torch.bfloat16 if bf16 else torch.float32
        from altxs_amd.model import build_itinerary

        self.n_slots = len(build_itinerary(cfg))

    def state_dict(self) -> dict:
        return self._sd

    def make_static_state(self, max_len: int, device, win: int = 1) -> RefStaticState:
        return RefStaticState(self.cfg, max_len, win, device, self._ac_compute_dtype, self.n_slots)

    def static_extend_fused(self, state: RefStaticState) -> None:
        from altxs_amd import dropin

        if int(state.win) > 1 and dropin.try_mega_encode(self, state):
            return
        if dropin.try_persistent_extend(self, state):
            return
        raise RuntimeError("no step tier ran (the reference would fall back to its eager step)")


class RefEngine:
    """StaticACEngine's slot-touching flow, on the device, W-window state plus
    the W=1 row state (XSA_AC_DECODE_ROW=1)."""

    def __init__(self, model: RefModel, oracle_cfg, oracle_sd: dict, *, win: int, block: int,
                 every: int, device="cuda"):
        self.model, self.win, self.block = model, int(win), int(block)
        self.vocab = int(model.cfg.vocab_size)
        self.device = torch.device(device)
        self.max_len = engine_max_len(block, every, win)
        self.state = model.make_static_state(self.max_len, self.device, win=self.win)
        self.row_state = model.make_static_state(self.max_len, self.device, win=1)
        self.oracle = OracleModel(oracle_cfg, oracle_sd, max_len=self.max_len)
        self._ctx_len = self._win_start = self._row_pos = 0
        self._carry = None
        self.uniform = np.full(self.vocab, 1.0 / self.vocab, dtype=np.float32)

    # -- incremental.py:858-897
    def reset_segment(self, prefix: np.ndarray, start: int) -> None:
        st = self.state
        _, ctx_start = chunk_ctx_start(int(start), self.block)
        ctx = np.asarray(prefix[ctx_start:start], dtype=np.int64)
        st.pos.fill_(0)
        self._ctx_len = self._win_start = int(ctx.shape[0])
        if ctx.size:
            st.set_step_mode(False)
            last = self._prefill(st, ctx)
            st.set_step_mode(True)
            st.prev_raw.copy_(self.oracle.sd["tok_emb.weight"][int(ctx[-1])].view(1, 1, -1))
            self._carry = softmax_np(last)
        else:
            st.prev_raw.zero_()
            self._carry = None
        self._rebind_packed_kv(st, getattr(self.model, "_encode_ws", None))
        self._sync_row_from_prefix()
        self._rebind_packed_kv(self.row_state, getattr(self.model, "_persist_ws", None))

    def _prefill(self, st: RefStaticState, ctx: np.ndarray) -> torch.Tensor:
        """prefill_cache(ids, kv_slots=st.slots): every slot's K/V rows [0, T)."""
        om = self.oracle
        ost = om.new_state()
        last = None
        for w0 in range(0, ctx.size, self.win):
            w = ctx[w0:w0 + self.win]
            last = om.step(ost, w)[-1]
            om.advance(ost, w.size)
        T = ctx.size
        dt = self.model._ac_compute_dtype
        for i, sk in enumerate(st.slots):
            like = torch.zeros(1, 1, om.Hkv, om.hd, dtype=dt, device=self.device)
            sk.ensure(like)
            sk.k[0, :T].copy_(ost.k[i][:T])
            sk.v[0, :T].copy_(ost.v[i][:T])
        return last

    # -- incremental.py:899-929
    def _rebind_packed_kv(self, state: RefStaticState, ws) -> None:
        if ws is None or getattr(ws, "k_pack", None) is None:
            return
        max_len, n_kv, hd = int(ws.max_len), int(ws.n_kv), int(ws.hd)
        n = min(int(self._ctx_len), max_len)
        for i, sk in enumerate(state.slots):
            if sk.k is None or sk.v is None:
                continue
            pack_k, pack_v = ws.k_pack[i], ws.v_pack[i]
            if sk.k.data_ptr() != pack_k.data_ptr():
                pack_k.copy_(sk.k.reshape(max_len, n_kv, hd).permute(1, 0, 2).to(dtype=pack_k.dtype))
                pack_v.copy_(sk.v.reshape(max_len, n_kv, hd).permute(1, 0, 2).to(dtype=pack_v.dtype))
                sk.k = pack_k.permute(1, 0, 2).unsqueeze(0)
                sk.v = pack_v.permute(1, 0, 2).unsqueeze(0)
            if n < max_len:
                pack_k[:, n:].zero_()
                pack_v[:, n:].zero_()

    # -- incremental.py:931-954
    def _sync_row_from_prefix(self) -> None:
        src, dst = self.state, self.row_state
        dst.prev_raw.copy_(src.prev_raw)
        dst.cand_prev_raw.zero_()
        dst.token.zero_()
        n = int(self._ctx_len)
        self._row_pos = n
        dst.pos.fill_(n)
        dst.set_step_mode(True)
        for a, b in zip(src.slots, dst.slots):
            if a.k is None:
                continue
            if b.k is None:
                b.ensure(a.k)
            if n > 0:
                b.k[:, :n].copy_(a.k[:, :n])
                b.v[:, :n].copy_(a.v[:, :n])
            if n < b.max_len:
                b.k[:, n:].zero_()
                b.v[:, n:].zero_()

    def carry_row(self) -> np.ndarray:
        return self.uniform if self._carry is None else self._carry

    def _probs(self, state: RefStaticState) -> np.ndarray:
        return torch.softmax(state.logits[0].float(), dim=-1).cpu().numpy().astype(np.float32)

    # -- incremental.py:1017-1052
    def run_window(self, tokens: np.ndarray, start_local: int) -> np.ndarray:
        st = self.state
        self._win_start = self._ctx_len + int(start_local)
        st.token.copy_(torch.as_tensor(np.asarray(tokens, np.int64)).view(1, -1))
        st.pos.fill_(self._win_start)
        self.model.static_extend_fused(st)
        return self._probs(st)

    def advance_window(self) -> None:
        self.state.commit_window(self._win_start)
        self.state.prev_raw.copy_(self.state.cand_prev_raw)

    # -- incremental.py:1054-1081
    def run_decode_row(self, token: int) -> np.ndarray:
        st = self.row_state
        st.token.fill_(int(token))
        st.pos.fill_(self._row_pos)
        self.model.static_extend_fused(st)
        probs = self._probs(st)
        st.commit_window(self._row_pos)
        st.prev_raw.copy_(st.cand_prev_raw)
        self._row_pos += 1
        return probs[0]

    # -- incremental.py:1238-1271
    def segment_rows_tf(self, arr: np.ndarray, seg, start: int) -> np.ndarray:
        self.reset_segment(arr, start)
        seg = np.asarray(seg, dtype=np.int64)
        n, win = seg.size, self.win
        rows = np.empty((n, self.vocab), dtype=np.float32)
        carry = self.carry_row()
        w0 = 0
        while w0 < n:
            valid = min(win, n - w0)
            tokens = np.zeros(win, dtype=np.int64)
            tokens[:valid] = seg[w0:w0 + valid]
            r = self.run_window(tokens, w0)
            rows[w0] = carry
            if valid > 1:
                rows[w0 + 1:w0 + valid] = r[:valid - 1]
            carry = r[valid - 1]
            if valid == win:
                self.advance_window()
            w0 += valid
        return rows

    # -- incremental.py:1221-1235
    def segment_rows_one_row(self, arr: np.ndarray, seg, start: int) -> np.ndarray:
        self.reset_segment(arr, start)
        seg = np.asarray(seg, dtype=np.int64)
        rows = np.empty((seg.size, self.vocab), dtype=np.float32)
        rows[0] = self.carry_row()
        for i in range(seg.size - 1):
            rows[i + 1] = self.run_decode_row(int(seg[i]))
        return rows
