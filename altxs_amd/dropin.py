"""The reference's own call signatures, served by libaltxs_hip.so.

A maintainer swaps these names into src/xsa_ttt and src/model without other
edits; every computation runs in the HIP library (no CPU path: a missing
library raises).

* :class:`GpuRangeCoder` <- ``GpuRangeCoder(device, *, max_bits, vocab)``
  (src/xsa_ttt/gpu_ac.py:397-479): ``encode_symbol(probs, symbol)``,
  ``finish() -> bytes``, ``begin_decode(payload)``, ``decode_symbol(probs)
  -> int64[1]``.  Tables come from the probabilities on the device by the
  reference's rule (``scale_p``, gpu_ac.py:38-42 == ``_scale_cum_np``); the
  bitstream is the reference's (MSB-first ``_pack_bits`` bytes).
* :func:`_scale_cum_np` / :func:`_scale_cum` <- src/model/arithmetic_coder_lm.py:49-87.
* :func:`encode_with_probs` / :func:`decode_with_probs` <-
  arithmetic_coder_lm.py:140-288 (same arguments, same bytes).
* :func:`try_persistent_extend` / :func:`try_mega_encode` <-
  persistent_step.py:1081-1119 / mega_encode.py:1693-1790: the W-token step
  into a reference-shaped ``StaticState`` (model.py:358-461) of a
  reference-shaped ``GPT`` (``model.cfg`` with the reference's config names,
  ``model.state_dict()`` with its parameter names).  The state's slots become
  views of the step's cache (:class:`_KVWorkspace`), so the engine's prefill,
  row sync and commits are what the step reads.  False (and disabled after an
  error, logged once) when the step cannot run, as the reference.
* :func:`prepare_persistent` / :func:`prepare_mega_encode` <-
  persistent_step.py:452-588 / mega_encode.py:1206-1351 (the workspace with
  ``k_pack`` / ``v_pack`` that ``_rebind_packed_kv`` and ``commit_packed_row``
  use); :func:`refresh_persistent_weights` / :func:`refresh_encode_weights`.
* :func:`load_codec` <- ``load_codec(codec_path, *, device)``
  (src/hyperflow_distillation/mixed_bit_delta.py:232-312), Init(seed)
  included (altxs_amd.init_seed).
* :func:`gemv_rows` / :func:`gemv_vec` / :func:`logits_stage_rows` <-
  src/xsa_ttt/ac_gemv.py:391-420, 562-582.
* :func:`ffn_stage_rows` <- ac_gemv.py:455-550 (the persistent tier's
  out-projection + MLP stages, with its rounding points) and
  :func:`run_split_attn` <- split_attn.py:341-425 (its decode / encode
  attention over ``ws.k_pack`` / ``ws.v_pack``), for callers that keep the
  reference's own workspace and swap only these stages.
"""

from __future__ import annotations

import ctypes
import dataclasses
import sys
from collections import OrderedDict
from typing import Callable, Sequence

import numpy as np
import torch

from . import _lib
from .codec import PackedTensor
from .coder import RangeCoder
from .config import AltxsConfig
from .model import CHUNK, StaticState, StepModel
from .synth import SynthModel

_CODE_BITS = 32


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(int(torch.cuda.current_stream(t.device).cuda_stream))


# ---- integer tables -----------------------------------------------------------
class _TableRows:
    """Device scratch for host probability rows -> integer tables."""

    def __init__(self):
        self.probs: torch.Tensor | None = None
        self.cum: torch.Tensor | None = None

    def tables(self, p: np.ndarray) -> np.ndarray:
        rows, V = p.shape
        if self.probs is None or self.probs.shape[0] < rows or self.probs.shape[1] != V:
            self.probs = torch.empty(max(rows, 1), V, dtype=torch.float64, device="cuda")
            self.cum = torch.empty(max(rows, 1), V + 1, dtype=torch.int32, device="cuda")
        pr, cm = self.probs[:rows], self.cum[:rows]
        pr.copy_(torch.from_numpy(p))
        rc = _lib.load().altxs_scale_cum_f64(pr.data_ptr(), rows, V, cm.data_ptr(), _stream(pr))
        _lib.check(rc, "altxs_scale_cum_f64")
        return cm.cpu().numpy().view(np.uint32).astype(np.int64)


_ROWS = _TableRows()


def _f64_rows(probs, n: int) -> np.ndarray:
    """One probability row as float64, the type the reference's rule converts
    every row to (arithmetic_coder_lm.py:56-59); fp32 values convert exactly."""
    if len(probs) != n:
        raise ValueError(f"probs_fn must return {n} probabilities, got {len(probs)}")
    return np.ascontiguousarray(np.asarray(probs, dtype=np.float64).reshape(1, n))


def _scale_cum_np(probs: Sequence[float], *, alphabet_size: int = 256) -> tuple[np.ndarray, int]:
    """probs -> (cum int64[V+1], total): f_i = max(1, floor(p_i * 1e6 + 0.5))
    in float64, cum_0 = 0 (arithmetic_coder_lm.py:49-64), computed by
    ``altxs_scale_cum_f64``."""
    n = int(alphabet_size)
    cum = _ROWS.tables(_f64_rows(probs, n))[0]
    return cum, int(cum[n])


def _scale_cum(probs: Sequence[float], *, alphabet_size: int = 256) -> tuple[list[int], int]:
    """The list form of :func:`_scale_cum_np` (arithmetic_coder_lm.py:67-87)."""
    cum, total = _scale_cum_np(probs, alphabet_size=alphabet_size)
    return cum.tolist(), total


# ---- range coder ----------------------------------------------------------------
class GpuRangeCoder:
    """One device range-coder stream with the reference's interface.  Buffer
    addresses never change, so a sequence of calls can be captured into a
    graph (the reference keeps its decode input fixed for the same reason)."""

    def __init__(self, device: torch.device, *, max_bits: int, vocab: int):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("GpuRangeCoder needs a GPU device")
        self.vocab = int(vocab)
        self.max_bits = int(max_bits)
        self._rc = RangeCoder(1, (self.max_bits + 7) // 8 + 8, device=self.device)
        self._cum = torch.zeros(1, self.vocab + 1, dtype=torch.int32, device=self.device)
        self._sym32 = torch.zeros(1, 1, dtype=torch.int32, device=self.device)
        self.sym = torch.zeros(1, dtype=torch.int64, device=self.device)
        self._lib = _lib.load()

    def _table(self, probs: torch.Tensor) -> None:
        # a float32 contiguous vector, cast like the reference's _probs_arg
        # (gpu_ac.py:415-426)
        p = probs.reshape(-1)
        if p.dtype != torch.float32 or not p.is_contiguous():
            p = p.float().contiguous()
        if p.numel() != self.vocab or p.device.type != "cuda":
            raise ValueError(f"probs must hold {self.vocab} values on the device")
        rc = self._lib.altxs_scale_cum(p.data_ptr(), 1, self.vocab, self._cum.data_ptr(), _stream(p))
        _lib.check(rc, "altxs_scale_cum")

    def encode_symbol(self, probs: torch.Tensor, symbol: torch.Tensor) -> None:
        self._table(probs)
        self._sym32.view(-1).copy_(symbol.view(-1)[:1])
        self._rc.encode(self._cum, self._sym32)

    def finish(self) -> bytes:
        return self._rc.finish()[0]

    def begin_decode(self, payload: bytes) -> None:
        if 8 * len(payload) > self.max_bits:
            raise ValueError(f"decode payload has {8 * len(payload)} bits, capacity is {self.max_bits}")
        self._rc.begin_decode([bytes(payload)])

    def decode_symbol(self, probs: torch.Tensor) -> torch.Tensor:
        self._table(probs)
        self._rc.decode(self._cum, self._sym32)
        self.sym.copy_(self._sym32.view(-1))
        return self.sym

    def check(self) -> None:
        """Raise if the device flagged a full buffer or an invalid symbol/table."""
        self._rc.check()


def encode_with_probs(symbols, probs_fn: Callable, *, desc: str | None = None,
                      alphabet_size: int = 256) -> bytes:
    """``probs_fn(i, symbols[:i])`` gives symbol i's distribution; returns the
    reference coder's bytes (arithmetic_coder_lm.py:140-191).  The rows are
    collected in order, turned into tables in one launch and coded in one
    launch on the device."""
    n = len(symbols)
    V = int(alphabet_size)
    syms = np.asarray(list(symbols) if isinstance(symbols, (bytes, bytearray, memoryview)) else symbols,
                      dtype=np.int64).reshape(-1)
    if ((syms < 0) | (syms >= V)).any():
        bad = int(syms[(syms < 0) | (syms >= V)][0])
        raise ValueError(f"symbol {bad} out of alphabet [0, {V})")
    if desc is not None:
        print(f"[{desc}] starting ({n} sym)…", file=sys.stderr, flush=True)
    rows = np.empty((max(n, 1), V), dtype=np.float64)
    for i in range(n):
        rows[i] = _f64_rows(probs_fn(i, symbols[:i]), V)[0]
    rc = RangeCoder(1, 64 + 4 * n)
    if n:
        pr = torch.from_numpy(rows[:n]).cuda()
        cum = torch.empty(n, V + 1, dtype=torch.int32, device="cuda")
        _lib.check(_lib.load().altxs_scale_cum_f64(pr.data_ptr(), n, V, cum.data_ptr(), _stream(pr)),
                   "altxs_scale_cum_f64")
        rc.encode(cum, torch.from_numpy(syms.astype(np.int32)).cuda().view(1, n))
    return rc.finish()[0]


def decode_with_probs(bitstream: bytes, n_symbols: int, probs_fn: Callable, *, desc: str | None = None,
                      out=None, hasher=None, return_bytes: bool = True, alphabet_size: int = 256):
    """Inverse of :func:`encode_with_probs` (arithmetic_coder_lm.py:194-288):
    ``probs_fn(i, decoded_so_far)`` per symbol; alphabets above 256 return a
    list of ids, 256 returns bytes (a bytearray with ``return_bytes=False``)."""
    V = int(alphabet_size)
    wide = V > 256
    buf = out if out is not None else ([] if wide else bytearray())
    if desc is not None:
        print(f"[{desc}] starting ({n_symbols} sym)…", file=sys.stderr, flush=True)
    rc = RangeCoder(1, len(bitstream) + 8)
    rc.begin_decode([bytes(bitstream)])
    dev_rows = torch.empty(1, V, dtype=torch.float64, device="cuda")
    cum = torch.empty(1, V + 1, dtype=torch.int32, device="cuda")
    sym = torch.empty(1, 1, dtype=torch.int32, device="cuda")
    L = _lib.load()
    for i in range(int(n_symbols)):
        dev_rows.copy_(torch.from_numpy(_f64_rows(probs_fn(i, buf), V)))
        _lib.check(L.altxs_scale_cum_f64(dev_rows.data_ptr(), 1, V, cum.data_ptr(), _stream(dev_rows)),
                   "altxs_scale_cum_f64")
        rc.decode(cum, sym)
        s = int(sym.item())
        buf.append(s)
        if hasher is not None:
            hasher.update(int(s).to_bytes(2, "little") if wide else bytes((s,)))
    rc.check()
    if wide:
        return list(buf)
    return bytes(buf) if return_bytes else buf


# ---- reference-shaped model and state ----------------------------------------------
def config_from_reference(ref_cfg) -> AltxsConfig:
    """The reference config object (XsaTttConfig field names) as an AltxsConfig."""
    fields = {f.name for f in dataclasses.fields(AltxsConfig)}
    src = ref_cfg if isinstance(ref_cfg, dict) else vars(ref_cfg)
    return AltxsConfig(**{k: v for k, v in src.items() if k in fields})


def dense_model_from_state(cfg: AltxsConfig, state: dict, device="cuda", bits: int = 16) -> SynthModel:
    """A reference-named state dict -> this build's weights: every matrix dense
    in the MFMA-tiled order, packed on the device -- bits 16: bf16, the
    reference's bf16 runtime banks (model.py:1183-1245); bits 32: the fp32
    values its fp32 compute mode keeps -- small parameters as fp32."""
    from .shipped import MODELED, pack_dense, split_init, tensor_shapes

    init = split_init(cfg, {k: v for k, v in state.items() if k in MODELED}, device)
    packed = {}
    for name, (n, k) in tensor_shapes(cfg).items():
        tiled = pack_dense(init[name].contiguous(), bits=bits)
        packed[name] = PackedTensor(name, bits, np.zeros((0, 0), np.uint16), np.zeros((0, 0), np.float16),
                                    tiled, np.zeros(0, np.float16), nk=(n, k))
    small = {k: torch.as_tensor(v).detach().float().cpu().numpy() for k, v in state.items()
             if k not in MODELED}
    return SynthModel(cfg, packed, small)


class _KVWorkspace:
    """The KV role of the reference's step workspaces (``_PersistWS`` /
    ``_EncodeWS``, persistent_step.py:452-588, mega_encode.py:1206-1351) over
    this build's cache.

    ``k_pack`` / ``v_pack`` are ``[n_slots, n_kv, max_len, hd]`` views of the
    step state's natural-order cache (bf16 for a bf16 model, fp32 otherwise),
    and every reference slot's ``k`` / ``v`` is re-pointed to a view of them
    exactly as ``prepare_persistent`` does (persistent_step.py:472-479), so the
    engine's eager prefill, ``_rebind_packed_kv``, ``_sync_row_from_prefix``
    (incremental.py:858-954), ``commit_window`` (model.py:449-461) and
    ``commit_packed_row`` (row_commit.py:59-98) all land in the memory the
    step reads.  The step keeps the reference's placement: prefix rows
    ``[0, pos)``, the window's K/V in the last W rows, committed by the caller.
    One workspace serves one state at a time, as the reference's does.
    """

    def __init__(self, adapter: "_Adapter", state):
        cfg = adapter.cfg
        self.win, self.max_len = int(state.win), int(state.max_len)
        self.n_slots, self.n_kv, self.hd = adapter.step.n_slots, cfg.num_kv_heads, cfg.head_dim
        self.d = cfg.model_dim
        if len(state.slots) not in (0, self.n_slots):
            raise ValueError(f"state has {len(state.slots)} slots, the model's itinerary {self.n_slots}")
        rows = (self.max_len + CHUNK - 1) // CHUNK * CHUNK
        self.st = adapter.step.make_static_state(rows, win=self.win, batch=1, want_probs=False,
                                                 want_cdf=False, rope_len=self.max_len,
                                                 kv_tail_end=self.max_len)
        self.k_pack = self.st.kv[:, 0, 0, :, :self.max_len]
        self.v_pack = self.st.kv[:, 0, 1, :, :self.max_len]
        self.adopt(state)

    def serves(self, state) -> bool:
        return (int(state.win) == self.win and int(state.max_len) == self.max_len
                and len(state.slots) in (0, self.n_slots))

    def adopt(self, state) -> None:
        """Point every slot of ``state`` at this cache, copying in what a slot
        held elsewhere (a fresh or reallocated ``StaticKV``)."""
        L, hkv, hd = self.max_len, self.n_kv, self.hd
        for i, sk in enumerate(state.slots):
            pk, pv = self.k_pack[i], self.v_pack[i]
            if sk.k is not None and sk.v is not None and sk.k.data_ptr() == pk.data_ptr() \
                    and sk.v.data_ptr() == pv.data_ptr() and sk.k.dtype == pk.dtype:
                continue
            if sk.k is not None and sk.v is not None:
                pk.copy_(sk.k.reshape(L, hkv, hd).permute(1, 0, 2))
                pv.copy_(sk.v.reshape(L, hkv, hd).permute(1, 0, 2))
            else:
                pk.zero_()
                pv.zero_()
            sk.k = pk.permute(1, 0, 2).unsqueeze(0)
            sk.v = pv.permute(1, 0, 2).unsqueeze(0)

    def run(self, step: StepModel, state) -> None:
        self.adopt(state)
        st, W = self.st, self.win
        V = step.cfg.vocab_size
        st.token.view(-1).copy_(state.token.view(-1)[:W])
        st.pos.view(-1).copy_(state.pos.view(-1)[:1])
        st.prev_raw.view(-1).copy_(state.prev_raw.reshape(-1)[:self.d])
        step.step(st, commit=False)
        state.logits.view(W, V).copy_(st.logits)
        state.cand_prev_raw.view(-1)[:self.d].copy_(st.cand_prev_raw.view(-1))


class _Adapter:
    """Per reference model: the step model built from its weights -- bf16
    banks and bf16 natural-order KV for a bf16 model; fp32 banks (bits 32) and
    fp32 KV for an fp32 one, the dtypes the reference computes in
    (model.py:1183-1196)."""

    def __init__(self, model, act: str):
        self.cfg = config_from_reference(model.cfg)
        sd = model.state_dict()
        dev = next((v.device for v in sd.values() if torch.is_tensor(v)), None)
        self.device = dev if dev is not None and dev.type == "cuda" else torch.device("cuda")
        self.act = act
        bits = 16 if act == "bf16" else 32
        self.step = StepModel(dense_model_from_state(self.cfg, sd, self.device, bits),
                              device=self.device, act=act, kv="bf16n" if act == "bf16" else "fp32")


def _adapter(model) -> _Adapter:
    ad = getattr(model, "_altxs_adapter", None)
    if ad is None:
        dt = getattr(model, "_ac_compute_dtype", None)
        ad = _Adapter(model, "bf16" if dt == torch.bfloat16 else "fp32")
        model._altxs_adapter = ad
    return ad


def _workspace(model, state, attr: str) -> _KVWorkspace:
    ws = getattr(model, attr, None)
    if not isinstance(ws, _KVWorkspace) or not ws.serves(state):
        ws = _KVWorkspace(_adapter(model), state)
        setattr(model, attr, ws)
    return ws


def prepare_persistent(model, state) -> _KVWorkspace | None:
    """The W=1 workspace (persistent_step.py:452-588): the cache the state's
    slots now view.  None when the step cannot serve this state."""
    if int(state.win) != 1:
        return None
    try:
        return _KVWorkspace(_adapter(model), state)
    except Exception as exc:  # noqa: BLE001 -- the reference returns None here
        print(f"[AC incr] altxs workspace unavailable ({exc!r})", file=sys.stderr, flush=True)
        return None


def prepare_mega_encode(model, state) -> _KVWorkspace | None:
    """The W-window workspace (mega_encode.py:1206-1351)."""
    if int(state.win) < 2:
        return None
    try:
        return _KVWorkspace(_adapter(model), state)
    except Exception as exc:  # noqa: BLE001
        print(f"[AC incr] altxs workspace unavailable ({exc!r})", file=sys.stderr, flush=True)
        return None


def refresh_weights(model) -> None:
    """Re-read the model's weights after an in-place update (e.g. a retrain;
    ``refresh_persistent_weights`` / ``refresh_encode_weights``,
    persistent_step.py:591-621); workspaces and their caches are kept."""
    ad = getattr(model, "_altxs_adapter", None)
    if ad is None:
        return
    new = _Adapter(model, ad.act)
    model._altxs_adapter = new
    for attr in ("_persist_ws", "_encode_ws"):
        ws = getattr(model, attr, None)
        if isinstance(ws, _KVWorkspace):  # same buffers, descriptors rebuilt for the new weights
            ws.st.model = new.step
            ws.st._descs.clear()


refresh_persistent_weights = refresh_weights
refresh_encode_weights = refresh_weights


def _try(model, state, flag: str, attr: str, what: str) -> bool:
    if getattr(model, flag, False):
        return False
    try:
        _workspace(model, state, attr).run(_adapter(model).step, state)
        return True
    except Exception as exc:  # noqa: BLE001 -- reference contract: log once, disable, fall back
        setattr(model, flag, True)
        print(f"[AC incr] {what} failed ({exc!r}); using the next tier", file=sys.stderr, flush=True)
        return False


def try_persistent_extend(model, state) -> bool:
    """The W=1 step (persistent_step.py:1081-1119): ``state.logits`` and
    ``state.cand_prev_raw`` from ``state.token``, ``state.pos``,
    ``state.prev_raw`` and the slots' prefix rows ``[0, pos)``; the token's
    K/V go to the slots' last row for the caller's commit.  False for W != 1
    (the reference's ``can_persistent``), and after an error (logged once)."""
    if int(state.win) != 1 or state.token.device.type != "cuda":
        return False
    return _try(model, state, "_persist_disabled", "_persist_ws", "altxs step")


def try_mega_encode(model, state) -> bool:
    """The W-token teacher-forced window (mega_encode.py:1693-1790), same
    placement: prefix ``[0, pos)``, window K/V in the last W rows.  False for
    W < 2 (``can_mega_encode``), and after an error."""
    if int(state.win) < 2 or state.token.device.type != "cuda":
        return False
    return _try(model, state, "_encode_disabled", "_encode_ws", "altxs window step")


# ---- shipped codec ------------------------------------------------------------------
def load_codec(codec_path, *, device, init_state: dict | None = None, act: str | None = None):
    """Decode a shipped codec into a step model: (StepModel, meta, small params)
    (mixed_bit_delta.py:232-312).

    Init(seed) is built here as the reference builds it (``enable_deterministic
    (seed)`` + ``build_model``; :func:`altxs_amd.init_seed.reference_init_state`)
    unless a state dict is passed in; the delta is decoded on the device, added
    to Init and packed (altxs_codec_decode, altxs_pack_dense[32]).  ``act``:
    "bf16" (bf16 banks, the reference's compute dtype with ``use_bf16``, its
    production setting) or "fp32" (fp32 banks); default from the codec's cfg."""
    import json

    from .init_seed import reference_init_state
    from .shipped import config_from_meta, load_shipped

    path = str(codec_path)
    stem = path[:-len(".safetensors")] if path.endswith(".safetensors") else path
    meta = json.load(open(stem + ".json", encoding="utf8"))
    if act is None:
        act = "bf16" if (meta.get("cfg") or {}).get("use_bf16", False) else "fp32"
    if act not in ("bf16", "fp32"):
        raise ValueError(act)
    if init_state is None:
        init_state = reference_init_state(config_from_meta(meta), int(meta["seed"]))
    cfg, weights, small = load_shipped(stem, init_state, device=device,
                                       bits=16 if act == "bf16" else 32)
    sm = SynthModel(cfg, weights, {k: np.asarray(v, np.float32) for k, v in small.items()})
    return StepModel(sm, device=device, act=act), meta, small


# ---- kernel-level helpers ------------------------------------------------------------
# Tiled bf16 copies of dense weights, keyed on where the values live; each entry
# keeps the weight's storage alive so its address cannot be reused by another
# tensor while cached, and the cache holds at most _TILED_MAX entries (oldest
# dropped first).
_TILED: "OrderedDict[tuple, tuple[int, object, torch.Tensor, _lib.QTensor]]" = OrderedDict()
_TILED_MAX = 256


def _tiled(weight: torch.Tensor) -> _lib.QTensor:
    """Dense [N, K] weight -> tiled copy (bits 16 for a bf16 weight, bits 32
    for an fp32 one: its exact value), cached until the weight changes in
    place (torch's version counter)."""
    from .shipped import pack_dense

    key = (weight.untyped_storage().data_ptr(), weight.storage_offset(), tuple(weight.shape),
           tuple(weight.stride()), weight.dtype, weight.device)
    hit = _TILED.get(key)
    ver = weight._version
    if hit is not None and hit[0] == ver:
        _TILED.move_to_end(key)
        return hit[3]
    n, k = weight.shape
    if n % 16 or k % 256:
        raise ValueError(f"weight [{n}, {k}]: N must be a multiple of 16 and K of 256")
    if weight.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("weights must be bf16 or fp32")
    bits = 16 if weight.dtype == torch.bfloat16 else 32
    tiled = pack_dense(weight.detach().float().contiguous(), bits=bits)
    qt = _lib.QTensor(tiled.data_ptr(), tiled.data_ptr(), n, k, bits, 0)
    _TILED[key] = (ver, weight.untyped_storage(), tiled, qt)
    _TILED.move_to_end(key)
    while len(_TILED) > _TILED_MAX:
        _TILED.popitem(last=False)
    return qt


_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}
_RMS_ROUND_ROW, _RMS_ROUND_SCALE = 1, 2  # ALTXS_RMS_ROUND_ROW / ALTXS_RMS_ROUND_SCALE


def gemv_rows(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor) -> None:
    """``out[r] = weight @ x[r]`` for x [win, K], out [win, N] (ac_gemv.py:391-420)."""
    win, k = int(x.shape[0]), int(weight.shape[1])
    n_out = int(weight.shape[0])
    if int(x.shape[1]) != k or tuple(out.shape) != (win, n_out):
        raise ValueError(f"gemv_rows shape mismatch x={tuple(x.shape)} w={tuple(weight.shape)} "
                         f"out={tuple(out.shape)}")
    if x.dtype not in _DT or not x.is_contiguous():
        raise ValueError("x must be a contiguous fp32/bf16/fp16 device tensor")
    qt = _tiled(weight)
    if qt.bits == 32 and x.dtype != torch.float32:  # fp32 weights: fp32 products of the widened x
        x = x.float()
    y = out if (out.dtype == torch.float32 and out.is_contiguous()) else \
        torch.empty(win, n_out, dtype=torch.float32, device=x.device)
    _lib.check(_lib.load().altxs_qgemm(ctypes.byref(qt), x.data_ptr(), _DT[x.dtype], win, y.data_ptr(),
                                       _stream(x)), "altxs_qgemm")
    if y is not out:
        out.copy_(y)


def gemv_vec(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor) -> None:
    """1-D ``out = weight @ x`` (ac_gemv.py:423-425)."""
    gemv_rows(x.view(1, -1), weight, out.view(1, -1))


def logits_stage_rows(src: torch.Tensor, weight: torch.Tensor, logit_buf: torch.Tensor, *,
                      eps: float = 1e-6) -> None:
    """Final RMS -> LM projection: ``logit_buf[r] = weight @ rms(src[r])``
    (ac_gemv.py:312-359, 562-582) with the reference's rounding points: the
    rsqrt factor in ``src``'s dtype, the product in ``src``'s dtype, then in
    the weight's dtype (bf16 ``src``: factor and row rounded to bf16; fp32
    ``src`` with a bf16 weight: the row rounded to bf16; both fp32: none)."""
    win, d = int(src.shape[0]), int(src.shape[1])
    vocab = int(weight.shape[0])
    if tuple(logit_buf.shape) != (win, vocab) or int(weight.shape[1]) != d:
        raise ValueError("stage-fused logit buffer shape mismatch")
    qt = _tiled(weight)
    x = src if (src.dtype == torch.float32 and src.is_contiguous()) else src.float().contiguous()
    y = logit_buf if (logit_buf.dtype == torch.float32 and logit_buf.is_contiguous()) else \
        torch.empty(win, vocab, dtype=torch.float32, device=src.device)
    if src.dtype == torch.bfloat16:
        if weight.dtype != torch.bfloat16:
            raise ValueError("a bf16 src row with an fp32 weight is not a reference combination")
        rounding = _RMS_ROUND_ROW | _RMS_ROUND_SCALE
    elif src.dtype == torch.float32:
        rounding = _RMS_ROUND_ROW if weight.dtype == torch.bfloat16 else 0
    else:
        raise ValueError("src must be fp32 or bf16")
    rc = _lib.load().altxs_rms_qgemm(ctypes.byref(qt), x.data_ptr(), win, 1.0, float(eps),
                                     rounding, y.data_ptr(), _stream(src))
    _lib.check(rc, "altxs_rms_qgemm")
    if y is not logit_buf:
        logit_buf.copy_(y)


# ---- stage-level helpers of the stage-fused row path ----------------------------

def _act_code(t: torch.Tensor, what: str) -> int:
    if t.dtype == torch.float32:
        return _lib.F32
    if t.dtype == torch.bfloat16:
        return _lib.BF16
    raise ValueError(f"{what} must be fp32 or bf16, got {t.dtype}")


def ffn_stage_rows(*, y: torch.Tensor, out_w: torch.Tensor, hid: torch.Tensor, a_sc: torch.Tensor,
                   xin: torch.Tensor, attn_s: torch.Tensor, src: torch.Tensor, up_w: torch.Tensor,
                   ln: torch.Tensor, scr: torch.Tensor, down_w: torch.Tensor, m_sc: torch.Tensor,
                   x: torch.Tensor, lane0: torch.Tensor, lane1: torch.Tensor, pr: torch.Tensor,
                   pp: torch.Tensor, skips: torch.Tensor, skip_dst: int, par: bool,
                   eps: float = 1e-6) -> None:
    """Out-projection -> MLP up/activation -> MLP down/commit for ``win`` rows
    as three stream-ordered launches (ac_gemv.py:455-550; stage kernels
    89-310), with the reference's rounding to the workspace dtype at every
    point its kernels round.  Activations and parameters (a_sc, m_sc, ln, pr,
    pp) share one dtype, fp32 or bf16; weights are dense bf16 or fp32 [N, K]
    tensors (tiled once and cached, like :func:`gemv_rows`).  ``src`` is
    ``xin`` for sequential slots and ``lane1`` for parallel ones
    (persistent_step.py:760-766)."""
    win, d = int(y.shape[0]), int(y.shape[1])
    mlp = int(scr.shape[1])
    if int(ln.numel()) != 1:
        raise ValueError(f"ln must be the per-layer scalar ln_scale_factor, got {ln.numel()} values")
    if tuple(hid.shape) != (win, d) or tuple(xin.shape) != (win, d):
        raise ValueError("stage-fused FFN hidden shape mismatch")
    act = _act_code(y, "y")
    named = dict(y=y, hid=hid, a_sc=a_sc, xin=xin, attn_s=attn_s, src=src, ln=ln, scr=scr, m_sc=m_sc,
                 x=x, lane0=lane0, lane1=lane1, pr=pr, pp=pp, skips=skips)
    for name, t in named.items():
        if t is None:
            continue
        if t.dtype != y.dtype or not t.is_contiguous() or t.device != y.device:
            raise ValueError(f"{name} must be a contiguous {y.dtype} tensor on {y.device}")
    for name, t, shape in (("a_sc", a_sc, (d,)), ("m_sc", m_sc, (d,)), ("scr", scr, (win, mlp)),
                           ("src", src, (win, d))):
        if tuple(t.shape) != shape:
            raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {shape}")
    if par:
        if int(pr.numel()) != 2 or int(pp.numel()) != 4:
            raise ValueError("pr must hold 2 and pp 4 values (the layer's parallel lambdas)")
        for name, t in (("attn_s", attn_s), ("lane0", lane0), ("lane1", lane1)):
            if t is None or tuple(t.shape) != (win, d):
                raise ValueError(f"{name} must be a [{win}, {d}] tensor in a parallel slot")
        if attn_s.data_ptr() == y.data_ptr():
            raise ValueError("attn_s must not alias y (stage 1 reads every column of y)")
    else:
        if x is None or tuple(x.shape) != (win, d):
            raise ValueError(f"x must be a [{win}, {d}] tensor in a sequential slot")
        if skip_dst >= 0 and (skips is None or skips.dim() != 3 or tuple(skips.shape[1:]) != (win, d)
                              or int(skips.shape[0]) <= skip_dst):
            raise ValueError(f"skip_dst={skip_dst}: skips must be [n > skip_dst, {win}, {d}]")
    a = _lib.FfnStageArgs()
    a.win, a.d, a.mlp, a.act_dtype = win, d, mlp, act
    a.parallel, a.skip_dst, a.eps = int(bool(par)), int(skip_dst) if not par else -1, float(eps)
    a.out_w, a.up_w, a.down_w = _tiled(out_w), _tiled(up_w), _tiled(down_w)
    for name, t in named.items():
        setattr(a, name, None if t is None else t.data_ptr())
    _lib.check(_lib.load().altxs_ffn_stage_rows(ctypes.byref(a), _stream(y)), "altxs_ffn_stage_rows")


_SPLIT_NORM_EPS = 1e-12  # the XSA norm floor the attention kernels use (persistent_step.py:36)


def run_split_attn(*, ws, pos: torch.Tensor, slot: int, rows: int, layer: int, use_xsa: int,
                   use_gate: int, v_cur: torch.Tensor, v_cur_row_stride: int, tail_at_pos: bool,
                   norm_eps: float, block_l: int) -> bool:
    """Decode / encode attention of one slot over ``ws.k_pack`` / ``ws.v_pack``
    ([slots, n_kv, max_len, hd], the reference's packed layout) into ``ws.y``
    (split_attn.py:341-425): row r attends to keys [0, pos + r) and then to
    the current key (row max_len - 1, or pos + r with ``tail_at_pos``), then
    XSA and the sparse gate sigmoid(attn_in[r, :gate_n] . gate_w[layer, h]).

    The natural-order MFMA decode kernel runs it (the key splits, ``block_l``
    and the split workspace are the reference kernel's own launch shape and
    have no role here; its work split is fixed, so its bits do not depend on
    them).  bf16 caches: q and the softmax weights enter the products in bf16
    as the reference's tl.dot operands; the current key is scored with the
    same bf16 q (the reference scores it with the fp32 q).  fp32 caches: fp32
    products.  ``v_cur`` equals the cache's current value row at both
    reference call sites (mega_step.py:1006, mega_encode.py:345-372); XSA
    reads it there.  Always True (the reference's False asks for its serial
    kernel)."""
    if abs(float(norm_eps) - _SPLIT_NORM_EPS) > 0:
        raise ValueError(f"norm_eps={norm_eps}: the attention kernels use {_SPLIT_NORM_EPS}")
    k_pack, v_pack = ws.k_pack, ws.v_pack
    if k_pack.shape != v_pack.shape or k_pack.dtype != v_pack.dtype or k_pack.dim() != 4:
        raise ValueError("k_pack/v_pack must be equal [slots, n_kv, max_len, hd] tensors")
    if not (k_pack.is_contiguous() and v_pack.is_contiguous()):
        raise ValueError("k_pack/v_pack must be contiguous")
    n_slots, n_kv, max_len, hd = (int(s) for s in k_pack.shape)
    H = int(ws.n_heads)
    if int(ws.n_kv) != n_kv or int(ws.hd) != hd or int(ws.max_len) != max_len:
        raise ValueError("ws.n_kv / hd / max_len disagree with k_pack")
    if not 0 <= int(slot) < n_slots:
        raise ValueError(f"slot {slot} outside k_pack's {n_slots} slots")
    if k_pack.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("k_pack must be bf16 or fp32")
    rows = int(rows)
    if rows < 1:
        raise ValueError(f"rows={rows}")
    if use_xsa and v_cur is None:
        raise ValueError("use_xsa needs v_cur")
    q_all = ws.q.reshape(-1, H, hd)
    if int(q_all.shape[0]) < rows or int(pos.numel()) < 1:
        raise ValueError(f"ws.q holds {q_all.shape[0]} rows of {H} heads, {rows} asked; pos must be set")
    q = q_all[:rows].float().contiguous()
    p0 = pos.reshape(-1)[:1].to(device=q.device, dtype=torch.int32)
    a = _lib.AttnArgs()
    a.H, a.Hkv, a.head_dim, a.max_len = H, n_kv, hd, max_len
    if tail_at_pos or rows == 1:
        # one sequence window: row r at pos + r (in place, or the tail row)
        a.B, a.W, pvec = 1, rows, p0
        a.kv_seg_stride = n_kv * max_len * hd
        a.kv_tail_end = 0 if tail_at_pos else max_len
    else:
        # every row scores the shared tail row: rows as segments of one cache
        a.B, a.W = rows, 1
        pvec = p0 + torch.arange(rows, dtype=torch.int32, device=q.device)
        a.kv_seg_stride = 0
        a.kv_tail_end = max_len
    a.kv_bf16 = _lib.KV_BF16_NATURAL if k_pack.dtype == torch.bfloat16 else _lib.KV_F32
    off = int(slot) * n_kv * max_len * hd * k_pack.element_size()
    a.q, a.k, a.v = q.data_ptr(), k_pack.data_ptr() + off, v_pack.data_ptr() + off
    a.pos = pvec.data_ptr()
    a.use_xsa = int(bool(use_xsa))
    a.flags = _lib.ATTN_OPS_BF16
    gate = None
    if use_gate:
        attn_in, gw = ws.attn_in, ws.gate_w[layer]
        gate_n = int(ws.gate_n)
        if attn_in.dtype != gw.dtype or not gw.is_contiguous() or attn_in.stride(-1) != 1:
            raise ValueError("attn_in and gate_w must share a dtype, unit-stride rows")
        if tuple(gw.shape) != (H, gate_n):
            raise ValueError(f"gate_w[layer] has shape {tuple(gw.shape)}, expected {(H, gate_n)}")
        if attn_in.dim() != 2 or int(attn_in.shape[0]) < rows or int(attn_in.shape[1]) < gate_n:
            raise ValueError(f"attn_in must hold {rows} rows of at least {gate_n} features")
        gate = torch.empty(rows, H, dtype=torch.float32, device=q.device)
        rc = _lib.load().altxs_attn_gate(attn_in.data_ptr(), _act_code(attn_in, "attn_in"),
                                         attn_in.stride(0), gw.data_ptr(), H, gate_n, rows,
                                         gate.data_ptr(), _stream(q))
        _lib.check(rc, "altxs_attn_gate")
    a.gate = None if gate is None else gate.data_ptr()
    y_out = ws.y
    if y_out.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("ws.y must be fp32 or bf16")
    a.y_bf16 = int(y_out.dtype == torch.bfloat16)
    direct = y_out.is_contiguous() and y_out.numel() >= rows * H * hd
    y = y_out if direct else torch.empty(rows, H * hd, dtype=y_out.dtype, device=q.device)
    a.y = y.data_ptr()
    a.err = None
    _lib.check(_lib.load().altxs_decode_attn(ctypes.byref(a), _stream(q)), "altxs_decode_attn")
    if not direct:
        y_out.reshape(-1, H * hd)[:rows].copy_(y)
    return True
