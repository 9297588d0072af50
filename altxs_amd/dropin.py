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
  ``model.state_dict()`` with its parameter names).  False (and disabled
  after an error, logged once) when the step cannot run, as the reference.
* :func:`load_codec` <- ``load_codec(codec_path, *, device)``
  (src/hyperflow_distillation/mixed_bit_delta.py:232-312).
* :func:`gemv_rows` / :func:`gemv_vec` / :func:`logits_stage_rows` <-
  src/xsa_ttt/ac_gemv.py:391-420, 562-582.

The reference's per-stage helpers ``ffn_stage_rows`` (ac_gemv.py:455-550) and
``run_split_attn`` (split_attn.py:341-425) act on the internal workspace of
the persistent tier (``_PersistWS``: its scratch rows and its packed KV
layout); ``try_persistent_extend`` replaces that tier whole, so they have no
standalone counterpart here.
"""

from __future__ import annotations

import ctypes
import dataclasses
import sys
from typing import Any, Callable, Sequence

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
            self.probs = torch.empty(max(rows, 1), V, dtype=torch.float32, device="cuda")
            self.cum = torch.empty(max(rows, 1), V + 1, dtype=torch.int32, device="cuda")
        pr, cm = self.probs[:rows], self.cum[:rows]
        pr.copy_(torch.from_numpy(p))
        rc = _lib.load().altxs_scale_cum(pr.data_ptr(), rows, V, cm.data_ptr(), _stream(pr))
        _lib.check(rc, "altxs_scale_cum")
        return cm.cpu().numpy().view(np.uint32).astype(np.int64)


_ROWS = _TableRows()


def _fp32_rows(probs, n: int) -> np.ndarray:
    p = np.asarray(probs)
    if p.size != n:
        raise ValueError(f"probs_fn must return {n} probabilities, got {p.size}")
    p32 = p.astype(np.float32).reshape(1, n)
    if p.dtype != np.float32 and not np.array_equal(p32.astype(np.float64), p.astype(np.float64).reshape(1, n)):
        raise ValueError("probabilities must be float32 values (the device rule reads fp32 rows)")
    return np.ascontiguousarray(p32)


def _scale_cum_np(probs: Sequence[float], *, alphabet_size: int = 256) -> tuple[np.ndarray, int]:
    """probs -> (cum int64[V+1], total): f_i = max(1, floor(p_i * 1e6 + 0.5)),
    cum_0 = 0 (arithmetic_coder_lm.py:49-64), computed by ``altxs_scale_cum``."""
    n = int(alphabet_size)
    cum = _ROWS.tables(_fp32_rows(probs, n))[0]
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
        p = probs.view(-1)
        if p.dtype != torch.float32 or not p.is_contiguous() or p.numel() != self.vocab:
            raise ValueError(f"probs must be {self.vocab} contiguous float32 values on the device")
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
    rows = np.empty((max(n, 1), V), dtype=np.float32)
    for i in range(n):
        rows[i] = _fp32_rows(probs_fn(i, symbols[:i]), V)[0]
    rc = RangeCoder(1, 64 + 4 * n)
    if n:
        pr = torch.from_numpy(rows[:n]).cuda()
        cum = torch.empty(n, V + 1, dtype=torch.int32, device="cuda")
        _lib.check(_lib.load().altxs_scale_cum(pr.data_ptr(), n, V, cum.data_ptr(), _stream(pr)),
                   "altxs_scale_cum")
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
    dev_rows = torch.empty(1, V, dtype=torch.float32, device="cuda")
    cum = torch.empty(1, V + 1, dtype=torch.int32, device="cuda")
    sym = torch.empty(1, 1, dtype=torch.int32, device="cuda")
    L = _lib.load()
    for i in range(int(n_symbols)):
        dev_rows.copy_(torch.from_numpy(_fp32_rows(probs_fn(i, buf), V)))
        _lib.check(L.altxs_scale_cum(dev_rows.data_ptr(), 1, V, cum.data_ptr(), _stream(dev_rows)),
                   "altxs_scale_cum")
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


def dense_model_from_state(cfg: AltxsConfig, state: dict, device="cuda") -> SynthModel:
    """A reference-named state dict -> this build's weights: every matrix as
    bf16 in the MFMA-tiled order (bits 16, the reference's runtime banks,
    model.py:1183-1245) packed on the device; small parameters as fp32."""
    from .shipped import MODELED, pack_dense, split_init, tensor_shapes

    init = split_init(cfg, {k: v for k, v in state.items() if k in MODELED}, device)
    packed = {}
    for name, (n, k) in tensor_shapes(cfg).items():
        tiled = pack_dense(init[name].contiguous())
        packed[name] = PackedTensor(name, 16, np.zeros((0, 0), np.uint16), np.zeros((0, 0), np.float16),
                                    tiled, np.zeros(0, np.float16), nk=(n, k))
    small = {k: torch.as_tensor(v).detach().float().cpu().numpy() for k, v in state.items()
             if k not in MODELED}
    return SynthModel(cfg, packed, small)


class _Adapter:
    """Per reference model: the step model and one mirror state per reference state."""

    def __init__(self, model, act: str):
        self.cfg = config_from_reference(model.cfg)
        dev = next((v.device for v in model.state_dict().values() if torch.is_tensor(v)), None)
        self.device = dev if dev is not None and dev.type == "cuda" else torch.device("cuda")
        self.step = StepModel(dense_model_from_state(self.cfg, model.state_dict(), self.device),
                              device=self.device, act=act, kv=act)
        self.states: dict[int, tuple[Any, StaticState]] = {}

    def mirror(self, state) -> StaticState:
        hit = self.states.get(id(state))
        if hit is not None and hit[0] is state:
            return hit[1]
        W, L = int(state.win), int(state.max_len)
        st = self.step.make_static_state((L + CHUNK - 1) // CHUNK * CHUNK, win=W, batch=1,
                                         want_probs=False, want_cdf=False, rope_len=L)
        self.states[id(state)] = (state, st)
        return st

    def run(self, state) -> None:
        st = self.mirror(state)
        W, D, V = st.win, self.cfg.model_dim, self.cfg.vocab_size
        st.token.view(-1).copy_(state.token.view(-1)[:W])
        st.pos.view(-1).copy_(state.pos.view(-1)[:1])
        st.prev_raw.view(-1).copy_(state.prev_raw.reshape(-1)[:D])
        self.step.step(st, commit=False)
        state.logits.view(W, V).copy_(st.logits)
        state.cand_prev_raw.view(-1)[:D].copy_(st.cand_prev_raw.view(-1))


def _adapter(model) -> _Adapter:
    ad = getattr(model, "_altxs_adapter", None)
    if ad is None:
        dt = getattr(model, "_ac_compute_dtype", None)
        ad = _Adapter(model, "bf16" if dt == torch.bfloat16 else "fp32")
        model._altxs_adapter = ad
    return ad


def refresh_weights(model) -> None:
    """Re-read the model's weights (after they were changed in place, e.g. by a
    retrain); states and their KV caches are kept."""
    ad = getattr(model, "_altxs_adapter", None)
    if ad is not None:
        states = ad.states
        new = _Adapter(model, "bf16" if ad.step.act_bf16 else "fp32")
        new.states = {}
        model._altxs_adapter = new
        for key, (ref_state, st) in states.items():  # keep the caches: rebuild descriptors only
            st.model = new.step
            st._descs.clear()
            new.states[key] = (ref_state, st)


def _try(model, state, flag: str, what: str) -> bool:
    if getattr(model, flag, False):
        return False
    try:
        _adapter(model).run(state)
        return True
    except Exception as exc:  # noqa: BLE001 -- reference contract: log once, disable, fall back
        setattr(model, flag, True)
        print(f"[AC incr] {what} failed ({exc!r}); using the next tier", file=sys.stderr, flush=True)
        return False


def try_persistent_extend(model, state) -> bool:
    """The W=1 step into ``state.logits`` / ``state.cand_prev_raw`` from
    ``state.token``, ``state.pos`` and ``state.prev_raw`` (persistent_step.py:1081)."""
    return _try(model, state, "_persist_disabled", "altxs step")


def try_mega_encode(model, state) -> bool:
    """The W-token teacher-forced window into ``state`` (mega_encode.py:1693)."""
    return _try(model, state, "_encode_disabled", "altxs window step")


# ---- shipped codec ------------------------------------------------------------------
def load_codec(codec_path, *, device, init_state: dict, act: str = "bf16"):
    """Decode a shipped codec into a step model: (StepModel, meta, small params).

    The reference builds Init(seed) itself (``build_model`` after
    ``enable_deterministic(seed)``, mixed_bit_delta.py:251-262); here it comes
    in as that model's state dict (``init_state``), and the delta is decoded,
    added and packed on the device (altxs_codec_decode, altxs_pack_dense)."""
    import json

    from .shipped import load_shipped

    path = str(codec_path)
    stem = path[:-len(".safetensors")] if path.endswith(".safetensors") else path
    cfg, weights, small = load_shipped(stem, init_state, device=device)
    meta = json.load(open(stem + ".json", encoding="utf8"))
    sm = SynthModel(cfg, weights, {k: np.asarray(v, np.float32) for k, v in small.items()})
    return StepModel(sm, device=device, act=act), meta, small


# ---- kernel-level helpers ------------------------------------------------------------
_TILED: dict[int, tuple[int, int, torch.Tensor, _lib.QTensor]] = {}


def _tiled(weight: torch.Tensor) -> _lib.QTensor:
    """Dense [N, K] weight -> bits-16 tiled copy, cached until the weight
    changes in place (torch's version counter)."""
    from .shipped import pack_dense

    key = weight.data_ptr()
    hit = _TILED.get(key)
    ver = weight._version
    if hit is not None and hit[0] == ver and hit[1] == tuple(weight.shape):
        return hit[3]
    n, k = weight.shape
    if n % 16 or k % 256:
        raise ValueError(f"weight [{n}, {k}]: N must be a multiple of 16 and K of 256")
    tiled = pack_dense(weight.detach().float().contiguous())
    qt = _lib.QTensor(tiled.data_ptr(), tiled.data_ptr(), n, k, 16, 0)
    _TILED[key] = (ver, (n, k), tiled, qt)
    return qt


_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


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
    (ac_gemv.py:562-582); bf16 ``src`` rounds the normalised row to bf16 for
    the products as the reference's bf16 path does."""
    win, d = int(src.shape[0]), int(src.shape[1])
    vocab = int(weight.shape[0])
    if tuple(logit_buf.shape) != (win, vocab) or int(weight.shape[1]) != d:
        raise ValueError("stage-fused logit buffer shape mismatch")
    qt = _tiled(weight)
    x = src if (src.dtype == torch.float32 and src.is_contiguous()) else src.float().contiguous()
    y = logit_buf if (logit_buf.dtype == torch.float32 and logit_buf.is_contiguous()) else \
        torch.empty(win, vocab, dtype=torch.float32, device=src.device)
    rc = _lib.load().altxs_rms_qgemm(ctypes.byref(qt), x.data_ptr(), win, 1.0, float(eps),
                                     int(src.dtype == torch.bfloat16), y.data_ptr(), _stream(src))
    _lib.check(rc, "altxs_rms_qgemm")
    if y is not logit_buf:
        logit_buf.copy_(y)
