"""Device model + static state for the per-symbol step (host side of the C-ABI).

Mirrors the reference's step surface (src/xsa_ttt/model.py):

* :meth:`StepModel.make_static_state` <- ``GPT.make_static_state``
  (model.py:1581-1615), batched over B independent segments;
* :meth:`StepModel.static_extend` <- ``GPT.static_extend`` /
  ``static_extend_fused`` (model.py:1617-1647): one W-token step, K/V written
  at ``pos + t``, logits into ``state.logits``, the window's last raw
  embedding into ``state.cand_prev_raw``; ``pos`` untouched;
* :meth:`StaticState.commit_window` / :meth:`StepModel.advance_window`
  <- ``StaticState.commit_window`` + the engine's ``advance_window``
  (model.py:449-461, incremental.py:1049-1052): here K/V already sit at their
  final rows, so committing is ``pos += W`` and ``prev_raw = cand``;
* :func:`try_persistent_extend` <- ``try_persistent_extend(model, state)``
  (persistent_step.py:1081-1119): returns False and disables itself on error.

All compute runs in libaltxs_hip.so on the current torch stream; there is no
CPU fallback.
"""

from __future__ import annotations

import ctypes
import sys

import numpy as np
import torch

from . import _lib, hiprt
from .config import AltxsConfig, slot_itinerary
from .synth import SynthModel, rope_table

NORM_EPS = float(np.finfo(np.float32).eps)  # F.rms_norm(eps=None) on fp32 (model.py:114-120)
CHUNK = 256


def build_itinerary(cfg: AltxsConfig) -> list[dict]:
    """Slot list as _static_extend_body walks it (model.py:1649-1781)."""
    enc, dec = slot_itinerary(cfg)
    n_skip = min(len(enc), len(dec))
    slots = []
    stack = []
    for i in enc:
        stack.append(len(slots))
        slots.append(dict(layer=i, kind=_lib.SLOT_SEQ, skip_idx=-1, skip_src=-1, first_parallel=0))
    psl = cfg.parallel_start_layer
    seen_par = False
    for j, i in enumerate(dec):
        par = psl > 0 and i >= psl
        if seen_par and not par:
            raise ValueError("a sequential decoder slot after a parallel one is not supported")
        src = stack.pop() if (j < n_skip and stack) else -1
        slots.append(dict(layer=i, kind=_lib.SLOT_PAR if par else _lib.SLOT_SEQ,
                          skip_idx=j if src >= 0 else -1, skip_src=src,
                          first_parallel=int(par and not seen_par)))
        seen_par = seen_par or par
    return slots


def _dev(a, device, dtype=torch.float32) -> torch.Tensor:
    return torch.as_tensor(np.ascontiguousarray(a)).to(device=device, dtype=dtype).contiguous()


def _stream_ptr(device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


# Steps of at least this many rows (B x W) run the large-tile GEMMs (the
# library's threshold), which read the expanded weight values when present.
BIG_ROWS = 1024


class StaticState:
    """Caller-owned device buffers of a B x W step (addresses stay fixed)."""

    def __init__(self, model: "StepModel", batch: int, win: int, max_len: int,
                 want_probs: bool = True, want_cdf: bool = True, split: bool = False,
                 persistent: bool = False, rope_len: int | None = None, kv_tail_end: int = 0):
        cfg, dev = model.cfg, model.device
        if max_len % CHUNK:
            raise ValueError(f"max_len must be a multiple of {CHUNK}")
        self.model = model
        self.batch, self.win, self.max_len = int(batch), int(win), int(max_len)
        # > 0: the window's K/V go to rows kv_tail_end - W + t (the reference's
        # tail rows) and the caller commits them into the prefix; natural layouts
        self.kv_tail_end = int(kv_tail_end)
        if self.kv_tail_end and (model.kv_layout == _lib.KV_BF16
                                 or not self.win <= self.kv_tail_end <= self.max_len):
            raise ValueError(f"kv_tail_end={kv_tail_end} needs a natural KV layout and "
                             f"W <= kv_tail_end <= max_len")
        # length the RoPE table is warmed at (sets the YaRN scale); rows kept = max_len
        self.rope_len = int(rope_len) if rope_len is not None else self.max_len
        B, W, V, D = self.batch, self.win, cfg.vocab_size, cfg.model_dim
        R = B * W
        self.token = torch.zeros(B, W, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(B, dtype=torch.int32, device=dev)
        self.prev_raw = torch.zeros(B, D, dtype=torch.float32, device=dev)
        self.cand_prev_raw = torch.zeros(B, D, dtype=torch.float32, device=dev)
        kv_dtype = torch.float32 if model.kv_layout == _lib.KV_F32 else torch.bfloat16
        self.kv = torch.zeros(model.n_slots, B, 2, cfg.num_kv_heads, self.max_len, cfg.head_dim,
                              dtype=kv_dtype, device=dev)
        self.logits = torch.zeros(R, V, dtype=torch.float32, device=dev)
        self.probs = torch.zeros(R, V, dtype=torch.float32, device=dev) if want_probs else None
        self.cum = torch.zeros(R, V + 1, dtype=torch.int32, device=dev) if want_cdf else None
        self.err = torch.zeros(1, dtype=torch.int32, device=dev)
        # split mode: a second stream + ordering events, owned here (the C-ABI never allocates)
        self.split = bool(split) and B >= 2
        self.aux_stream = torch.cuda.Stream(device=dev) if self.split else None
        self.sync_events = (hiprt.EventArray(2 * model.n_slots + 2, timing=False)
                            if self.split else None)
        if R >= BIG_ROWS and model.act_bf16 and model.expand is not False:
            model.expand_codes()  # the large-tile GEMMs of this state read the expanded values
        self._descs: dict[int, _lib.StepDesc] = {}
        # decode states reserve the fused out-projection's terms (StepModel.fuse_o)
        desc = self._desc(_lib.F_FUSE_O if win == 1 else 0)
        nbytes = _lib.load().altxs_step_workspace_bytes(ctypes.byref(desc))
        self.ws = torch.empty(int(nbytes), dtype=torch.uint8, device=dev)
        self._descs.clear()
        # persistent layer kernel: plan built once for these buffers (device copy + host image)
        self.persistent = False  # set once the plan exists (the descriptor then points at it)
        if persistent:
            L = _lib.load()
            desc = self._desc(0)
            nb = int(L.altxs_step_plan_bytes(ctypes.byref(desc)))
            if nb <= 0:
                raise RuntimeError("altxs_step_plan_bytes failed")
            self.plan_dev = torch.empty(nb, dtype=torch.uint8, device=dev)
            self.plan_host = (ctypes.c_uint8 * nb)()
            rc = L.altxs_step_plan_build(ctypes.byref(desc), ctypes.cast(self.plan_host, ctypes.c_void_p),
                                         ctypes.c_void_p(self.plan_dev.data_ptr()), nb,
                                         ctypes.c_void_p(_stream_ptr(dev)))
            _lib.check(rc, "altxs_step_plan_build")
            self.persistent = True
            self._descs.clear()

    def kv_slot(self, slot: int) -> torch.Tensor:
        """[B, 2, Hkv, max_len, hd] view of one slot's cache."""
        return self.kv[slot]

    def _desc(self, flags: int, width: int | None = None) -> _lib.StepDesc:
        w = self.win if width is None else int(width)
        d = self._descs.get((flags, w))
        if d is None:
            d = self.model._fill_desc(self, flags)
            if w != self.win:  # a narrower window over the same buffers (first B*w rows)
                if not 1 <= w <= self.win or self.split or self.persistent:
                    raise ValueError(f"width {w} not usable on this state")
                d.W = w
            self._descs[(flags, w)] = d
        return d

    def tokens(self, width: int | None = None) -> torch.Tensor:
        """The [B, width] token buffer a step of that width reads (a view)."""
        w = self.win if width is None else int(width)
        return self.token.view(-1)[:self.batch * w].view(self.batch, w)

    def commit_window(self) -> None:
        """pos += W; prev_raw = cand (K/V rows are already in place)."""
        self.pos += self.win
        self.prev_raw.copy_(self.cand_prev_raw)

    def check_errors(self) -> None:
        e = int(self.err.item())
        if e:
            raise RuntimeError(f"altxs device error flags 0x{e:x} (1 = position >= max_len, "
                               "2 = token id out of range, 4 = a persistent-kernel wait gave up)")


class StepModel:
    """Packed weights + small params resident in HBM."""

    def __init__(self, synth: SynthModel, *, device="cuda", act: str = "bf16",
                 kv: str | None = None, expand: bool | None = None):
        """``expand``: expanded copies of the packed tensors (altxs_expand_codes,
        N*K*2 bytes each) for steps of at least BIG_ROWS rows, whose large-tile
        GEMMs then read them instead of decoding codes -- the same operands, the
        same bits.  None: made when the first such state is; False: never;
        True: now."""
        cfg = synth.cfg
        cfg.validate()
        if act not in ("bf16", "fp32"):
            raise ValueError(act)
        kv = kv or act
        if kv not in ("bf16", "fp32", "bf16n"):
            raise ValueError(kv)
        if cfg.head_dim != 64:
            raise ValueError("head_dim must be 64")
        if cfg.model_dim % 256 or cfg.hidden_dim % 256:
            raise ValueError("model_dim and hidden dim must be multiples of 256")
        self.lib = _lib.load()
        self.cfg = cfg
        self.device = torch.device(device)
        self.act_bf16 = act == "bf16"
        # "bf16": MFMA-tiled bf16 cache; "bf16n": bf16 in the natural (reference
        # k_pack) order; "fp32": natural fp32
        self.kv_layout = {"fp32": _lib.KV_F32, "bf16": _lib.KV_BF16, "bf16n": _lib.KV_BF16_NATURAL}[kv]
        self.kv_bf16 = kv == "bf16"
        self.slots = build_itinerary(cfg)
        self.n_slots = len(self.slots)
        dev = self.device
        self._keep: list[torch.Tensor] = []
        self.qt: dict[str, _lib.QTensor] = {}
        for name, p in synth.packed.items():
            if isinstance(p.tiled, torch.Tensor):  # tiles built on the device (shipped codec)
                codes = p.tiled.to(dev)
            else:
                codes = torch.from_numpy(np.ascontiguousarray(p.tiled)).to(dev)
            scales = torch.from_numpy(np.ascontiguousarray(p.tiled_scales).view(np.int16)).to(dev)
            self._keep += [codes, scales]
            n, k = p.shape
            self.qt[name] = _lib.QTensor(codes.data_ptr(), scales.data_ptr(), n, k, p.bits, 0)
        sm = synth.small
        self.small = {k: _dev(v, dev) for k, v in sm.items() if "_loras." not in k}
        # LoRA matrices in fp16 (the values are fp16-exact), as the C-ABI reads them
        self.lora = {k: _dev(v, dev, torch.float16) for k, v in sm.items() if "_loras." in k}
        self.synth = synth
        self._cos_cache: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}
        self._disabled = False
        # True: decode steps form the out-projection inside the attention
        # launch and finish it where it is read (ALTXS_F_FUSE_O; the same bits,
        # slower on the benchmark model)
        self.fuse_o = False
        self.expand = expand
        self._expanded = False
        if expand:
            self.expand_codes()

    def expand_codes(self) -> None:
        """Expanded copies of the packed QKV, out-projection and MLP-up tensors
        (the stages whose large-row GEMMs read them; bits 2/3/4/6), once; each
        QTensor's ``expanded`` then points at its copy."""
        if self._expanded:
            return
        stream = ctypes.c_void_p(_stream_ptr(self.device))
        for name, qt in self.qt.items():
            if qt.bits not in (2, 3, 4, 6) or not name.endswith((".qkv", ".o", ".up")):
                continue
            out = torch.empty(qt.N * qt.K, dtype=torch.bfloat16, device=self.device)
            _lib.check(self.lib.altxs_expand_codes(ctypes.byref(qt), out.data_ptr(), stream),
                       "altxs_expand_codes")
            self._keep.append(out)
            qt.expanded = out.data_ptr()
        self._expanded = True

    def rope(self, max_len: int, rope_len: int | None = None):
        """cos/sin rows [0, max_len) of the table warmed at ``rope_len`` (default
        max_len), as ``Rotary.forward(rope_len)`` builds it (model.py:147-192)."""
        key = (int(max_len), int(rope_len) if rope_len is not None else int(max_len))
        t = self._cos_cache.get(key)
        if t is None:
            cos, sin = rope_table(self.cfg, key[0], key[1])
            t = (cos.to(self.device).contiguous(), sin.to(self.device).contiguous())
            self._cos_cache[key] = t
        return t

    def make_static_state(self, max_len: int, device=None, win: int = 1, batch: int = 1,
                          want_probs: bool = True, want_cdf: bool = True,
                          split: bool = False, persistent: bool = False,
                          rope_len: int | None = None, kv_tail_end: int = 0) -> StaticState:
        """``split``: run the segments as two groups on two streams (B >= 2).
        ``persistent``: run every slot in one persistent launch (bf16 KV, W | 16).
        ``rope_len``: the length the RoPE table is warmed at (default max_len);
        the reference engine warms it at its static length (incremental.py:239-242).
        ``kv_tail_end``: keep the window's K/V in rows kv_tail_end - W + t, the
        reference StaticKV's tail (model.py:259-461), for the caller to commit."""
        return StaticState(self, batch, win, max_len, want_probs, want_cdf, split, persistent,
                           rope_len, kv_tail_end)

    def _fill_desc(self, st: StaticState, flags: int) -> _lib.StepDesc:
        cfg = self.cfg
        d = _lib.StepDesc()
        d.abi_version = _lib.ABI_VERSION
        d.B, d.W, d.D, d.H, d.Hkv = st.batch, st.win, cfg.model_dim, cfg.num_heads, cfg.num_kv_heads
        d.head_dim, d.F, d.V = cfg.head_dim, cfg.hidden_dim, cfg.vocab_size
        d.n_layers, d.n_slots, d.max_len = cfg.num_layers, self.n_slots, st.max_len
        d.gate_window, d.rope_dims = cfg.gate_window, cfg.rope_dims_eff
        d.lora_rank = cfg.lora_rank if self.lora else 0
        d.act_bf16, d.kv_bf16 = int(self.act_bf16), int(self.kv_layout)
        d.kv_tail_end = int(getattr(st, "kv_tail_end", 0))
        f = flags
        if cfg.smear_gate_enabled:
            f |= _lib.F_SMEAR
        if cfg.sparse_attn_gate_enabled:
            f |= _lib.F_SPARSE_GATE
        if cfg.skip_gates_enabled:
            f |= _lib.F_SKIP_GATES
        if cfg.asym_logit_rescale:
            f |= _lib.F_ASYM_SOFTCAP
        lane = cfg.parallel_final_lane.lower()
        if lane == "attn":
            f |= _lib.F_FINAL_ATTN
        elif lane == "mlp":
            f |= _lib.F_FINAL_MLP
        d.flags = f
        d.norm_eps, d.gate_scale, d.logit_softcap = NORM_EPS, cfg.sparse_attn_gate_scale, cfg.logit_softcap
        sm = self.small
        L = cfg.num_layers
        for i in range(L):
            ly = d.layers[i]
            ly.qkv, ly.o = self.qt[f"l{i}.qkv"], self.qt[f"l{i}.o"]
            ly.up, ly.down = self.qt[f"l{i}.up"], self.qt[f"l{i}.down"]
            ly.resid_mix = sm[f"blocks.{i}.resid_mix"].data_ptr()
            ly.attn_scale = sm[f"blocks.{i}.attn_scale"].data_ptr()
            ly.mlp_scale = sm[f"blocks.{i}.mlp_scale"].data_ptr()
            ly.q_gain = sm[f"blocks.{i}.attn.q_gain"].data_ptr()
            g = sm.get(f"blocks.{i}.attn.attn_gate_w")
            ly.attn_gate_w = g.data_ptr() if g is not None else None
            ly.par_resid = sm["parallel_resid_lambdas"][i].data_ptr()
            ly.par_post = sm["parallel_post_lambdas"][i].data_ptr()
            ly.ln_scale = float(1.0 / np.sqrt(i + 1)) if cfg.ln_scale else 1.0
            ly.use_xsa = int(cfg.xsa_last_n > 0 and i >= L - cfg.xsa_last_n)
        for s, sl in enumerate(self.slots):
            o = d.slots[s]
            o.layer, o.kind, o.skip_idx = sl["layer"], sl["kind"], sl["skip_idx"]
            o.skip_src, o.first_parallel = sl["skip_src"], sl["first_parallel"]
            if self.lora:
                o.lora_scale = cfg.lora_alpha / cfg.lora_rank
                o.lora_q_a = self.lora[f"q_loras.{s}.A"].data_ptr()
                o.lora_q_b = self.lora[f"q_loras.{s}.B"].data_ptr()
                o.lora_v_a = self.lora[f"v_loras.{s}.A"].data_ptr()
                o.lora_v_b = self.lora[f"v_loras.{s}.B"].data_ptr()
        d.emb = self.qt["emb"]
        d.skip_weights = sm["skip_weights"].data_ptr()
        d.skip_gates = sm["skip_gates"].data_ptr() if "skip_gates" in sm else None
        if cfg.smear_gate_enabled:
            d.smear_w = sm["smear_gate.weight"].data_ptr()
            d.smear_lambda = sm["smear_lambda"].data_ptr()
        if cfg.asym_logit_rescale:
            if "softcap_pn" not in sm:
                sm["softcap_pn"] = torch.stack([sm["softcap_pos"].reshape(()),
                                                sm["softcap_neg"].reshape(())]).contiguous()
            d.softcap_pn = sm["softcap_pn"].data_ptr()
        cos, sin = self.rope(st.max_len, getattr(st, "rope_len", None))
        d.rope_cos, d.rope_sin = cos.data_ptr(), sin.data_ptr()
        d.tokens, d.pos = st.token.data_ptr(), st.pos.data_ptr()
        d.prev_raw, d.cand_raw = st.prev_raw.data_ptr(), st.cand_prev_raw.data_ptr()
        d.kv = st.kv.data_ptr()
        if hasattr(st, "ws"):
            d.ws, d.ws_bytes = st.ws.data_ptr(), st.ws.numel()
        d.logits = st.logits.data_ptr()
        d.probs = st.probs.data_ptr() if st.probs is not None else None
        d.cum = st.cum.data_ptr() if st.cum is not None else None
        d.err = st.err.data_ptr()
        if getattr(st, "split", False):
            d.aux_stream = int(st.aux_stream.cuda_stream)
            d.sync_events = st.sync_events.ptr
        if getattr(st, "persistent", False):
            d.plan_dev = st.plan_dev.data_ptr()
            d.plan_host = ctypes.cast(st.plan_host, ctypes.c_void_p)
            d.plan_bytes = st.plan_dev.numel()
        return d

    # ---- the step -------------------------------------------------------------
    def step(self, st: StaticState, *, commit: bool = False, renorm: bool = False,
             attn_events: int | None = None, width: int | None = None) -> None:
        """Enqueue one step on the current stream.

        ``attn_events``: optional address of 2*n_slots hipEvent_t handles,
        recorded around each slot's attention launch (timing hook); with a
        persistent state, events 0 and 1 bracket the layer kernel.
        ``width``: run a window of that many tokens (<= the state's W) over the
        same buffers -- tokens in ``st.tokens(width)``, outputs in the first
        B*width rows; a commit advances pos by width.
        """
        flags = (_lib.F_COMMIT if commit else 0) | (_lib.F_RENORM if renorm else 0)
        if self.fuse_o:
            flags |= _lib.F_FUSE_O
        d = st._desc(flags, width)
        d.attn_events = attn_events
        rc = self.lib.altxs_step(ctypes.byref(d), ctypes.c_void_p(_stream_ptr(self.device)))
        _lib.check(rc, "altxs_step")

    def fuses_out_proj(self, st: StaticState, slot: int = 0) -> bool:
        """Whether a step on ``st`` forms slot ``slot``'s out-projection inside
        its attention launch (altxs_step_fuses_out_proj)."""
        flags = _lib.F_FUSE_O if self.fuse_o else 0
        v = int(self.lib.altxs_step_fuses_out_proj(ctypes.byref(st._desc(flags)), int(slot)))
        if v < 0:
            raise ValueError(f"altxs_step_fuses_out_proj: bad slot {slot}")
        return v == 1

    def static_extend(self, st: StaticState) -> None:
        """One W-token window at ``pos`` (logits, probs, CDFs); pos unchanged."""
        self.step(st, commit=False)

    static_extend_fused = static_extend

    def advance_window(self, st: StaticState) -> None:
        st.commit_window()

    def decode_row(self, st: StaticState, tokens) -> None:
        """W=1 step that also commits (run_decode_row_dev, incremental.py:1083-1101)."""
        if st.win != 1:
            raise ValueError("decode_row needs a W=1 state")
        st.token.copy_(torch.as_tensor(np.asarray(tokens).reshape(st.batch, 1), dtype=torch.int32))
        self.step(st, commit=True)


def try_persistent_extend(model: StepModel, state: StaticState) -> bool:
    """Drop-in for persistent_step.try_persistent_extend: True if the HIP step ran."""
    if model._disabled:
        return False
    try:
        model.static_extend(state)
        return True
    except Exception as exc:  # noqa: BLE001 -- reference contract: log once, disable, fall back
        model._disabled = True
        print(f"[altxs] HIP step disabled: {exc!r}", file=sys.stderr, flush=True)
        return False
