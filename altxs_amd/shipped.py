"""The reference's shipped codec -> dense bf16 weights for the step, on the device.

The reference ships a model as Init(seed) + a per-channel mixed-bit delta
(src/hyperflow_distillation/mixed_bit_delta.py: ``load_codec`` 232-312,
``dequantize_channels`` 172-229, ``_from_channels`` 116-144) and runs it on
dense bf16 banks (model.py:1183-1245).  Here the deltas are decoded by
``altxs_codec_decode`` straight into this build's per-layer tensors (q/k/v
rows of ``l{i}.qkv``; o and down channels land as columns), the reference's
own Init(seed) state is added and the sum is rounded to bf16 in the
MFMA-tiled order by ``altxs_pack_dense``: the result is a set of bits-16
weights the step reads like the packed ones.

Init(seed) is the reference model's construction (``build_model`` after
``enable_deterministic(seed)``); it is passed in as its state dict
(reference names), so no part of the reference's init is restated here.
"""

from __future__ import annotations

import dataclasses
import json
from typing import Callable

import numpy as np
import torch

from . import _lib
from .codec import PackedTensor
from .config import AltxsConfig

MODELED = ("tok_emb.weight", "qo_bank", "kv_bank", "mlp_up_bank", "mlp_down_bank")


def channel_ranks(bits: np.ndarray) -> np.ndarray:
    """Rank of each channel among the channels of its width (int32; 0 for dead ones)."""
    bits = np.asarray(bits).reshape(-1)
    rank = np.zeros(bits.size, dtype=np.int32)
    for b in (2, 3, 4):
        idx = np.flatnonzero(bits == b)
        rank[idx] = np.arange(idx.size, dtype=np.int32)
    return rank


@dataclasses.dataclass
class Part:
    """Channels [c0, c0 + n) of a bank -> tensor `dest` at `offset`, channel j
    at offset + j*stride_ch, value i at + i*stride_el (elements)."""

    c0: int
    n: int
    dest: str
    offset: int
    stride_ch: int
    stride_el: int


def bank_parts(cfg: AltxsConfig) -> dict[str, list[Part]]:
    """Where each channel of each modeled bank goes in this build's tensors
    (the inverse of synth.SynthModel.state_dict; _from_channels semantics)."""
    L, d, kvd, F = cfg.num_layers, cfg.model_dim, cfg.kv_dim, cfg.hidden_dim
    parts: dict[str, list[Part]] = {n: [] for n in MODELED}
    parts["tok_emb.weight"].append(Part(0, cfg.vocab_size, "emb", 0, d, 1))
    for l in range(L):
        parts["qo_bank"].append(Part(l * d, d, f"l{l}.qkv", 0, d, 1))            # q rows
        parts["qo_bank"].append(Part(L * d + l * d, d, f"l{l}.o", 0, 1, d))      # o columns
        parts["kv_bank"].append(Part(l * kvd, kvd, f"l{l}.qkv", d * d, d, 1))    # k rows
        parts["kv_bank"].append(Part(L * kvd + l * kvd, kvd, f"l{l}.qkv", (d + kvd) * d, d, 1))
        parts["mlp_up_bank"].append(Part(l * F, F, f"l{l}.up", 0, d, 1))         # up rows
        parts["mlp_down_bank"].append(Part(l * F, F, f"l{l}.down", 0, 1, F))     # down columns
    return parts


def tensor_shapes(cfg: AltxsConfig) -> dict[str, tuple[int, int]]:
    from .synth import tensor_list

    return {name: (n, k) for name, n, k in tensor_list(cfg)}


def split_init(cfg: AltxsConfig, init_state: dict[str, torch.Tensor], device) -> dict[str, torch.Tensor]:
    """Reference-named Init(seed) banks -> this build's tensors (fp32, device)."""
    L = cfg.num_layers
    f = {k: torch.as_tensor(v).to(device=device, dtype=torch.float32) for k, v in init_state.items()
         if k in MODELED}
    out = {"emb": f["tok_emb.weight"].contiguous()}
    for l in range(L):
        out[f"l{l}.qkv"] = torch.cat([f["qo_bank"][l], f["kv_bank"][l], f["kv_bank"][L + l]]).contiguous()
        out[f"l{l}.o"] = f["qo_bank"][L + l].contiguous()
        out[f"l{l}.up"] = f["mlp_up_bank"][l].contiguous()
        out[f"l{l}.down"] = f["mlp_down_bank"][l].contiguous()
    return out


class DeviceBank:
    """One modeled bank's codec arrays on the device (the three width groups)."""

    def __init__(self, bits: np.ndarray, packed: dict[int, np.ndarray], codebooks: dict[int, np.ndarray],
                 mode: str, scales: dict[int, np.ndarray] | None, device):
        mode = str(mode).lower().strip()
        if mode not in _lib.CODEBOOK_MODES:
            raise ValueError(f"unsupported codebook mode {mode!r}")
        bits = np.asarray(bits, dtype=np.uint8).reshape(-1).copy()
        if mode == "fp4":  # dequantize_channels: every live channel is 4-bit FP4
            bits[bits > 0] = 4
        self.n_channels = bits.size
        self.bits = torch.from_numpy(bits).to(device)
        self.rank = torch.from_numpy(channel_ranks(bits)).to(device)
        self.g = _lib.CodecGroups()
        self.g.mode = _lib.CODEBOOK_MODES[mode]
        self._keep = [self.bits, self.rank]
        for b in (2, 3, 4):
            pk = np.ascontiguousarray(packed.get(b, np.zeros(0, np.uint8)), dtype=np.uint8).reshape(-1)
            if mode == "shared":  # per-channel scales in `codebook`, the shared levels aside
                cb = np.asarray(scales[b], dtype=np.float16).reshape(-1) if scales and b in scales \
                    else np.zeros(0, np.float16)
                sh = np.asarray(codebooks.get(b, np.zeros(0)), dtype=np.float16).reshape(-1)
            else:
                cb = np.asarray(codebooks.get(b, np.zeros(0)), dtype=np.float16).reshape(-1)
                sh = np.zeros(0, np.float16)
            tp = torch.from_numpy(pk.copy()).to(device)
            tc = torch.from_numpy(cb.view(np.int16).copy()).to(device)
            ts = torch.from_numpy(sh.view(np.int16).copy()).to(device)
            self._keep += [tp, tc, ts]
            codes = (pk.size // 3) * 8 if b == 3 else pk.size * (8 // b)
            self.g.packed[b - 2] = tp.data_ptr() if tp.numel() else None
            self.g.codebook[b - 2] = tc.data_ptr() if tc.numel() else None
            self.g.shared[b - 2] = ts.data_ptr() if (ts.numel() >= (1 << b)) else None
            self.g.n_codes[b - 2] = codes if tp.numel() and tc.numel() else 0
            self.g.n_book[b - 2] = cb.size

    def decode(self, part: Part, width: int, out: torch.Tensor, err: torch.Tensor) -> None:
        """Decode the part's channels into `out` (fp32, contiguous) at its offsets."""
        if part.c0 < 0 or part.c0 + part.n > self.n_channels:
            raise ValueError("bank part outside the bank")
        need = part.offset + (part.n - 1) * part.stride_ch + (width - 1) * part.stride_el + 1
        if out.dtype != torch.float32 or not out.is_contiguous() or need > out.numel():
            raise ValueError("destination too small or not contiguous fp32")
        L = _lib.load()
        stream = ctypes_stream(out)
        _lib.check(L.altxs_codec_decode(self.g, self.bits.data_ptr() + part.c0,
                                        self.rank.data_ptr() + 4 * part.c0, part.n, width,
                                        out.data_ptr() + 4 * part.offset, part.stride_ch, part.stride_el,
                                        err.data_ptr(), stream), "altxs_codec_decode")


def ctypes_stream(t: torch.Tensor):
    import ctypes

    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def pack_dense(delta: torch.Tensor, base: torch.Tensor | None = None, bits: int = 16) -> torch.Tensor:
    """base + delta in the MFMA-tiled order (uint8 device tensor): bits 16
    rounds it to bf16, bits 32 keeps the fp32 value as three exact bf16 planes."""
    n, k = delta.shape
    if delta.dtype != torch.float32 or not delta.is_contiguous():
        raise ValueError("delta must be contiguous fp32 [N, K]")
    if base is not None and (base.shape != delta.shape or base.dtype != torch.float32
                             or not base.is_contiguous()):
        raise ValueError("base must match delta")
    nbytes = dense_bytes(n, k, bits)
    out = torch.empty(nbytes, dtype=torch.uint8, device=delta.device)
    L = _lib.load()
    b = base.data_ptr() if base is not None else None
    if bits == 16:
        rc = L.altxs_pack_dense(b, delta.data_ptr(), n, k, k, out.data_ptr(), ctypes_stream(delta))
    else:
        rc = L.altxs_pack_dense32(b, delta.data_ptr(), n, k, k, out.data_ptr(), nbytes, ctypes_stream(delta))
    _lib.check(rc, "altxs_pack_dense")
    return out


def dense_bytes(n: int, k: int, bits: int) -> int:
    """Bytes of a dense [n, k] tensor: bf16 values (bits 16), or three bf16
    planes of the fp32 values (bits 32)."""
    if bits == 16:
        return n * k * 2
    if bits == 32:
        return n * k * 6
    raise ValueError(f"dense bits {bits} not in (16, 32)")


def decode_to_dense(cfg: AltxsConfig, banks: dict[str, DeviceBank], width: int,
                    init: dict[str, torch.Tensor] | None, device, bits: int = 16) -> dict[str, PackedTensor]:
    """Every modeled bank decoded into this build's tensors, Init added, packed
    as dense weights (bits 16: bf16, the reference's bf16 banks; bits 32:
    fp32; PackedTensor with device-resident tiles)."""
    shapes = tensor_shapes(cfg)
    deltas = {name: torch.zeros(n * k, dtype=torch.float32, device=device) for name, (n, k) in shapes.items()}
    err = torch.zeros(1, dtype=torch.int32, device=device)
    for bank, parts in bank_parts(cfg).items():
        for part in parts:
            banks[bank].decode(part, width, deltas[part.dest], err)
    if int(err.item()):
        raise RuntimeError("shipped codec: a channel's codes or codebook entries are out of range")
    out = {}
    for name, (n, k) in shapes.items():
        d = deltas[name].view(n, k)
        base = init[name] if init is not None else None
        tiled = pack_dense(d, base, bits)
        out[name] = PackedTensor(name, bits, np.zeros((0, 0), np.uint16), np.zeros((0, 0), np.float16),
                                 tiled, np.zeros(0, np.float16), nk=(n, k))
    return out


def config_from_meta(meta: dict) -> AltxsConfig:
    """The codec's ``cfg`` block (reference config names) as an AltxsConfig."""
    fields = {f.name for f in dataclasses.fields(AltxsConfig)}
    return AltxsConfig(**{k: v for k, v in (meta.get("cfg") or {}).items() if k in fields})


def load_shipped(codec_path: str, init_state: dict[str, torch.Tensor],
                 config_from_meta: Callable[[dict], AltxsConfig] = config_from_meta, device="cuda",
                 bits: int = 16):
    """Read a shipped codec (``<stem>.json`` + ``<stem>.safetensors``, loaded
    with safetensors: no code runs from the file) and return (cfg, dense
    tensors on the device -- bits 16 or 32, as :func:`decode_to_dense` --,
    small params as reference-named numpy arrays)."""
    from safetensors.numpy import load_file

    stem = codec_path[:-len(".safetensors")] if codec_path.endswith(".safetensors") else codec_path
    meta = json.load(open(stem + ".json", encoding="utf8"))
    if meta.get("format") != "hope_mixed_bit_delta":
        raise ValueError("not a mixed-bit delta codec")
    if meta.get("compact"):
        raise ValueError("compact (zlib) payloads are not supported")
    if meta.get("global_lora"):
        raise ValueError("codecs with a global-LoRA residual are not supported")
    cfg = config_from_meta(meta)
    state = load_file(stem + ".safetensors")
    mode = str(meta.get("codebook_mode", "lloyd"))
    width = None
    banks = {}
    for name in MODELED:
        layout = meta["layouts"][name]
        w = int(layout["channel_width"])
        if width is None:
            width = w
        if w != width or w != cfg.model_dim:
            raise ValueError("channel width must equal model_dim")
        key = lambda kind, *rest: "/".join((kind, name) + rest)  # noqa: E731
        if key("fp16") in state:
            raise ValueError(f"{name}: fp16 channels are not supported")
        packed = {b: state[key("packed", f"b{b}")] for b in (2, 3, 4) if key("packed", f"b{b}") in state}
        books = {b: state[key("codebook", f"b{b}")] for b in (2, 3, 4) if key("codebook", f"b{b}") in state}
        scales = {b: state[key("scale", f"b{b}")] for b in (2, 3, 4) if key("scale", f"b{b}") in state}
        banks[name] = DeviceBank(state[key("bits")], packed, books, mode, scales or None, device)
    init = split_init(cfg, init_state, device)
    weights = decode_to_dense(cfg, banks, width, init, device, bits)
    small = {n: state["small/" + n] for n in meta["small_params"] if "small/" + n in state}
    return cfg, weights, small
