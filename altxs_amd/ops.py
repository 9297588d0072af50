"""torch-facing wrappers of the standalone C-ABI entry points.

Each wrapper validates shapes on the host, launches on the current torch
stream and never synchronises.  Names follow the reference call sites they
replace:

* :func:`scale_cum`     <- ``_scale_cum_np(probs, alphabet_size)``
  (src/model/arithmetic_coder_lm.py:49-64), batched over rows;
* :func:`softmax_cdf`   <- ``torch.softmax(logits, -1, out=probs_dev)``
  (src/xsa_ttt/incremental.py:603-605) + ``_scale_cum_np``;
* :func:`dequant`       <- ``dequantize_channels`` (mixed_bit_delta.py:172-229);
* :func:`qgemm`         <- ``gemv_rows(x, w, out)`` (src/xsa_ttt/ac_gemv.py:391-420);
* :func:`decode_attn`   <- ``run_split_attn`` (src/xsa_ttt/split_attn.py:341-425).
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from .codec import PackedTensor


def _s(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(int(torch.cuda.current_stream(t.device).cuda_stream))


def _need(t: torch.Tensor, dtype, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def scale_cum(probs: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """probs fp32 [..., V] -> cum int32 (uint32 values) [..., V+1]."""
    _need(probs, torch.float32, "probs")
    V = probs.shape[-1]
    rows = probs.numel() // V
    if out is None:
        out = torch.empty(probs.shape[:-1] + (V + 1,), dtype=torch.int32, device=probs.device)
    _need(out, torch.int32, "out")
    rc = _lib.load().altxs_scale_cum(probs.data_ptr(), rows, V, out.data_ptr(), _s(probs))
    _lib.check(rc, "altxs_scale_cum")
    return out


def softmax_cdf(logits: torch.Tensor, *, renorm: bool = False, want_probs: bool = True,
                want_cdf: bool = True):
    """Deterministic fp32 softmax (+ renorm) and integer CDF rows."""
    _need(logits, torch.float32, "logits")
    V = logits.shape[-1]
    rows = logits.numel() // V
    probs = torch.empty_like(logits) if want_probs else None
    cum = (torch.empty(logits.shape[:-1] + (V + 1,), dtype=torch.int32, device=logits.device)
           if want_cdf else None)
    rc = _lib.load().altxs_softmax_cdf(
        logits.data_ptr(), rows, V, _lib.CDF_RENORM if renorm else 0,
        probs.data_ptr() if probs is not None else None,
        cum.data_ptr() if cum is not None else None, _s(logits))
    _lib.check(rc, "altxs_softmax_cdf")
    return probs, cum


class DeviceQTensor:
    """A packed tensor uploaded to HBM (keeps its buffers alive)."""

    def __init__(self, p: PackedTensor, device="cuda"):
        self.codes = torch.from_numpy(np.ascontiguousarray(p.tiled)).to(device)
        self.scales = torch.from_numpy(np.ascontiguousarray(p.tiled_scales).view(np.int16)).to(device)
        self.N, self.K = p.shape
        self.bits = p.bits
        self.qt = _lib.QTensor(self.codes.data_ptr(), self.scales.data_ptr(), self.N, self.K,
                               self.bits, 0)


def dequant(w: DeviceQTensor) -> torch.Tensor:
    out = torch.empty(w.N, w.K, dtype=torch.float32, device=w.codes.device)
    rc = _lib.load().altxs_dequant(ctypes.byref(w.qt), out.data_ptr(), _s(out))
    _lib.check(rc, "altxs_dequant")
    return out


_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def qgemm(w: DeviceQTensor, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """y[rows, N] = x[rows, K] . W^T (fp32 out)."""
    if x.dtype not in _DT:
        raise ValueError(f"x dtype {x.dtype} not supported")
    if not x.is_cuda or not x.is_contiguous() or x.shape[-1] != w.K:
        raise ValueError("x must be a contiguous device tensor [..., K]")
    rows = x.numel() // w.K
    if out is None:
        out = torch.empty(x.shape[:-1] + (w.N,), dtype=torch.float32, device=x.device)
    _need(out, torch.float32, "out")
    rc = _lib.load().altxs_qgemm(ctypes.byref(w.qt), x.data_ptr(), _DT[x.dtype], rows,
                                 out.data_ptr(), _s(x))
    _lib.check(rc, "altxs_qgemm")
    return out


def qgemm_stream(codes: torch.Tensor, scales: torch.Tensor, count: int, N: int, K: int, bits: int,
                 codes_stride: int, scales_stride: int, x: torch.Tensor,
                 out: torch.Tensor) -> torch.Tensor:
    """One launch over ``count`` packed tensors at fixed byte strides."""
    qt = _lib.QTensor(codes.data_ptr(), scales.data_ptr(), N, K, bits, 0)
    rows = x.numel() // K
    rc = _lib.load().altxs_qgemm_stream(ctypes.byref(qt), count, codes_stride, scales_stride,
                                        x.data_ptr(), _DT[x.dtype], rows, out.data_ptr(), _s(x))
    _lib.check(rc, "altxs_qgemm_stream")
    return out


def qgemv(w: DeviceQTensor, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """y[rows, N] = x[rows, K] . W^T for 1..4 fp16/bf16 rows, each row on its
    own (VALU dot arithmetic; a row's bits depend on that row alone)."""
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"x dtype {x.dtype} not supported (fp16 or bf16)")
    if not x.is_cuda or not x.is_contiguous() or x.shape[-1] != w.K:
        raise ValueError("x must be a contiguous device tensor [..., K]")
    rows = x.numel() // w.K
    if out is None:
        out = torch.empty(x.shape[:-1] + (w.N,), dtype=torch.float32, device=x.device)
    _need(out, torch.float32, "out")
    rc = _lib.load().altxs_qgemv(ctypes.byref(w.qt), x.data_ptr(), _DT[x.dtype], rows,
                                 out.data_ptr(), _s(x))
    _lib.check(rc, "altxs_qgemv")
    return out


def qgemv_stream(codes: torch.Tensor, scales: torch.Tensor, count: int, N: int, K: int, bits: int,
                 codes_stride: int, scales_stride: int, x: torch.Tensor,
                 out: torch.Tensor) -> torch.Tensor:
    """:func:`qgemv` over ``count`` packed tensors at fixed byte strides."""
    qt = _lib.QTensor(codes.data_ptr(), scales.data_ptr(), N, K, bits, 0)
    rows = x.numel() // K
    rc = _lib.load().altxs_qgemv_stream(ctypes.byref(qt), count, codes_stride, scales_stride,
                                        x.data_ptr(), _DT[x.dtype], rows, out.data_ptr(), _s(x))
    _lib.check(rc, "altxs_qgemv_stream")
    return out


def decode_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor, *,
                W: int = 1, gate: torch.Tensor | None = None, use_xsa: bool = False,
                y_bf16: bool = False, ops_bf16: bool = False, tiled: bool = False,
                err: torch.Tensor | None = None, rows: bool = False,
                xcd_rows: bool = False, natural: bool = False, kv_tail_end: int = 0) -> torch.Tensor:
    """q [B*W, H, 64] fp32; k/v [B, Hkv, max_len, 64] (fp32 or bf16); pos [B] int32.

    bf16 k/v are given in natural [key][dim] order and tiled here
    (:func:`altxs_amd.codec.tile_kv`) unless ``tiled`` says they already are.
    ``ops_bf16`` rounds q and the softmax weights to bf16 for the MFMA products
    (the reference's tl.dot arithmetic); otherwise fp32-faithful splits.
    ``rows`` runs windows (W > 1) of a bf16 cache one row per workgroup (the
    decode kernel) instead of the window kernel; the bits are the same.
    ``xcd_rows`` places the one-row kernel's workgroups in 8-row tiles, tile t
    on XCD t % 8 (B*W a multiple of 64; otherwise ignored); the bits are the same.
    ``natural`` keeps bf16 k/v in their natural order (the reference's k_pack
    layout; the MFMA kernel reads them in place, with the tiled layout's bits).  ``kv_tail_end`` (natural
    layouts): window token t's K/V sit in row kv_tail_end - W + t and query t
    attends to rows [0, pos) and then to those rows (the reference's
    StaticKV tail, model.py:259-461).
    """
    from .codec import tile_kv

    _need(q, torch.float32, "q")
    _need(pos, torch.int32, "pos")
    B, Hkv, max_len, hd = k.shape
    if v.shape != k.shape or v.dtype != k.dtype or not (k.is_contiguous() and v.is_contiguous()):
        raise ValueError("k and v must be contiguous with equal shape/dtype")
    if k.dtype == torch.bfloat16 and not tiled and not natural:
        k = tile_kv(k, "k").contiguous()
        v = tile_kv(v, "v").contiguous()
    H = q.shape[1]
    a = _lib.AttnArgs()
    a.B, a.W, a.H, a.Hkv, a.head_dim, a.max_len = B, W, H, Hkv, hd, max_len
    a.kv_bf16 = (_lib.KV_F32 if k.dtype != torch.bfloat16 else
                 _lib.KV_BF16_NATURAL if natural else _lib.KV_BF16)
    a.kv_tail_end = int(kv_tail_end)
    a.y_bf16 = int(y_bf16)
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.kv_seg_stride = Hkv * max_len * hd
    a.pos = pos.data_ptr()
    a.gate = gate.data_ptr() if gate is not None else None
    a.use_xsa = int(use_xsa)
    a.flags = ((_lib.ATTN_OPS_BF16 if ops_bf16 else 0) | (_lib.ATTN_ROWS if rows else 0)
               | (_lib.ATTN_XCD_ROWS if xcd_rows else 0))
    y = torch.empty(B * W, H * hd, dtype=torch.bfloat16 if y_bf16 else torch.float32,
                    device=q.device)
    a.y = y.data_ptr()
    a.err = err.data_ptr() if err is not None else None
    rc = _lib.load().altxs_decode_attn(ctypes.byref(a), _s(q))
    _lib.check(rc, "altxs_decode_attn")
    return y
