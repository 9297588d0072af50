"""Mixed-bit codec arithmetic, numpy -- TEST INFRASTRUCTURE ONLY.

* :func:`unpack_codes` restates ``unpack_codes``
  (src/hyperflow_distillation/mixed_bit_delta.py:96-113): unsigned fixed-width
  codes, LSB first; 3-bit codes pack 8 per 3 bytes.  Pinned by hand-built
  known answers (tests/test_oracle_codec.py) and by the byte sizes of the
  shipped asset's packed tensors, which must equal channels*512*bits/8
  (weights/mixed_da_bpw3.15_upb1.8.json layouts).
* :func:`symmetric_levels` restates ``_symmetric_levels`` (147-152).
* :func:`dequantize_channels` restates ``dequantize_channels`` (172-229) for the
  lloyd, symmetric, shared, fp4 and hybrid modes; pinned bit for bit by the
  reference's own outputs in every mode (tests/golden/codec_modes.npz) and on
  channels of every bank of the shipped asset (tests/golden/shipped_slice.npz).
* :func:`from_channels` restates ``_from_channels`` (116-144); pinned by a
  hand-built 2-layer example (tests/test_codec.py).
* :func:`dequant_group64` is the symmetric rule with 64-wide groups along K
  (the build's device format); pinned against the closed form on all codes.
* :func:`unpack_tiled` reads the device layout back to (codes, scales); it is
  written from the layout description, independently of the packer.
"""

from __future__ import annotations

import numpy as np


def unpack_codes(packed: np.ndarray, bits: int, count: int) -> np.ndarray:
    bits, count = int(bits), int(count)
    if bits not in (2, 3, 4):
        raise ValueError(f"bits must be 2/3/4, got {bits}")
    p = np.asarray(packed, dtype=np.uint8).reshape(-1)
    group = 3 if bits == 3 else 1  # bytes per little-endian word
    if p.size % group:
        raise ValueError("packed byte count not a multiple of the word size")
    words = np.zeros(p.size // group, dtype=np.uint32)
    for i in range(group):
        words |= p[i::group].astype(np.uint32) << np.uint32(8 * i)
    per_word = (8 * group) // bits
    out = np.empty((words.size, per_word), dtype=np.uint8)
    for j in range(per_word):
        out[:, j] = (words >> np.uint32(j * bits)) & np.uint32((1 << bits) - 1)
    return out.reshape(-1)[:count]


def symmetric_levels(scales: np.ndarray, bits: int) -> np.ndarray:
    n = 1 << int(bits)
    s = np.asarray(scales, dtype=np.float16).astype(np.float32).reshape(-1)
    return (np.arange(n, dtype=np.float32)[None, :] - (n - 1) / 2.0) * s[:, None]


def fp4_e2m1() -> np.ndarray:
    t = np.zeros(16, dtype=np.float32)
    for code in range(16):
        sign = -1.0 if code & 8 else 1.0
        e, m = (code >> 1) & 3, code & 1
        t[code] = sign * (0.5 * m if e == 0 else (1.0 + 0.5 * m) * 2.0 ** (e - 1))
    return t


def dequantize_channels(channel_bits, codebooks, packed, *, channel_width, mode="lloyd",
                        scales=None) -> np.ndarray:
    mode = str(mode).lower().strip()
    bits = np.asarray(channel_bits, dtype=np.uint8).reshape(-1).copy()
    if mode == "fp4":
        bits[bits > 0] = 4
    out = np.zeros((bits.size, int(channel_width)), dtype=np.float32)
    for b in (2, 3, 4):
        idx = np.flatnonzero(bits == b)
        if idx.size == 0:
            continue
        codes = unpack_codes(packed[b], b, idx.size * channel_width).reshape(idx.size, channel_width)
        codes = codes.astype(np.int64)
        cb = np.asarray(codebooks[b], dtype=np.float16).astype(np.float32)
        nl = 1 << b
        if mode in ("fp4", "hybrid_fp4_symmetric") and b == 4:
            out[idx] = fp4_e2m1()[codes] * cb.reshape(-1)[:, None]
        elif mode == "lloyd" or (cb.ndim == 2 and cb.shape == (idx.size, nl)):
            out[idx] = np.take_along_axis(cb.reshape(idx.size, nl), codes, axis=1)
        elif mode in ("symmetric", "hybrid_fp4_symmetric") or (cb.ndim == 2 and cb.shape == (idx.size, 1)):
            out[idx] = np.take_along_axis(symmetric_levels(cb, b), codes, axis=1)
        elif mode == "shared":
            sc = np.asarray(scales[b], dtype=np.float16).astype(np.float32).reshape(-1)
            out[idx] = cb.reshape(nl)[codes] * sc[:, None]
        else:
            raise ValueError(f"unsupported mode {mode} for {b}-bit")
    return out


def from_channels(name: str, channels: np.ndarray, shape, n_layers: int) -> np.ndarray:
    """Decoded channels -> the bank tensor (``_from_channels``,
    mixed_bit_delta.py:116-144): q/k/v/up/emb channels are rows; o and down
    channels are columns (their banks store the transpose)."""
    x = np.asarray(channels, dtype=np.float32)
    L = int(n_layers)
    if name == "qo_bank":
        d = int(shape[-1])
        q = x[:L * d].reshape(L, d, d)
        o = x[L * d:].reshape(L, d, d).transpose(0, 2, 1)
        return np.concatenate([q, o], axis=0)
    if name == "kv_bank":
        kv, d = int(shape[1]), int(shape[2])
        return np.concatenate([x[:L * kv].reshape(L, kv, d), x[L * kv:].reshape(L, kv, d)], axis=0)
    if name in ("mlp_up_bank", "tok_emb.weight"):
        return x.reshape(shape)
    if name == "mlp_down_bank":
        return x.reshape(shape[0], shape[2], shape[1]).transpose(0, 2, 1)
    raise KeyError(name)


def dequant_group64(codes: np.ndarray, scales: np.ndarray, bits: int) -> np.ndarray:
    """w[n,k] = (code[n,k] - (2^b-1)/2) * float(scale[n, k//64])."""
    codes = np.asarray(codes)
    n, k = codes.shape
    lv = np.arange(1 << bits, dtype=np.float32) - np.float32(((1 << bits) - 1) / 2.0)
    s = np.asarray(scales, dtype=np.float16).astype(np.float32)
    return lv[codes.astype(np.int64)] * np.repeat(s, 64, axis=1)


_PLANES = {2: (2,), 3: (2, 1), 4: (4,), 6: (4, 2)}


def unpack_tiled(tiled: np.ndarray, tiled_scales: np.ndarray, n: int, k: int, bits: int):
    """Device layout -> (codes [n,k] uint8, scales [n, k//64] fp16), element by element."""
    t = np.asarray(tiled, dtype=np.uint8).reshape(-1)
    kb_n = k // 256
    codes = np.zeros((n, k), dtype=np.uint8)
    rows = np.arange(n)[:, None]
    cols = np.arange(k)[None, :]
    blk = (rows // 16) * kb_n + cols // 256
    kk = cols % 256
    s, lg, i = kk // 32, (kk % 32) // 8, kk % 8
    lane = rows % 16 + 16 * lg
    j = 8 * s + i  # code index within the lane
    base = blk * (512 * bits)
    off, shift = 0, 0
    val = np.zeros((n, k), dtype=np.uint32)
    for pb in _PLANES[bits]:
        bit = pb * j
        byte = base + off + lane * (8 * pb) + bit // 8
        part = (t[byte].astype(np.uint32) >> (bit % 8).astype(np.uint32)) & np.uint32((1 << pb) - 1)
        val |= part << np.uint32(shift)
        off += 512 * pb
        shift += pb
    codes[:] = val.astype(np.uint8)
    ts = np.asarray(tiled_scales, dtype=np.float16).reshape(-1)
    g = np.arange(k // 64)[None, :]
    r = np.arange(n)[:, None]
    sidx = ((r // 16) * kb_n + g // 4) * 64 + (r % 16) * 4 + g % 4
    return codes, ts[sidx]
