"""Mixed-bit weight format: group-64 symmetric quantisation + the MFMA-tiled layout.

Math (per tensor W[N, K], bits b in {2, 3, 4, 6}, groups of 64 along K):

    w[n, k] = (code[n, k] - (2^b - 1) / 2) * scale[n, k // 64],  scale in fp16

This is the reference's "symmetric" codebook mode
(src/hyperflow_distillation/mixed_bit_delta.py:147-152, dequantize_channels
172-229) with the channel width set to 64 and b = 6 added (the reference
accepts only b in {2, 3, 4}, mixed_bit_delta.py:100-101).

Device layout (``pack_tiled``), consumed by libaltxs_hip's MFMA GEMM:

* the tensor is cut into blocks of 16 rows x 256 columns, block (nb, kb) at
  index ``nb * (K // 256) + kb``;
* inside a block, wave lane ``l`` (0..63) owns row ``l % 16`` and the columns
  ``32*s + 8*(l // 16) + i`` for k-step ``s`` = 0..7 and ``i`` = 0..7 -- the B
  operand of one v_mfma_f32_16x16x32 per k-step;
* each code splits into bit planes (b=2: 2; b=3: 2+1; b=4: 4; b=6: 4+2); plane
  ``p`` of width ``pb`` stores, per lane, the 64 codes LSB-first (code index
  ``8*s + i`` at bit ``pb * (8*s + i)``) in ``8*pb`` bytes, lanes contiguous,
  so a block is ``512*b`` bytes and each lane's share is whole 16/8-byte words;
* scales per block: 16 rows x 4 groups fp16, row-major (128 bytes).

Dense weights (``bits = 16``, e.g. the reference's runtime banks, which are
Init(seed) + the decoded delta in bf16) use the same block and lane order
with each value stored as its bf16 bits (lane ``l``: 64 values, k-step ``s``
in bytes 16s..16s+15), 8192 bytes per block and no scales.
"""

from __future__ import annotations

import dataclasses

import numpy as np

BITS = (2, 3, 4, 6)
PLANES = {2: (2,), 3: (2, 1), 4: (4,), 6: (4, 2)}
GROUP = 64
BLOCK_N = 16
BLOCK_K = 256


def quantize_group64(w: np.ndarray, bits: int) -> tuple[np.ndarray, np.ndarray]:
    """fp32 [N, K] -> (codes uint8 [N, K], scales fp16 [N, K // 64]).

    scale = fp16(max|w_g| / ((2^b - 1) / 2)); code = clip(rint(w/scale + c), 0, 2^b - 1)
    with c = (2^b - 1) / 2, computed against the fp16-rounded scale.
    """
    if bits not in BITS:
        raise ValueError(f"bits must be one of {BITS}, got {bits}")
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % GROUP:
        raise ValueError(f"K={k} is not a multiple of {GROUP}")
    c = (2 ** bits - 1) / 2.0
    g = w.reshape(n, k // GROUP, GROUP)
    amax = np.abs(g).max(axis=-1)
    scale = (amax / c).astype(np.float16)
    s32 = scale.astype(np.float32)
    safe = np.where(s32 > 0, s32, 1.0).astype(np.float32)
    q = np.rint(g / safe[..., None] + c)
    q = np.where(s32[..., None] > 0, q, np.floor(c))
    codes = np.clip(q, 0, 2 ** bits - 1).astype(np.uint8).reshape(n, k)
    return codes, scale


def dequantize_group64(codes: np.ndarray, scales: np.ndarray, bits: int) -> np.ndarray:
    """(codes [N, K], scales fp16 [N, K//64]) -> fp32 [N, K] (exact)."""
    n, k = codes.shape
    c = np.float32((2 ** bits - 1) / 2.0)
    v = codes.astype(np.float32) - c
    s = np.repeat(scales.astype(np.float32), GROUP, axis=1)
    return (v * s).astype(np.float32)


def _lane_order(n: int, k: int) -> np.ndarray:
    """Index array mapping tiled (block, lane, code) order -> flat [N*K] index."""
    nb, kb = n // BLOCK_N, k // BLOCK_K
    blk_n = np.arange(nb)[:, None, None, None, None]
    blk_k = np.arange(kb)[None, :, None, None, None]
    lane = np.arange(64)[None, None, :, None, None]
    s = np.arange(8)[None, None, None, :, None]
    i = np.arange(8)[None, None, None, None, :]
    row = blk_n * BLOCK_N + lane % 16
    col = blk_k * BLOCK_K + 32 * s + 8 * (lane // 16) + i
    return (row * k + col).reshape(nb * kb, 64, 64)  # [block, lane, code j = 8s+i]


def _pack_plane(vals: np.ndarray, pb: int) -> np.ndarray:
    """vals uint [blocks, 64 lanes, 64 codes] (each < 2^pb) -> bytes [blocks, 64*8*pb]."""
    nblk = vals.shape[0]
    per_word = 32 // pb
    v = vals.astype(np.uint32).reshape(nblk, 64, 64 // per_word, per_word)
    shifts = (np.arange(per_word, dtype=np.uint32) * pb)[None, None, None, :]
    words = np.bitwise_or.reduce(v << shifts, axis=-1).astype("<u4")  # [blk, lane, 2*pb]
    return words.view(np.uint8).reshape(nblk, 64 * 8 * pb)


def _unpack_plane(raw: np.ndarray, pb: int) -> np.ndarray:
    nblk = raw.shape[0]
    per_word = 32 // pb
    words = np.ascontiguousarray(raw).view("<u4").reshape(nblk, 64, 2 * pb).astype(np.uint32)
    shifts = (np.arange(per_word, dtype=np.uint32) * pb)[None, None, None, :]
    v = (words[..., None] >> shifts) & np.uint32((1 << pb) - 1)
    return v.reshape(nblk, 64, 64)


def pack_tiled(codes: np.ndarray, scales: np.ndarray, bits: int) -> tuple[np.ndarray, np.ndarray]:
    """(codes [N, K] uint8, scales fp16 [N, K//64]) -> (tiled code bytes, tiled fp16 scales)."""
    n, k = codes.shape
    if n % BLOCK_N or k % BLOCK_K:
        raise ValueError(f"tensor [{n}, {k}] must be a multiple of [{BLOCK_N}, {BLOCK_K}]")
    if bits not in BITS:
        raise ValueError(f"bits must be one of {BITS}")
    if int(codes.max(initial=0)) >= 2 ** bits:
        raise ValueError("code out of range for the bit width")
    order = _lane_order(n, k)
    lane_codes = codes.reshape(-1)[order].astype(np.uint32)  # [blk, lane, 64]
    planes = []
    shift = 0
    for pb in PLANES[bits]:
        planes.append(_pack_plane((lane_codes >> shift) & ((1 << pb) - 1), pb))
        shift += pb
    packed = np.concatenate(planes, axis=1).reshape(-1)
    nb, kb = n // BLOCK_N, k // BLOCK_K
    sc = scales.astype(np.float16).reshape(nb, BLOCK_N, kb, BLOCK_K // GROUP)
    sc = np.ascontiguousarray(sc.transpose(0, 2, 1, 3)).reshape(-1)
    return packed, sc


def bf16_bits(w: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(w, dtype=np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    return np.where(nan, (u >> np.uint32(16)) | np.uint32(0x40), r).astype(np.uint16)


def pack_dense_tiled(w: np.ndarray) -> np.ndarray:
    """fp32 [N, K] -> the dense bf16 tiled bytes (module docstring)."""
    n, k = w.shape
    if n % BLOCK_N or k % BLOCK_K:
        raise ValueError(f"tensor [{n}, {k}] must be a multiple of [{BLOCK_N}, {BLOCK_K}]")
    vals = bf16_bits(w).reshape(-1)[_lane_order(n, k)]  # [blk, lane, 64]
    return np.ascontiguousarray(vals).astype("<u2").view(np.uint8).reshape(-1)


def split3_bf16(w: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """fp32 -> three bf16 bit patterns hi, mid, lo with hi + mid + lo == w
    exactly: hi = bf16(w), mid = bf16(w - hi), lo = bf16(w - hi - mid), where
    both differences are exact in fp32 and the last one is a bf16 value."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    hi = bf16_bits(w)
    r1 = w - (hi.astype(np.uint32) << np.uint32(16)).view(np.float32)
    mid = bf16_bits(r1)
    r2 = r1 - (mid.astype(np.uint32) << np.uint32(16)).view(np.float32)
    return hi, mid, bf16_bits(r2)


def pack_dense32_tiled(w: np.ndarray) -> np.ndarray:
    """fp32 [N, K] -> the dense bits-32 bytes: per 16 x 256 block the tiled
    bytes of the hi, mid and lo planes one after the other."""
    n, k = w.shape
    if n % BLOCK_N or k % BLOCK_K:
        raise ValueError(f"tensor [{n}, {k}] must be a multiple of [{BLOCK_N}, {BLOCK_K}]")
    order = _lane_order(n, k)  # [blk, lane, 64]
    planes = [np.ascontiguousarray(p.reshape(-1)[order]).astype("<u2").view(np.uint8).reshape(order.shape[0], -1)
              for p in split3_bf16(w)]
    return np.ascontiguousarray(np.stack(planes, axis=1)).reshape(-1)


def unpack_dense_tiled(packed: np.ndarray, n: int, k: int) -> np.ndarray:
    """Inverse of :func:`pack_dense_tiled`: fp32 [N, K] of the bf16 values."""
    vals = np.ascontiguousarray(packed, dtype=np.uint8).view("<u2").astype(np.uint32)
    out = np.zeros(n * k, dtype=np.uint32)
    out[_lane_order(n, k).reshape(-1)] = vals
    return (out << np.uint32(16)).view(np.float32).reshape(n, k)


def unpack_tiled(packed: np.ndarray, scales_t: np.ndarray, n: int, k: int,
                 bits: int) -> tuple[np.ndarray, np.ndarray]:
    """Inverse of :func:`pack_tiled`."""
    nb, kb = n // BLOCK_N, k // BLOCK_K
    blk = np.asarray(packed, dtype=np.uint8).reshape(nb * kb, 512 * bits)
    lane_codes = np.zeros((nb * kb, 64, 64), dtype=np.uint32)
    off = 0
    shift = 0
    for pb in PLANES[bits]:
        lane_codes |= _unpack_plane(blk[:, off:off + 512 * pb], pb) << shift
        off += 512 * pb
        shift += pb
    codes = np.zeros(n * k, dtype=np.uint8)
    codes[_lane_order(n, k).reshape(-1)] = lane_codes.reshape(-1).astype(np.uint8)
    sc = np.asarray(scales_t, dtype=np.float16).reshape(nb, kb, BLOCK_N, BLOCK_K // GROUP)
    sc = np.ascontiguousarray(sc.transpose(0, 2, 1, 3)).reshape(n, k // GROUP)
    return codes.reshape(n, k), sc


@dataclasses.dataclass
class PackedTensor:
    """One quantised tensor on the host: logical codes/scales + the device layout."""

    name: str
    bits: int
    codes: np.ndarray   # uint8 [N, K]
    scales: np.ndarray  # fp16 [N, K//64]
    tiled: np.ndarray   # uint8 bytes (or a device tensor built there, see altxs_amd.shipped)
    tiled_scales: np.ndarray  # fp16
    nk: tuple[int, int] | None = None  # the shape when `codes` is not kept on the host

    @property
    def shape(self) -> tuple[int, int]:
        return self.nk if self.nk is not None else tuple(self.codes.shape)  # type: ignore[return-value]

    @property
    def nbytes_codes(self) -> int:
        return int(self.tiled.size)

    @property
    def nbytes_scales(self) -> int:
        return int(self.tiled_scales.size * 2)

    def dense(self) -> np.ndarray:
        if self.bits == 16:  # codes hold the bf16 bit patterns
            return (self.codes.astype(np.uint32) << np.uint32(16)).view(np.float32)
        if self.bits == 32:  # codes hold the fp32 bit patterns
            return self.codes.astype(np.uint32).view(np.float32).copy()
        return dequantize_group64(self.codes, self.scales, self.bits)

    @classmethod
    def from_dense(cls, name: str, w: np.ndarray, bits: int) -> "PackedTensor":
        if bits == 16:  # dense bf16 weights, no quantisation
            n = w.shape[0]
            return cls(name, 16, bf16_bits(w), np.zeros((n, 0), np.float16), pack_dense_tiled(w),
                       np.zeros(0, np.float16))
        if bits == 32:  # dense fp32 weights as three exact bf16 planes
            n = w.shape[0]
            w = np.ascontiguousarray(w, dtype=np.float32)
            return cls(name, 32, w.view(np.uint32).copy(), np.zeros((n, 0), np.float16),
                       pack_dense32_tiled(w), np.zeros(0, np.float16))
        codes, scales = quantize_group64(w, bits)
        tiled, tsc = pack_tiled(codes, scales, bits)
        return cls(name, bits, codes, scales, tiled, tsc)


def allocate_bits(sizes: list[tuple[str, int]], target: float) -> dict[str, int]:
    """Deterministic per-tensor widths from {2,3,4,6} near a mean of ``target`` bits.

    Role recipe (names as in altxs_amd.synth.tensor_list): the first layer's
    QKV at 6 bits, other QKV at 4, out-projection / MLP-up / embedding at 3,
    MLP-down at 2; then MLP-down tensors are raised to 3 bits, in layer order,
    while that moves the weighted mean closer to ``target``.
    """
    total = sum(n for _, n in sizes)
    bits: dict[str, int] = {}
    for name, _ in sizes:
        role = name.rsplit(".", 1)[-1]
        if name == "l0.qkv":
            bits[name] = 6
        elif role == "qkv":
            bits[name] = 4
        elif role == "down":
            bits[name] = 2
        else:
            bits[name] = 3

    def err() -> float:
        return abs(sum(bits[nm] * n for nm, n in sizes) / total - target)

    for name, _ in sizes:
        if not name.endswith(".down"):
            continue
        before = err()
        bits[name] = 3
        if err() >= before:
            bits[name] = 2
            break
    return bits


# ---- bf16 KV cache tile layout (include/altxs.h, ALTXS_KV_TILE) -------------

KV_TILE = 64


def tile_kv(x, which: str):
    """Natural [..., max_len, 64] K or V -> the bf16 cache's tiled operand order.

    Works on numpy arrays and torch tensors (any device).  Per 64-key tile the
    4096 elements are reordered so each lane's MFMA operand is 16 contiguous
    bytes: K as (block, kstep, lanegroup, key%16, dim%8), V as (kstep,
    dimblock, lanegroup, dim%16, key-half, key%4) -- the index formulas
    kv_tile_k / kv_tile_v of altxs_amd/csrc/common.h.
    """
    *lead, L, hd = x.shape
    if hd != 64 or L % KV_TILE:
        raise ValueError(f"expected [..., multiple of {KV_TILE}, 64], got {tuple(x.shape)}")
    nt = L // KV_TILE
    n = len(lead)
    if which == "k":   # key = 16*blk + r ; dim = 32*ks + 8*g + j
        y = x.reshape(*lead, nt, 4, 16, 2, 4, 8)
        perm = (0, 1, 3, 4, 2, 5)
    elif which == "v":  # key = 32*s + 16*jb + 4*g + jr ; dim = 16*nb + dd
        y = x.reshape(*lead, nt, 2, 2, 4, 4, 4, 16)
        perm = (0, 1, 5, 3, 6, 2, 4)
    else:
        raise ValueError(which)
    perm = tuple(range(n)) + tuple(n + p for p in perm)
    y = y.transpose(perm) if isinstance(y, np.ndarray) else y.permute(perm)
    return y.reshape(*lead, L, hd)


def untile_kv(x, which: str):
    """Inverse of :func:`tile_kv`."""
    *lead, L, hd = x.shape
    nt = L // KV_TILE
    n = len(lead)
    if which == "k":
        y = x.reshape(*lead, nt, 4, 2, 4, 16, 8)   # (T, blk, ks, g, r, j)
        perm = (0, 1, 4, 2, 3, 5)                  # -> (T, blk, r, ks, g, j)
    elif which == "v":
        y = x.reshape(*lead, nt, 2, 4, 4, 16, 2, 4)  # (T, s, nb, g, dd, jb, jr)
        perm = (0, 1, 5, 3, 6, 2, 4)                 # -> (T, s, jb, g, jr, nb, dd)
    else:
        raise ValueError(which)
    perm = tuple(range(n)) + tuple(n + p for p in perm)
    y = y.transpose(perm) if isinstance(y, np.ndarray) else y.permute(perm)
    return y.reshape(*lead, L, hd)
