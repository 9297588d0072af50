"""Mixed-bit codec: reference per-channel arithmetic KATs and the group-64 tiled format."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

from altxs_amd import codec
from oracle import codec_ref

REF_WEIGHTS = "/root/reference/weights/mixed_da_bpw3.15_upb1.8"


def test_unpack_codes_known_answers():
    # 2-bit: 0b11_10_01_00 -> [0, 1, 2, 3] (LSB first)
    assert list(codec_ref.unpack_codes(np.array([0b11100100], np.uint8), 2, 4)) == [0, 1, 2, 3]
    # 4-bit: 0x21 -> [1, 2]
    assert list(codec_ref.unpack_codes(np.array([0x21], np.uint8), 4, 2)) == [1, 2]
    # 3-bit: codes 0..7 in one little-endian 24-bit word
    word = sum(c << (3 * c) for c in range(8))
    b = np.array([word & 255, (word >> 8) & 255, (word >> 16) & 255], np.uint8)
    assert list(codec_ref.unpack_codes(b, 3, 8)) == list(range(8))
    with pytest.raises(ValueError):
        codec_ref.unpack_codes(b, 6, 8)


def test_symmetric_levels_closed_form():
    lv = codec_ref.symmetric_levels(np.array([0.5], np.float16), 3)
    assert np.allclose(lv[0], (np.arange(8) - 3.5) * 0.5)


def test_fp4_table():
    t = codec_ref.fp4_e2m1()
    assert list(t[:8]) == [0, 0.5, 1, 1.5, 2, 3, 4, 6]
    assert np.array_equal(t[8:], -t[:8])


@pytest.mark.parametrize("bits", codec.BITS)
def test_quantize_roundtrip_error(bits):
    rng = np.random.default_rng(bits)
    w = rng.standard_normal((32, 512)).astype(np.float32) * 0.02
    codes, scales = codec.quantize_group64(w, bits)
    deq = codec_ref.dequant_group64(codes, scales, bits)
    s = np.repeat(scales.astype(np.float32), 64, axis=1)
    assert np.all(np.abs(deq - w) <= 0.5 * s * (1 + 1e-3) + 1e-7)
    assert codes.max() <= 2 ** bits - 1
    assert np.array_equal(deq, codec.dequantize_group64(codes, scales, bits))


@pytest.mark.parametrize("bits", codec.BITS)
@pytest.mark.parametrize("shape", [(16, 256), (48, 512), (32, 2048)])
def test_tiled_layout_roundtrip(bits, shape):
    rng = np.random.default_rng(1)
    n, k = shape
    codes = rng.integers(0, 2 ** bits, size=(n, k)).astype(np.uint8)
    scales = rng.standard_normal((n, k // 64)).astype(np.float16)
    tiled, tsc = codec.pack_tiled(codes, scales, bits)
    assert tiled.size == n * k * bits // 8
    c2, s2 = codec.unpack_tiled(tiled, tsc, n, k, bits)
    assert np.array_equal(c2, codes) and np.array_equal(s2.view(np.uint16), scales.view(np.uint16))
    # independent element-by-element reader of the layout description
    c3, s3 = codec_ref.unpack_tiled(tiled, tsc, n, k, bits)
    assert np.array_equal(c3, codes) and np.array_equal(s3.view(np.uint16), scales.view(np.uint16))


def test_tiled_lane_ownership():
    """Lane l of block (0,0) owns row l%16, columns 32s + 8(l//16) + i (s, i < 8)."""
    n, k, bits = 16, 256, 4
    codes = np.zeros((n, k), np.uint8)
    codes[5, 32 * 3 + 8 * 2 + 7] = 9  # lane 5 + 16*2 = 37, k-step 3, i = 7
    tiled, _ = codec.pack_tiled(codes, np.ones((n, k // 64), np.float16), bits)
    lane_bytes = tiled.reshape(64, 32)
    nz = np.nonzero(lane_bytes)
    assert list(nz[0]) == [37]
    word = lane_bytes[37].view("<u4")
    assert word[3] == 9 << 28  # k-step 3 -> word 3, code i=7 -> bits 28..31


def test_allocate_bits_hits_budget():
    from altxs_amd.config import make_config
    from altxs_amd.synth import tensor_list

    cfg = make_config("cfg3")
    sizes = [(nm, n * k) for nm, n, k in tensor_list(cfg)]
    bits = codec.allocate_bits(sizes, 3.15)
    mean = sum(bits[nm] * n for nm, n in sizes) / sum(n for _, n in sizes)
    assert abs(mean - 3.15) < 0.01
    assert set(bits.values()) == {2, 3, 4, 6}


@pytest.mark.skipif(not os.path.exists(REF_WEIGHTS + ".json"), reason="reference asset absent")
def test_shipped_asset_sizes_match_closed_forms():
    """The shipped codec's packed tensors have the byte sizes the layout implies."""
    from safetensors.numpy import load_file

    meta = json.load(open(REF_WEIGHTS + ".json", encoding="utf8"))
    st = load_file(REF_WEIGHTS + ".safetensors")
    for name, layout in meta["layouts"].items():
        bits = st[f"bits/{name}"]
        width = int(layout["channel_width"])
        for b in (2, 3, 4):
            nch = int((bits == b).sum())
            key = f"packed/{name}/b{b}"
            if key in st:
                assert st[key].size == nch * width * b // 8, key
        # decode the whole bank with the oracle (lloyd codebooks) -> finite values
        cbs = {b: st.get(f"codebook/{name}/b{b}", np.empty((0, 1 << b), np.float16)) for b in (2, 3, 4)}
        pk = {b: st.get(f"packed/{name}/b{b}", np.zeros(0, np.uint8)) for b in (2, 3, 4)}
        ch = codec_ref.dequantize_channels(bits, cbs, pk, channel_width=width,
                                           mode=meta.get("codebook_mode", "lloyd"))
        assert ch.shape == (bits.size, width) and np.isfinite(ch).all()
        assert np.all(ch[bits == 0] == 0)


def test_kv_tile_layout_roundtrip_and_operand_runs():
    """tile_kv/untile_kv are inverse permutations; each MFMA operand is a 16-byte run.

    K: lane 16g + r of k-step ks in block blk reads key 16*blk + r, dims
    32*ks + 8*g + [0, 8); V: lane 16g + c of k-step s, dim block nb reads dim
    16*nb + c of keys 16*(2s + j//4) + 4g + j%4 for j = 0..7.  Both must be the
    8 consecutive elements at offset 8 * (64 * step + lane) of the tile.
    """
    from altxs_amd.codec import tile_kv, untile_kv

    rng = np.random.default_rng(5)
    x = rng.integers(0, 1 << 30, size=(2, 3, 192, 64))
    for which in ("k", "v"):
        t = tile_kv(x, which)
        assert np.array_equal(untile_kv(t, which), x)
        assert sorted(t.reshape(-1).tolist()) == sorted(x.reshape(-1).tolist())
    tk = tile_kv(x, "k").reshape(2, 3, 3, 4096)
    tv = tile_kv(x, "v").reshape(2, 3, 3, 4096)
    for T in range(3):
        for lane in range(64):
            g, c = divmod(lane, 16)
            for blk in range(4):
                for ks in range(2):
                    run = tk[1, 2, T, 8 * (64 * (2 * blk + ks) + lane):][:8]
                    want = x[1, 2, 64 * T + 16 * blk + c, 32 * ks + 8 * g: 32 * ks + 8 * g + 8]
                    assert np.array_equal(run, want)
            for s in range(2):
                for nb in range(4):
                    run = tv[1, 2, T, 8 * (64 * (4 * s + nb) + lane):][:8]
                    keys = [64 * T + 16 * (2 * s + j // 4) + 4 * g + j % 4 for j in range(8)]
                    assert np.array_equal(run, x[1, 2, keys, 16 * nb + c])


def test_dense_bf16_tiled_layout():
    """Dense bf16 weights: each value at the byte offset the layout states
    (block (n//16, k//256), lane n%16 + 16*((k%32)//8), k-step (k%256)//32,
    element k%8), as its round-to-nearest-even bf16 bits."""
    import torch

    from altxs_amd import codec

    rng = np.random.default_rng(3)
    n, k = 48, 768
    w = (rng.standard_normal((n, k)) * 3).astype(np.float32)
    w[0, :4] = [0.0, -0.0, 1e-40, 65504.0]
    t = codec.pack_dense_tiled(w)
    assert t.size == n * k * 2
    want = torch.from_numpy(w).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    rows, cols = np.meshgrid(np.arange(n), np.arange(k), indexing="ij")
    blk = (rows // 16) * (k // 256) + cols // 256
    kk = cols % 256
    lane = rows % 16 + 16 * ((kk % 32) // 8)
    off = blk * 8192 + lane * 128 + (kk // 32) * 16 + (kk % 8) * 2
    got = t[off].astype(np.uint16) | (t[off + 1].astype(np.uint16) << 8)
    assert np.array_equal(got, want)
    assert np.array_equal(codec.unpack_dense_tiled(t, n, k),
                          torch.from_numpy(w).to(torch.bfloat16).float().numpy())
    p = codec.PackedTensor.from_dense("w", w, 16)
    assert p.bits == 16 and p.nbytes_scales == 0 and np.array_equal(p.dense(), codec.unpack_dense_tiled(t, n, k))


def test_from_channels_hand_built():
    """_from_channels (mixed_bit_delta.py:116-144) on a 2-layer, d=2 example
    written out by hand: q/k/v/up rows are channels, o/down columns are."""
    x = np.arange(16, dtype=np.float32).reshape(8, 2)  # channel c holds (2c, 2c+1)
    qo = codec_ref.from_channels("qo_bank", x, [4, 2, 2], 2)
    assert np.array_equal(qo[0], [[0, 1], [2, 3]]) and np.array_equal(qo[1], [[4, 5], [6, 7]])
    # o of layer 0 is channels 4, 5 as columns: o0[i][c] = channel(4 + c)[i]
    assert np.array_equal(qo[2], [[8, 10], [9, 11]]) and np.array_equal(qo[3], [[12, 14], [13, 15]])
    kv = codec_ref.from_channels("kv_bank", x[:4], [4, 1, 2], 2)
    assert np.array_equal(kv[:, 0], [[0, 1], [2, 3], [4, 5], [6, 7]])
    down = codec_ref.from_channels("mlp_down_bank", x[:8], [2, 2, 4], 2)  # [L, d=2, F=4]
    assert np.array_equal(down[0], [[0, 2, 4, 6], [1, 3, 5, 7]])
    up = codec_ref.from_channels("mlp_up_bank", x[:8], [2, 4, 2], 2)
    assert np.array_equal(up[1], [[8, 9], [10, 11], [12, 13], [14, 15]])


def test_bank_parts_place_channels_like_from_channels():
    """altxs_amd.shipped.bank_parts (where the device decoder writes each
    channel) equals from_channels followed by the split into this build's
    per-layer tensors."""
    from altxs_amd import shipped
    from altxs_amd.config import make_config

    cfg = make_config("tiny")
    L, d, kvd, F, V = cfg.num_layers, cfg.model_dim, cfg.kv_dim, cfg.hidden_dim, cfg.vocab_size
    shapes = {"tok_emb.weight": [V, d], "qo_bank": [2 * L, d, d], "kv_bank": [2 * L, kvd, d],
              "mlp_up_bank": [L, F, d], "mlp_down_bank": [L, d, F]}
    rng = np.random.default_rng(0)
    bank = {n: rng.standard_normal((int(np.prod(s)) // d, d)).astype(np.float32) for n, s in shapes.items()}
    dst = {n: np.zeros(a * b, np.float32) for n, (a, b) in shipped.tensor_shapes(cfg).items()}
    for name, parts in shipped.bank_parts(cfg).items():
        covered = 0
        for p in parts:
            for j in range(p.n):
                idx = p.offset + j * p.stride_ch + np.arange(d) * p.stride_el
                dst[p.dest][idx] = bank[name][p.c0 + j]
            covered += p.n
        assert covered == bank[name].shape[0]
    full = {n: codec_ref.from_channels(n, bank[n], shapes[n], L) for n in shapes}
    assert np.array_equal(dst["emb"].reshape(V, d), full["tok_emb.weight"])
    for l in range(L):
        qkv = np.concatenate([full["qo_bank"][l], full["kv_bank"][l], full["kv_bank"][L + l]])
        assert np.array_equal(dst[f"l{l}.qkv"].reshape(qkv.shape), qkv)
        assert np.array_equal(dst[f"l{l}.o"].reshape(d, d), full["qo_bank"][L + l])
        assert np.array_equal(dst[f"l{l}.up"].reshape(F, d), full["mlp_up_bank"][l])
        assert np.array_equal(dst[f"l{l}.down"].reshape(d, F), full["mlp_down_bank"][l])


@pytest.mark.skipif(not os.path.exists("/root/reference/weights/mixed_da_bpw3.15_upb1.8.json"),
                    reason="the reference asset is only in the build container")
def test_shipped_layouts_match_bank_parts():
    """The shipped student's layouts (channel counts, widths) are what the
    device decoder's placement expects for its config."""
    from altxs_amd import shipped

    meta = json.load(open("/root/reference/weights/mixed_da_bpw3.15_upb1.8.json"))
    cfg = shipped.config_from_meta(meta)
    assert cfg.num_layers == meta["n_layers"] and cfg.vocab_size == 256
    for name, parts in shipped.bank_parts(cfg).items():
        lay = meta["layouts"][name]
        assert lay["channel_width"] == cfg.model_dim
        assert sum(p.n for p in parts) == lay["channels"]
        assert sorted((p.c0, p.c0 + p.n) for p in parts)[-1][1] == lay["channels"]


# ---- reference-written vectors (tests/golden/make_golden.py) ---------------------

MODES = ["lloyd", "symmetric", "shared", "fp4", "hybrid_fp4_symmetric"]


def _mode_inputs(z, mode):
    books = {b: z[f"{mode}/codebook_b{b}"] for b in (2, 3, 4)}
    packed = {b: z[f"{mode}/packed_b{b}"] for b in (2, 3, 4)}
    scales = {b: z[f"{mode}/scale_b{b}"] for b in (2, 3, 4) if f"{mode}/scale_b{b}" in z.files}
    return packed, books, scales or None


@pytest.mark.parametrize("mode", MODES)
def test_dequantize_channels_matches_reference(golden_dir, mode):
    """The oracle decoder equals the reference's dequantize_channels
    (mixed_bit_delta.py:172-229) bit for bit in every codebook mode, on
    seeded channels of mixed width with dead ones."""
    z = np.load(os.path.join(golden_dir, "codec_modes.npz"))
    packed, books, scales = _mode_inputs(z, mode)
    bits = z["bits"].copy()
    got = codec_ref.dequantize_channels(bits, books, packed, channel_width=int(z["width"]),
                                        mode=mode, scales=scales)
    assert np.array_equal(got, z[f"{mode}/out"])


def test_dequantize_channels_mode_mistakes_fail(golden_dir):
    """Plausible mistakes fail the reference vectors: decoding lloyd codebooks
    with the symmetric rule, or codes MSB-first."""
    z = np.load(os.path.join(golden_dir, "codec_modes.npz"))
    packed, books, scales = _mode_inputs(z, "symmetric")
    bits = z["bits"].copy()
    want = z["symmetric/out"]
    flipped = {b: np.unpackbits(p, bitorder="little").reshape(-1, 8)[:, ::-1].copy() for b, p in packed.items()}
    flipped = {b: np.packbits(f.reshape(-1), bitorder="little") for b, f in flipped.items()}
    got = codec_ref.dequantize_channels(bits, books, flipped, channel_width=int(z["width"]),
                                        mode="symmetric")
    assert not np.array_equal(got, want)
    lp, lb, _ = _mode_inputs(z, "lloyd")
    got = codec_ref.dequantize_channels(bits, {b: lb[b][:, :1] for b in lb}, lp,
                                        channel_width=int(z["width"]), mode="symmetric")
    assert not np.array_equal(got, z["lloyd/out"])


def test_shipped_slice_matches_reference(golden_dir):
    """Channels of every bank of the shipped asset, decoded by the oracle from
    their packed bytes and codebook rows, equal what the reference decoded
    from the whole bank (so rank -> byte offset and codebook row mapping
    are pinned on the real file)."""
    z = np.load(os.path.join(golden_dir, "shipped_slice.npz"))
    assert str(z["mode"]) == "lloyd"
    for bank in ("tok_emb.weight", "qo_bank", "kv_bank", "mlp_up_bank", "mlp_down_bank"):
        bits = z[f"{bank}/bits"]
        packed = {b: z[f"{bank}/packed_b{b}"] for b in (2, 3, 4)}
        books = {b: z[f"{bank}/codebook_b{b}"] for b in (2, 3, 4)}
        got = codec_ref.dequantize_channels(bits, books, packed, channel_width=int(z[f"{bank}/width"]),
                                            mode="lloyd")
        assert np.array_equal(got, z[f"{bank}/out"]), bank
        assert (bits == 0).any() == (~z[f"{bank}/out"].any(axis=1)).any() or not (bits == 0).any()
