"""The shipped per-channel codec on the device (altxs_codec_decode,
altxs_pack_dense) and the dense bf16 step it feeds.

* decode: every codebook mode of the reference (lloyd, symmetric, shared,
  fp4, hybrid) over random channel widths incl. dead channels, written as rows
  and as columns, equals the oracle's ``dequantize_channels`` bit for bit;
* pack: bf16(base + delta) in the tiled order equals the host packer's bytes;
* end to end: a codec written in the reference's file format (json +
  safetensors) for the "tiny" config, plus an Init state, decodes and packs on
  the device, and the step on those weights matches the fp32 oracle run on
  bf16(Init + delta);
* the real asset: slices of every bank of the reference's shipped codec
  (weights/mixed_da_bpw3.15_upb1.8; packed bytes, bit widths and codebook
  rows, tests/golden/shipped_slice.npz) decode on the device to exactly the
  values the reference's own decoder produced from the whole bank, and the
  five codebook modes decode to the reference's outputs on its vectors
  (tests/golden/codec_modes.npz);
* the whole asset (a copy in tests/golden/shipped/) through
  ``dropin.load_codec(path, device=...)`` with Init(seed) built here: the
  student's logits against the ones the reference's load_codec model wrote.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """LSB-first packing of the reference format (3-bit: 8 codes per 3 bytes)."""
    c = np.asarray(codes, dtype=np.uint32).reshape(-1)
    per = 8 if bits == 3 else 8 // bits
    nbytes = 3 if bits == 3 else 1
    pad = (-c.size) % per
    c = np.concatenate([c, np.zeros(pad, np.uint32)]).reshape(-1, per)
    words = np.bitwise_or.reduce(c << (np.arange(per, dtype=np.uint32) * bits), axis=1)
    return np.stack([(words >> (8 * i)) & 0xFF for i in range(nbytes)], axis=1).astype(np.uint8).reshape(-1)


def random_bank(rng, n_ch: int, width: int, mode: str):
    bits = rng.choice([0, 2, 3, 4], size=n_ch, p=[0.05, 0.3, 0.35, 0.3]).astype(np.uint8)
    if mode == "fp4":
        bits[bits > 0] = 4
    packed, books, scales = {}, {}, {}
    for b in (2, 3, 4):
        n = int((bits == b).sum())
        packed[b] = pack_codes(rng.integers(0, 1 << b, n * width), b)
        if mode == "lloyd":
            books[b] = (rng.standard_normal((n, 1 << b)) * 0.05).astype(np.float16)
        elif mode == "shared":
            books[b] = (rng.standard_normal(1 << b)).astype(np.float16)
            scales[b] = (rng.random(n) * 0.05 + 0.001).astype(np.float16)
        else:
            books[b] = (rng.random((n, 1)) * 0.05 + 0.001).astype(np.float16)
    return bits, packed, books, scales


@pytest.mark.parametrize("mode", ["lloyd", "symmetric", "shared", "fp4", "hybrid_fp4_symmetric"])
def test_codec_decode_matches_oracle(mode):
    from altxs_amd import shipped
    from oracle import codec_ref

    _log(f"codec decode {mode}")
    rng = np.random.default_rng(len(mode))
    n_ch, width = 96, 512
    bits, packed, books, scales = random_bank(rng, n_ch, width, mode)
    for b in (2, 3, 4):  # the test packer inverts the oracle's unpacker
        n = int((bits == b).sum())
        assert codec_ref.unpack_codes(packed[b], b, n * width).size == n * width
    want = codec_ref.dequantize_channels(bits, books, packed, channel_width=width, mode=mode,
                                         scales=scales or None)
    bank = shipped.DeviceBank(bits, packed, books, mode, scales or None, "cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    rows = torch.full((n_ch * width,), 7.0, device="cuda")
    bank.decode(shipped.Part(0, n_ch, "x", 0, width, 1), width, rows, err)
    cols = torch.full((n_ch * width,), 7.0, device="cuda")
    bank.decode(shipped.Part(0, n_ch, "x", 0, 1, n_ch), width, cols, err)
    part = torch.full((40 * width + 3,), 7.0, device="cuda")  # a channel range at an offset
    bank.decode(shipped.Part(50, 40, "x", 3, width, 1), width, part, err)
    assert int(err.item()) == 0
    assert np.array_equal(rows.cpu().numpy().reshape(n_ch, width), want)
    assert np.array_equal(cols.cpu().numpy().reshape(width, n_ch), want.T)
    assert np.array_equal(part.cpu().numpy()[3:].reshape(40, width), want[50:90])


def test_codec_decode_flags_missing_codebook_rows():
    from altxs_amd import shipped

    _log("codec decode error flag")
    rng = np.random.default_rng(1)
    bits, packed, books, _ = random_bank(rng, 32, 512, "lloyd")
    books[3] = books[3][:2]  # two channels' worth of levels only
    bank = shipped.DeviceBank(bits, packed, books, "lloyd", None, "cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.zeros(32 * 512, device="cuda")
    bank.decode(shipped.Part(0, 32, "x", 0, 512, 1), 512, out, err)
    assert int(err.item()) == 2
    rank3 = np.flatnonzero(bits == 3)
    if rank3.size > 2:  # channels past the codebook are zero, the others decoded
        assert not out.view(32, 512)[int(rank3[2])].any()


def test_pack_dense_matches_host_packer():
    from altxs_amd import codec, shipped

    _log("pack dense")
    rng = np.random.default_rng(2)
    base = rng.standard_normal((48, 768)).astype(np.float32)
    delta = (rng.standard_normal((48, 768)) * 1e-3).astype(np.float32)
    got = shipped.pack_dense(torch.from_numpy(delta).cuda(), torch.from_numpy(base).cuda())
    want = codec.pack_dense_tiled(base + delta)
    assert np.array_equal(got.cpu().numpy(), want)
    got32 = shipped.pack_dense(torch.from_numpy(delta).cuda(), torch.from_numpy(base).cuda(), bits=32)
    assert np.array_equal(got32.cpu().numpy(), codec.pack_dense32_tiled(base + delta))
    hi, mid, lo = codec.split3_bf16(base + delta)  # the planes sum back to the fp32 value exactly
    planes = [(p.astype(np.uint32) << np.uint32(16)).view(np.float32) for p in (hi, mid, lo)]
    assert np.array_equal((planes[0] + planes[1]) + planes[2], base + delta)
    got0 = shipped.pack_dense(torch.from_numpy(delta).cuda())
    assert np.array_equal(got0.cpu().numpy(), codec.pack_dense_tiled(delta))


def test_shipped_codec_end_to_end(tmp_path):
    from safetensors.numpy import save_file

    from altxs_amd import codec, shipped, synth
    from altxs_amd.config import make_config
    from altxs_amd.model import StepModel
    from oracle import codec_ref
    from oracle.model_ref import OracleModel

    _log("shipped codec end to end (tiny)")
    cfg = make_config("tiny")
    L, d, kvd, F, V = cfg.num_layers, cfg.model_dim, cfg.kv_dim, cfg.hidden_dim, cfg.vocab_size
    shapes = {"tok_emb.weight": [V, d], "qo_bank": [2 * L, d, d], "kv_bank": [2 * L, kvd, d],
              "mlp_up_bank": [L, F, d], "mlp_down_bank": [L, d, F]}
    rng = np.random.default_rng(11)
    sm0 = synth.make_model(cfg, std=0.08, softcap=(2.0, 1.5))
    init = {n: (rng.standard_normal(s) * 0.06).astype(np.float32) for n, s in shapes.items()}
    state, layouts = {}, {}
    delta = {}
    for name, shape in shapes.items():
        n_ch = int(np.prod(shape)) // d
        bits, packed, books, _ = random_bank(rng, n_ch, d, "lloyd")
        state[f"bits/{name}"] = bits
        for b in (2, 3, 4):
            state[f"packed/{name}/b{b}"] = packed[b]
            state[f"codebook/{name}/b{b}"] = books[b]
        layouts[name] = {"shape": shape, "channels": n_ch, "channel_width": d, "fp16": False}
        ch = codec_ref.dequantize_channels(bits, books, packed, channel_width=d, mode="lloyd")
        delta[name] = codec_ref.from_channels(name, ch, shape, L)
    small_names = sorted(sm0.small)
    for n in small_names:
        state[f"small/{n}"] = np.ascontiguousarray(sm0.small[n], dtype=np.float32)
    cfg_meta = {f: getattr(cfg, f) for f in ("vocab_size", "num_layers", "xsa_last_n", "model_dim",
                                              "num_heads", "num_kv_heads", "mlp_mult", "rope_dims",
                                              "rope_yarn", "num_loops", "loop_start", "loop_end",
                                              "parallel_start_layer", "block_size")}
    meta = {"format": "hope_mixed_bit_delta", "format_version": 5, "seed": 1, "cfg": cfg_meta,
            "codebook_mode": "lloyd", "n_layers": L, "layouts": layouts, "small_params": small_names}
    stem = str(tmp_path / "codec")
    save_file(state, stem + ".safetensors")
    json.dump(meta, open(stem + ".json", "w"))

    cfg2, weights, small = shipped.load_shipped(stem + ".safetensors", init)
    assert cfg2 == cfg
    model_sm = synth.SynthModel(cfg2, weights, {k: np.asarray(v) for k, v in small.items()})
    # the oracle runs bf16(Init + delta), reassembled into reference banks
    dense = {n: torch.from_numpy(init[n] + delta[n]).to(torch.bfloat16).float().numpy() for n in shapes}
    sd = dict(sm0.small)
    sd.update(dense)
    for l in range(L):  # the device tiles hold exactly these values
        qkv = np.concatenate([dense["qo_bank"][l], dense["kv_bank"][l], dense["kv_bank"][L + l]])
        assert np.array_equal(weights[f"l{l}.qkv"].tiled.cpu().numpy(), codec.pack_dense_tiled(qkv))
        assert np.array_equal(weights[f"l{l}.down"].tiled.cpu().numpy(),
                              codec.pack_dense_tiled(dense["mlp_down_bank"][l]))
    toks = synth.zipf_tokens(V, (2, 10), seed=4).astype(np.int32)
    model = StepModel(model_sm, act="fp32")
    st = model.make_static_state(256, win=1, batch=2)
    got = []
    for t in range(toks.shape[1]):
        st.token.copy_(torch.from_numpy(toks[:, t:t + 1]))
        model.step(st, commit=True)
        got.append(st.logits.cpu().numpy().copy())
    st.check_errors()
    got = np.stack(got, 1)
    om = OracleModel(cfg, sd, max_len=256)
    want = np.stack([om.decode_rows(t).numpy() for t in toks.astype(np.int64)])
    err = np.abs(got - want).max()
    _log(f"max |dlogit| = {err:.3e}")
    assert err < 2e-4, err
    # the reference-named loader in the fp32 mode keeps Init + delta in fp32
    # (bits-32 banks): the oracle on the unrounded sum
    from altxs_amd import dropin

    model2, meta2, _ = dropin.load_codec(stem + ".safetensors", device="cuda", init_state=init, act="fp32")
    assert meta2["codebook_mode"] == "lloyd"
    assert all(model2.qt[n].bits == 32 for n in model2.qt)
    st2 = model2.make_static_state(256, win=1, batch=2)
    got2 = []
    for t in range(toks.shape[1]):
        st2.token.copy_(torch.from_numpy(toks[:, t:t + 1]))
        model2.step(st2, commit=True)
        got2.append(st2.logits.cpu().numpy().copy())
    st2.check_errors()
    sd32 = dict(sm0.small)
    sd32.update({n: init[n] + delta[n] for n in shapes})
    om32 = OracleModel(cfg, sd32, max_len=256)
    want32 = np.stack([om32.decode_rows(t).numpy() for t in toks.astype(np.int64)])
    err32 = np.abs(np.stack(got2, 1) - want32).max()
    _log(f"fp32 banks: max |dlogit| = {err32:.3e}")
    assert err32 < 2e-4, err32


def test_real_student_decodes_whole_asset(golden_dir):
    """The reference's shipped codec (tests/golden/shipped/, its
    weights/mixed_da_bpw3.15_upb1.8.*) through ``dropin.load_codec(path,
    device=...)``: Init(seed) restated, the whole delta decoded and added on
    the device, the 17-slot student (GQA, depth loops, parallel lanes, XSA,
    gates) stepped W=1 from the stream start.
    * fp32 banks: logits within 2e-3 of the fp32 logits the reference's own
      load_codec model wrote (tests/golden/shipped_full.npz);
    * bf16 banks and bf16 activations (the reference's production dtypes,
      model.py:1183-1245, compress.py:58-61): no farther from the fp32
      reference logits than the reference's own eager step under its bf16
      autocast policy is (rows_w1_autocast_bf16, written by the reference:
      0.52 max, 0.083 mean on this student), in max and in mean."""
    import os

    from altxs_amd import dropin
    from oracle import coder

    z = np.load(os.path.join(golden_dir, "shipped_full.npz"))
    path = os.path.join(golden_dir, "shipped", "mixed_da_bpw3.15_upb1.8.safetensors")
    toks = z["tokens"].astype(np.int32)
    ref = z["rows_w1"]
    ref_bf16 = np.abs(z["rows_w1_autocast_bf16"] - ref)
    for act in ("fp32", "bf16"):
        _log(f"real student, {act} banks")
        model, meta, small = dropin.load_codec(path, device="cuda", act=act)
        assert model.n_slots == 17 and model.cfg.vocab_size == 256
        st = model.make_static_state(int(z["max_len"]), win=1, batch=1)
        rows, cums = [], []
        for t in range(toks.size):
            st.token.fill_(int(toks[t]))
            model.step(st, commit=True)
            rows.append(st.logits[0].cpu().numpy().copy())
            cums.append(st.cum[0].cpu().numpy().copy())
        st.check_errors()
        d = np.abs(np.stack(rows) - ref)
        _log(f"{act}: max |dlogit| = {d.max():.3e}, mean {d.mean():.3e} (reference bf16 autocast: "
             f"{ref_bf16.max():.3e}, {ref_bf16.mean():.3e}; logits up to {np.abs(ref).max():.1f})")
        if act == "fp32":
            assert d.max() < 2e-3, d.max()
        else:
            assert d.max() <= ref_bf16.max() and d.mean() <= ref_bf16.mean(), (d.max(), d.mean())
        # the last row's table is the rule applied to the device probabilities
        assert np.array_equal(cums[-1].astype(np.int64), coder.scale_cum(st.probs[0].cpu().numpy()[None])[0])


def _decode_on_device(bits, packed, books, mode, width, scales=None):
    from altxs_amd import shipped

    bank = shipped.DeviceBank(bits, packed, books, mode, scales, "cuda")
    n = int(np.asarray(bits).size)
    out = torch.full((n * width,), float("nan"), dtype=torch.float32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    bank.decode(shipped.Part(0, n, "x", 0, width, 1), width, out, err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    return out.view(n, width).cpu().numpy()


def test_shipped_asset_slices_decode_like_the_reference(golden_dir):
    import os

    _log("shipped asset slices on the device")
    z = np.load(os.path.join(golden_dir, "shipped_slice.npz"))
    mode = str(z["mode"])
    for bank in ("tok_emb.weight", "qo_bank", "kv_bank", "mlp_up_bank", "mlp_down_bank"):
        bits = z[f"{bank}/bits"]
        packed = {b: z[f"{bank}/packed_b{b}"] for b in (2, 3, 4)}
        books = {b: z[f"{bank}/codebook_b{b}"] for b in (2, 3, 4)}
        got = _decode_on_device(bits, packed, books, mode, int(z[f"{bank}/width"]))
        want = z[f"{bank}/out"]
        assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist(), bank


@pytest.mark.parametrize("mode", ["lloyd", "symmetric", "shared", "fp4", "hybrid_fp4_symmetric"])
def test_codec_modes_decode_like_the_reference(golden_dir, mode):
    import os

    _log(f"codec mode {mode} vs reference vectors")
    z = np.load(os.path.join(golden_dir, "codec_modes.npz"))
    bits, width = z["bits"], int(z["width"])
    packed = {b: z[f"{mode}/packed_b{b}"] for b in (2, 3, 4)}
    books = {b: z[f"{mode}/codebook_b{b}"] for b in (2, 3, 4)}
    scales = {b: z[f"{mode}/scale_b{b}"] for b in (2, 3, 4) if f"{mode}/scale_b{b}" in z.files} or None
    got = _decode_on_device(bits, packed, books, mode, width, scales)
    want = z[f"{mode}/out"]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), mode
