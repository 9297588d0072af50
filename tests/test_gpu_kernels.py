"""GPU parity of the standalone kernels (through the C-ABI) against the CPU oracle."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


# ---------------------------------------------------------------- CDF ----------

def _adversarial_rows(V: int, rng) -> np.ndarray:
    rows = []
    rows.append(np.full(V, 1.0 / V, np.float32))
    r = np.zeros(V, np.float32)
    r[V // 3] = 1.0
    rows.append(r)
    # values straddling the (k - 1/2) * 1e-6 rounding boundaries
    ks = rng.integers(1, 5000, V)
    r = ((ks - 0.5) * 1e-6).astype(np.float32)
    r = np.nextafter(r, np.where(rng.random(V) < 0.5, 0, 1).astype(np.float32))
    rows.append(r)
    rows.append(np.full(V, 1e-40, np.float32))  # denormals
    return np.stack(rows)


@pytest.mark.parametrize("V", [256, 4096, 16384, 65536])
def test_scale_cum_bit_exact(V):
    from altxs_amd import ops
    from oracle import coder

    _log(f"scale_cum V={V}")
    rng = np.random.default_rng(V)
    lg = rng.standard_normal((37, V)).astype(np.float32) * 3
    p = np.exp(lg - lg.max(1, keepdims=True))
    p = (p / p.sum(1, keepdims=True)).astype(np.float32)
    p = np.concatenate([p, _adversarial_rows(V, rng)])
    got = ops.scale_cum(torch.from_numpy(p).to(DEV)).cpu().numpy().astype(np.int64)
    torch.cuda.synchronize()
    assert np.array_equal(got, coder.scale_cum(p))


@pytest.mark.parametrize("V", [256, 4096, 16384])
def test_softmax_cdf_matches_torch_and_is_batch_invariant(V):
    from altxs_amd import ops
    from oracle import coder

    _log(f"softmax_cdf V={V}")
    rng = np.random.default_rng(1)
    lg = torch.from_numpy(rng.standard_normal((64, V)).astype(np.float32) * 4).to(DEV)
    probs, cum = ops.softmax_cdf(lg)
    ref = torch.softmax(lg.double().cpu(), -1)
    assert (probs.double().cpu() - ref).abs().max() < 1e-6 * max(1.0, float(ref.max()))
    # the CDF is exactly the count rule on the kernel's own probabilities
    assert np.array_equal(cum.cpu().numpy().astype(np.int64), coder.scale_cum(probs.cpu().numpy()))
    # a row alone gives the same bits as inside a batch, and reruns agree
    for r in (0, 17, 63):
        p1, c1 = ops.softmax_cdf(lg[r:r + 1].contiguous())
        assert torch.equal(p1[0], probs[r]) and torch.equal(c1[0], cum[r])
    p2, c2 = ops.softmax_cdf(lg)
    assert torch.equal(p2, probs) and torch.equal(c2, cum)
    # renormalised mode sums to one
    pr, _ = ops.softmax_cdf(lg, renorm=True, want_cdf=False)
    assert (pr.double().sum(-1) - 1).abs().max() < 1e-5


# --------------------------------------------------------------- GEMM ----------

def _packed(bits, n, k, seed, std=0.02):
    from altxs_amd.codec import PackedTensor

    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k)).astype(np.float32) * std
    return PackedTensor.from_dense("w", w, bits)


@pytest.mark.parametrize("bits", [2, 3, 4, 6])
@pytest.mark.parametrize("shape", [(512, 2048), (2048, 512)])
def test_dequant_bit_exact(bits, shape):
    from altxs_amd import ops
    from oracle import codec_ref

    _log(f"dequant bits={bits} shape={shape}")
    p = _packed(bits, *shape, seed=bits)
    w = ops.DeviceQTensor(p)
    got = ops.dequant(w).cpu().numpy()
    want = codec_ref.dequant_group64(p.codes, p.scales, bits)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bits", [2, 3, 4, 6])
@pytest.mark.parametrize("shape", [(512, 2048), (2048, 512)])
@pytest.mark.parametrize("B", [1, 64])
@pytest.mark.parametrize("xdt", ["f16", "bf16", "f32"])
def test_qgemm_against_fp32_matmul(bits, shape, B, xdt):
    from altxs_amd import ops
    from oracle import codec_ref

    _log(f"qgemm bits={bits} shape={shape} B={B} x={xdt}")
    n, k = shape
    p = _packed(bits, n, k, seed=10 + bits)
    w = ops.DeviceQTensor(p)
    rng = np.random.default_rng(B)
    x32 = torch.from_numpy(rng.standard_normal((B, k)).astype(np.float32))
    dt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[xdt]
    x = x32.to(dt)
    y = ops.qgemm(w, x.to(DEV).contiguous()).cpu().double()
    wd = torch.from_numpy(codec_ref.dequant_group64(p.codes, p.scales, bits)).double()
    ref = x.double() @ wd.T
    err = (y - ref).abs().max().item()
    assert err < 1e-3, err  # fp32 accumulation of exact products
    assert err < 1e-5 * max(1.0, ref.abs().max().item()) * math.sqrt(k)


@pytest.mark.parametrize("shape", [(512, 2048), (2048, 512), (16, 256)])
@pytest.mark.parametrize("B", [1, 5, 64])
def test_qgemm_dense_fp32_weights(shape, B):
    """bits 32 (fp32 weights as three exact bf16 planes) with fp32 x: the
    products of an fp32 matmul to ~2^-24 relative per term; bits 16 of the
    same weights misses that bound (the planes matter); bf16 or fp16 x is
    refused."""
    from altxs_amd import ops
    from altxs_amd.codec import PackedTensor

    _log(f"qgemm bits=32 shape={shape} B={B}")
    n, k = shape
    rng = np.random.default_rng(40 + B)
    w32 = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    x32 = torch.from_numpy(rng.standard_normal((B, k)).astype(np.float32))
    ref = x32.double() @ torch.from_numpy(w32).double().T
    bound = 1e-6 * math.sqrt(k) * max(1.0, ref.abs().max().item())
    w = ops.DeviceQTensor(PackedTensor.from_dense("w", w32, 32))
    y = ops.qgemm(w, x32.to(DEV).contiguous()).cpu().double()
    err = (y - ref).abs().max().item()
    assert err < bound, (err, bound)
    w16 = ops.DeviceQTensor(PackedTensor.from_dense("w", w32, 16))
    y16 = ops.qgemm(w16, x32.to(DEV).contiguous()).cpu().double()
    assert (y16 - ref).abs().max().item() > 10 * bound
    with pytest.raises(RuntimeError):
        ops.qgemm(w, x32.to(torch.bfloat16).to(DEV).contiguous())


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(2048, 512), (512, 2048)])
@pytest.mark.parametrize("bits", [2, 3, 4, 6])
def test_qgemm_batch_invariant(xdt, shape, bits):
    """Rows of 1, 17 and 64 (16-row tiles) equal the same rows of a 4200-row
    launch (64 x 128 tiles for 16-bit x, enough of them to fill the chip) bit
    for bit."""
    from altxs_amd import ops

    _log(f"qgemm batch invariance {xdt} {shape} b={bits}")
    n, k = shape
    p = _packed(bits, n, k, seed=3)
    w = ops.DeviceQTensor(p)
    x = torch.randn(4200, k, generator=torch.Generator().manual_seed(0)).to(xdt).to(DEV)
    y_all = ops.qgemm(w, x)
    y64 = ops.qgemm(w, x[:64].contiguous())
    assert torch.equal(y_all[:64], y64)
    for r in (0, 5, 31, 63, 100, 4199):
        y1 = ops.qgemm(w, x[r:r + 1].contiguous())
        assert torch.equal(y1[0], y_all[r])
    y17 = ops.qgemm(w, x[:17].contiguous())
    assert torch.equal(y17, y64[:17])


def test_qgemm_stream_matches_single():
    from altxs_amd import ops

    _log("qgemm_stream")
    count, n, k, bits = 5, 512, 2048, 3
    ps = [_packed(bits, n, k, seed=100 + i) for i in range(count)]
    cs, ss = ps[0].tiled.size, ps[0].tiled_scales.size * 2
    codes = torch.from_numpy(np.concatenate([p.tiled for p in ps])).to(DEV)
    scales = torch.from_numpy(np.concatenate([p.tiled_scales for p in ps]).view(np.int16)).to(DEV)
    x = torch.randn(3, k).to(torch.float16).to(DEV)
    out = torch.empty(count, 3, n, device=DEV)
    ops.qgemm_stream(codes, scales, count, n, k, bits, cs, ss, x, out)
    for i, p in enumerate(ps):
        assert torch.equal(out[i], ops.qgemm(ops.DeviceQTensor(p), x))
    # 80 matrices x 40 rows: the stream takes the 64 x 128 tiles (320
    # workgroups), a single matrix the 16-row tiles; the same bits
    g = torch.Generator(device=DEV).manual_seed(1)
    many = 80
    codes2 = torch.randint(0, 256, (many * cs,), dtype=torch.uint8, device=DEV, generator=g)
    scales2 = (torch.rand(many * ss // 2, device=DEV, generator=g) * 0.05 + 0.001).half().view(torch.int16)
    x = torch.randn(40, k, device=DEV, generator=g).to(torch.float16)
    out = torch.empty(many, 40, n, device=DEV)
    ops.qgemm_stream(codes2, scales2, many, n, k, bits, cs, ss, x, out)
    for i in (0, 37, many - 1):
        one = torch.empty(40, n, device=DEV)
        ops.qgemm_stream(codes2[i * cs:], scales2[i * ss // 2:], 1, n, k, bits, cs, ss, x, one)
        assert torch.equal(out[i], one)


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bits", [3, 6])
def test_qgemm_stream_row_band_matches_single(xdt, bits):
    """K = 512 matrices streamed 60 at a time with 100 rows: the batched
    row-band kernel (its one band per matrix partly past the 100 rows) gives
    the bits of each matrix alone on the 16-row tiles."""
    from altxs_amd import ops

    _log(f"qgemm_stream row band {xdt} b={bits}")
    many, n, k, rows = 60, 1024, 512, 100
    g = torch.Generator(device=DEV).manual_seed(7)
    cs = n * k * bits // 8
    ss = n * k // 64 * 2
    codes = torch.randint(0, 256, (many * cs,), dtype=torch.uint8, device=DEV, generator=g)
    scales = (torch.rand(many * ss // 2, device=DEV, generator=g) * 0.05 + 0.001).half().view(torch.int16)
    x = torch.randn(rows, k, device=DEV, generator=g).to(xdt)
    out = torch.empty(many, rows, n, device=DEV)
    ops.qgemm_stream(codes, scales, many, n, k, bits, cs, ss, x, out)
    for i in (0, 29, many - 1):
        for r0, r1 in ((0, 16), (16, 33), (84, 100)):  # 16-row tiles
            one = torch.empty(r1 - r0, n, device=DEV)
            ops.qgemm_stream(codes[i * cs:], scales[i * ss // 2:], 1, n, k, bits, cs, ss,
                             x[r0:r1].contiguous(), one)
            assert torch.equal(out[i, r0:r1], one), (i, r0)


# ---------------------------------------------------------- attention ----------

def _attn_ref(q, k, v, pos, W, gate, use_xsa):
    """fp64 reference on the (already rounded) cache values. q [R,H,64]; k/v [B,Hkv,L,64]."""
    R, H, hd = q.shape
    B, Hkv = k.shape[0], k.shape[1]
    g = H // Hkv
    out = torch.zeros(R, H, hd, dtype=torch.float64)
    for r in range(R):
        b, t = divmod(r, W)
        p = int(pos[b]) + t
        for h in range(H):
            kk = k[b, h // g, : p + 1].double()
            vv = v[b, h // g, : p + 1].double()
            s = (kk @ q[r, h].double()) / 8.0
            y = torch.softmax(s, 0) @ vv
            if use_xsa:
                vc = v[b, h // g, p].double()
                vn = vc / max(vc.norm().item(), 1e-12)
                y = y - (y @ vn) * vn
            if gate is not None:
                y = y * float(gate[r, h])
            out[r, h] = y
    return out.reshape(R, H * hd)


@pytest.mark.parametrize("kv", ["fp32", "bf16"])
@pytest.mark.parametrize("H,Hkv", [(4, 4), (4, 2), (8, 2)])
def test_decode_attention_against_reference(kv, H, Hkv):
    from altxs_amd import ops

    _log(f"attn kv={kv} H={H} Hkv={Hkv}")
    B, W, L = 3, 2, 768
    gen = torch.Generator().manual_seed(H * 10 + Hkv)
    pos = torch.tensor([0, 300, 700], dtype=torch.int32)  # ragged; 700+1 < 768
    dt = torch.bfloat16 if kv == "bf16" else torch.float32
    k = torch.randn(B, Hkv, L, 64, generator=gen).to(dt)
    v = torch.randn(B, Hkv, L, 64, generator=gen).to(dt)
    q = torch.randn(B * W, H, 64, generator=gen) * 3
    gate = torch.rand(B * W, H, generator=gen)
    y = ops.decode_attn(q.to(DEV), k.to(DEV), v.to(DEV), pos.to(DEV), W=W, gate=gate.to(DEV),
                        use_xsa=True)
    ref = _attn_ref(q, k.float(), v.float(), pos, W, gate, True)
    assert (y.cpu().double() - ref).abs().max() < 2e-5


@pytest.mark.parametrize("H,Hkv", [(4, 4), (8, 2), (8, 8)])
def test_decode_attention_bf16_operands(H, Hkv):
    """bf16 q and softmax weights (the reference's tl.dot arithmetic).

    Against an fp64 reference on the bf16-rounded q: what remains is the bf16
    rounding of the unnormalised weights exp(s - m) in [0, 1] (relative error
    <= 2^-9 each), so |y - ref| <= 2^-8 * max|v| bounds it with margin.
    """
    from altxs_amd import ops

    _log(f"attn bf16 operands H={H} Hkv={Hkv}")
    B, W, L = 3, 2, 768
    gen = torch.Generator().manual_seed(H * 100 + Hkv)
    pos = torch.tensor([0, 300, 700], dtype=torch.int32)
    k = torch.randn(B, Hkv, L, 64, generator=gen).to(torch.bfloat16)
    v = torch.randn(B, Hkv, L, 64, generator=gen).to(torch.bfloat16)
    q = torch.randn(B * W, H, 64, generator=gen) * 3
    y = ops.decode_attn(q.to(DEV), k.to(DEV), v.to(DEV), pos.to(DEV), W=W, ops_bf16=True)
    qr = (q * 0.125).to(torch.bfloat16).float() * 8.0
    ref = _attn_ref(qr, k.float(), v.float(), pos, W, None, False)
    err = (y.cpu().double() - ref).abs().max().item()
    vmax = v.float().abs().max().item()
    assert err <= vmax * 2.0 ** -8, err
    # the fp32-faithful path on the same inputs is an order of magnitude closer
    y32 = ops.decode_attn(q.to(DEV), k.to(DEV), v.to(DEV), pos.to(DEV), W=W)
    ref32 = _attn_ref(q, k.float(), v.float(), pos, W, None, False)
    assert (y32.cpu().double() - ref32).abs().max().item() < 2e-5


@pytest.mark.parametrize("H,Hkv,W", [(8, 8, 2), (8, 8, 16), (8, 8, 17), (8, 2, 33), (4, 1, 64),
                                     (8, 8, 100), (4, 4, 257)])
def test_window_kernel_bit_identical_to_rows(H, Hkv, W):
    """The window kernel (up to 64 rows of a segment per K/V read) gives every
    row the bits of the one-row decode kernel: ragged last blocks, GQA, XSA,
    the sparse gate, windows starting at 0 (prefill) and ending at max_len."""
    from altxs_amd import ops

    _log(f"window kernel H={H} Hkv={Hkv} W={W}")
    B, L = 3, 512
    gen = torch.Generator().manual_seed(W * 10 + H + Hkv)
    k = torch.randn(B, Hkv, L, 64, generator=gen).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, Hkv, L, 64, generator=gen).to(torch.bfloat16).to(DEV)
    q = (torch.randn(B * W, H, 64, generator=gen) * 3).to(DEV)
    gate = torch.rand(B * W, H, generator=gen).to(DEV)
    pos = torch.tensor([0, 61, L - W], dtype=torch.int32, device=DEV)
    for ob in (False, True):
        for yb in (False, True):
            got = ops.decode_attn(q, k, v, pos, W=W, gate=gate, use_xsa=True, ops_bf16=ob, y_bf16=yb)
            want = ops.decode_attn(q, k, v, pos, W=W, gate=gate, use_xsa=True, ops_bf16=ob, y_bf16=yb,
                                   rows=True)
            assert torch.equal(got, want), (ob, yb)


def test_decode_attention_window_equals_rows():
    """Row at position p computes the same bits as W=1 and inside a W=4 window."""
    from altxs_amd import ops

    _log("attn W=4 vs W=1 bit equality")
    B, L, H = 2, 1024, 8
    gen = torch.Generator().manual_seed(7)
    k = torch.randn(B, H, L, 64, generator=gen).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, H, L, 64, generator=gen).to(torch.bfloat16).to(DEV)
    q = (torch.randn(B * 4, H, 64, generator=gen) * 3).to(DEV)
    pos = torch.tensor([253, 510], dtype=torch.int32, device=DEV)  # windows cross chunk edges
    for ob in (False, True):
        y4 = ops.decode_attn(q, k, v, pos, W=4, use_xsa=True, ops_bf16=ob)
        for t in range(4):
            q1 = q.view(B, 4, H, 64)[:, t].contiguous()
            y1 = ops.decode_attn(q1, k, v, pos + t, W=1, use_xsa=True, ops_bf16=ob)
            assert torch.equal(y1, y4.view(B, 4, -1)[:, t])


def test_decode_attention_xcd_row_placement_same_bits():
    """The row-local XCD placement (8-row tiles, tile t on XCD t % 8) through the
    public entry gives the bits of the linear placement, for 64 and 128 rows,
    MHA and GQA; at 24 rows (not a multiple of 64) the flag is ignored."""
    from altxs_amd import ops

    _log("attn xcd row placement vs linear")
    L = 512
    for B, H, Hkv in ((64, 8, 8), (128, 8, 4), (24, 8, 8)):
        gen = torch.Generator().manual_seed(B + Hkv)
        k = torch.randn(B, Hkv, L, 64, generator=gen).to(torch.bfloat16).to(DEV)
        v = torch.randn(B, Hkv, L, 64, generator=gen).to(torch.bfloat16).to(DEV)
        q = (torch.randn(B, H, 64, generator=gen) * 3).to(DEV)
        pos = torch.randint(0, L, (B,), generator=gen, dtype=torch.int32).to(DEV)
        for ob in (False, True):
            want = ops.decode_attn(q, k, v, pos, use_xsa=True, ops_bf16=ob, y_bf16=True)
            got = ops.decode_attn(q, k, v, pos, use_xsa=True, ops_bf16=ob, y_bf16=True, xcd_rows=True)
            assert torch.equal(got, want), (B, Hkv, ob)


def test_attention_position_error_flag():
    from altxs_amd import ops

    _log("attn pos out of range -> error flag, no fault")
    k = torch.zeros(1, 1, 256, 64, device=DEV)
    q = torch.zeros(1, 1, 64, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.decode_attn(q, k, k.clone(), torch.tensor([999], dtype=torch.int32, device=DEV), err=err)
    assert int(err.item()) & 1
