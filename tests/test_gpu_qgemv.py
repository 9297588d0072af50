"""The row GEMV (altxs_qgemv / altxs_qgemv_stream) against the oracle.

* Results against x . dequant(W)^T in float64 (the oracle's dequantisation),
  elementwise within a rounding bound of the kernel's fp32 arithmetic: the
  group sums of |x| weighted by the code range plus the operand offset (128
  for bf16 x), times (40 + 2 K / 64) units of 2^-24 -- the staged group sum
  and its scaling, the eight-step dot2 chain, the scale FMA and the sum over
  groups and lane groups.  A mispaired code or x value is off by a whole
  weight * x term, ~10^5 times the bound.
* Row independence: each row of a 2-, 3- and 4-row call equals that row
  alone, bit for bit.
* The stream form equals single calls bit for bit (other grids and wave
  assignments, the same per-column arithmetic).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def _packed(bits, n, k, seed, std=0.02):
    from altxs_amd.codec import PackedTensor

    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k)).astype(np.float32) * std
    return PackedTensor.from_dense("w", w, bits)


def _bound(p, x: torch.Tensor, off: float) -> torch.Tensor:
    """[rows, N] rounding bound of the kernel's fp32 arithmetic (see module doc)."""
    n, k = p.codes.shape
    s = torch.from_numpy(np.asarray(p.scales, dtype=np.float16).astype(np.float64)).abs()  # [N, K/64]
    ax = x.double().abs().view(-1, k // 64, 64).sum(-1)  # [rows, K/64]
    t = ax @ s.T * (off + 2.0 ** p.bits)
    return t * (40 + 2 * k / 64) * 2.0 ** -24


@pytest.mark.parametrize("bits", [2, 3, 4, 6])
@pytest.mark.parametrize("shape", [(512, 2048), (2048, 512), (48, 768)])
@pytest.mark.parametrize("xdt", ["f16", "bf16"])
def test_qgemv_against_fp64(bits, shape, xdt):
    from altxs_amd import ops
    from oracle import codec_ref

    _log(f"qgemv bits={bits} shape={shape} x={xdt}")
    n, k = shape
    p = _packed(bits, n, k, seed=20 + bits)
    w = ops.DeviceQTensor(p)
    rng = np.random.default_rng(bits + k)
    dt = torch.float16 if xdt == "f16" else torch.bfloat16
    x = torch.from_numpy(rng.standard_normal((4, k)).astype(np.float32) * 2).to(dt)
    y = ops.qgemv(w, x.to(DEV).contiguous()).cpu().double()
    wd = torch.from_numpy(codec_ref.dequant_group64(p.codes, p.scales, bits)).double()
    ref = x.double() @ wd.T
    err = (y - ref).abs()
    bound = _bound(p, x, 0.0 if xdt == "f16" else 128.0)
    _log(f"max err {err.max().item():.2e}, max err/bound {(err / bound).max().item():.3f}")
    assert (err <= bound).all()
    assert err.max().item() < 1e-3  # the benchmark config's tolerance


@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("xdt", ["f16", "bf16"])
def test_qgemv_rows_independent(bits, xdt):
    from altxs_amd import ops

    _log(f"qgemv rows bits={bits} x={xdt}")
    n, k = 512, 2048
    w = ops.DeviceQTensor(_packed(bits, n, k, seed=30 + bits))
    dt = torch.float16 if xdt == "f16" else torch.bfloat16
    g = torch.Generator(device=DEV).manual_seed(bits)
    x = torch.randn(4, k, device=DEV, generator=g).to(dt)
    alone = torch.stack([ops.qgemv(w, x[r:r + 1].contiguous())[0] for r in range(4)])
    for rows in (2, 3, 4):
        got = ops.qgemv(w, x[:rows].contiguous())
        assert torch.equal(got, alone[:rows]), rows


@pytest.mark.parametrize("bits", [2, 6])
def test_qgemv_stream_matches_single(bits):
    from altxs_amd import ops

    _log(f"qgemv_stream bits={bits}")
    n, k = 2048, 512
    g = torch.Generator(device=DEV).manual_seed(7)
    p0 = _packed(bits, n, k, seed=1)
    cs, ss = p0.tiled.size, p0.tiled_scales.size * 2
    # 300 matrices: 38400 wave tasks, more than the grid, so waves walk several
    many = 300
    codes = torch.randint(0, 256, (many * cs,), dtype=torch.uint8, device=DEV, generator=g)
    scales = (torch.rand(many * ss // 2, device=DEV, generator=g) * 0.05 + 0.001).half().view(torch.int16)
    for rows in (1, 3):
        x = torch.randn(rows, k, device=DEV, generator=g).to(torch.float16)
        out = torch.empty(many, rows, n, device=DEV)
        ops.qgemv_stream(codes, scales, many, n, k, bits, cs, ss, x, out)
        for i in (0, 151, many - 1):
            one = torch.empty(rows, n, device=DEV)
            ops.qgemv_stream(codes[i * cs:], scales[i * ss // 2:], 1, n, k, bits, cs, ss, x, one)
            assert torch.equal(out[i], one), (rows, i)
