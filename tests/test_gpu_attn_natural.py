"""Attention on the natural-order bf16 cache (ALTXS_KV_BF16_NATURAL).

The natural order is the reference's own k_pack layout, which the drop-in's
states share.  Its launches run the MFMA kernel of the tiled layout with the V
tiles staged through LDS, so:

* on the same cache values, natural and tiled launches give the same output
  bits: decode rows and windows, MHA and GQA, XSA and the sparse gate, both
  operand modes, small launches (two tiles in flight plus prefetch
  workgroups) and large ones;
* with the tail placement (the window's K/V in rows kv_tail_end - W + t, the
  reference StaticKV's tail), a row gives the bits of the same logical cache
  with the window rows at pos + t.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def _case(B, W, H, Hkv, L, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(B, Hkv, L, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, L, 64, generator=g).to(torch.bfloat16)
    q = torch.randn(B * W, H, 64, generator=g) * 2
    gate = torch.rand(B * W, H, generator=g)
    return k.to(DEV), v.to(DEV), q.to(DEV), gate.to(DEV)


@pytest.mark.parametrize("B,W,H,Hkv", [(3, 1, 8, 8), (40, 1, 8, 8), (2, 37, 8, 8), (5, 1, 8, 2),
                                       (2, 9, 8, 4)])
@pytest.mark.parametrize("ops_bf16", [True, False])
def test_natural_equals_tiled(B, W, H, Hkv, ops_bf16):
    from altxs_amd import ops

    _log(f"natural vs tiled B={B} W={W} H={H} Hkv={Hkv} ops_bf16={ops_bf16}")
    L = 512
    k, v, q, gate = _case(B, W, H, Hkv, L, seed=B * 100 + W)
    pos = torch.tensor([(37 * b + 11) % (L - W) for b in range(B)], dtype=torch.int32, device=DEV)
    pos[0] = 0
    for xsa, gt in ((False, None), (True, gate)):
        kw = dict(W=W, gate=gt, use_xsa=xsa, ops_bf16=ops_bf16, y_bf16=ops_bf16)
        nat = ops.decode_attn(q, k.contiguous(), v.contiguous(), pos, natural=True, **kw)
        til = ops.decode_attn(q, k.contiguous(), v.contiguous(), pos, **kw)
        rows = ops.decode_attn(q, k.contiguous(), v.contiguous(), pos, rows=True, **kw)
        torch.cuda.synchronize()
        assert torch.equal(til, rows)
        assert torch.equal(nat, til), (xsa, (nat.float() - til.float()).abs().max().item())


@pytest.mark.parametrize("ops_bf16", [True, False])
def test_natural_tail_rows_equal_logical_rows(ops_bf16):
    from altxs_amd import ops

    _log(f"natural tail placement ops_bf16={ops_bf16}")
    B, W, H, Hkv, L = 3, 6, 8, 8, 256
    E = L  # window rows at E - W + t
    k, v, q, gate = _case(B, W, H, Hkv, L, seed=7)
    pos = torch.tensor([0, 100, 249 - W], dtype=torch.int32, device=DEV)
    # the logical cache: row pos + t holds the tail row E - W + t
    kl, vl = k.clone(), v.clone()
    for b in range(B):
        p = int(pos[b])
        kl[b, :, p:p + W] = k[b, :, E - W:E]
        vl[b, :, p:p + W] = v[b, :, E - W:E]
    kw = dict(W=W, gate=gate, use_xsa=True, ops_bf16=ops_bf16, natural=True)
    tail = ops.decode_attn(q, k.contiguous(), v.contiguous(), pos, kv_tail_end=E, **kw)
    logical = ops.decode_attn(q, kl.contiguous(), vl.contiguous(), pos, **kw)
    torch.cuda.synchronize()
    assert torch.equal(tail, logical)
