"""The C-ABI library loads, exports every declared symbol and matches the header layout.

No compute calls: these run without a GPU.
"""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from altxs_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "altxs.h")


def _declared() -> list[str]:
    text = open(HEADER, encoding="utf8").read()
    return sorted(set(re.findall(r"^\s*(?:int32_t|int64_t|const char \*)\s*(altxs_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} missing: run `python -m altxs_amd.build`")
    L = _lib.load()
    declared = _declared()
    assert set(declared) == set(_lib.EXPORTS)
    for name in declared:
        assert hasattr(L, name), name
    assert L.altxs_abi_version() == _lib.ABI_VERSION
    assert L.altxs_last_error() == b""


def test_bad_arguments_return_errors_without_gpu():
    L = _lib.load()
    rc = L.altxs_scale_cum(None, 1, 256, None, None)
    assert rc == -1 and b"null" in L.altxs_last_error()
    d = _lib.StepDesc()
    d.abi_version = 999
    assert L.altxs_step(ctypes.byref(d), None) == -1
    assert b"abi_version" in L.altxs_last_error()
    assert L.altxs_range_encode(None, 1, 1, None, None, 256, None, 64, None) == -1
    assert b"altxs_range_encode" in L.altxs_last_error()
    assert L.altxs_range_decode(None, 1, None, 1, None, 64, None, 1, None) == -1
    assert L.altxs_codec_decode(None, None, None, 1, 512, None, 512, 1, None, None) == -1
    assert L.altxs_pack_dense(None, None, 16, 256, 256, None, None) == -1
    assert b"altxs_pack_dense" in L.altxs_last_error()
    # a bits-32 buffer smaller than N*K*6 bytes is refused before any launch
    fake = ctypes.c_void_p(1 << 20)
    assert L.altxs_pack_dense32(None, fake, 16, 256, 256, fake, 16 * 256 * 4, None) == -1
    assert b"bytes" in L.altxs_last_error()
    # the row GEMV takes 1..4 fp16/bf16 rows of packed (not dense) weights
    qt = _lib.QTensor(1 << 20, 1 << 20, 512, 2048, 4, 0)
    for rows, xdt, bits, what in ((5, _lib.F16, 4, b"rows"), (0, _lib.F16, 4, b"rows"),
                                  (1, _lib.F32, 4, b"fp16 or bf16"), (1, _lib.F16, 16, b"bits")):
        qt.bits = bits
        assert L.altxs_qgemv(ctypes.byref(qt), fake, xdt, rows, fake, None) == -1
        assert what in L.altxs_last_error(), L.altxs_last_error()
    # the stage entry points check shapes and pointers before any launch
    a = _lib.FfnStageArgs()
    a.win, a.d, a.mlp, a.act_dtype = 4, 384, 2048, _lib.BF16
    assert L.altxs_ffn_stage_rows(ctypes.byref(a), None) == -1
    assert b"d=384" in L.altxs_last_error()
    a.d = 512
    assert L.altxs_ffn_stage_rows(ctypes.byref(a), None) == -1
    assert b"out_w" in L.altxs_last_error()
    assert L.altxs_attn_gate(fake, _lib.F16, 16, fake, 8, 12, 1, fake, None) == -1
    assert b"x_dtype" in L.altxs_last_error()
    qt.bits = 4
    assert L.altxs_qgemv_stream(ctypes.byref(qt), 2, 512 * 1024, 16, fake, _lib.F16, 1, fake, None) == -1
    assert b"strides" in L.altxs_last_error()


def test_dense_sizes():
    from altxs_amd import codec, shipped

    assert shipped.dense_bytes(48, 768, 16) == 48 * 768 * 2
    assert shipped.dense_bytes(48, 768, 32) == 48 * 768 * 6
    w = np.zeros((48, 768), np.float32)
    assert codec.pack_dense32_tiled(w).size == shipped.dense_bytes(48, 768, 32)
    assert codec.pack_dense_tiled(w).size == shipped.dense_bytes(48, 768, 16)
    with pytest.raises(ValueError):
        shipped.dense_bytes(48, 768, 8)


def test_struct_layout_matches_header(tmp_path):
    """sizeof/offsetof from the C compiler equal the ctypes mirror."""
    src = tmp_path / "layout.c"
    src.write_text(f"""
#include <stdio.h>
#include <stddef.h>
#include "{HEADER}"
int main(void) {{
  printf("%zu %zu %zu %zu %zu\\n", sizeof(AltxsQTensor), sizeof(AltxsAttnArgs), sizeof(AltxsLayer),
         sizeof(AltxsSlot), sizeof(AltxsStepDesc));
  printf("%zu %zu %zu %zu\\n", offsetof(AltxsStepDesc, layers), offsetof(AltxsStepDesc, emb),
         offsetof(AltxsStepDesc, tokens), offsetof(AltxsStepDesc, err));
  printf("%zu %zu %zu\\n", sizeof(AltxsCoderState), offsetof(AltxsCoderState, nbytes),
         offsetof(AltxsCoderState, err));
  printf("%zu %zu %zu\\n", sizeof(AltxsCodecGroups), offsetof(AltxsCodecGroups, n_codes),
         offsetof(AltxsCodecGroups, mode));
  printf("%zu %zu %zu %zu\\n", sizeof(AltxsFfnStageArgs), offsetof(AltxsFfnStageArgs, out_w),
         offsetof(AltxsFfnStageArgs, y), offsetof(AltxsFfnStageArgs, skips));
  return 0;
}}
""")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    c_sizes = [int(x) for x in out]
    py = [ctypes.sizeof(_lib.QTensor), ctypes.sizeof(_lib.AttnArgs), ctypes.sizeof(_lib.Layer),
          ctypes.sizeof(_lib.Slot), ctypes.sizeof(_lib.StepDesc),
          _lib.StepDesc.layers.offset, _lib.StepDesc.emb.offset, _lib.StepDesc.tokens.offset,
          _lib.StepDesc.err.offset, ctypes.sizeof(_lib.CoderState), _lib.CoderState.nbytes.offset,
          _lib.CoderState.err.offset, ctypes.sizeof(_lib.CodecGroups), _lib.CodecGroups.n_codes.offset,
          _lib.CodecGroups.mode.offset, ctypes.sizeof(_lib.FfnStageArgs), _lib.FfnStageArgs.out_w.offset,
          _lib.FfnStageArgs.y.offset, _lib.FfnStageArgs.skips.offset]
    assert c_sizes == py


def test_fused_out_projection_query_host_logic():
    """altxs_step_fuses_out_proj reads only the descriptor (no GPU): the fused
    out-projection is taken with ALTXS_F_FUSE_O for W = 1, bf16 activations,
    the tiled bf16 cache, MHA and a packed out-projection, and not otherwise;
    it also sizes the workspace for the head terms."""
    L = _lib.load()
    d = _lib.StepDesc()
    d.abi_version = _lib.ABI_VERSION
    d.B, d.W, d.D, d.H, d.Hkv, d.head_dim, d.F, d.V = 4, 1, 512, 8, 8, 64, 2048, 16384
    d.n_layers, d.n_slots, d.max_len = 2, 2, 256
    d.act_bf16, d.kv_bf16 = 1, _lib.KV_BF16
    for i in range(2):
        d.layers[i].o = _lib.QTensor(1 << 20, 1 << 20, 512, 512, 3, 0)
        d.slots[i].layer = i
    q = lambda s=0: L.altxs_step_fuses_out_proj(ctypes.byref(d), s)
    assert q() == 0  # off by default
    base = L.altxs_step_workspace_bytes(ctypes.byref(d))
    d.flags = _lib.F_FUSE_O
    assert q(0) == 1 and q(1) == 1
    # Rp x H x D fp32 per segment group (the split layout's two groups of 16 rows are the larger)
    assert L.altxs_step_workspace_bytes(ctypes.byref(d)) == base + 2 * 16 * 8 * 512 * 4
    assert q(2) == -1 and q(-1) == -1
    assert L.altxs_step_fuses_out_proj(None, 0) == -1
    for field, value in (("W", 4), ("act_bf16", 0), ("kv_bf16", _lib.KV_BF16_NATURAL), ("Hkv", 4)):
        old = getattr(d, field)
        setattr(d, field, value)
        assert q() == 0, field
        setattr(d, field, old)
    d.D = 384  # the prologue's row mapping covers D = 256 and 512
    assert q() == 0
    d.D = 512
    d.layers[0].o.bits = 16  # dense bf16 out-projection
    assert q(0) == 0 and q(1) == 1
