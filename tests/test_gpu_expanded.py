"""Expanded weight values (altxs_expand_codes, AltxsQTensor.expanded).

* The expanded buffer equals the numpy tiler's bits-16 layout of the values
  code - (2^b - 1)/2 (codec.PackedTensor.from_dense at bits 16 on those
  values) with each block's (lane, k-step) operands transposed to k-step
  order, byte for byte, for every packed width.
* Steps of >= 1024 rows read the expanded values in their large-tile GEMMs
  (QKV / MLP-up / out-projection / LM head row bands, the K = 2048 MLP-down
  tiles): the same windows with and without the expanded copies give the same
  logits, probabilities and tables bit for bit (the row-count tests in
  tests/test_gpu_step.py compare them with the 16-row GEMMs as well).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


@pytest.mark.parametrize("bits", [2, 3, 4, 6])
def test_expand_codes_matches_tiled_values(bits):
    from altxs_amd import _lib, ops
    from altxs_amd.codec import PackedTensor

    _log(f"expand codes bits={bits}")
    n, k = 48, 768
    rng = np.random.default_rng(bits)
    p = PackedTensor.from_dense("w", rng.standard_normal((n, k)).astype(np.float32) * 0.02, bits)
    w = ops.DeviceQTensor(p)
    out = torch.empty(n * k, dtype=torch.bfloat16, device="cuda")
    L = _lib.load()
    _lib.check(L.altxs_expand_codes(ctypes.byref(w.qt), out.data_ptr(),
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
               "altxs_expand_codes")
    vals = p.codes.astype(np.float32) - np.float32(((1 << bits) - 1) / 2)
    # bits-16 tiles hold lane l's eight 16-byte k-step operands together; the
    # expanded blocks hold k-step s's 64 lane operands together
    t16 = np.asarray(PackedTensor.from_dense("e", vals, 16).tiled).view(np.uint8).reshape(-1, 64, 8, 16)
    want = t16.transpose(0, 2, 1, 3).reshape(-1)
    got = out.cpu().view(torch.int16).numpy().view(np.uint8)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("profile", ["cfg4", "tiny512"])
def test_windows_expanded_equal_packed(profile):
    from altxs_amd import synth
    from altxs_amd.config import make_config
    from altxs_amd.model import StepModel

    _log(f"expanded vs packed large tiles: {profile}")
    cfg = (make_config("tiny", model_dim=512, num_heads=8, num_kv_heads=4) if profile == "tiny512"
           else make_config(profile))
    sm = synth.make_model(cfg, std=0.02, softcap=(30.0, 24.0))
    B, T, L = 3, 361, 512
    toks = torch.from_numpy(np.random.default_rng(13).integers(0, cfg.vocab_size, (B, T)).astype(np.int32))
    out = []
    for expand in (False, True):
        model = StepModel(sm, act="bf16", expand=expand)
        assert model._expanded == expand
        st = model.make_static_state(L, win=T, batch=B, want_probs=True)
        st.token.copy_(toks)
        model.step(st)
        torch.cuda.synchronize()
        st.check_errors()
        out.append((st.logits.cpu(), st.probs.cpu(), st.cum.cpu()))
    for a, b in zip(*out):
        assert torch.equal(a, b)
