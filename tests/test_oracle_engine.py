"""Pins the oracle's probability-engine row semantics (CPU only).

``oracle.model_ref.segment_rows_tf`` restates ``_segment_rows_tf`` +
``reset_segment`` (src/xsa_ttt/incremental.py:858-897, 1238-1271): the carry
row is ``_softmax_np`` (fp32 softmax, then ``p /= p.sum()``, compress.py:
64-85) of the logits after the segment's context window, uniform at the
stream start; later rows are the softmax of each window's logits.  The
fixture tests/golden/engine_rows.npz holds rows the reference's own
``StaticACEngine`` produced on its CPU path ("tiny" weights, W=16, block 64,
retrain every 64, so the engine's static length -- and RoPE table -- is 128);
engine_rows_bf16w.npz the same with the weight matrices rounded to bf16.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from altxs_amd import synth
from altxs_amd.config import make_config
from oracle import model_ref as mr

from .refshape import bf16_banks


@pytest.fixture(scope="module")
def eng(golden_dir):
    z = np.load(os.path.join(golden_dir, "engine_rows.npz"))
    cfg = make_config("tiny")
    sm = synth.make_model(cfg, std=float(z["std"]), softcap=tuple(z["softcap"].tolist()))
    return z, cfg, sm


def test_engine_length_rule(eng):
    z, _, _ = eng
    assert mr.engine_max_len(int(z["block"]), int(z["every"]), int(z["win"])) == int(z["max_len"])
    assert mr.engine_max_len(64, 100, 16) == 64 + 112


@pytest.mark.parametrize("fixture", ["engine_rows.npz", "engine_rows_bf16w.npz"])
@pytest.mark.parametrize("key,start", [("rows_start", 0), ("rows_ctx", 100)])
def test_segment_rows_match_reference_engine(eng, golden_dir, fixture, key, start):
    _, cfg, sm = eng
    z = np.load(os.path.join(golden_dir, fixture))
    block, win = int(z["block"]), int(z["win"])
    sd = sm.state_dict() if fixture == "engine_rows.npz" else bf16_banks(sm.state_dict())
    om = mr.OracleModel(cfg, sd, max_len=int(z["max_len"]))
    rows = mr.segment_rows_tf(om, z["arr"], z["arr"][start:start + 64], start, block, win)
    assert np.abs(rows - z[key]).max() < 1e-6
    if start == 0:
        assert np.array_equal(rows[0], np.full(cfg.vocab_size, 1.0 / cfg.vocab_size, np.float32))


def test_bf16_bank_fixture_differs_from_fp32_weights(golden_dir):
    """The two fixtures are different models: rounding the banks to bf16 moves
    the reference's rows well past the 1e-6 above."""
    a = np.load(os.path.join(golden_dir, "engine_rows.npz"))["rows_ctx"]
    b = np.load(os.path.join(golden_dir, "engine_rows_bf16w.npz"))["rows_ctx"]
    assert np.abs(a - b).max() > 1e-4


def test_rope_length_matters(eng):
    """A RoPE table warmed at another length (YaRN scale 4 instead of 2) moves
    the rows far past the tolerance above: the fixture pins the length rule."""
    z, cfg, sm = eng
    om = mr.OracleModel(cfg, sm.state_dict(), max_len=256)
    rows = mr.segment_rows_tf(om, z["arr"], z["arr"][100:164], 100, int(z["block"]), int(z["win"]))
    assert np.abs(rows - z["rows_ctx"]).max() > 1e-3


def test_softmax_np_renormalises():
    rng = np.random.default_rng(3)
    lg = torch.from_numpy(rng.standard_normal(4096).astype(np.float32) * 4)
    p = mr.softmax_np(lg)
    q = torch.softmax(lg, -1).numpy()
    s = float(q.sum())
    assert p.dtype == np.float32
    assert np.array_equal(p, (q / np.float32(s)).astype(np.float32)) or np.array_equal(p, q / s)
    assert np.array_equal(mr.softmax_np(torch.full((8,), float("nan"))), np.full(8, 0.125, np.float32))
