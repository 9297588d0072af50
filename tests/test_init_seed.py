"""Init(seed) and the shipped student on the CPU (no GPU).

* ``altxs_amd.init_seed.reference_init_state`` for the shipped codec's seed and
  config equals the reference's own Init(seed) (``enable_deterministic`` +
  ``build_model``, recorded in tests/golden/shipped_full.npz): per-matrix sums
  and sums of squares, first rows and sampled values of every modeled bank,
  bit for bit; another seed does not.
* The oracle on the whole shipped student -- Init(seed) plus the delta the
  oracle's codec decodes from tests/golden/shipped/ (the reference's asset,
  weights/mixed_da_bpw3.15_upb1.8.*) -- gives the fp32 logits the reference's
  ``load_codec`` model wrote (W=1 ``static_extend`` rows from the stream start).
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import pytest
import torch

from altxs_amd.init_seed import reference_init_state
from altxs_amd.shipped import MODELED, config_from_meta

STEM = os.path.join("shipped", "mixed_da_bpw3.15_upb1.8")


@pytest.fixture(scope="module")
def full(golden_dir):
    z = np.load(os.path.join(golden_dir, "shipped_full.npz"))
    meta = json.load(open(os.path.join(golden_dir, STEM + ".json"), encoding="utf8"))
    return z, meta, config_from_meta(meta)


def _sample_index(shape):
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    from make_golden import init_sample_index

    return init_sample_index(shape)


def _fingerprint_errors(sd, z):
    errs = {}
    for name in MODELED:
        t = sd[name].float()
        t = t.reshape(-1, t.shape[-2], t.shape[-1]).numpy().astype(np.float64)
        idx = _sample_index(t.shape)
        errs[name] = max(float(np.abs(t.sum(axis=(1, 2)) - z[f"{name}/sum"]).max()),
                         float(np.abs((t * t).sum(axis=(1, 2)) - z[f"{name}/sumsq"]).max()),
                         float(np.abs(t[:, 0, :] - z[f"{name}/row0"]).max()),
                         float(np.abs(t.reshape(t.shape[0], -1)[:, idx] - z[f"{name}/sample"]).max()))
    return errs


def test_init_seed_equals_reference_init(full):
    z, meta, cfg = full
    assert int(z["seed"]) == int(meta["seed"])
    errs = _fingerprint_errors(reference_init_state(cfg, int(meta["seed"])), z)
    assert all(e == 0.0 for e in errs.values()), errs


def test_init_seed_depends_on_seed_and_order(full):
    """The fingerprint catches a plausible slip: another seed misses it, and so
    does the tied embedding drawn without nn.Embedding's own N(0, 1) draw
    first (the draw the restatement's step 1 makes)."""
    z, meta, cfg = full
    errs = _fingerprint_errors(reference_init_state(cfg, int(meta["seed"]) + 1), z)
    assert all(e > 1e-3 for k, e in errs.items() if k != "mlp_down_bank"), errs
    g = torch.Generator().manual_seed(int(meta["seed"]))
    emb = torch.empty(cfg.vocab_size, cfg.model_dim)
    torch.nn.init.normal_(emb, mean=0.0, std=cfg.tied_embed_init_std, generator=g)
    assert np.abs(emb[0].numpy() - z["tok_emb.weight/row0"][0]).max() > 1e-4


def test_oracle_student_matches_reference_logits(full, golden_dir):
    from oracle.model_ref import OracleModel

    from .refshape import student_state_dict

    z, _, _ = full
    cfg, meta, sd = student_state_dict(golden_dir)
    om = OracleModel(cfg, sd, max_len=int(z["max_len"]))
    rows = om.decode_rows(z["tokens"]).numpy()
    err = float(np.abs(rows - z["rows_w1"]).max())
    print(f"oracle vs reference student rows: max |dlogit| = {err:.3e}")
    assert err < 1e-4, err
