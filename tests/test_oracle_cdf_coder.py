"""Pins the C oracle for the integer CDF rule and the WNC coder (CPU only)."""

from __future__ import annotations

import math
import os
from fractions import Fraction

import numpy as np
import pytest

from oracle import coder


def _two_round(p: float) -> int:
    """max(1, floor(rd(rd(p*1e6) + 0.5))) with exact rationals; rd = nearest double."""
    t1 = float(Fraction(p) * 1_000_000)  # float(Fraction) rounds to nearest double
    t2 = float(Fraction(t1) + Fraction(1, 2))
    return max(1, math.floor(t2))


def _exact(p: float) -> int:
    """max(1, floor(p*1e6 + 1/2)) over the rationals.

    For a float32 p the double product has <= 38 significant bits and the sum
    stays within 53, so both double roundings of the reference rule are exact
    and the rule equals this closed form (which also makes FMA contraction
    harmless).  What would break it is float32 arithmetic.
    """
    return max(1, math.floor(Fraction(p) * 1_000_000 + Fraction(1, 2)))


def _float32_rule(p: np.ndarray) -> np.ndarray:
    """A plausible wrong implementation: the same expression in float32."""
    t = (p.astype(np.float32) * np.float32(1e6)) + np.float32(0.5)
    return np.maximum(1, np.floor(t).astype(np.int64))


@pytest.mark.parametrize("V,f", [(256, 3906), (4096, 244), (16384, 61)])
def test_uniform_known_answers(V, f):
    cum = coder.scale_cum(np.full((1, V), 1.0 / V, np.float32))[0]
    assert np.all(np.diff(cum) == f)
    assert cum[0] == 0 and cum[-1] == f * V


def test_zero_and_one():
    cum = coder.scale_cum(np.array([[0.0, 1.0, 0.0, 1e-30]], np.float32))[0]
    assert list(np.diff(cum)) == [1, 1_000_000, 1, 1]


def test_rounding_boundaries_exact():
    """Every float32 within +-6 ULP of (k - 1/2) * 1e-6 for many k, against exact rationals."""
    ks = list(range(1, 2000)) + list(range(10_000, 1_000_001, 9973))
    vals = []
    for k in ks:
        x = np.float32((k - 0.5) * 1e-6)
        v = x
        for _ in range(6):
            v = np.nextafter(v, np.float32(0))
        for _ in range(13):
            vals.append(float(v))
            v = np.nextafter(v, np.float32(2))
    p = np.array(vals, np.float32)
    got = np.diff(coder.scale_cum(p[None, :])[0])
    want = np.array([_two_round(float(x)) for x in p])
    assert np.array_equal(got, want)
    assert np.array_equal(want, np.array([_exact(float(x)) for x in p]))
    # The inputs discriminate: a float32-arithmetic implementation differs somewhere.
    assert not np.array_equal(_float32_rule(p), want)


def test_f64_rule_rounding_boundaries():
    """float64 rows: doubles within +-8 ULP of (k - 1/2) * 1e-6 and of the
    doubles whose product lands on a half, against exact rationals of the two
    double roundings (which are not exact here, unlike float32 input)."""
    ks = list(range(1, 3000)) + list(range(10_000, 1_000_001, 7919))
    vals = []
    for k in ks:
        for base in ((k - 0.5) * 1e-6, (k - 0.5) / 1e6):
            v = np.float64(base)
            for _ in range(8):
                v = np.nextafter(v, 0.0)
            for _ in range(17):
                vals.append(float(v))
                v = np.nextafter(v, 1.0)
    p = np.array(vals, np.float64)
    got = np.diff(coder.scale_cum_f64(p[None])[0])
    want = np.array([_two_round(x) for x in vals], np.int64)
    assert np.array_equal(got, want)
    # numpy's own evaluation of the reference expression
    assert np.array_equal(got, np.maximum(1, np.floor(p * 1_000_000.0 + 0.5).astype(np.int64)))
    # where the double roundings matter, the closed form differs (the check can fail)
    assert any(_two_round(x) != _exact(x) for x in vals)


def test_f64_rule_equals_f32_rule_on_float32_values():
    rng = np.random.default_rng(5)
    p = (rng.random((3, 4096)) ** 3).astype(np.float32)
    assert np.array_equal(coder.scale_cum_f64(p.astype(np.float64)), coder.scale_cum(p))


def test_matches_reference_tables(golden_dir):
    g = np.load(os.path.join(golden_dir, "coder_ref.npz"))
    assert np.array_equal(coder.scale_cum(g["a_rows"]), g["a_cum"])


def test_bitstream_matches_reference_v256(golden_dir):
    g = np.load(os.path.join(golden_dir, "coder_ref.npz"))
    cum = coder.scale_cum(g["a_rows"])
    bits = coder.wnc_encode(g["a_syms"], cum)
    assert bits == g["a_bits"].tobytes()
    assert np.array_equal(coder.wnc_decode(bits, cum), g["a_syms"])


def test_bitstream_matches_reference_v4096(golden_dir):
    from tests.golden.make_golden import coder_stream_b

    g = np.load(os.path.join(golden_dir, "coder_ref.npz"))
    p, syms = coder_stream_b()
    assert float(p.astype(np.float64).sum()) == float(g["b_rows_sum"])
    assert np.array_equal(syms, g["b_syms"])
    cum = coder.scale_cum(p)
    bits = coder.wnc_encode(syms, cum)
    assert bits == g["b_bits"].tobytes()
    assert np.array_equal(coder.wnc_decode(bits, cum), syms)


@pytest.mark.parametrize("V", [2, 256, 16384])
def test_roundtrip_random(V):
    rng = np.random.default_rng(V)
    n = 500
    logits = rng.standard_normal((n, V)).astype(np.float32) * 4
    p = np.exp(logits - logits.max(1, keepdims=True))
    p = (p / p.sum(1, keepdims=True)).astype(np.float32)
    syms = rng.integers(0, V, n)
    cum = coder.scale_cum(p)
    bits = coder.wnc_encode(syms, cum)
    assert np.array_equal(coder.wnc_decode(bits, cum), syms)
    # coded length tracks the ideal code length of the integer model
    ideal = -np.log2((cum[np.arange(n), syms + 1] - cum[np.arange(n), syms]) / cum[:, -1]).sum()
    assert abs(8 * len(bits) - ideal) <= 40


def test_empty_stream():
    cum = np.zeros((0, 5), np.int64)
    bits = coder.wnc_encode(np.zeros(0, np.int64), cum)
    assert len(bits) == 1  # the flush alone: 2 bits padded to a byte
