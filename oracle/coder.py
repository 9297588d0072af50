"""ctypes bindings for oracle/cdf_coder.c -- TEST INFRASTRUCTURE ONLY.

* :func:`scale_cum` restates ``_scale_cum_np`` (src/model/arithmetic_coder_lm.py:49-64).
  Pinned by closed-form known answers (uniform rows: V=256 -> f=3906,
  total 999,936; V=4096 -> 244, 999,424; V=16384 -> 61, 999,424; p=0 -> 1),
  by exact-rational brute force around every rounding boundary (tests), and by
  numpy's own evaluation of the same expression.  :func:`scale_cum_f64`
  is the rule on float64 rows, pinned by exact-rational emulation of its two
  double roundings around every boundary and by numpy's float64 evaluation.
* :func:`wnc_encode` / :func:`wnc_decode` restate ``encode_with_probs`` /
  ``decode_with_probs`` (arithmetic_coder_lm.py:140-288).  Pinned by
  round-trip identity and by byte equality with bitstreams written by the
  reference coder itself (tests/golden/coder_*.npz, made by
  tests/golden/make_golden.py).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle_cdf.so")
_lib = None


def build() -> str:
    """Compile the C restatement (always, even when a built library exists)."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i64, p = ctypes.c_int64, ctypes.c_void_p
        L.oracle_scale_cum.restype = i64
        L.oracle_scale_cum.argtypes = [p, i64, p]
        L.oracle_scale_cum_rows.restype = None
        L.oracle_scale_cum_rows.argtypes = [p, i64, i64, p]
        L.oracle_scale_cum_rows_f64.restype = None
        L.oracle_scale_cum_rows_f64.argtypes = [p, i64, i64, p]
        L.oracle_wnc_encode.restype = i64
        L.oracle_wnc_encode.argtypes = [p, i64, p, i64, p, i64]
        L.oracle_wnc_decode.restype = ctypes.c_int
        L.oracle_wnc_decode.argtypes = [p, i64, i64, p, i64, p]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def scale_cum(probs: np.ndarray) -> np.ndarray:
    """probs float32 [..., V] -> cum int64 [..., V+1]."""
    p = np.ascontiguousarray(probs, dtype=np.float32)
    V = p.shape[-1]
    rows = p.reshape(-1, V)
    out = np.empty((rows.shape[0], V + 1), dtype=np.int64)
    lib().oracle_scale_cum_rows(_ptr(rows), rows.shape[0], V, _ptr(out))
    return out.reshape(p.shape[:-1] + (V + 1,))


def scale_cum_f64(probs: np.ndarray) -> np.ndarray:
    """probs float64 [..., V] -> cum int64 [..., V+1] (the rule on float64 rows)."""
    p = np.ascontiguousarray(probs, dtype=np.float64)
    V = p.shape[-1]
    rows = p.reshape(-1, V)
    out = np.empty((rows.shape[0], V + 1), dtype=np.int64)
    lib().oracle_scale_cum_rows_f64(_ptr(rows), rows.shape[0], V, _ptr(out))
    return out.reshape(p.shape[:-1] + (V + 1,))


def wnc_encode(symbols: np.ndarray, cum_rows: np.ndarray) -> bytes:
    syms = np.ascontiguousarray(symbols, dtype=np.int64).reshape(-1)
    cum = np.ascontiguousarray(cum_rows, dtype=np.int64)
    n, V = syms.size, cum.shape[-1] - 1
    if cum.reshape(-1, V + 1).shape[0] != n:
        raise ValueError("need one CDF row per symbol")
    cap = 64 + n * 8
    out = np.zeros(cap, dtype=np.uint8)
    nb = lib().oracle_wnc_encode(_ptr(syms), n, _ptr(cum), V, _ptr(out), cap)
    if nb < 0:
        raise ValueError("oracle_wnc_encode failed (bad symbol or overflow)")
    return out[:nb].tobytes()


def wnc_decode(data: bytes, cum_rows: np.ndarray) -> np.ndarray:
    cum = np.ascontiguousarray(cum_rows, dtype=np.int64)
    V = cum.shape[-1] - 1
    n = cum.reshape(-1, V + 1).shape[0]
    buf = np.frombuffer(data, dtype=np.uint8).copy() if len(data) else np.zeros(1, np.uint8)
    out = np.empty(n, dtype=np.int64)
    lib().oracle_wnc_decode(_ptr(buf), len(data), n, _ptr(cum), V, _ptr(out))
    return out


def bits_per_symbol(symbols: np.ndarray, cum_rows: np.ndarray) -> float:
    return 8.0 * len(wnc_encode(symbols, cum_rows)) / max(1, np.asarray(symbols).size)
