"""GPU range coder (altxs_range_*) against the CPU oracle coder.

The oracle (oracle/cdf_coder.c) is the reference's 32-bit WNC coder, pinned by
byte equality with bitstreams the reference coder wrote (tests/golden).  Here:
the device encoder's bytes equal the oracle's for the same symbols and
tables, whether symbols arrive one per call (decode rows) or in windows; the
device decoder recovers the symbols from the oracle's bytes; skewed tables
(long E3 runs), V = 2 and V = 65536; and a compress -> decompress round trip
through the model step, the decoder writing each symbol into the next step's
token buffer.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def _tables(rng, n_rows: int, V: int, skew: bool = False) -> np.ndarray:
    from oracle import coder

    if skew:
        p = np.full((n_rows, V), 1e-9, np.float32)
        p[np.arange(n_rows), rng.integers(0, V, n_rows)] = 1.0
    else:
        p = rng.random((n_rows, V)).astype(np.float32) ** 3
    p /= p.sum(-1, keepdims=True)
    return coder.scale_cum(p.astype(np.float32))  # [n_rows, V+1] int64


def _dev_u32(cum: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(cum.astype(np.uint32).view(np.int32)).cuda()


@pytest.mark.parametrize("V,n,T,W,skew", [(256, 5, 300, 1, False), (256, 5, 300, 37, False),
                                          (4096, 3, 200, 200, False), (2, 4, 500, 5, False),
                                          (1000, 4, 400, 1, True), (65536, 2, 40, 4, False)])
def test_encode_matches_oracle_and_decodes(V, n, T, W, skew):
    from altxs_amd.coder import RangeCoder
    from oracle import coder

    _log(f"coder V={V} n={n} T={T} W={W} skew={skew}")
    rng = np.random.default_rng(V + n + T + W)
    cum = _tables(rng, n * T, V, skew).reshape(n, T, V + 1)
    if skew:  # mostly the likely symbol, sometimes a 1e-9 one
        likely = np.argmax(np.diff(cum, axis=-1), axis=-1)
        syms = np.where(rng.random((n, T)) < 0.97, likely, rng.integers(0, V, (n, T)))
    else:
        syms = rng.integers(0, V, (n, T))
    want = [coder.wnc_encode(syms[b], cum[b]) for b in range(n)]
    rc = RangeCoder(n, max(len(w) for w in want) + 64)
    for t0 in range(0, T, W):
        w = min(W, T - t0)
        s = torch.from_numpy(syms[:, t0:t0 + w].astype(np.int32)).cuda().contiguous()
        c = _dev_u32(np.ascontiguousarray(cum[:, t0:t0 + w].reshape(n * w, V + 1)))
        rc.encode(c, s)
    got = rc.finish()
    for b in range(n):
        assert got[b] == want[b], (b, len(got[b]), len(want[b]))
    # decode the oracle's bytes on the device, one symbol per stream and call
    rc.begin_decode(want)
    out = torch.zeros(n, dtype=torch.int32, device="cuda")
    dec = []
    for t in range(T):
        rc.decode(_dev_u32(np.ascontiguousarray(cum[:, t])), out)
        dec.append(out.cpu().numpy().copy())
    rc.check()
    assert np.array_equal(np.stack(dec, 1), syms)


def test_empty_streams_and_capacity_error():
    from altxs_amd.coder import RangeCoder
    from oracle import coder

    _log("coder empty / capacity")
    rc = RangeCoder(3, 16)
    got = rc.finish()
    V = 8
    empty = coder.wnc_encode(np.zeros(0, np.int64), np.zeros((0, V + 1), np.int64))
    assert got == [empty] * 3
    rng = np.random.default_rng(1)
    cum = _tables(rng, 3 * 400, 4096).reshape(3, 400, 4097)
    rc.reset()
    syms = rng.integers(0, 4096, (3, 400))
    rc.encode(_dev_u32(np.ascontiguousarray(cum.reshape(1200, 4097))),
              torch.from_numpy(syms.astype(np.int32)).cuda().contiguous())
    with pytest.raises(RuntimeError, match="buffer full"):
        rc.finish()


def test_step_compress_decompress_roundtrip():
    """Encoder: step, then code the next token with the step's CDFs.  Decoder:
    step, then decode straight into the state's token buffer for the next step.
    The payloads equal the oracle coder's on the same tables."""
    from altxs_amd import synth
    from altxs_amd.coder import RangeCoder, frame, iter_framed_segments
    from altxs_amd.config import make_config
    from altxs_amd.model import StepModel
    from oracle import coder

    _log("coder round trip through the step")
    cfg = make_config("cfg1")
    sm = synth.make_model(cfg)
    B, T = 3, 24
    toks = synth.zipf_tokens(cfg.vocab_size, (B, T), seed=9).astype(np.int32)
    V = cfg.vocab_size

    model = StepModel(sm, act="bf16")
    st = model.make_static_state(256, win=1, batch=B, want_probs=False)
    enc = RangeCoder(B, 4096)
    tables = []
    for t in range(T - 1):
        st.token.copy_(torch.from_numpy(toks[:, t:t + 1]))
        model.step(st, commit=True)
        nxt = torch.from_numpy(toks[:, t + 1:t + 2].copy()).cuda()
        enc.encode(st.cum, nxt)
        tables.append(st.cum.cpu().numpy().astype(np.int64))
    payloads = enc.finish()
    tab = np.stack(tables, 1)  # [B, T-1, V+1]
    for b in range(B):
        assert payloads[b] == coder.wnc_encode(toks[b, 1:].astype(np.int64), tab[b])
    blob = frame(payloads)
    assert list(iter_framed_segments(blob)) == payloads

    model2 = StepModel(sm, act="bf16")
    st2 = model2.make_static_state(256, win=1, batch=B, want_probs=False)
    dec = RangeCoder(B, 4096)
    dec.begin_decode(list(iter_framed_segments(blob)))
    st2.token.copy_(torch.from_numpy(toks[:, :1]))
    got = [toks[:, 0]]
    for t in range(T - 1):
        model2.step(st2, commit=True)
        dec.decode(st2.cum, st2.token)  # the next step's input, on the device
        got.append(st2.token.cpu().numpy()[:, 0].copy())
    dec.check()
    st2.check_errors()
    assert np.array_equal(np.stack(got, 1), toks)
