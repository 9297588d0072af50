"""The probability engine (altxs_amd.engine, after StaticACEngine).

* teacher-forced tables from windows (the last one narrower) equal the tables
  of width-1 decode rows, with a context prefilled by committed windows; the
  carry is the renormalised table after the context (reference rule);
* the stream-start carry is the count rule applied to the uniform row (the
  oracle's scale_cum on p = 1/V);
* a compress -> decompress round trip of two segments after a context: the
  device decoder recovers every symbol, writing each into the next step's
  token buffer, and the payloads equal the oracle coder's bytes on the
  engine's teacher-forced tables.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


_M = {}


def _model():
    if "m" not in _M:
        from altxs_amd import synth
        from altxs_amd.config import make_config
        from altxs_amd.model import StepModel

        cfg = make_config("cfg1")
        _M["m"] = StepModel(synth.make_model(cfg, std=0.02, softcap=(30.0, 24.0)), act="bf16")
    return _M["m"]


def _stream(n: int, seed: int):
    from altxs_amd import synth

    return synth.zipf_tokens(4096, (n,), seed=seed).astype(np.int64)


def test_window_rows_equal_decode_rows_after_context():
    from altxs_amd.engine import StaticACEngine, segment_rows_one_row, segment_rows_tf

    _log("engine rows: windows vs decode rows")
    model = _model()
    eng = StaticACEngine(model, batch=2, win=16, max_len=256, block=64)
    streams = [_stream(200, 1), _stream(200, 2)]
    starts = [100, 100]  # context = stream[36:100] (block 64)
    segs = [s[100:140] for s in streams]  # 40 symbols: windows of 16, 16 and 8
    tf = segment_rows_tf(eng, streams, segs, starts)
    one = segment_rows_one_row(eng, streams, segs, starts)
    assert np.array_equal(tf, one)
    assert (tf[:, :, -1] > 0).all() and (np.diff(tf, axis=-1) >= 1).all()
    # the carry is the table after the context's last token, as a decode row
    # with the renormalising count rule gives it (_softmax_np, incremental.py:878-886)
    eng.reset_segment([s[:0] for s in streams], [0, 0])
    for t in range(36, 100):
        tok = torch.from_numpy(np.stack([s[t] for s in streams]).astype(np.int32)).cuda()
        if t < 99:
            eng.run_decode_row_dev(tok)
        else:
            eng._run(tok.reshape(2, 1), commit=True, renorm=True)
    assert np.array_equal(eng.st.cum[:2].cpu().numpy(), tf[:, 0])


def test_stream_start_carry_is_uniform_rule():
    from altxs_amd.engine import StaticACEngine
    from oracle import coder

    _log("engine uniform carry")
    eng = StaticACEngine(_model(), batch=1, win=8, max_len=256, block=64)
    eng.reset_segment(_stream(10, 3), 0)
    V = 4096
    want = coder.scale_cum(np.full((1, V), 1.0 / V, np.float32))[0]
    assert np.array_equal(eng.carry_row_dev()[0].cpu().numpy().astype(np.int64), want)


def test_compress_decompress_round_trip():
    from altxs_amd.coder import frame, iter_framed_segments
    from altxs_amd.engine import (StaticACEngine, decode_segments_gpu, encode_segments_gpu,
                                  segment_rows_tf)
    from oracle import coder

    _log("engine compress / decompress")
    model = _model()
    eng = StaticACEngine(model, batch=2, win=16, max_len=256, block=64)
    streams = [_stream(300, 5), _stream(300, 6)]
    starts = [150, 150]
    segs = [s[150:187] for s in streams]  # 37 symbols
    payloads = encode_segments_gpu(eng, streams, segs, starts)
    tables = segment_rows_tf(eng, streams, segs, starts)
    for b in range(2):
        assert payloads[b] == coder.wnc_encode(segs[b], tables[b])
    blob = frame(payloads)
    back = decode_segments_gpu(eng, streams, list(iter_framed_segments(blob)), starts, n_seg=37)
    assert np.array_equal(back, np.stack(segs))
    eng.st.check_errors()
