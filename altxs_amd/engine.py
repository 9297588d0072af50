"""Probability engine over the step: segment resets, windows, decode rows.

Mirrors the reference's ``StaticACEngine`` (src/xsa_ttt/incremental.py:203-1218)
and its segment drivers (``_segment_rows_tf`` 1238-1271, ``_segment_rows_one_row``
1221-1235, ``_encode_segment_gpu`` 1280-1305, ``_decode_segment_gpu`` 1308-1337)
for B segments in lockstep (B = 1 is the reference's per-segment use).  One
state (window width ``win``) serves every call: encode windows run at width
``win`` (the last one of a segment narrower), decode rows at width 1, and the
context prefill of ``reset_segment`` is a run of committed windows; all of them
give the rows of decode bit for bit (the step is batch- and window-invariant).

Row semantics (incremental.py:1238-1271): ``rows[0]`` is the carry -- the
distribution after the segment's context (uniform at the stream start) -- and
``rows[i + 1] = P(. | context, seg[:i + 1])``.  Here every row is the step's
integer CDF (and, on request, its fp32 probabilities).  The carry follows the
reference's rule for it (``reset_segment`` applies ``_softmax_np``: fp32
softmax, then ``p /= sum(p)``, compress.py:64-85, incremental.py:878-886): the
context's last window runs with the step's renormalisation flag, so the
carry's counts come from renormalised probabilities while every later row
uses the plain softmax, as the reference's device rows do.  Encoder and
decoder both form it this way.

Lengths: the engine's static length is ``block + ceil(every / W) * W``
(incremental.py:239-242) and the RoPE table is warmed at that length
(warm_rotary, 106-113), which sets the YaRN scale; the KV cache is that
length rounded up to the step's 256-key granule unless ``max_len`` is given.
"""

from __future__ import annotations

import numpy as np
import torch

from .coder import RangeCoder
from .model import CHUNK, StaticState, StepModel


def chunk_ctx_start(start: int, block: int) -> tuple[int, int]:
    """``(p0, ctx_start)`` of a chunk starting at ``start`` (compress.py:122-125)."""
    p0 = 1 if start == 0 else int(start)
    return p0, max(0, p0 - int(block))


def engine_length(block: int, every: int, win: int) -> int:
    """Static length of the engine (incremental.py:239-242): the context block
    plus whole windows covering one retrain segment of ``every`` symbols."""
    return int(block) + (max(1, int(every)) + int(win) - 1) // int(win) * int(win)


def uniform_cum(V: int, device) -> torch.Tensor:
    """The CDF of the uniform row, by the step's count rule max(1, floor(p*1e6 + 0.5))."""
    f = max(1, int(np.floor(np.float64(np.float32(1.0 / V)) * 1e6 + 0.5)))
    return (torch.arange(V + 1, dtype=torch.int64) * f).to(torch.int32).to(device)


class StaticACEngine:
    """B segments stepped in lockstep; every segment of a batch has the same
    context length and position (the reference runs one segment at a time)."""

    def __init__(self, model: StepModel, *, batch: int = 1, win: int = 64, max_len: int | None = None,
                 block: int | None = None, every: int | None = None, want_probs: bool = False):
        self.model = model
        self.batch, self.win = int(batch), int(win)
        self.block = int(block if block is not None else model.cfg.block_size)
        self.every = int(every if every is not None else model.cfg.online_retrain_every)
        self.V = model.cfg.vocab_size
        self.rope_len = engine_length(self.block, self.every, self.win)
        if max_len is None:
            max_len = (self.rope_len + CHUNK - 1) // CHUNK * CHUNK
        self.st: StaticState = model.make_static_state(int(max_len), win=self.win, batch=self.batch,
                                                       want_probs=want_probs,
                                                       rope_len=self.rope_len)
        self.uniform = uniform_cum(self.V, model.device)
        self.carry = torch.empty(self.batch, self.V + 1, dtype=torch.int32, device=model.device)
        self.ctx_len = 0
        self.pos = 0  # committed position of the batch (host copy, no device sync)
        self.n_steps = 0

    # ---- segment start ---------------------------------------------------------
    def reset_segment(self, prefixes, starts) -> None:
        """Rewind to segment starts and prefill their context windows
        (incremental.py:858-897).  ``prefixes``: one token array per segment
        (the stream so far), ``starts``: each segment's start offset."""
        if self.batch == 1 and not isinstance(starts, (list, tuple)):
            prefixes, starts = [prefixes], [starts]
        ctxs = []
        for pre, start in zip(prefixes, starts):
            _, c0 = chunk_ctx_start(int(start), self.block)
            ctxs.append(np.asarray(pre[c0:int(start)], dtype=np.int64))
        n = {c.size for c in ctxs}
        if len(ctxs) != self.batch or len(n) != 1:
            raise ValueError("one prefix per segment, all with the same context length")
        L = n.pop()
        if L >= self.st.max_len:
            raise ValueError(f"context of {L} tokens does not fit max_len {self.st.max_len}")
        st = self.st
        st.pos.zero_()
        st.prev_raw.zero_()
        st.cand_prev_raw.zero_()
        self.ctx_len = L
        self.pos = 0
        if L == 0:  # stream start: uniform first row, smear sees zeros
            self.carry.copy_(self.uniform.expand(self.batch, -1))
            if st.probs is not None:
                self.carry_probs = torch.full((self.batch, self.V), 1.0 / self.V,
                                              dtype=torch.float32, device=self.model.device)
            return
        ctx = np.stack(ctxs)
        w0 = 0
        while w0 < L:  # committed windows; the last one is narrower and renormalises
            w = min(self.win, L - w0)
            self._run(ctx[:, w0:w0 + w], commit=True, renorm=w0 + w >= L)
            w0 += w
        self.carry.copy_(st.cum[:self.batch * w].view(self.batch, w, -1)[:, w - 1])
        if st.probs is not None:
            self.carry_probs = st.probs[:self.batch * w].view(self.batch, w, -1)[:, w - 1].clone()

    def carry_row_dev(self) -> torch.Tensor:
        """[B, V+1] table of each segment's first symbol (rows[0])."""
        return self.carry

    # ---- steps ----------------------------------------------------------------
    def _run(self, tokens, *, commit: bool, renorm: bool = False) -> int:
        toks = torch.as_tensor(np.asarray(tokens) if not torch.is_tensor(tokens) else tokens)
        w = int(toks.shape[-1])
        if self.pos + w > self.st.max_len:
            raise ValueError("window past max_len")
        self.st.tokens(w).copy_(toks.reshape(self.batch, w).to(torch.int32))
        self.model.step(self.st, commit=commit, renorm=renorm, width=w)
        if commit:
            self.pos += w
        self.n_steps += 1
        return w

    def run_window(self, tokens, start_local: int, *, commit: bool = False) -> torch.Tensor:
        """One W-token step at segment offset ``start_local`` (incremental.py:991-1015);
        returns the [B, W, V+1] tables (device): row j = P(symbol start_local+j+1 | ...)."""
        if self.pos != self.ctx_len + int(start_local):
            raise ValueError("windows must follow the committed position")
        w = self._run(tokens, commit=commit)
        return self.st.cum[:self.batch * w].view(self.batch, w, -1)

    def advance_window(self, width: int) -> None:
        """Commit a window that ran without commit (incremental.py:1049-1052)."""
        self.st.pos += int(width)
        self.st.prev_raw.copy_(self.st.cand_prev_raw)
        self.pos += int(width)

    def run_decode_row_dev(self, tokens: torch.Tensor) -> torch.Tensor:
        """One confirmed token per segment on the width-1 step, committed
        (incremental.py:1083-1101); returns the [B, V+1] tables of the next symbols."""
        self._run(tokens.reshape(self.batch, 1), commit=True)
        return self.st.cum[:self.batch]


def segment_rows_tf(engine: StaticACEngine, prefixes, segs, starts) -> np.ndarray:
    """Teacher-forced tables for B equal-length segments (``_segment_rows_tf``):
    [B, n, V+1] int64, rows[:, 0] = carry."""
    engine.reset_segment(prefixes, starts)
    seg = np.stack([np.asarray(s, dtype=np.int64) for s in segs])
    B, n = seg.shape
    out = np.empty((B, n, engine.V + 1), dtype=np.int64)
    carry = engine.carry_row_dev().cpu().numpy()
    w0 = 0
    while w0 < n:
        w = min(engine.win, n - w0)
        rows = engine.run_window(seg[:, w0:w0 + w], w0, commit=True).cpu().numpy()
        out[:, w0] = carry
        if w > 1:
            out[:, w0 + 1:w0 + w] = rows[:, :w - 1]
        carry = rows[:, w - 1]
        w0 += w
    return out


def segment_rows_one_row(engine: StaticACEngine, prefixes, segs, starts) -> np.ndarray:
    """The same tables from width-1 decode rows (``_segment_rows_one_row``)."""
    engine.reset_segment(prefixes, starts)
    seg = np.stack([np.asarray(s, dtype=np.int64) for s in segs])
    B, n = seg.shape
    out = np.empty((B, n, engine.V + 1), dtype=np.int64)
    out[:, 0] = engine.carry_row_dev().cpu().numpy()
    dev = torch.from_numpy(seg.astype(np.int32)).to(engine.model.device)
    for i in range(n - 1):
        out[:, i + 1] = engine.run_decode_row_dev(dev[:, i]).cpu().numpy()
    return out


def encode_segments_gpu(engine: StaticACEngine, prefixes, segs, starts, max_bytes: int | None = None
                        ) -> list[bytes]:
    """``_encode_segment_gpu`` for B segments: rows on the device, the range
    coder on the device, one copy of the bytes at the end.  Windows of the
    engine's width carry the teacher-forced tokens."""
    engine.reset_segment(prefixes, starts)
    dev = engine.model.device
    seg = np.stack([np.asarray(s, dtype=np.int64) for s in segs])
    B, n = seg.shape
    if n == 0:
        return [b""] * B
    seg_d = torch.from_numpy(seg.astype(np.int32)).to(dev)
    rc = RangeCoder(B, max_bytes or (64 + 4 * n))
    rc.encode(engine.carry_row_dev(), seg_d[:, :1].contiguous())
    w0 = 0
    while w0 < n - 1:  # window of tokens seg[w0 : w0+w] predicts seg[w0+1 : w0+w+1]
        w = min(engine.win, n - 1 - w0)
        rows = engine.run_window(seg_d[:, w0:w0 + w], w0, commit=True)
        rc.encode(rows.reshape(B * w, -1), seg_d[:, w0 + 1:w0 + w + 1].contiguous())
        w0 += w
    return rc.finish()


def decode_segments_gpu(engine: StaticACEngine, prefixes, payloads: list[bytes], starts, n_seg: int,
                        max_bytes: int | None = None) -> np.ndarray:
    """``_decode_segment_gpu`` for B segments: each decoded symbol goes into
    the token buffer of the next width-1 step on the device; [B, n] int64."""
    engine.reset_segment(prefixes, starts)
    B, n = engine.batch, int(n_seg)
    dev = engine.model.device
    out = torch.empty(B, n, dtype=torch.int32, device=dev)
    if n == 0:
        return out.cpu().numpy().astype(np.int64)
    rc = RangeCoder(B, max_bytes or max(64, max(len(p) for p in payloads) + 8))
    rc.begin_decode(payloads)
    rc.decode(engine.carry_row_dev(), out[:, 0:1], out_stride=n)
    for i in range(n - 1):
        rows = engine.run_decode_row_dev(out[:, i])
        rc.decode(rows, out[:, i + 1:i + 2], out_stride=n)
    rc.check()
    return out.cpu().numpy().astype(np.int64)


def segment_prob_rows_tf(engine: StaticACEngine, prefixes, segs, starts):
    """The teacher-forced rows of :func:`segment_rows_tf` as probabilities
    too (the engine must keep them: ``want_probs=True``): returns
    ``(probs [B, n, V] fp32, cum [B, n, V+1] int64)``; ``probs[:, 0]`` is the
    renormalised carry (incremental.py:878-886)."""
    if engine.st.probs is None:
        raise ValueError("segment_prob_rows_tf needs an engine built with want_probs=True")
    engine.reset_segment(prefixes, starts)
    seg = np.stack([np.asarray(s, dtype=np.int64) for s in segs])
    B, n = seg.shape
    probs = np.empty((B, n, engine.V), dtype=np.float32)
    cum = np.empty((B, n, engine.V + 1), dtype=np.int64)
    cprob = engine.carry_probs.cpu().numpy()
    ccum = engine.carry_row_dev().cpu().numpy()
    w0 = 0
    while w0 < n:
        w = min(engine.win, n - w0)
        rows = engine.run_window(seg[:, w0:w0 + w], w0, commit=True).cpu().numpy()
        pr = engine.st.probs[:B * w].view(B, w, -1).cpu().numpy()
        probs[:, w0], cum[:, w0] = cprob, ccum
        if w > 1:
            probs[:, w0 + 1:w0 + w], cum[:, w0 + 1:w0 + w] = pr[:, :w - 1], rows[:, :w - 1]
        cprob, ccum = pr[:, w - 1], rows[:, w - 1]
        w0 += w
    return probs, cum
