"""The reference-named surface (altxs_amd.dropin) driven with reference-shaped
arguments, checked against the oracle and the reference's own vectors.

* ``_scale_cum_np`` / ``_scale_cum``: the reference's (cum, total) for V = 256,
  4096 and 16384, equal to the pinned CDF oracle and to the tables the
  reference coder wrote (tests/golden/coder_ref.npz);
* ``GpuRangeCoder``: encode_symbol / finish give the bytes the reference coder
  wrote for the rows and symbols of its own test; begin_decode /
  decode_symbol return the symbols as int64[1];
* ``encode_with_probs`` / ``decode_with_probs``: same bytes as the oracle
  coder, round trip for a byte alphabet (bytes out) and a wide one (ids);
* ``try_persistent_extend`` / ``try_mega_encode`` on a reference-shaped GPT
  (``cfg`` with the reference's field names, ``state_dict()`` with its
  parameter names) and StaticState (token [1, W] int64, pos int64[1],
  prev_raw / cand_prev_raw [1, 1, D], logits [1, W, V]): logits within 2e-4
  of the fp32 oracle over 20 positions, windows equal to rows bit for bit,
  False plus a sticky disable on a broken state;
* ``gemv_rows`` / ``logits_stage_rows`` against fp64 products.
"""

from __future__ import annotations

import os
import types

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def _rows(rng, n, V):
    p = rng.random((n, V)).astype(np.float32) ** 4
    return (p / p.sum(1, keepdims=True)).astype(np.float32)


def test_scale_cum_np_matches_oracle_and_reference(golden_dir):
    from altxs_amd import dropin
    from oracle import coder

    _log("dropin _scale_cum_np")
    rng = np.random.default_rng(3)
    for V in (256, 4096, 16384):
        p = _rows(rng, 3, V)
        p[0, :5] = 0.0
        for r in p:
            cum, total = dropin._scale_cum_np(r, alphabet_size=V)
            want = coder.scale_cum(r[None])[0]
            assert cum.dtype == np.int64 and np.array_equal(cum, want) and total == int(want[-1])
        lst, tot = dropin._scale_cum(list(map(float, p[1])), alphabet_size=V)
        assert lst == coder.scale_cum(p[1:2])[0].tolist() and tot == lst[-1]
    z = np.load(os.path.join(golden_dir, "coder_ref.npz"))
    for r, want in zip(z["a_rows"], z["a_cum"]):
        assert np.array_equal(dropin._scale_cum_np(r, alphabet_size=256)[0], want)
    with pytest.raises(ValueError):
        dropin._scale_cum_np(np.ones(10, np.float32) / 10, alphabet_size=256)


def test_gpu_range_coder_reference_interface(golden_dir):
    from altxs_amd import dropin

    _log("dropin GpuRangeCoder")
    z = np.load(os.path.join(golden_dir, "coder_ref.npz"))
    rows, syms = z["a_rows"], z["a_syms"]
    want = z["a_bits"].tobytes()  # the bytes the reference coder wrote for its own test
    dev = torch.device("cuda")
    enc = dropin.GpuRangeCoder(dev, max_bits=4096, vocab=256)
    prow = torch.from_numpy(rows).cuda()
    for i, s in enumerate(syms):
        enc.encode_symbol(prow[i], torch.tensor([int(s)], dtype=torch.int64, device=dev))
    got = enc.finish()
    assert got == want
    dec = dropin.GpuRangeCoder(dev, max_bits=4096, vocab=256)
    dec.begin_decode(got)
    out = []
    for i in range(len(syms)):
        t = dec.decode_symbol(prow[i])
        assert t.dtype == torch.int64 and tuple(t.shape) == (1,)
        out.append(int(t.item()))
    assert out == syms.tolist()
    dec.check()


def test_encode_decode_with_probs():
    from altxs_amd import dropin
    from oracle import coder

    _log("dropin encode_with_probs / decode_with_probs")
    rng = np.random.default_rng(8)
    for V, n in ((256, 300), (4096, 120)):
        table = _rows(rng, n, V)
        p64 = table.astype(np.float64)
        p64 /= p64.sum(1, keepdims=True)
        syms = np.array([rng.choice(V, p=p64[i]) for i in range(n)])
        seen = []

        def probs_fn(i, prefix):
            seen.append((i, len(prefix)))
            return table[i]

        data = bytes(syms.astype(np.uint8)) if V == 256 else syms
        blob = dropin.encode_with_probs(data, probs_fn, alphabet_size=V)
        assert seen == [(i, i) for i in range(n)]
        assert blob == coder.wnc_encode(syms, coder.scale_cum(table))
        back = dropin.decode_with_probs(blob, n, lambda i, buf: table[i], alphabet_size=V)
        if V == 256:
            assert isinstance(back, bytes) and back == data
        else:
            assert back == syms.tolist()


def _reference_shaped(profile: str, bf16: bool):
    """A stand-in for the reference GPT: cfg with its field names and a
    state_dict() with its parameter names (weights rounded to bf16 so the
    dense bf16 banks hold them exactly)."""
    from altxs_amd import synth
    from altxs_amd.config import make_config

    cfg = make_config(profile)
    sm = synth.make_model(cfg, std=0.08, softcap=(2.0, 1.5), dense=True)
    sd = {k: torch.from_numpy(np.asarray(v, np.float32)).to(torch.bfloat16).float()
          for k, v in sm.state_dict().items()}
    ref_cfg = types.SimpleNamespace(**{f: getattr(cfg, f) for f in cfg.__dataclass_fields__})
    sd_dev = {k: v.cuda() for k, v in sd.items()}
    model = types.SimpleNamespace(cfg=ref_cfg, state_dict=lambda: sd_dev,
                                  _ac_compute_dtype=torch.bfloat16 if bf16 else None)
    return cfg, model, {k: v.numpy() for k, v in sd.items()}


def _reference_state(cfg, win: int, max_len: int):
    dev = "cuda"
    return types.SimpleNamespace(
        token=torch.zeros(1, win, dtype=torch.long, device=dev),
        prev_raw=torch.zeros(1, 1, cfg.model_dim, device=dev),
        cand_prev_raw=torch.zeros(1, 1, cfg.model_dim, device=dev),
        pos=torch.zeros(1, dtype=torch.long, device=dev),
        logits=torch.zeros(1, win, cfg.vocab_size, device=dev),
        slots=[], max_len=max_len, win=win)


def test_try_persistent_extend_on_reference_shaped_objects():
    from altxs_amd import dropin, synth
    from oracle.model_ref import OracleModel

    _log("dropin try_persistent_extend / try_mega_encode (tiny, fp32)")
    cfg, model, sd = _reference_shaped("tiny", bf16=False)
    T = 20
    toks = synth.zipf_tokens(cfg.vocab_size, (T,), seed=21)
    st = _reference_state(cfg, 1, 256)
    rows = []
    for t in range(T):  # the engine's decode-row loop (incremental.py:1083-1101)
        st.token.fill_(int(toks[t]))
        st.pos.fill_(t)
        assert dropin.try_persistent_extend(model, st)
        rows.append(st.logits[0, 0].cpu().clone())
        st.prev_raw.copy_(st.cand_prev_raw)
    got = torch.stack(rows).numpy()
    want = OracleModel(cfg, sd, max_len=256).decode_rows(toks).numpy()
    err = np.abs(got - want).max()
    _log(f"max |dlogit| = {err:.3e}")
    assert err < 2e-4, err
    # W = 4 windows on the same model: the same rows, bit for bit
    sw = _reference_state(cfg, 4, 256)
    win_rows = []
    for w0 in range(0, T, 4):
        sw.token.copy_(torch.from_numpy(toks[w0:w0 + 4].astype(np.int64)).view(1, 4))
        sw.pos.fill_(w0)
        assert dropin.try_mega_encode(model, sw)
        win_rows.append(sw.logits[0].cpu().clone())
        sw.prev_raw.copy_(sw.cand_prev_raw)
    assert np.array_equal(torch.cat(win_rows).numpy(), got)
    # a state the step cannot serve: False, logged, and disabled from then on
    bad = _reference_state(cfg, 1, 256)
    bad.logits = torch.zeros(1, 1, cfg.vocab_size + 1, device="cuda")
    assert not dropin.try_persistent_extend(model, bad)
    assert model._persist_disabled and not dropin.try_persistent_extend(model, st)


def test_gemv_rows_and_logits_stage_rows():
    from altxs_amd import dropin

    _log("dropin gemv_rows / logits_stage_rows")
    g = torch.Generator().manual_seed(4)
    w = (torch.randn(1024, 512, generator=g) * 0.05).to(torch.bfloat16).float().cuda()
    for dt in (torch.float32, torch.bfloat16):
        x = torch.randn(5, 512, generator=g).to(dt).cuda()
        out = torch.empty(5, 1024, dtype=torch.float32, device="cuda")
        dropin.gemv_rows(x, w, out)
        want = x.double() @ w.double().T
        assert (out.double() - want).abs().max().item() < 1e-4 * want.abs().max().item()
    v = torch.randn(512, generator=g).cuda()
    o = torch.empty(1024, device="cuda")
    dropin.gemv_vec(v, w, o)
    assert (o.double() - w.double() @ v.double()).abs().max().item() < 1e-3
    src = torch.randn(7, 512, generator=g).cuda()
    lg = torch.empty(7, 1024, device="cuda")
    dropin.logits_stage_rows(src, w, lg, eps=1e-6)
    s = src.double()
    nrm = s * torch.rsqrt((s * s).mean(-1, keepdim=True) + 1e-6)
    want = nrm @ w.double().T
    assert (lg.double() - want).abs().max().item() < 1e-4 * want.abs().max().item()
    w.mul_(2.0)  # an in-place weight update is picked up (version counter)
    dropin.gemv_rows(src, w, lg)
    assert (lg.double() - s @ w.double().T).abs().max().item() < 1e-4 * (s @ w.double().T).abs().max().item()
