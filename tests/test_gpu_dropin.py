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
  and StaticState (tests/refshape.py: the reference's slots, tail rows and
  commits): the slots become views of the step's cache; logits within 2e-4
  of the fp32 oracle, windows equal to rows bit for bit; the engine's own
  flow (prefill into the slots, rebind, row-state sync, windows and rows)
  within 2e-5 of rows the reference's StaticACEngine wrote (fp32 weights, or
  bf16-valued ones); fp32 models on fp32 banks; False plus a sticky disable
  on a broken state;
* ``gemv_rows`` / ``logits_stage_rows`` against fp64 products.
"""

from __future__ import annotations

import os

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
    # float64 rows (the reference's own input type) that are not float32 values
    p64 = rng.random((2, 4096)) ** 3
    p64 /= p64.sum(1, keepdims=True)
    for r in p64:
        cum, total = dropin._scale_cum_np(r, alphabet_size=4096)
        want = coder.scale_cum_f64(r[None])[0]
        assert np.array_equal(cum, want) and total == int(want[-1])
    lst, _ = dropin._scale_cum(list(map(float, p64[0])), alphabet_size=4096)
    assert lst == coder.scale_cum_f64(p64[:1])[0].tolist()


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
    # probabilities handed over as float64 or as a strided view are cast to a
    # contiguous float32 vector first (the reference's _probs_arg)
    enc2 = dropin.GpuRangeCoder(dev, max_bits=4096, vocab=256)
    wide = torch.zeros(len(syms), 512, dtype=torch.float64, device=dev)
    wide[:, ::2] = prow.double()
    for i, s in enumerate(syms):
        p = wide[i, ::2] if i % 2 else prow[i].double()
        enc2.encode_symbol(p, torch.tensor([int(s)], dtype=torch.int64, device=dev))
    assert enc2.finish() == want


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


def _ref_model(profile: str, bf16: bool, *, round_banks: bool = True, std: float = 0.08,
               softcap=(2.0, 1.5)):
    """A reference-shaped GPT (tests/refshape.py) on synthetic weights whose
    matrices are rounded to bf16 values (the dense bank format) unless
    ``round_banks`` is False."""
    from altxs_amd import synth
    from altxs_amd.config import make_config

    from .refshape import RefModel, bf16_banks

    cfg = make_config(profile)
    sm = synth.make_model(cfg, std=std, softcap=softcap)
    sd = {k: np.asarray(v, np.float32) for k, v in sm.state_dict().items()}
    if round_banks:
        sd = bf16_banks(sd)
    return cfg, RefModel(cfg, sd, bf16=bf16), sd


def test_try_persistent_extend_shares_the_state_kv():
    """W=1 rows with the reference's commits (model.py:449-461) and W=4 windows
    (mega_encode) on the same model: the slots of each state view the step's
    cache, the committed K/V rows and the logits of both agree bit for bit, and
    the logits match the fp32 oracle."""
    from altxs_amd import dropin, synth
    from oracle.model_ref import OracleModel

    _log("dropin try_persistent_extend / try_mega_encode on shared slots (tiny, fp32)")
    cfg, model, sd = _ref_model("tiny", bf16=False)
    T, L = 20, 256
    toks = synth.zipf_tokens(cfg.vocab_size, (T,), seed=21)
    st = model.make_static_state(L, "cuda", win=1)
    rows = []
    for t in range(T):  # the engine's decode-row loop (incremental.py:1054-1081)
        st.token.fill_(int(toks[t]))
        st.pos.fill_(t)
        model.static_extend_fused(st)
        rows.append(st.logits[0, 0].cpu().clone())
        st.commit_window(t)
        st.prev_raw.copy_(st.cand_prev_raw)
    ws = model._persist_ws
    for i, sk in enumerate(st.slots):
        assert sk.k.data_ptr() == ws.k_pack[i].data_ptr() and sk.v.data_ptr() == ws.v_pack[i].data_ptr()
        assert tuple(sk.k.shape) == (1, L, cfg.num_kv_heads, cfg.head_dim)
    got = torch.stack(rows).numpy()
    want = OracleModel(cfg, sd, max_len=L).decode_rows(toks).numpy()
    err = np.abs(got - want).max()
    _log(f"max |dlogit| = {err:.3e}")
    assert err < 2e-4, err
    sw = model.make_static_state(L, "cuda", win=4)
    win_rows = []
    for w0 in range(0, T, 4):  # run_window + advance_window
        sw.token.copy_(torch.from_numpy(toks[w0:w0 + 4].astype(np.int64)).view(1, 4))
        sw.pos.fill_(w0)
        model.static_extend_fused(sw)
        win_rows.append(sw.logits[0].cpu().clone())
        sw.commit_window(w0)
        sw.prev_raw.copy_(sw.cand_prev_raw)
    assert model._encode_ws is not ws
    assert np.array_equal(torch.cat(win_rows).numpy(), got)
    for a, b in zip(st.slots, sw.slots):  # the same committed prefix rows in both states
        assert torch.equal(a.k[:, :T], b.k[:, :T]) and torch.equal(a.v[:, :T], b.v[:, :T])
        assert a.k[:, :T].abs().sum() > 0
    # a state the step cannot serve: False, logged, and disabled from then on
    bad = model.make_static_state(L, "cuda", win=1)
    bad.logits = torch.zeros(1, 1, cfg.vocab_size + 1, device="cuda")
    assert not dropin.try_persistent_extend(model, bad)
    assert model._persist_disabled and not dropin.try_persistent_extend(model, st)


def _engine(bf16: bool, golden_dir, fixture: str = "engine_rows_bf16w.npz"):
    from .refshape import RefEngine

    z = np.load(os.path.join(golden_dir, fixture))
    cfg, model, sd = _ref_model("tiny", bf16=bf16, std=float(z["std"]),
                                softcap=tuple(z["softcap"].tolist()),
                                round_banks=fixture == "engine_rows_bf16w.npz")
    eng = RefEngine(model, cfg, sd, win=int(z["win"]), block=int(z["block"]), every=int(z["every"]))
    assert eng.max_len == int(z["max_len"])
    return z, eng


@pytest.mark.parametrize("fixture", ["engine_rows.npz", "engine_rows_bf16w.npz"])
@pytest.mark.parametrize("key,start", [("rows_ctx", 100), ("rows_start", 0)])
def test_engine_flow_matches_reference_engine(golden_dir, fixture, key, start):
    """The engine's own flow through the drop-in (reset_segment's eager prefill
    into the slots, _rebind_packed_kv, W=16 windows through try_mega_encode
    with commit_window, the row state synced from the prefix and stepped
    through try_persistent_extend) on an fp32 model -- its fp32 weights
    (engine_rows.npz) or the same rounded to bf16 values (_bf16w): rows within
    2e-5 of the rows the reference's StaticACEngine wrote on those weights,
    and the window rows equal the decode rows bit for bit (encode/decode
    lockstep)."""
    from oracle import coder

    _log(f"dropin engine flow {fixture} {key} (tiny, fp32)")
    z, eng = _engine(False, golden_dir, fixture)
    arr, seg = z["arr"], z["arr"][start:start + 64]
    enc = eng.segment_rows_tf(arr, seg, start)
    err = float(np.abs(enc - z[key]).max())
    _log(f"windows: max |dp| = {err:.3e}")
    assert err < 2e-5, err
    dec = eng.segment_rows_one_row(arr, seg, start)
    assert np.array_equal(enc, dec)
    assert np.array_equal(coder.scale_cum(enc), coder.scale_cum(dec))
    # the slots of both states are views of the step's caches
    for st, ws in ((eng.state, eng.model._encode_ws), (eng.row_state, eng.model._persist_ws)):
        assert all(sk.k.data_ptr() == ws.k_pack[i].data_ptr() for i, sk in enumerate(st.slots))


def test_engine_flow_bf16_lockstep(golden_dir):
    """A bf16 model (bf16 activations, bf16 KV in the reference's natural
    order): the window rows equal the decode rows bit for bit, and stay within
    the bf16 mode's distance of the fp32 reference rows."""
    _log("dropin engine flow (tiny, bf16)")
    z, eng = _engine(True, golden_dir)
    arr, seg = z["arr"], z["arr"][100:164]
    enc = eng.segment_rows_tf(arr, seg, 100)
    dec = eng.segment_rows_one_row(arr, seg, 100)
    assert np.array_equal(enc, dec)
    err = float(np.abs(enc - z["rows_ctx"]).max())
    _log(f"bf16 windows vs fp32 reference: max |dp| = {err:.3e}")
    assert err < 5e-3, err
    assert eng.model._encode_ws.k_pack.dtype == torch.bfloat16


def test_fp32_model_keeps_fp32_weights():
    """An fp32 model whose matrices are not bf16 values runs on fp32 banks
    (bits 32): logits within 2e-4 of the fp32 oracle on the same weights."""
    from altxs_amd import synth
    from oracle.model_ref import OracleModel

    _log("dropin fp32 model, fp32 weights")
    cfg, model, sd = _ref_model("tiny", bf16=False, round_banks=False)
    st = model.make_static_state(256, "cuda", win=1)
    toks = synth.zipf_tokens(cfg.vocab_size, (12,), seed=3)
    rows = []
    for t, tk in enumerate(toks):
        st.token.fill_(int(tk))
        st.pos.fill_(t)
        model.static_extend_fused(st)
        rows.append(st.logits[0, 0].cpu().clone())
        st.commit_window(t)
        st.prev_raw.copy_(st.cand_prev_raw)
    assert all(q.bits == 32 for q in model._altxs_adapter.step.qt.values())
    err = float(np.abs(torch.stack(rows).numpy() - OracleModel(cfg, sd, max_len=256).decode_rows(toks).numpy()).max())
    _log(f"max |dlogit| = {err:.3e}")
    assert err < 2e-4, err


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


def test_logits_stage_rows_reference_rounding():
    """_logits_fused_rows (ac_gemv.py:312-359): the rsqrt factor is cast to
    src's dtype, the product formed in src's dtype, then cast to the weight's
    dtype.  bf16 src: factor and row rounded to bf16; fp32 src with a bf16
    weight: the row rounded to bf16."""
    from altxs_amd import dropin

    _log("dropin logits_stage_rows rounding points")
    g = torch.Generator().manual_seed(9)
    w32 = (torch.randn(1024, 512, generator=g) * 0.05).to(torch.bfloat16).float()
    src = torch.randn(6, 512, generator=g) * 3.0

    def ref(sv: torch.Tensor, wt: torch.Tensor) -> torch.Tensor:  # the reference's steps
        scale = torch.rsqrt((sv.float() ** 2).sum(-1, keepdim=True) / 512 + 1e-6).to(sv.dtype)
        norm = (sv * scale).to(wt.dtype)
        return norm.double() @ wt.double().T

    cases = [(src.to(torch.bfloat16), w32.to(torch.bfloat16)), (src, w32.to(torch.bfloat16)), (src, w32)]
    for sv, wt in cases:
        out = torch.empty(6, 1024, device="cuda")
        dropin.logits_stage_rows(sv.cuda(), wt.cuda(), out, eps=1e-6)
        want = ref(sv, wt)
        tol = 1e-5 * want.abs().max().item()
        err = (out.cpu().double() - want).abs().max().item()
        _log(f"src {sv.dtype} w {wt.dtype}: max err {err:.3e} (tol {tol:.3e})")
        assert err < tol, (sv.dtype, wt.dtype, err)
    # the rounding points matter at this tolerance: without them the bf16 case misses
    sv = src.to(torch.bfloat16)
    s = sv.double()
    plain = (s * torch.rsqrt((s * s).mean(-1, keepdim=True) + 1e-6)) @ w32.double().T
    assert (plain - ref(sv, w32.to(torch.bfloat16))).abs().max().item() > 1e-5 * plain.abs().max().item()
