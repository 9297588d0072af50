#!/usr/bin/env python3
"""Scored symbols/sec of the altxs per-symbol step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload (benchmark config "cfg3"): a ~40M-weight GPT (10 layers, d=512,
8 heads MHA of 64, FFN 2048, V=16384, mixed 2/3/4/6-bit group-64 weights at
~3.16 bpw) scoring one symbol for each of 64 independent segments whose KV
caches hold 2047 previous tokens, so every attention row reads 2048 keys.  A
step = embedding -> 10 slots -> LM head -> softmax -> integer CDFs for all 64
segments; ``value`` = 64 / step time.  The KV cache is filled with N(0, 1)
bf16 values (the scale of QK-RMS-normalised keys) and the step runs at a
fixed position, overwriting the same cache row, so each step moves the same
bytes.  Weights are seeded N(0, 0.02^2) then quantised; tokens are Zipf(1.1).
The timed K steps run as K/S replays of a HIP graph of S consecutive steps
(``--graph-steps``, default 10; ``config.graph_steps``).

The line also carries:
* ``roofline``: the decode-attention kernel (the dominant one), algorithmic
  bytes per launch / its mean launch duration, timed with HIP events around
  replays of a HIP graph of 20 launches that walk the ten slots' caches in
  turn (the same kernel, launch shape and cache footprint as in the step's
  graph: each launch reads a 268 MB cache the previous nine launches did not
  touch, so nothing is served from the 256 MB Infinity Cache);
  ``us_per_launch_in_step`` is the mean of events recorded around every
  attention launch inside the timed steps, which also includes each launch's
  gap after the preceding kernel;
  ``traffic`` comes from profiles/traffic_attn.txt (rocprofv3 FETCH_SIZE +
  WRITE_SIZE, scaled by a plain copy of known size);
* ``step_roofline``: algorithmic bytes of the whole step / step time;
* ``cpu_baseline``: the CPU oracle (op-for-op fp32 PyTorch restatement of the
  reference eager step, B=1 per segment as the reference runs) timed on this
  host on a bounded sample of the same workload;
* ``secondary`` (default workload only; ``--no-secondary`` skips it): the other
  regimes of the benchmark set measured in the same run, after the timed
  region -- the batch-1 decode step at ctx 2048, the headline step with fp32
  activations (the mode within 2e-3 of the fp32 oracle's logits), cfg4 chunk
  scoring (64 x 2048 tokens), the cfg5 LoRA step (256 segments at ctx 4096)
  and the cfg2 batch-1 row GEMV over >= 2 GB streams.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

METRIC = "scored symbols/sec @32M mixed-3.15bpw, 64 segs ctx2048; % HBM roofline"


def decode_metric(profile: str, B: int, ctx: int, bpw: float | None) -> str:
    """The headline metric string for the default workload; the same wording
    with this run's model, bit width, segment count and context otherwise."""
    if (profile, B, ctx) == ("cfg3", 64, 2048) and bpw is not None:
        return METRIC
    w = "dense bf16" if bpw is None else f"mixed-{bpw:.2f}bpw"
    return f"scored symbols/sec @{profile} {w}, {B} segs ctx{ctx}; % HBM roofline"


HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def read_traffic(kernel: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/traffic_<kernel>.txt)."""
    path = os.path.join(HERE, "profiles", f"traffic_{kernel}.txt")
    if not os.path.exists(path):
        return None
    for line in open(path, encoding="utf8"):
        if line.startswith("traffic_bytes_per_launch"):
            return float(line.split("=")[1].split()[0])
    return None


def attn_kernel_ms(model, st, reps: int = 20, replays: int = 5) -> float:
    """Mean duration of the decode-attention kernel: ``reps`` launches with the
    step's launch configuration (XSA on, bf16 operands), launch i reading slot
    i's cache (mod the slot count) as the step's launches do, captured in one
    HIP graph (back to back as in the step's own graph, no host launch gaps)
    and replayed ``replays`` times between HIP events on the replay stream."""
    import ctypes

    import torch

    from altxs_amd import _lib

    cfg = model.cfg
    B, H, Hkv, max_len = st.batch, cfg.num_heads, cfg.num_kv_heads, st.max_len
    g = torch.Generator(device="cuda").manual_seed(5)
    q = torch.randn(B, H, 64, generator=g, device="cuda")
    y = torch.empty(B, H * 64, dtype=torch.bfloat16 if model.act_bf16 else torch.float32, device="cuda")
    args = []
    for s in range(model.n_slots):
        kv = st.kv[s]
        a = _lib.AttnArgs()
        a.B, a.W, a.H, a.Hkv, a.head_dim, a.max_len = B, 1, H, Hkv, 64, max_len
        a.kv_bf16, a.y_bf16 = int(model.kv_bf16), int(model.act_bf16)
        esz = kv.element_size()
        a.q, a.k = q.data_ptr(), kv.data_ptr()
        a.v = kv.data_ptr() + Hkv * max_len * 64 * esz
        a.kv_seg_stride = 2 * Hkv * max_len * 64
        a.pos, a.gate, a.use_xsa = st.pos.data_ptr(), None, 1
        a.flags = _lib.ATTN_OPS_BF16 if model.act_bf16 else 0
        a.y, a.err = y.data_ptr(), st.err.data_ptr()
        args.append(a)
    L = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for a in args:
        _lib.check(L.altxs_decode_attn(ctypes.byref(a), stream), "altxs_decode_attn")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for i in range(reps):
            _lib.check(L.altxs_decode_attn(ctypes.byref(args[i % len(args)]), cap), "altxs_decode_attn")
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    del graph
    return e0.elapsed_time(e1) / (reps * replays)


def decode_measure(sm, B: int, ctx: int, steps: int = 50, gs: int = 10, warmup: int = 5,
                   act: str = "bf16") -> dict:
    """The decode step of B segments at context ctx (``act`` activations, bf16
    KV): ms per step over steps // gs replays of a graph of gs steps, and the
    attention kernel's own launch time (attn_kernel_ms)."""
    import numpy as np
    import torch

    from altxs_amd import synth
    from altxs_amd.model import StepModel

    cfg = sm.cfg
    model = StepModel(sm, act=act, kv="bf16")
    st = model.make_static_state((ctx + 255) // 256 * 256, win=1, batch=B, want_probs=False, want_cdf=True)
    g = torch.Generator(device="cuda").manual_seed(0)
    st.kv.normal_(generator=g)
    st.pos.fill_(ctx - 1)
    st.token.copy_(torch.from_numpy(synth.zipf_tokens(cfg.vocab_size, (B, 1)).astype(np.int32)))
    for _ in range(warmup):
        model.step(st)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(gs):
            model.step(st)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps // gs):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (steps // gs * gs)
    st.check_errors()
    attn_ms = attn_kernel_ms(model, st)
    ab = synth.algorithmic_step_bytes(sm, B, ctx, kv_bytes=2)
    attn_bytes = ab["kv_read"] // ab["n_slots"] + B * cfg.num_heads * cfg.head_dim * 6 + B * cfg.num_heads * 4
    del graph, st, model  # blocks stay in torch's cache (see main)
    return {"segments": B, "ctx": ctx, "act": act, "ms_per_step": round(ms, 4),
            "value": round(B / (ms * 1e-3), 1),
            "unit": "sym/s", "steps": steps // gs * gs, "graph_steps": gs,
            "attn_us_per_launch": round(attn_ms * 1e3, 2),
            "attn_GBps": round(attn_bytes / (attn_ms * 1e-3) / 1e9, 1)}


def secondary_measures(sm) -> dict:
    """The other regimes of the benchmark set, measured in the same run (each
    a few seconds): the batch-1 decode step (the reference's production
    regime), the headline step with fp32 activations (the mode whose logits
    stay within 2e-3 of the fp32 oracle), cfg4 chunk scoring (64 x 2048
    tokens from position 0), the cfg5 LoRA step (256 segments at ctx 4096)
    and the cfg2 batch-1 row GEMV over >= 2 GB streams."""
    import numpy as np

    from altxs_amd import synth
    from altxs_amd.config import make_config

    out = {}
    try:
        out["b1_decode_step"] = decode_measure(sm, 1, 2048)
        log(f"secondary: batch-1 decode step {out['b1_decode_step']['ms_per_step']:.3f} ms")
    except Exception as exc:  # noqa: BLE001
        out["b1_decode_step"] = {"error": repr(exc)}
    try:
        out["fp32_act_decode_step"] = decode_measure(sm, 64, 2048, act="fp32")
        log(f"secondary: fp32-activation decode step {out['fp32_act_decode_step']['ms_per_step']:.3f} ms")
    except Exception as exc:  # noqa: BLE001
        out["fp32_act_decode_step"] = {"error": repr(exc)}
    try:
        sm4 = synth.make_model(make_config("cfg4"))
        ms, flops = window_measure(sm4, 64, 2048, 0, "bf16", "bf16", steps=3, warmup=1)
        tf = flops / (ms * 1e-3) / 1e12
        out["cfg4_window"] = {"workload": "cfg4: 64 segments x 2048 tokens from position 0, bf16",
                              "ms_per_step": round(ms, 3), "value": round(64 * 2048 / (ms * 1e-3), 1),
                              "unit": "sym/s", "TFLOPs": round(tf, 1), "mfma_frac": round(tf / 2500.0, 4),
                              "steps": 3}
        log(f"secondary: cfg4 {ms:.2f} ms/step, {tf:.0f} TFLOP/s")
    except Exception as exc:  # noqa: BLE001
        out["cfg4_window"] = {"error": repr(exc)}
    try:
        sm5 = synth.make_model(make_config("cfg5"))
        r5 = decode_measure(sm5, 256, 4096, steps=20)
        ab5 = synth.algorithmic_step_bytes(sm5, 256, 4096, kv_bytes=2)
        gbs5 = ab5["total"] / (r5["ms_per_step"] * 1e-3) / 1e9
        r5.update({"workload": "cfg5: 256 segments at ctx 4096, rank-16 q/v LoRA on every slot, bf16",
                   "step_GBps": round(gbs5, 1), "step_hbm_frac": round(gbs5 / HBM_PEAK_GBS, 4)})
        out["cfg5_decode_step"] = r5
        log(f"secondary: cfg5 {r5['ms_per_step']:.3f} ms/step, {gbs5:.0f} GB/s")
        del sm5
    except Exception as exc:  # noqa: BLE001
        out["cfg5_decode_step"] = {"error": repr(exc)}
    try:
        res = cfg2_measure(2.0, (("qgemv", 1),))
        gbs = float(np.mean([r["GBps"] for r in res]))
        out["cfg2_gemv_b1"] = {"workload": "cfg2 B=1 row GEMV (altxs_qgemv_stream), >= 2 GB streams, "
                                           "512x2048 / 2048x512 x 2/3/4/6 bits",
                               "mean_GBps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                               "lines": [{k: r[k] for k in ("N", "K", "bits", "GBps")} for r in res]}
        log(f"secondary: cfg2 row GEMV {gbs:.0f} GB/s")
    except Exception as exc:  # noqa: BLE001
        out["cfg2_gemv_b1"] = {"error": repr(exc)}
    return out


def cpu_model() -> str:
    """The host CPU's model name (lscpu "Model name", else /proc/cpuinfo)."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.strip().lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except Exception:  # noqa: BLE001
        pass
    try:
        for line in open("/proc/cpuinfo", encoding="utf8"):
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(sm, ctx: int, seconds: float, seed: int = 0) -> dict:
    """Time the CPU oracle on single-segment decode steps at context ``ctx``."""
    import numpy as np
    import torch

    from altxs_amd import synth
    from oracle.model_ref import OracleModel

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    om = OracleModel(sm.cfg, sm.state_dict(), max_len=ctx)
    st = om.new_state(ctx)
    g = torch.Generator().manual_seed(seed)
    for s in range(om.n_slots):
        st.k[s].normal_(generator=g)
        st.v[s].normal_(generator=g)
    toks = synth.zipf_tokens(sm.cfg.vocab_size, (4096,), seed=seed + 1)
    om.step(st, [int(toks[0])])  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        st.pos = ctx - 1
        om.step(st, [int(toks[n % len(toks)])])
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 8) or n >= 100000:
            break
    return {"value": n / el, "unit": "sym/s", "cores": cores, "kind": "port", "cpu": cpu_model(),
            "sample": f"{n} single-segment decode steps at ctx {ctx} (fp32 oracle, B=1, "
                      f"{el:.1f} s, torch threads={cores})"}


def window_bench(a) -> int:
    """--window W > 1: one step scores W tokens of each of B segments from position 0
    (the prefill-style chunk scoring of benchmark cfg4: causal attention over the
    chunk, MFMA GEMMs, one CDF per token).  MFMA-bound, so ``roofline`` is in
    TFLOP/s against the dense bf16 peak."""
    import numpy as np
    import torch

    from altxs_amd import synth
    from altxs_amd.config import make_config
    from altxs_amd.model import StepModel

    B, W = a.segments, a.window
    # --ctx C > W: windows at the end of a C-token context (steady-state encode,
    # the cache holding C - W earlier positions); otherwise from position 0
    p0 = max(0, a.ctx - W) if a.ctx > W else 0
    max_len = (p0 + W + 255) // 256 * 256
    cfg = make_config(a.profile)
    sm = synth.make_model(cfg, dense=a.dense)
    ms, flops = window_measure(sm, B, W, p0, a.act, a.kv, a.steps, a.warmup)
    R = B * W
    tflops = flops / (ms * 1e-3) / 1e12
    peak = 2500.0 if a.act == "bf16" else 157.3
    log(f"window W={W} x {B} segments at position {p0}: {ms:.3f} ms/step, "
        f"{R / (ms * 1e-3) / 1e6:.2f} M sym/s, {tflops:.0f} TFLOP/s")
    cpu = None
    if not a.no_cpu:
        from oracle.model_ref import OracleModel

        cores = len(os.sched_getaffinity(0))
        torch.set_num_threads(cores)
        om = OracleModel(cfg, sm.state_dict(), max_len=max_len)
        ids = synth.zipf_tokens(cfg.vocab_size, (W,), seed=3)
        t0 = time.perf_counter()
        om.forward_logits(ids)
        el = time.perf_counter() - t0
        cpu = {"value": W / el, "unit": "sym/s", "cores": cores, "kind": "port", "cpu": cpu_model(),
               "sample": f"one segment of {W} tokens, fp32 oracle full causal forward, {el:.1f} s"}
    out = {
        "metric": (f"scored symbols/sec, {a.profile} chunk scoring {B} segments x {W} tokens"
                   + (f" after {p0} cached positions" if p0 else "")),
        "value": round(R / (ms * 1e-3), 1), "unit": "sym/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": a.kv if a.act == a.kv else f"{a.act}-act/{a.kv}-kv", "data": "synthetic",
        "config": {"workload": f"{a.profile} window scoring: {B} segments x {W} tokens from position {p0}",
                   "segments": B, "window": W, "position": p0, "timing": "hip-graph"},
        "roofline": {"kernel": "whole step (MFMA GEMMs + window attention)", "bound": "mfma",
                     "achieved": round(tflops, 1), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(tflops / peak, 4), "traffic": None, "flops": int(flops)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


def window_measure(sm, B: int, W: int, p0: int, act: str, kv: str, steps: int, warmup: int):
    """(ms per window step, useful flops per step) of B segments x W tokens
    from position p0, timed over ``steps`` replays of a one-step HIP graph."""
    import numpy as np
    import torch

    from altxs_amd import synth
    from altxs_amd.model import StepModel

    cfg = sm.cfg
    max_len = (p0 + W + 255) // 256 * 256
    model = StepModel(sm, act=act, kv=kv)
    st = model.make_static_state(max_len, win=W, batch=B, want_probs=False, want_cdf=True)
    if p0:
        g = torch.Generator(device="cuda").manual_seed(0)
        st.kv.normal_(generator=g)
    st.pos.fill_(p0)
    st.token.copy_(torch.from_numpy(synth.zipf_tokens(cfg.vocab_size, (B, W)).astype(np.int32)))
    for _ in range(warmup):
        model.step(st)
    torch.cuda.synchronize()
    st.check_errors()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        model.step(st)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    st.check_errors()
    R = B * W
    body = sum(p.codes.size for n, p in sm.packed.items() if n != "emb")
    attn = 4 * 64 * (W * (W + 1) // 2 + W * p0) * cfg.num_heads * B * model.n_slots
    flops = 2 * R * body + 2 * R * cfg.vocab_size * cfg.model_dim + attn
    del graph, st, model  # blocks stay in torch's cache (see main)
    return ms, flops


def cfg2_bench(a) -> int:
    """--cfg2: the fused dequant-GEMV/GEMM microbenchmark (benchmark config 2).

    Weight matrices [N, K] = 512 x 2048 and 2048 x 512 packed at 2, 3, 4 and 6
    bits (uniform random codes -- uniform random bytes in the tiled planes --
    and random fp16 group-64 scales), fp16 activations ~N(0, 1), B = 1 and 64
    rows.  One matrix is at most 0.8 MB and would sit in the 256 MB Infinity
    Cache, so the HBM figure streams >= 2 GB of distinct matrices through one
    ``altxs_qgemv_stream`` / ``altxs_qgemm_stream`` launch (each matrix's y
    written to its own rows); algorithmic bytes per launch = codes + scales +
    y of every matrix + x once.  B = 1 runs both the row GEMV (altxs_qgemv:
    VALU dot arithmetic, the batch-1 kernel; ``value`` is its mean) and the
    16-row MFMA tiles of altxs_qgemm (15 empty rows, for comparison); B = 64
    runs altxs_qgemm.  The single-call latency is one matrix, replayed from a
    HIP graph (cache-resident, launch included).  MFMA figures count the
    useful 2*N*K*B flops against the dense fp16 peak (2.5 PFLOP/s)."""
    import numpy as np

    results = cfg2_measure(a.cfg2_gb, (("qgemv", 1), ("qgemm", 1), ("qgemm", 64)))
    b1 = [r for r in results if r["B"] == 1 and r["api"] == "qgemv"]
    value = float(np.mean([r["GBps"] for r in b1]))
    mfma_b1 = float(np.mean([r["GBps"] for r in results if r["B"] == 1 and r["api"] == "qgemm"]))
    out = {
        "metric": "cfg2 fused dequant-GEMV HBM throughput (B=1, >=2 GB of distinct packed matrices, "
                  "mean over 512x2048 / 2048x512 and 2/3/4/6 bits)",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": 5, "warmup": 1,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "cfg2: packed group-64 weights, fp16 scales, fp16 activations, B in {1, 64}",
                   "stream_gb": a.cfg2_gb},
        "roofline": {"kernel": "qgemv_kernel (altxs_qgemv_stream), B=1", "bound": "hbm",
                     "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": None},
        "mfma_tile_b1_GBps": round(mfma_b1, 1),
        "results": results,
    }
    print(json.dumps(out), flush=True)
    return 0


def cfg2_measure(gb: float, runs) -> list:
    """cfg2 lines for ``runs`` = ((api, B), ...) over >= ``gb`` GB streams of
    each shape and width (each launch checked against dequant + fp64 matmul)."""
    import ctypes

    import torch

    from altxs_amd import _lib

    L = _lib.load()
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    g = torch.Generator(device="cuda").manual_seed(2)
    target = float(gb) * 1e9
    results = []
    for (N, K) in ((512, 2048), (2048, 512)):
        for bits in (2, 3, 4, 6):
            cb = N * K * bits // 8
            sb = N * K // 64 * 2
            cs, ss = (cb + 255) // 256 * 256, (sb + 255) // 256 * 256
            count = int(min(65535, max(1, -(-target // (cb + sb)))))
            codes = torch.randint(0, 256, (count * cs,), dtype=torch.uint8, device="cuda", generator=g)
            scales = (torch.rand(count * ss // 2, device="cuda", generator=g) * 0.05 + 0.001).half()
            qt = _lib.QTensor(codes.data_ptr(), scales.data_ptr(), N, K, bits, 0)
            for api, B in runs:
                x = torch.randn(B, K, device="cuda", generator=g).half()
                y = torch.empty(count, B, N, dtype=torch.float32, device="cuda")
                fn_stream = L.altxs_qgemv_stream if api == "qgemv" else L.altxs_qgemm_stream
                fn_one = L.altxs_qgemv if api == "qgemv" else L.altxs_qgemm
                run = lambda: _lib.check(fn_stream(  # noqa: E731
                    ctypes.byref(qt), count, cs, ss, x.data_ptr(), _lib.F16, B, y.data_ptr(), stream()),
                    f"altxs_{api}_stream")
                run()
                torch.cuda.synchronize()
                # spot check: the first and last matrix against dequant + fp64 matmul
                for i in (0, count - 1):
                    qi = _lib.QTensor(codes.data_ptr() + i * cs, scales.data_ptr() + i * ss, N, K, bits, 0)
                    w = torch.empty(N, K, device="cuda")
                    _lib.check(L.altxs_dequant(ctypes.byref(qi), w.data_ptr(), stream()), "altxs_dequant")
                    ref = x.double() @ w.double().T
                    err = (y[i].double() - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)
                    if err > 1e-3:
                        raise RuntimeError(f"cfg2 check failed: {api} [{N},{K}] b={bits} B={B} matrix {i}: "
                                           f"{err:.2e}")
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                reps = 5
                e0.record()
                for _ in range(reps):
                    run()
                e1.record()
                torch.cuda.synchronize()
                ms = e0.elapsed_time(e1) / reps
                nbytes = count * (cb + sb + B * N * 4) + B * K * 2
                flops = 2.0 * N * K * B * count
                # single call on one matrix, from a graph of 50 calls
                y1 = torch.empty(B, N, dtype=torch.float32, device="cuda")
                one = lambda: fn_one(ctypes.byref(qt), x.data_ptr(), _lib.F16, B,  # noqa: E731
                                     y1.data_ptr(), stream())
                one()
                torch.cuda.synchronize()
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr):
                    for _ in range(50):
                        one()
                gr.replay()
                torch.cuda.synchronize()
                e0.record()
                gr.replay()
                e1.record()
                torch.cuda.synchronize()
                us1 = e0.elapsed_time(e1) / 50 * 1e3
                r = {"api": api, "N": N, "K": K, "bits": bits, "B": B, "matrices": count,
                     "stream_bytes": int(nbytes), "ms_per_launch": round(ms, 4),
                     "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1),
                     "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / 2500.0, 4),
                     "single_call_us": round(us1, 2)}
                log(f"{api} [{N},{K}] b={bits} B={B}: {count} matrices, {ms:.3f} ms, {r['GBps']:.0f} GB/s "
                    f"({100 * r['hbm_frac']:.1f}% HBM), {r['TFLOPs']:.1f} TFLOP/s; single call {us1:.2f} us")
                results.append(r)
                del y, y1, gr
            del codes, scales  # blocks stay in torch's cache (see main)
    return results


def coder_bench(a) -> int:
    """--coder: the closed loop of compression on the cfg3 decode workload.
    Compress = step + the range coder encoding each segment's next symbol with
    the step's integer CDF; decompress = step + the decoder writing the decoded
    symbol into the token buffer the next step reads (no host round trip).
    Each is timed over K steps captured in one HIP graph; the coder kernels
    alone are timed the same way (latency-bound: one lane per stream to
    encode, one wave per stream to decode)."""
    import numpy as np
    import torch

    from altxs_amd import synth
    from altxs_amd.coder import RangeCoder
    from altxs_amd.config import make_config
    from altxs_amd.model import StepModel

    B, ctx = a.segments, a.ctx
    max_len = (ctx + 255) // 256 * 256
    cfg = make_config(a.profile)
    sm = synth.make_model(cfg)
    model = StepModel(sm, act=a.act, kv=a.kv)
    st = model.make_static_state(max_len, win=1, batch=B, want_probs=False, want_cdf=True)
    g = torch.Generator(device="cuda").manual_seed(0)
    st.kv.normal_(generator=g)
    st.pos.fill_(ctx - 1)
    toks = torch.from_numpy(synth.zipf_tokens(cfg.vocab_size, (B, 1)).astype(np.int32)).cuda()
    st.token.copy_(toks)
    nxt = torch.from_numpy(synth.zipf_tokens(cfg.vocab_size, (B, 1), seed=7).astype(np.int32)).cuda()
    K = a.steps
    enc = RangeCoder(B, 64 + 8 * (K + a.warmup + 8))
    dec = RangeCoder(B, 64 + 8 * (K + a.warmup + 8))
    model.step(st)
    torch.cuda.synchronize()
    dec.begin_decode([bytes(16)] * B)

    def timed(body) -> float:
        for _ in range(a.warmup):
            body()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(K):
                body()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        gr.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / K

    step_ms = timed(lambda: model.step(st))
    enc_ms = timed(lambda: enc.encode(st.cum, nxt))
    dec_ms = timed(lambda: dec.decode(st.cum, st.token))
    comp_ms = timed(lambda: (model.step(st), enc.encode(st.cum, nxt)))
    dec.begin_decode([bytes(16)] * B)
    decomp_ms = timed(lambda: (model.step(st), dec.decode(st.cum, st.token)))
    st.check_errors()
    enc.check()
    dec.check()
    log(f"step {step_ms * 1e3:.1f} us; encode {enc_ms * 1e3:.2f} us, decode {dec_ms * 1e3:.2f} us "
        f"per call ({B} streams); compress {comp_ms * 1e3:.1f} us/step, decompress "
        f"{decomp_ms * 1e3:.1f} us/step")
    out = {
        "metric": f"compressed symbols/sec, {a.profile} decode step + GPU range coder, {B} segments "
                  f"ctx{ctx}",
        "value": round(B / (comp_ms * 1e-3), 1), "unit": "sym/s", "n_gpus": 1, "steps": K,
        "warmup": a.warmup, "ms_per_step": round(comp_ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": a.kv, "data": "synthetic",
        "config": {"workload": f"{a.profile} compress: step + encode of one symbol per segment",
                   "segments": B, "ctx": ctx, "timing": "hip-graph"},
        "decompress": {"value": round(B / (decomp_ms * 1e-3), 1), "unit": "sym/s",
                       "ms_per_step": round(decomp_ms, 4)},
        "coder_us_per_call": {"encode": round(enc_ms * 1e3, 2), "decode": round(dec_ms * 1e3, 2),
                              "step_alone": round(step_ms * 1e3, 1)},
    }
    print(json.dumps(out), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--profile", default="cfg3")
    ap.add_argument("--segments", type=int, default=64)
    ap.add_argument("--ctx", type=int, default=2048)
    ap.add_argument("--act", default="bf16", choices=["bf16", "fp32"])
    ap.add_argument("--kv", default="bf16", choices=["bf16", "fp32"])
    ap.add_argument("--no-graph", action="store_true", help="time eager launches instead of a HIP graph")
    ap.add_argument("--graph-steps", type=int, default=10, metavar="S",
                    help="decode steps captured per HIP graph (the timed K steps replay K/S graphs; "
                         "S must divide K, else 1)")
    ap.add_argument("--streams", type=int, default=1, choices=[1, 2],
                    help="2: two segment groups on two streams, the second chain started half a slot later")
    ap.add_argument("--window", type=int, default=1, metavar="W",
                    help="W > 1: score W-token windows from position 0 (prefill-style "
                         "chunk scoring, cfg4 = --profile cfg4 --window 2048); value = B*W / step")
    ap.add_argument("--dense", action="store_true",
                    help="dense bf16 weights (bits 16, the reference's runtime banks) instead of "
                         "the mixed-bit packing")
    ap.add_argument("--coder", action="store_true",
                    help="time compression (step + GPU range coder encode) and decompression "
                         "(step + decode into the next step's token buffer) instead")
    ap.add_argument("--cfg2", action="store_true",
                    help="the fused dequant-GEMV/GEMM microbenchmark (512x2048 and 2048x512, 2/3/4/6 bits, "
                         "B=1 and 64) over >= --cfg2-gb GB of distinct packed matrices")
    ap.add_argument("--cfg2-gb", type=float, default=2.0)
    ap.add_argument("--fuse-o", action="store_true",
                    help="decode: form the out-projection inside the attention launch and finish "
                         "it where it is read, instead of its own launch (the same bits)")
    ap.add_argument("--persistent", action="store_true",
                    help="run every slot in one persistent launch (tasks in dependency order)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB five times (the known-size "
                         "reference kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE), then exit")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the batch-1 step, cfg4 window and cfg2 row-GEMV lines the default "
                         "workload adds under \"secondary\"")
    a = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py: this build runs on one GPU only (independent segments would shard "
              "across GPUs with no per-step communication); --gpus must be 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    if a.cfg2:
        return cfg2_bench(a)
    if a.window > 1:
        return window_bench(a)
    if a.coder:
        return coder_bench(a)
    if a.copy_calibration > 0:
        n = a.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "launches": 5}), flush=True)
        return 0

    from altxs_amd import hiprt, synth
    from altxs_amd.config import make_config
    from altxs_amd.model import StepModel

    B, ctx = a.segments, a.ctx
    max_len = (ctx + 255) // 256 * 256
    cfg = make_config(a.profile)
    t0 = time.time()
    sm = synth.make_model(cfg, dense=a.dense)
    log(f"model {a.profile}: {sm.bits_summary()['bpw']:.4f} bpw, built in {time.time() - t0:.1f}s")
    model = StepModel(sm, act=a.act, kv=a.kv)
    model.fuse_o = a.fuse_o
    st = model.make_static_state(max_len, win=1, batch=B, want_probs=False, want_cdf=True,
                                 split=a.streams == 2, persistent=a.persistent)
    groups = 2 if st.split else 1
    g = torch.Generator(device="cuda").manual_seed(0)
    st.kv.normal_(generator=g)
    st.pos.fill_(ctx - 1)
    st.token.copy_(torch.from_numpy(synth.zipf_tokens(cfg.vocab_size, (B, 1)).astype(np.int32)))
    torch.cuda.synchronize()

    for _ in range(a.warmup):
        model.step(st)
    torch.cuda.synchronize()
    st.check_errors()
    log(f"warmup done ({a.warmup} steps)")

    # S consecutive steps per graph: the steps are device-resident end to end
    # (the engine's decode loop feeds each decoded symbol to the next step on
    # the device), so a graph of S steps is a launch strategy a caller can use;
    # it removes S - 1 of every S gaps between graph launches (~8 us each here).
    gs = a.graph_steps if a.graph_steps >= 1 and a.steps % a.graph_steps == 0 else 1
    graph = None
    if not a.no_graph:
        try:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(gs):
                    model.step(st)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
        except Exception as exc:  # noqa: BLE001
            log(f"graph capture failed ({exc!r}); timing eager launches")
            graph = None

    # ---- timed region: exactly K steps -------------------------------------
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    if graph is not None:
        for _ in range(a.steps // gs):
            graph.replay()
    else:
        for _ in range(a.steps):
            model.step(st)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / a.steps
    st.check_errors()
    log(f"timed {a.steps} steps ({f'graphs of {gs} steps' if graph is not None else 'eager'}): "
        f"{ms:.3f} ms/step")

    # ---- dominant kernel: HIP events around every attention launch ----------
    # The K instrumented steps are captured into one graph (distinct events per
    # step) and replayed once, so the events see the graph's launch spacing;
    # if capture is unavailable they run eagerly.
    n_slots = model.n_slots
    per_step = 2 * n_slots * groups
    ev = hiprt.EventArray(per_step * a.steps)
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s0.record()
    for k in range(a.steps):
        model.step(st, attn_events=ev.ptr + k * per_step * 8)
    s1.record()
    torch.cuda.synchronize()
    eager_ms = s0.elapsed_time(s1) / a.steps
    event_timing = "eager"
    if graph is not None:
        try:
            g2 = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g2):
                for k in range(a.steps):
                    model.step(st, attn_events=ev.ptr + k * per_step * 8)
            torch.cuda.synchronize()
            g2.replay()
            torch.cuda.synchronize()
            event_timing = "hip-graph"
        except Exception as exc:  # noqa: BLE001
            log(f"instrumented graph failed ({exc!r}); using the eager event times")
            torch.cuda.synchronize()
    kvb = 2 if a.kv == "bf16" else 4
    ab = synth.algorithmic_step_bytes(sm, B, ctx, kv_bytes=kvb)
    ybytes = 2 if a.act == "bf16" else 4
    if a.persistent:
        # one layer-kernel launch per step (events 0/1 of each step's block)
        durs = [ev.elapsed_ms(k * per_step, k * per_step + 1) for k in range(a.steps)]
        layer_w = sum(p.nbytes_codes + p.nbytes_scales for n, p in sm.packed.items() if n != "emb")
        # algorithmic bytes of the launch: every slot's KV read + append, layer weights
        attn_bytes = ab["kv_read"] + ab["kv_write"] + layer_w
        kname = "layers_kernel (persistent: every slot's QKV, attention, O, MLP)"
    else:
        durs = [ev.elapsed_ms(2 * i, 2 * i + 1) for i in range(n_slots * groups * a.steps)]
        # algorithmic bytes of one attention launch (one slot, one group: B/groups segments)
        attn_bytes = (ab["kv_read"] // ab["n_slots"] + B * cfg.num_heads * cfg.head_dim * (4 + ybytes)
                      + B * cfg.num_heads * 4) / groups
        kname = "attn_mfma_kernel (decode attention)"
    ev.close()
    in_step_ms = float(np.mean(durs))  # events around each launch inside the step (incl. launch gaps)
    if a.persistent or groups > 1 or a.kv != "bf16":
        attn_ms = in_step_ms
    else:
        attn_ms = attn_kernel_ms(model, st)
        st.check_errors()
    achieved = attn_bytes / (attn_ms * 1e-3) / 1e9
    step_gbs = ab["total"] / (ms * 1e-3) / 1e9
    log(f"{kname.split(' ')[0]}: {attn_ms * 1e3:.1f} us/launch, {achieved:.0f} GB/s; eager step {eager_ms:.3f} ms; "
        f"step {step_gbs:.0f} GB/s of algorithmic traffic")

    cpu = None
    if not a.no_cpu:
        log(f"cpu baseline (~{a.cpu_seconds:.0f}s)")
        cpu = cpu_baseline(sm, ctx, a.cpu_seconds)
        log(f"cpu baseline: {cpu['value']:.1f} sym/s on {cpu['cores']} cores")

    value = B / (ms * 1e-3)
    graphed = graph is not None
    secondary = None
    if not a.no_secondary and (a.profile, B, ctx, a.act, a.kv, a.dense, a.persistent, a.streams) == (
            "cfg3", 64, 2048, "bf16", "bf16", False, False, 1):
        # The freed buffers stay in torch's cache, for the later measurements to
        # reuse: memory handed back to the driver (empty_cache) and allocated
        # again measured slower here -- cfg3 0.687 against 0.668 ms per step,
        # attention 44.3 against 43.0 us -- while cached blocks and first-time
        # allocations measure alike.
        del graph, st, model
        secondary = secondary_measures(sm)
    out = {
        "metric": decode_metric(a.profile, B, ctx, None if a.dense else sm.bits_summary()["bpw"]),
        "value": round(value, 1),
        "unit": "sym/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": a.kv if a.act == a.kv else f"{a.act}-act/{a.kv}-kv",
        "data": "synthetic",
        "config": {
            "workload": (f"{a.profile} decode step: {B} segments x 1 symbol, ctx {ctx}, "
                         f"{cfg.num_layers} layers d={cfg.model_dim} H={cfg.num_heads} "
                         f"FFN={cfg.hidden_dim} V={cfg.vocab_size}, "
                         + ("dense bf16 weights, " if a.dense else
                            f"{sm.bits_summary()['bpw']:.3f} bpw group-64 weights, ")
                         + f"{a.act} activations, {a.kv} KV"),
            "segments": B, "ctx": ctx, "timing": "hip-graph" if graphed else "eager",
            "graph_steps": gs if graphed else 0,
            "streams": groups, "persistent": bool(a.persistent),
            "eager_ms_per_step": round(eager_ms, 4), "kernel_event_timing": event_timing,
        },
        "roofline": {
            "kernel": kname,
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            # measured for the default workload only (cfg3, 64 segments, ctx 2048)
            "traffic": (read_traffic("layers" if a.persistent else "attn")
                        if (a.profile, B, ctx, a.act, a.kv, a.dense) == ("cfg3", 64, 2048, "bf16", "bf16", False)
                        else None),
            "bytes_per_launch": int(attn_bytes),
            "us_per_launch": round(attn_ms * 1e3, 2),
            "us_per_launch_in_step": round(in_step_ms * 1e3, 2),
        },
        "step_roofline": {
            "algorithmic_bytes": int(ab["total"]),
            "achieved": round(step_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(step_gbs / HBM_PEAK_GBS, 4),
        },
        "cpu_baseline": cpu,
    }
    if secondary is not None:
        out["secondary"] = secondary
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
