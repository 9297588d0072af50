"""Several committed decode steps captured in one HIP graph.

The step's inputs and outputs stay on the device, so a caller can capture S
consecutive decode steps (each committing its token) in one graph, the tokens
fed from a device array inside the graph -- the launch strategy bench.py times
with ``--graph-steps``.  Every replay must give the tables of the same steps
launched one by one, also with eager work and synchronisation between replays.
The graph holds kernels only: tokens go in and tables come out through
elementwise kernels (no memset or memcpy nodes).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _log(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


@pytest.mark.parametrize("profile,B,S", [("cfg1", 4, 6), ("tiny", 3, 5)])
def test_committed_steps_in_one_graph_equal_eager(profile, B, S):
    from altxs_amd import synth
    from altxs_amd.config import make_config
    from altxs_amd.model import StepModel

    _log(f"graph of {S} committed steps, {profile} B={B}")
    cfg = make_config(profile)
    sm = synth.make_model(cfg, std=0.02 if profile == "cfg1" else 0.08,
                          softcap=(30.0, 24.0) if profile == "cfg1" else (2.0, 1.5))
    toks = torch.from_numpy(synth.zipf_tokens(cfg.vocab_size, (B, S), seed=7).astype(np.int32)).to(DEV)
    model = StepModel(sm, device=DEV, act="bf16")
    st = model.make_static_state(256, win=1, batch=B, want_probs=False)

    def reset():
        st.pos.zero_()
        st.prev_raw.zero_()
        st.cand_prev_raw.zero_()
        st.kv.zero_()

    reset()
    want = []
    for i in range(S):
        torch.add(toks[:, i:i + 1], 0, out=st.token)
        model.step(st, commit=True)
        want.append(st.cum.clone())
    torch.cuda.synchronize()
    st.check_errors()
    want = torch.stack(want)

    rec = torch.zeros_like(want)
    reset()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(S):
            torch.add(toks[:, i:i + 1], 0, out=st.token)
            model.step(st, commit=True)
            torch.add(st.cum, 0, out=rec[i])
    torch.cuda.synchronize()
    for rep in range(3):
        reset()
        rec.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        st.check_errors()
        assert torch.equal(rec, want), f"replay {rep}"
        assert int(st.pos[0].item()) == S
        # eager work between replays
        torch.add(toks[:, 0:1], 0, out=st.token)
        model.step(st, commit=False)
        torch.cuda.synchronize()
