"""Init(seed): the reference model's initial weights, for decoding a shipped codec.

A shipped codec stores ``W - Init(seed)`` (src/hyperflow_distillation/
mixed_bit_delta.py:232-312): ``load_codec`` seeds the RNGs
(``enable_deterministic(seed)``, src/xsa_ttt/device.py:19-31 ->
src/model/deterministic_mode.py:20-80: ``torch.manual_seed(seed)``), builds
the model (``build_model``, src/xsa_ttt/model.py:2102-2108 -> ``GPT.__init__``
982-1117 -> ``_init_weights`` 1139-1163) and adds the decoded delta.  This
module restates that construction as the sequence of torch init calls it
makes on the CPU generator, in the order the constructor makes them:

1. ``nn.Embedding(V, D)`` draws its default N(0, 1) weight (later redrawn);
2. per block (``CausalSelfAttention.__init__`` 703-758): the optional gate
   weights -- ``attn_gate_proj`` (a ``CastedLinear``: kaiming-uniform, later
   zeroed), ``gated_attn`` N(0, 0.01), the sparse gate N(0, std) when its
   init std is positive;
3. ``lm_head`` when the embedding is not tied (kaiming-uniform, later zeroed);
4. ``smear_gate`` (``CastedLinear(gate_window, 1)``: kaiming-uniform, later
   zeroed);
5. ``_init_weights``: the tied embedding N(0, tied_embed_init_std); for each
   layer i the orthogonal q bank ``qo[i]``, zero out-projection ``qo[n + i]``,
   orthogonal ``kv[i]`` and ``kv[n + i]``; then for each layer the orthogonal
   MLP up bank and a zero down bank.

Everything else starts at a constant (model.py:925-932, 1085-1113).  The
result is pinned against the reference's own Init(seed) for the shipped
codec's seed and config (tests/golden/init_seed.npz, written by
tests/golden/make_golden.py: per-matrix sums and sampled values).  Host-side
set-up only: it runs once, before the weights are packed for the device.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from .config import AltxsConfig, slot_itinerary


def _kaiming_linear(out_f: int, in_f: int, g: torch.Generator) -> None:
    """``nn.Linear.reset_parameters`` of a bias-free linear: the draws only."""
    nn.init.kaiming_uniform_(torch.empty(out_f, in_f), a=math.sqrt(5), generator=g)


@torch.no_grad()
def reference_init_state(cfg: AltxsConfig, seed: int) -> dict[str, torch.Tensor]:
    """The reference-named state dict of ``GPT(cfg)`` built after
    ``torch.manual_seed(seed)`` (CPU, fp32)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(int(seed))
    V, D, L = cfg.vocab_size, cfg.model_dim, cfg.num_layers
    H, kvd, F, gw = cfg.num_heads, cfg.kv_dim, cfg.hidden_dim, cfg.gate_window
    emb = torch.empty(V, D)
    nn.init.normal_(emb, generator=g)  # 1. nn.Embedding's own init
    qo = torch.empty(2 * L, D, D)
    kv = torch.empty(2 * L, kvd, D)
    up = torch.empty(L, F, D)
    down = torch.empty(L, D, F)
    gate_w = []
    for _ in range(L):  # 2. the blocks' gate weights
        if cfg.attn_out_gate_enabled:
            _kaiming_linear(H, gw, g)
        if cfg.gated_attn_enabled:
            nn.init.normal_(torch.empty(H, D), mean=0.0, std=0.01, generator=g)
        w = torch.zeros(H, gw)
        if cfg.sparse_attn_gate_enabled and cfg.sparse_attn_gate_init_std > 0:
            nn.init.normal_(w, mean=0.0, std=cfg.sparse_attn_gate_init_std, generator=g)
        gate_w.append(w)
    if not cfg.tie_embeddings:  # 3. the untied head (zeroed by _init_weights)
        _kaiming_linear(V, D, g)
    if cfg.smear_gate_enabled:  # 4. the smear gate (zeroed by _init_weights)
        _kaiming_linear(1, gw, g)
    # 5. _init_weights
    if cfg.tie_embeddings:
        nn.init.normal_(emb, mean=0.0, std=cfg.tied_embed_init_std, generator=g)
    for i in range(L):
        nn.init.orthogonal_(qo[i], gain=1.0, generator=g)
        qo[L + i].zero_()
        nn.init.orthogonal_(kv[i], gain=1.0, generator=g)
        nn.init.orthogonal_(kv[L + i], gain=1.0, generator=g)
    for i in range(L):
        nn.init.orthogonal_(up[i], gain=1.0, generator=g)
        down[i].zero_()
    sd: dict[str, torch.Tensor] = {"tok_emb.weight": emb, "qo_bank": qo, "kv_bank": kv,
                                   "mlp_up_bank": up, "mlp_down_bank": down}
    # constants (model.py:925-932, 1085-1113)
    enc, dec = slot_itinerary(cfg)
    n_skip = min(len(enc), len(dec))
    sd["skip_weights"] = torch.ones(n_skip, D)
    if cfg.skip_gates_enabled:
        sd["skip_gates"] = torch.zeros(n_skip, D)
    sd["parallel_post_lambdas"] = torch.ones(L, 2, 2)
    sd["parallel_resid_lambdas"] = torch.full((L, 2), 1.1)
    if cfg.asym_logit_rescale:
        sd["softcap_pos"] = torch.tensor(cfg.logit_softcap)
        sd["softcap_neg"] = torch.tensor(cfg.logit_softcap)
    if cfg.smear_gate_enabled:
        sd["smear_gate.weight"] = torch.zeros(1, gw)
        sd["smear_lambda"] = torch.zeros(1)
    for i in range(L):
        sd[f"blocks.{i}.attn_scale"] = torch.ones(D)
        sd[f"blocks.{i}.mlp_scale"] = torch.ones(D)
        sd[f"blocks.{i}.resid_mix"] = torch.stack((torch.ones(D), torch.zeros(D)))
        sd[f"blocks.{i}.attn.q_gain"] = torch.full((H,), float(cfg.qk_gain_init))
        if cfg.sparse_attn_gate_enabled:
            sd[f"blocks.{i}.attn.attn_gate_w"] = gate_w[i]
    return sd
