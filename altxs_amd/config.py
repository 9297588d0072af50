"""Model configuration for the per-symbol step.

Mirrors the step-relevant fields of the reference ``XsaTttConfig``
(src/xsa_ttt/config.py:20-53) with the same names and defaults, plus the
profiles of ``make_config`` (config.py:195-228) and the synthetic
configurations this build is measured on:

* ``cfg1``: 2 layers, d=256, 4 heads (head_dim 64), FFN 1024, V=4096 -- the
  CPU-runnable configuration (fp32).
* ``cfg3``: 10 layers, d=512, 8 heads MHA (head_dim 64), FFN 2048, V=16384 --
  the production-scale decode step (bf16 activations, 64 segments, ctx 2048).
* ``cfg5``: cfg3 with rank-16 q/v LoRA (256 segments, ctx 4096).

The cfg* profiles keep the reference's "large" motif switches (XSA on every
layer, SmearGate, sparse attention gate, gated U-Net skips, asymmetric
softcap, ln_scale, partial RoPE over 16 dims) and turn off depth loops and
parallel lanes, so the slot count equals the layer count.
"""

from __future__ import annotations

import dataclasses
from dataclasses import dataclass


@dataclass
class AltxsConfig:
    # architecture (reference names, config.py:22-53)
    vocab_size: int = 256
    num_layers: int = 11
    xsa_last_n: int = 11
    model_dim: int = 512
    num_heads: int = 8
    num_kv_heads: int = 4
    mlp_mult: float = 4.0
    tie_embeddings: bool = True
    tied_embed_init_std: float = 0.005  # Init(seed) only (model.py:1139-1141)
    logit_softcap: float = 30.0
    asym_logit_rescale: bool = True
    rope_base: float = 1e4
    rope_dims: int = 16
    rope_yarn: bool = False
    ln_scale: bool = True
    qk_gain_init: float = 5.0
    skip_gates_enabled: bool = True
    num_loops: int = 2
    loop_start: int = 3
    loop_end: int = 5
    parallel_start_layer: int = 8
    parallel_final_lane: str = "mean"
    smear_gate_enabled: bool = True
    gate_window: int = 12
    sparse_attn_gate_enabled: bool = True
    sparse_attn_gate_scale: float = 0.5
    sparse_attn_gate_init_std: float = 0.0  # Init(seed) only (model.py:750-756)
    attn_out_gate_enabled: bool = False
    gated_attn_enabled: bool = False
    block_size: int = 2048  # RoPE train_seq_len (model.py:1023)
    online_retrain_every: int = 2048  # segment length (config.py:58); sets the engine length
    # build-only fields
    lora_rank: int = 0  # unmerged q/v LoRA rank (0 = off); ttt_lora.py:22-55
    lora_alpha: float = 16.0
    bpw_target: float = 3.15  # mixed-bit weight budget (bits per weight)

    @property
    def head_dim(self) -> int:
        return self.model_dim // self.num_heads

    @property
    def kv_dim(self) -> int:
        return self.num_kv_heads * self.head_dim

    @property
    def hidden_dim(self) -> int:
        return int(self.mlp_mult * self.model_dim)

    @property
    def rope_dims_eff(self) -> int:
        return self.rope_dims if self.rope_dims > 0 else self.head_dim

    def replace(self, **kw) -> "AltxsConfig":
        return dataclasses.replace(self, **kw)

    def validate(self) -> None:
        if self.model_dim % self.num_heads:
            raise ValueError("model_dim must be divisible by num_heads")
        if self.num_heads % self.num_kv_heads:
            raise ValueError("num_heads must be divisible by num_kv_heads")
        if self.head_dim % 2:
            raise ValueError("head_dim must be even for RoPE")
        if self.attn_out_gate_enabled or self.gated_attn_enabled:
            raise ValueError(
                "attn_out_gate / gated_attn are not part of the large motif and "
                "are not implemented by this step"
            )
        if self.logit_softcap <= 0:
            raise ValueError("logit_softcap must be positive")


def slot_itinerary(cfg: AltxsConfig) -> tuple[list[int], list[int]]:
    """Encoder and decoder layer indices with depth loops active.

    Follows GPT.__init__ (model.py:1063-1077): with ``num_loops > 0`` the
    layers ``[loop_start, loop_end]`` repeat ``num_loops + 1`` times and the
    flat list splits in half (encoder gets the floor); without loops the
    layers split at ``num_layers // 2``.
    """
    n = cfg.num_layers
    if cfg.num_loops > 0:
        seg = list(range(cfg.loop_start, cfg.loop_end + 1))
        flat = list(range(cfg.loop_start))
        for _ in range(cfg.num_loops + 1):
            flat.extend(seg)
        flat.extend(range(cfg.loop_end + 1, n))
        ne = len(flat) // 2
        return flat[:ne], flat[ne:]
    ne = n // 2
    return list(range(ne)), list(range(ne, n))


def make_config(profile: str = "large", **overrides) -> AltxsConfig:
    """Profiles of the reference (config.py:195-228) plus the benchmark configs cfg1-cfg5."""
    cfg = AltxsConfig()
    p = profile.strip().lower()
    if p == "large":
        pass
    elif p == "smoke":
        cfg = cfg.replace(num_layers=2, xsa_last_n=2, model_dim=64, num_heads=4,
                          num_kv_heads=2, mlp_mult=2.0, block_size=128,
                          num_loops=0, parallel_start_layer=99, rope_dims=8)
    elif p == "tiny":
        # Every motif feature on at a size the CPU oracle runs in milliseconds:
        # GQA, depth loops, parallel lanes, skips, smear, XSA, sparse gate.
        cfg = cfg.replace(vocab_size=256, num_layers=4, xsa_last_n=3, model_dim=256,
                          num_heads=4, num_kv_heads=2, mlp_mult=2.0, block_size=64,
                          num_loops=1, loop_start=1, loop_end=2,
                          parallel_start_layer=3, rope_dims=16, rope_yarn=True)
    elif p == "cfg1":
        cfg = cfg.replace(vocab_size=4096, num_layers=2, xsa_last_n=2, model_dim=256,
                          num_heads=4, num_kv_heads=4, mlp_mult=4.0, num_loops=0,
                          parallel_start_layer=0)
    elif p in ("cfg3", "cfg4"):
        cfg = cfg.replace(vocab_size=16384, num_layers=10, xsa_last_n=10, model_dim=512,
                          num_heads=8, num_kv_heads=8, mlp_mult=4.0, num_loops=0,
                          parallel_start_layer=0)
    elif p == "cfg5":
        cfg = cfg.replace(vocab_size=16384, num_layers=10, xsa_last_n=10, model_dim=512,
                          num_heads=8, num_kv_heads=8, mlp_mult=4.0, num_loops=0,
                          parallel_start_layer=0, lora_rank=16, lora_alpha=16.0)
    else:
        raise ValueError(f"unknown profile {profile!r}")
    cfg = cfg.replace(**overrides)
    cfg.validate()
    return cfg
