"""Seeded synthetic workloads: model weights, token streams, KV fill.

Weights use the reference's state_dict names (src/xsa_ttt/model.py:982-1163)
so the same tensors can be loaded into the reference GPT:

* matrices (tok_emb.weight, qo_bank, kv_bank, mlp_up_bank, mlp_down_bank) are
  N(0, std^2) from ``np.random.default_rng(seed)`` and then quantised per
  tensor with :mod:`altxs_amd.codec` (the packed copy is what the GPU reads;
  the dequantised copy is what the CPU oracle reads -- identical values);
* small parameters are their reference init values plus seeded noise, so
  every motif term (skips, gates, smear, lanes, softcap) is exercised.

Tokens are Zipf(s) over the vocabulary: p_k ~ k^-s with rank k <-> id k-1,
drawn with ``default_rng(seed).choice``.
"""

from __future__ import annotations

import dataclasses

import numpy as np

from .codec import PackedTensor, allocate_bits
from .config import AltxsConfig, slot_itinerary

TOKEN_SEED = 20261201
WEIGHT_SEED = 1337


def zipf_tokens(vocab: int, shape, s: float = 1.1, seed: int = TOKEN_SEED) -> np.ndarray:
    ranks = np.arange(1, vocab + 1, dtype=np.float64)
    p = ranks ** (-s)
    p /= p.sum()
    return np.random.default_rng(seed).choice(vocab, size=shape, p=p).astype(np.int64)


def tensor_list(cfg: AltxsConfig) -> list[tuple[str, int, int]]:
    """(name, N, K) of every packed tensor, most sensitive first."""
    d, kvd, f = cfg.model_dim, cfg.kv_dim, cfg.hidden_dim
    out = [("emb", cfg.vocab_size, d)]
    for i in range(cfg.num_layers):
        out.append((f"l{i}.qkv", d + 2 * kvd, d))
    for i in range(cfg.num_layers):
        out.append((f"l{i}.o", d, d))
    for i in range(cfg.num_layers):
        out.append((f"l{i}.up", f, d))
    for i in range(cfg.num_layers):
        out.append((f"l{i}.down", d, f))
    return out


@dataclasses.dataclass
class SynthModel:
    cfg: AltxsConfig
    packed: dict[str, PackedTensor]
    small: dict[str, np.ndarray]  # reference-named small params (fp32)

    def state_dict(self) -> dict[str, np.ndarray]:
        """Dense fp32 state dict (reference names) from the dequantised tensors."""
        cfg = self.cfg
        n, d, kvd = cfg.num_layers, cfg.model_dim, cfg.kv_dim
        sd = dict(self.small)
        sd["tok_emb.weight"] = self.packed["emb"].dense()
        qo = np.zeros((2 * n, d, d), np.float32)
        kv = np.zeros((2 * n, kvd, d), np.float32)
        up = np.zeros((n, cfg.hidden_dim, d), np.float32)
        down = np.zeros((n, d, cfg.hidden_dim), np.float32)
        for i in range(n):
            qkv = self.packed[f"l{i}.qkv"].dense()
            qo[i] = qkv[:d]
            kv[i] = qkv[d:d + kvd]
            kv[n + i] = qkv[d + kvd:]
            qo[n + i] = self.packed[f"l{i}.o"].dense()
            up[i] = self.packed[f"l{i}.up"].dense()
            down[i] = self.packed[f"l{i}.down"].dense()
        sd["qo_bank"], sd["kv_bank"] = qo, kv
        sd["mlp_up_bank"], sd["mlp_down_bank"] = up, down
        return sd

    def bits_summary(self) -> dict:
        vals = sum(p.codes.size * p.bits for p in self.packed.values())
        nw = sum(p.codes.size for p in self.packed.values())
        return {
            "weights": int(nw),
            "value_bits": int(vals),
            "bpw": vals / nw,
            "code_bytes": int(sum(p.nbytes_codes for p in self.packed.values())),
            "scale_bytes": int(sum(p.nbytes_scales for p in self.packed.values())),
            "bits": {k: p.bits for k, p in self.packed.items()},
        }


def make_model(cfg: AltxsConfig, *, seed: int = WEIGHT_SEED, std: float = 0.02,
               softcap: tuple[float, float] | None = None, dense: bool | int = False,
               bits: dict[str, int] | None = None) -> SynthModel:
    """``dense``: every matrix kept dense instead of the mixed-bit packing --
    True or 16: bf16 (the reference's runtime banks); 32: fp32 (its fp32
    compute mode).  ``bits``: widths of named tensors (e.g. ``{"l0.o": 6}``)
    in place of the allocation's."""
    cfg.validate()
    rng = np.random.default_rng(seed)
    d, kvd, f = cfg.model_dim, cfg.kv_dim, cfg.hidden_dim
    names = tensor_list(cfg)
    override = dict(bits or {})
    if dense:
        bits = {nm: (32 if dense == 32 else 16) for nm, _, _ in names}
    else:
        bits = allocate_bits([(nm, nn * kk) for nm, nn, kk in names], cfg.bpw_target)
    unknown = set(override) - set(bits)
    if unknown:
        raise ValueError(f"no tensors named {sorted(unknown)}")
    bits.update(override)
    packed = {}
    for nm, nn, kk in names:
        w = rng.standard_normal((nn, kk), dtype=np.float32) * np.float32(std)
        packed[nm] = PackedTensor.from_dense(nm, w, bits[nm])

    srng = np.random.default_rng(seed + 1)
    L, H, gw = cfg.num_layers, cfg.num_heads, cfg.gate_window

    def noise(*shape, scale=1.0):
        return (srng.standard_normal(shape) * scale).astype(np.float32)

    small: dict[str, np.ndarray] = {}
    enc, dec = slot_itinerary(cfg)
    n_skip = min(len(enc), len(dec))
    small["skip_weights"] = 1.0 + noise(n_skip, d, scale=0.1)
    if cfg.skip_gates_enabled:
        small["skip_gates"] = noise(n_skip, d, scale=0.5)
    small["parallel_post_lambdas"] = 1.0 + noise(L, 2, 2, scale=0.1)
    small["parallel_resid_lambdas"] = 1.1 + noise(L, 2, scale=0.05)
    if cfg.smear_gate_enabled:
        small["smear_gate.weight"] = noise(1, gw, scale=0.3)
        small["smear_lambda"] = np.array([0.5], np.float32)
    if cfg.asym_logit_rescale:
        sp, sn = softcap if softcap is not None else (cfg.logit_softcap, 0.8 * cfg.logit_softcap)
        small["softcap_pos"] = np.array(sp, np.float32)
        small["softcap_neg"] = np.array(sn, np.float32)
    for i in range(L):
        small[f"blocks.{i}.attn_scale"] = 1.0 + noise(d, scale=0.1)
        small[f"blocks.{i}.mlp_scale"] = 1.0 + noise(d, scale=0.1)
        small[f"blocks.{i}.resid_mix"] = np.stack(
            [1.0 + noise(d, scale=0.1), noise(d, scale=0.1)]).astype(np.float32)
        small[f"blocks.{i}.attn.q_gain"] = cfg.qk_gain_init + noise(H, scale=0.3)
        if cfg.sparse_attn_gate_enabled:
            small[f"blocks.{i}.attn.attn_gate_w"] = noise(H, gw, scale=0.3)
    if cfg.lora_rank > 0:
        # per-slot q/v adapters (TTTLoRA.q_loras/v_loras, ttt_lora.py:64-120), fp16
        # values N(0, 0.01^2) for A and B (benchmark cfg5; the reference starts B at 0)
        lrng = np.random.default_rng(seed + 2)
        r = cfg.lora_rank
        for sl in range(len(enc) + len(dec)):
            for kind, n_out in (("q", d), ("v", kvd)):
                a = lrng.standard_normal((r, d)) * 0.01
                b = lrng.standard_normal((n_out, r)) * 0.01
                small[f"{kind}_loras.{sl}.A"] = a.astype(np.float16).astype(np.float32)
                small[f"{kind}_loras.{sl}.B"] = b.astype(np.float16).astype(np.float32)
    return SynthModel(cfg, packed, small)


def rope_table(cfg: AltxsConfig, max_len: int, rope_len: int | None = None):
    """cos/sin [max_len, rope_dims/2] fp32, built as Rotary.forward does.

    Follows src/xsa_ttt/model.py:130-192: inv_freq = 1 / base^(arange(0, rd, 2)/rd)
    in fp32; with YaRN and a table longer than train_seq_len (= block_size),
    base <- base * (len/train_seq_len)^(rd/(rd-2)); freqs = outer(t, inv_freq).
    ``len`` is the length the table is warmed at, ``rope_len`` (default
    max_len): the engine warms it once at its static length
    (incremental.py:106-113, 239-242), which can differ from the rows kept.
    """
    import torch

    rd = cfg.rope_dims_eff
    base = cfg.rope_base
    L = int(rope_len) if rope_len is not None else int(max_len)
    if cfg.rope_yarn and L > cfg.block_size:
        scale = L / cfg.block_size
        new_base = base * scale ** (rd / (rd - 2))
        inv_freq = 1.0 / new_base ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd)
    else:
        inv_freq = 1.0 / base ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd)
    t = torch.arange(max_len, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return freqs.cos().contiguous(), freqs.sin().contiguous()


def algorithmic_step_bytes(model: SynthModel, B: int, ctx: int, kv_bytes: int = 2,
                           with_probs: bool = False) -> dict:
    """Algorithmic HBM bytes of one W=1 decode step over B segments at context ctx.

    KV read (ctx keys per row, K and V, every slot) + packed weights + scales +
    KV append + logits (fp32) + CDF (uint32, V+1) [+ probs].
    """
    cfg = model.cfg
    enc, dec = slot_itinerary(cfg)
    n_slots = len(enc) + len(dec)
    kvd = cfg.kv_dim
    kv_read = B * n_slots * 2 * ctx * kvd * kv_bytes
    kv_write = B * n_slots * 2 * kvd * kv_bytes
    codes = sum(p.nbytes_codes for p in model.packed.values())
    scales = sum(p.nbytes_scales for p in model.packed.values())
    logits = B * cfg.vocab_size * 4
    cdf = B * (cfg.vocab_size + 1) * 4
    probs = B * cfg.vocab_size * 4 if with_probs else 0
    total = kv_read + kv_write + codes + scales + logits + cdf + probs
    return {"kv_read": kv_read, "kv_write": kv_write, "weight_codes": codes,
            "weight_scales": scales, "logits": logits, "cdf": cdf, "probs": probs,
            "total": total, "n_slots": n_slots}


def flops_per_step(cfg: AltxsConfig, B: int, ctx: int) -> float:
    enc, dec = slot_itinerary(cfg)
    n_slots = len(enc) + len(dec)
    d, kvd, f = cfg.model_dim, cfg.kv_dim, cfg.hidden_dim
    per_slot = 2 * (d * (d + 2 * kvd) + d * d + 2 * d * f)
    gemm = B * (n_slots * per_slot + 2 * cfg.vocab_size * d)
    attn = B * n_slots * cfg.num_heads * 2 * 2 * ctx * cfg.head_dim
    return float(gemm + attn)
