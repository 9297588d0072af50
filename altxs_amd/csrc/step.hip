// The whole per-symbol step for B independent segments x W window tokens.
//
// Per slot (one transformer layer application) five launches:
//   QKV  : prologue = U-Net skip + resid_mix + RMSNorm*ln_scale (+ sparse-gate
//          logits), MFMA dequant GEMM, epilogue = per-head QK-RMSNorm, RoPE,
//          q_gain, K/V written into the cache at pos+t.
//   ATTN : attn.hip (fixed 64-key tiles, per-wave online softmax, fixed-order merge).
//   O    : out-projection; epilogue = attention residual (or parallel lane term).
//   UP   : prologue = RMSNorm*ln_scale of the attention output; epilogue =
//          LeakyReLU(0.5)^2.
//   DOWN : down-projection; epilogue = MLP residual / parallel-lane update.
// Then the LM head (final RMSNorm prologue, tanh softcap epilogue), the
// deterministic softmax -> CDF, and an optional commit (pos += W,
// prev_raw = last raw embedding).  Every kernel computes each row from that
// row's inputs only, so a decode row (W = 1) and the same position inside an
// encode window (W > 1) or a larger batch produce identical bits.
//
// Semantics follow src/xsa_ttt/model.py: Block.forward 932-979,
// CausalSelfAttention.forward 770-871, MLP 874-882, _parallel_block
// 1293-1355, _apply_decoder_skip 1275-1291, _embed_tokens_window 1559-1579,
// _project_logits/_apply_asym_softcap 1463-1500, _static_extend_body
// 1649-1781.
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "common.h"
#include "kernels.h"
#include "persist.h"
#include "step_ops.h"

using namespace altxs;
using namespace altxs_sk;

namespace {

// ---- host side --------------------------------------------------------------


int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

// LM head: workgroups per 16-row tile (0 = one per 64-column tile).  128 (two
// column tiles each, V = 16384): cfg3 11.9 us against 12.9 (64: 15.5).
constexpr int kLmHeadColWgs = 128;
// Launches with at least this many rows use the 64 x 128 tile GEMMs
// (gemm_big_kernel, bit-identical to the 16-row tasks); bf16 activations only.
// cfg3 windows at ctx 2048: W = 16 (1024 rows) 1.43 ms per step against 1.51
// on the 16-row tasks; W = 8 (512 rows) 1.34 against 1.09.
constexpr int kBigRows = 1024;
// Decode launches (W = 1, rows a multiple of 64, at most kXcdRowsMax) place row
// tile t (8 rows) on XCD t % 8 (xcd_row_split) in the out-projection, MLP,
// attention, embedding and CDF launches, so each reads the rows the previous
// one wrote from its own XCD's L2.  QKV and the LM head keep the column-task
// placement: their 8-row tiles would decode each weight twice as often, which
// measured slower than the reads it makes local (cfg3: 0.677 ms per step
// against 0.687 with them, 0.693 with none).  At 256 rows (cfg5) the doubled
// weight decoding costs more than it saves (3.79 against 3.58 ms).
// ALTXS_XCD_ROWS=0 turns it off (same bits either way; for measurement).
constexpr int kXcdRowsMax = 64;
bool xcd_rows_on() {
  static int v = -1;
  if (v < 0) {
    const char* e = getenv("ALTXS_XCD_ROWS");
    v = (e && atoi(e) == 0) ? 0 : 1;
  }
  return v != 0;
}
// Preferred K-splits of the 4-wave GEMM stages (QKV and the LM head use
// (NB, KS) = (4, 1): one 64-column head tile per task).
constexpr int kKsO = 2, kKsUp = 2, kKsDown = 4;
// Sync area layout (ints): persistent-kernel role counter at 0, GEMM-queue
// and attention-queue tickets at 16 and 32 (one 64-byte line each), counters
// of (slot s, row tile m) at kTicketPad + (s * nrt + m) * kCtrStride + stage.
constexpr int kTicketPad = 64, kCtrStride = 16;
// Persistent kernel: workgroups that run the GEMM chain; the rest stream
// attention (ALTXS_PERSIST_NG overrides, for tuning).
int persist_gemm_workers() {
  static int ng = -1;
  if (ng < 0) {
    const char* e = getenv("ALTXS_PERSIST_NG");
    ng = e ? atoi(e) : 96;
    if (ng < 1) ng = 1;
  }
  return ng;
}
static_assert(N_ST <= kCtrStride, "counter group too small");

int64_t carve(const AltxsStepDesc* d, int nb, WS* w, char* base) {
  const int64_t R = (int64_t)nb * d->W, Rp = align_up(R, 16);
  const int64_t D = d->D, n = d->n_slots;
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align_up(bytes, 256);
    return p;
  };
  char* x0 = take((n + 1) * Rp * D * 4);
  char* x1 = take((n + 1) * Rp * D * 4);
  char* xin = take(2 * Rp * D * 4);
  char* qin = take(2 * Rp * D * 4);
  char* xout = take(Rp * D * 4);
  char* q = take(Rp * d->H * HD * 4);
  char* gate = take(Rp * d->H * 4);
  char* y = take(Rp * D * 4);
  char* hb = take(Rp * (int64_t)d->F * 4);
  char* stats = take(Rp * (int64_t)(d->V / 64 + 1) * 8);
  // persistent-kernel counters: role counter and queue tickets, then one
  // 64-byte group of completion counters per (slot, row tile)
  const int nsync = kTicketPad + (int)(n * (Rp / 16)) * kCtrStride;
  char* sync = take(nsync * 4);
  // ALTXS_F_FUSE_O decode steps: the out-projection's per-head terms
  char* opart = take(d->W == 1 && (d->flags & ALTXS_F_FUSE_O) ? Rp * d->H * D * 4 : 0);
  if (w) {
    w->X0 = (float*)x0; w->X1 = (float*)x1; w->XIN = (float*)xin; w->QIN = (float*)qin;
    w->XOUT = (float*)xout;
    w->Q = (float*)q; w->GATE = (float*)gate; w->Y = y; w->HB = hb;
    w->STATS = (float2*)stats; w->SYNC = (int*)sync; w->nsync = nsync;
    w->OPART = (float*)opart;
  }
  return off;
}

// Split mode: the second group's chain starts after the first group's slot-0
// QKV (0), attention (1) or MLP (2) -- ALTXS_SPLIT_FORK, for tuning.
int split_fork_stage() {
  static int f = -1;
  if (f < 0) {
    const char* e = getenv("ALTXS_SPLIT_FORK");
    f = e ? atoi(e) : 0;
    if (f < 0 || f > 2) f = 0;
  }
  return f;
}

// ALTXS_F_FUSE_O, for decode steps (R rows) on the tiled bf16 cache with
// bf16 activations and a packed MHA out-projection: the attention launch also
// forms the out-projection's per-head terms, and the out-projection is
// finished where its result is read -- the MLP-up prologue of a sequential
// slot (ProOutNorm), the MLP-down epilogue of a parallel one (OutFin) -- one
// launch fewer per slot, the same bits.  Not the default: every MLP-up
// column task of a sequential slot then reads H terms per element instead of
// one, and each attention workgroup decodes the out-projection's codes of its
// head for its one row (the GEMM decodes them once per 8-row tile); cfg3,
// per slot: attention +2.5 us (B = 64) / +2.0 us (B = 1), MLP up +5.6 / +1.8 us,
// against the 4.4-4.6 us launch saved.
bool out_proj_fused(const AltxsStepDesc* d, int s, int R) {
  const AltxsLayer& L = d->layers[d->slots[s].layer];
  return d->act_bf16 && (d->flags & ALTXS_F_FUSE_O) && d->W == 1 && R < kBigRows &&
         !d->plan_dev && d->kv_bf16 == ALTXS_KV_BF16 && d->kv_tail_end == 0 && d->H == d->Hkv &&
         d->H % 4 == 0 && (d->D == 256 || d->D == 512) && L.o.N == d->D && L.o.K == (int64_t)d->H * HD &&
         (L.o.bits == 2 || L.o.bits == 3 || L.o.bits == 4 || L.o.bits == 6);
}

// Two segment groups (split mode) when the caller hands in a second stream.
bool split_mode(const AltxsStepDesc* d) { return d->aux_stream != nullptr && d->B >= 2; }
int64_t ws_bytes_needed(const AltxsStepDesc* d) {
  const int nb0 = (d->B + 1) / 2;
  const int64_t one = carve(d, d->B, nullptr, nullptr);
  const int64_t two = carve(d, nb0, nullptr, nullptr) + carve(d, d->B - nb0, nullptr, nullptr);
  return one > two ? one : two;
}

QT qt_of(const AltxsQTensor& t) {
  QT q;
  q.codes = (const uint8_t*)t.codes;
  q.scales = (const uint16_t*)t.scales;
  q.N = (int)t.N;
  q.K = (int)t.K;
  q.bits = t.bits;
  return q;
}

int check_tensor(const AltxsQTensor& t, int64_t N, int64_t K, const char* what, int li, int act_bf16) {
  const bool dense = t.bits == 16 || t.bits == 32;  // bf16 / fp32 values in the tiled order, no scales
  ALTXS_REQUIRE(t.codes && (dense || t.scales), "altxs_step: layer %d %s: null tensor", li, what);
  ALTXS_REQUIRE(t.N == N && t.K == K, "altxs_step: layer %d %s: shape [%lld,%lld] != [%lld,%lld]",
                li, what, (long long)t.N, (long long)t.K, (long long)N, (long long)K);
  ALTXS_REQUIRE(t.bits == 2 || t.bits == 3 || t.bits == 4 || t.bits == 6 || dense,
                "altxs_step: layer %d %s: bits=%d", li, what, t.bits);
  ALTXS_REQUIRE(t.bits != 32 || !act_bf16, "altxs_step: layer %d %s: fp32 weights (bits 32) need "
                "fp32 activations", li, what);
  ALTXS_REQUIRE(((uintptr_t)t.codes & 15) == 0 && ((uintptr_t)t.scales & 7) == 0,
                "altxs_step: layer %d %s: misaligned", li, what);
  ALTXS_REQUIRE(!t.expanded || (!dense && ((uintptr_t)t.expanded & 15) == 0),
                "altxs_step: layer %d %s: expanded values need a packed width and 16-byte alignment", li,
                what);
  return ALTXS_OK;
}

// A tensor as the large-tile kernels read it: its expanded values (the same
// operands, without the decoding) when the caller supplies them.  Used by the
// K = 512 row-band stages QKV, out-projection and MLP up, whose expanded
// weights (<= 1.5 MB) stay in an XCD's L2 (cfg4: 585 / 174 / 419 us against
// 640 / 180 / 495 packed).  The MLP down-projection (K = 2048 tiles, whose
// k-block barriers leave one group of loads in flight: 943 against 628 us)
// and the LM head (16 MB expanded, re-read from the memory-side cache by
// every row band: 5.10 against 4.71 ms) stay on the packed codes.
QT qt_big(const AltxsQTensor& t) {
  QT q = qt_of(t);
  if (t.expanded) {
    q.codes = (const uint8_t*)t.expanded;
    q.bits = kExpBits;
  }
  return q;
}

int validate(const AltxsStepDesc* d) {
  ALTXS_REQUIRE(d, "altxs_step: null descriptor");
  ALTXS_REQUIRE(d->abi_version == ALTXS_ABI_VERSION, "altxs_step: abi_version %d != %d",
                d->abi_version, ALTXS_ABI_VERSION);
  ALTXS_REQUIRE(d->head_dim == HD, "altxs_step: head_dim=%d (only 64 is built)", d->head_dim);
  ALTXS_REQUIRE(d->D == d->H * HD, "altxs_step: D != H*head_dim");
  ALTXS_REQUIRE(d->D % 256 == 0 && d->D <= 512, "altxs_step: D=%d must be 256 or 512",
                d->D);
  ALTXS_REQUIRE(d->F % 256 == 0 && d->F <= 8192, "altxs_step: F=%d must be a multiple of 256", d->F);
  ALTXS_REQUIRE(d->V >= 16 && d->V % 16 == 0 && d->V <= 65536, "altxs_step: V=%d must be a multiple of 16 in [16, 65536]",
                d->V);
  ALTXS_REQUIRE(d->Hkv >= 1 && d->H % d->Hkv == 0, "altxs_step: H %% Hkv != 0");
  const int group = d->H / d->Hkv;
  ALTXS_REQUIRE(group == 1 || group == 2 || group == 4, "altxs_step: H/Hkv=%d not in {1,2,4}", group);
  ALTXS_REQUIRE(d->B >= 1 && d->W >= 1 && (int64_t)d->B * d->W <= (1 << 20), "altxs_step: bad B/W");
  ALTXS_REQUIRE(d->n_layers >= 1 && d->n_layers <= ALTXS_MAX_LAYERS, "altxs_step: n_layers");
  ALTXS_REQUIRE(d->n_slots >= 1 && d->n_slots <= ALTXS_MAX_SLOTS, "altxs_step: n_slots");
  ALTXS_REQUIRE(d->max_len >= 256 && d->max_len % 256 == 0, "altxs_step: max_len=%d must be a multiple of 256",
                d->max_len);
  ALTXS_REQUIRE(d->kv_bf16 == ALTXS_KV_F32 || d->kv_bf16 == ALTXS_KV_BF16 || d->kv_bf16 == ALTXS_KV_BF16_NATURAL,
                "altxs_step: kv_bf16=%d is not a KV layout", d->kv_bf16);
  ALTXS_REQUIRE(d->kv_tail_end == 0 || (d->kv_bf16 != ALTXS_KV_BF16 && d->kv_tail_end >= d->W &&
                                        d->kv_tail_end <= d->max_len),
                "altxs_step: kv_tail_end=%d needs a natural KV layout and W <= kv_tail_end <= max_len",
                d->kv_tail_end);
  ALTXS_REQUIRE(d->rope_dims >= 8 && d->rope_dims <= HD && d->rope_dims % 8 == 0,
                "altxs_step: rope_dims=%d", d->rope_dims);
  ALTXS_REQUIRE(d->gate_window >= 0 && d->gate_window <= d->D, "altxs_step: gate_window");
  ALTXS_REQUIRE(d->lora_rank >= 0 && d->lora_rank <= 16, "altxs_step: lora_rank=%d not in [0, 16]",
                d->lora_rank);
  ALTXS_REQUIRE(d->tokens && d->pos && d->prev_raw && d->cand_raw && d->kv && d->ws && d->logits &&
                    d->rope_cos && d->rope_sin && d->err,
                "altxs_step: null state/output pointer");
  ALTXS_REQUIRE(d->ws_bytes >= ws_bytes_needed(d), "altxs_step: workspace too small");
  if (d->aux_stream) ALTXS_REQUIRE(d->sync_events, "altxs_step: aux_stream needs sync_events");
  if (d->flags & ALTXS_F_SMEAR)
    ALTXS_REQUIRE(d->smear_w && d->smear_lambda, "altxs_step: smear params missing");
  if (d->flags & ALTXS_F_RENORM)
    ALTXS_REQUIRE(d->V <= 16384, "altxs_step: renormalised rows need V <= 16384 (V=%d)", d->V);
  if (d->flags & ALTXS_F_ASYM_SOFTCAP) ALTXS_REQUIRE(d->softcap_pn, "altxs_step: softcap_pn missing");
  const int kvd = d->Hkv * HD;
  for (int l = 0; l < d->n_layers; ++l) {
    const AltxsLayer& L = d->layers[l];
    int rc;
    if ((rc = check_tensor(L.qkv, d->D + 2 * kvd, d->D, "qkv", l, d->act_bf16))) return rc;
    if ((rc = check_tensor(L.o, d->D, d->D, "o", l, d->act_bf16))) return rc;
    if ((rc = check_tensor(L.up, d->F, d->D, "up", l, d->act_bf16))) return rc;
    if ((rc = check_tensor(L.down, d->D, d->F, "down", l, d->act_bf16))) return rc;
    ALTXS_REQUIRE(L.resid_mix && L.attn_scale && L.mlp_scale && L.q_gain,
                  "altxs_step: layer %d small params missing", l);
    // read with 16-byte vector loads (embedding and strip epilogues)
    ALTXS_REQUIRE((((uintptr_t)L.resid_mix | (uintptr_t)L.attn_scale | (uintptr_t)L.mlp_scale) & 15) == 0,
                  "altxs_step: layer %d resid_mix / attn_scale / mlp_scale must be 16-byte aligned", l);
    if (d->flags & ALTXS_F_SPARSE_GATE)
      ALTXS_REQUIRE(L.attn_gate_w, "altxs_step: layer %d attn_gate_w missing", l);
  }
  ALTXS_REQUIRE((((uintptr_t)d->skip_weights | (uintptr_t)d->skip_gates) & 15) == 0,
                "altxs_step: skip_weights / skip_gates must be 16-byte aligned");
  int rc;
  if ((rc = check_tensor(d->emb, d->V, d->D, "emb", -1, d->act_bf16))) return rc;
  for (int s = 0; s < d->n_slots; ++s) {
    const AltxsSlot& S = d->slots[s];
    ALTXS_REQUIRE(S.layer >= 0 && S.layer < d->n_layers, "altxs_step: slot %d layer", s);
    ALTXS_REQUIRE(S.kind == ALTXS_SLOT_SEQ || S.kind == ALTXS_SLOT_PAR, "altxs_step: slot %d kind", s);
    ALTXS_REQUIRE(S.skip_src < s, "altxs_step: slot %d pops a later slot", s);
    if (s == 0)
      ALTXS_REQUIRE(S.kind == ALTXS_SLOT_SEQ && S.skip_src < 0,
                    "altxs_step: slot 0 must be a sequential slot without a skip");
    if (S.skip_src >= 0) ALTXS_REQUIRE(S.skip_idx >= 0 && d->skip_weights, "altxs_step: slot %d skip", s);
    if (S.kind == ALTXS_SLOT_PAR)
      ALTXS_REQUIRE(d->layers[S.layer].par_resid && d->layers[S.layer].par_post,
                    "altxs_step: slot %d parallel lambdas missing", s);
    const int nl = (S.lora_q_a != nullptr) + (S.lora_q_b != nullptr) + (S.lora_v_a != nullptr) +
                   (S.lora_v_b != nullptr);
    ALTXS_REQUIRE(nl == 0 || (nl == 4 && d->lora_rank > 0),
                  "altxs_step: slot %d LoRA needs all four matrices and lora_rank > 0", s);
    if (nl)
      ALTXS_REQUIRE(((uintptr_t)S.lora_q_a & 15) == 0 && ((uintptr_t)S.lora_v_a & 15) == 0 &&
                        ((uintptr_t)S.lora_q_b & 1) == 0 && ((uintptr_t)S.lora_v_b & 1) == 0,
                    "altxs_step: slot %d LoRA A must be 16-byte aligned", s);
  }
  return ALTXS_OK;
}

// Final hidden state: 0 = x (or the attention lane), 1 = mean of the two
// parallel lanes, 2 = the MLP lane (model.py:1357-1362).
int final_mode(const AltxsStepDesc* d) {
  bool any_par = false;
  for (int s = 0; s < d->n_slots; ++s) any_par |= d->slots[s].kind == ALTXS_SLOT_PAR;
  if (!any_par) return 0;
  if (d->flags & ALTXS_F_FINAL_MLP) return 2;
  if (d->flags & ALTXS_F_FINAL_ATTN) return 0;
  return 1;
}

// A contiguous range of segments run as one batch: segments [b0, b0 + nb).
// Pointers are the caller's state offset to the group; the KV slot stride
// stays that of the whole batch.
struct Group {
  int b0, nb;
  const int32_t* tokens;
  int32_t* pos;
  float* prev_raw;
  float* cand_raw;
  char* kv;  // slot 0, segment b0
  float* logits;
  float* probs;
  uint32_t* cum;
  WS w;
};

Group make_group(const AltxsStepDesc* d, int b0, int nb, char* ws) {
  Group g;
  g.b0 = b0; g.nb = nb;
  const int64_t r0 = (int64_t)b0 * d->W;
  const int64_t esz = d->kv_bf16 ? 2 : 4;
  g.tokens = d->tokens + r0;
  g.pos = d->pos + b0;
  g.prev_raw = d->prev_raw + (int64_t)b0 * d->D;
  g.cand_raw = d->cand_raw + (int64_t)b0 * d->D;
  g.kv = (char*)d->kv + (int64_t)b0 * 2 * d->Hkv * d->max_len * HD * esz;
  g.logits = d->logits + r0 * d->V;
  g.probs = d->probs ? d->probs + r0 * d->V : nullptr;
  g.cum = d->cum ? d->cum + r0 * (d->V + 1) : nullptr;
  carve(d, nb, &g.w, ws);
  return g;
}

template <int AM>
struct StepRun {
  const AltxsStepDesc* d;
  static constexpr int hb16 = AM == A_BF16 ? 1 : 0;

  // row-local XCD placement for this group's launches
  bool xr(const Group& G) const {
    const int R = G.nb * d->W;
    return d->W == 1 && R % 64 == 0 && R <= kXcdRowsMax && xcd_rows_on();
  }

  hipError_t embed(const Group& G, hipStream_t st) const {
    const WS& w = G.w;
    EmbedP p;
    p.emb = qt_of(d->emb); p.bits = d->emb.bits; p.V = d->V; p.D = d->D; p.W = d->W;
    p.gw = d->gate_window; p.smear = (d->flags & ALTXS_F_SMEAR) ? 1 : 0; p.eps = d->norm_eps;
    p.tokens = G.tokens; p.prev_raw = G.prev_raw; p.cand_raw = G.cand_raw;
    p.smear_w = d->smear_w; p.smear_lambda = d->smear_lambda; p.x0 = w.X0; p.err = d->err;
    p.sync = w.SYNC; p.nsync = w.nsync;
    p.mix0 = d->layers[d->slots[0].layer].resid_mix; p.xin0 = w.XIN;
    p.R = G.nb * d->W;
    // many rows: four per workgroup (cfg4: 0.68 ms with one-wave workgroups)
    const int rpw = p.R >= 4096 ? 4 : 1;
    p.xcd_rows = (rpw == 1 && xr(G)) ? 1 : 0;
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)((p.R + rpw - 1) / rpw)), dim3(64 * rpw), 0, st, p);
    return hipGetLastError();
  }

  // QKV of slot s: RMSNorm * ln_scale of the attention input (+ sparse-gate
  // multipliers) in the prologue; QK-RMS, RoPE, q_gain and the K/V write in the
  // epilogue.
  void qkv_parts(const Group& G, int s, ProNorm& pro, EpiQKV& epi) const {
    const WS& w = G.w;
    const int R = G.nb * d->W;
    const int64_t Rp = align_up(R, 16), D = d->D;
    const AltxsSlot& S = d->slots[s];
    const AltxsLayer& L = d->layers[S.layer];
    const bool par = S.kind == ALTXS_SLOT_PAR;
    const float* attn_in = par ? w.QIN + (s & 1) * Rp * D : w.XIN + (s & 1) * Rp * D;
    pro = ProNorm{attn_in, nullptr, 0, L.ln_scale, d->norm_eps, d->D};
    pro.gate_w = (d->flags & ALTXS_F_SPARSE_GATE) ? L.attn_gate_w : nullptr;
    pro.gate_out = w.GATE; pro.gate_scale = d->gate_scale; pro.H = d->H; pro.gw = d->gate_window;
    epi = EpiQKV{};
    epi.q = w.Q; epi.kv = slot_kv(G, s); epi.kv_bf16 = d->kv_bf16; epi.H = d->H; epi.Hkv = d->Hkv;
    epi.W = d->W; epi.max_len = d->max_len; epi.rd = d->rope_dims; epi.pos = G.pos;
    epi.kv_tail = d->kv_tail_end > 0 ? d->kv_tail_end - d->W : -1;
    epi.cosb = d->rope_cos; epi.sinb = d->rope_sin; epi.q_gain = L.q_gain; epi.eps = d->norm_eps;
    epi.err = d->err;
    if (S.lora_q_a) {
      epi.lqa = S.lora_q_a; epi.lqb = S.lora_q_b; epi.lva = S.lora_v_a; epi.lvb = S.lora_v_b;
      epi.lora_s = S.lora_scale; epi.rank = d->lora_rank;
    }
    epi.D = d->D; epi.a_f32 = AM == A_F32 ? 1 : 0;
  }

  hipError_t qkv(const Group& G, int s, hipStream_t st) const {
    const WS& w = G.w;
    const int R = G.nb * d->W;
    const AltxsSlot& S = d->slots[s];
    const AltxsLayer& L = d->layers[S.layer];
    ProNorm pro{};
    EpiQKV epi{};
    qkv_parts(G, s, pro, epi);
    if (big(R, L.qkv) && !S.lora_q_a) {
      const QT q = qt_big(L.qkv);
      if (band_norm_fits(q)) return launch_gemm_band_norm<4, 1>(q.bits, q, R, pro, epi, st);
      // normalised rows in Y (free until the attention)
      hipError_t e = launch_norm_rows(pro, R, d->D, (uint16_t*)w.Y, st);
      if (e != hipSuccess) return e;
      return launch_gemm_big<4, 1>(q.bits, q, R, (const uint16_t*)w.Y, epi, st);
    }
    // fp32 rows: staged pre-split (A_F32S) unless the LoRA epilogue reads them
    if constexpr (AM == A_F32) {
      if (!S.lora_q_a)
        return launch_gemm_bits<A_F32S, 4, 1>(L.qkv.bits, qt_of(L.qkv), R, 1, 0, 0, ADirect{nullptr, 0},
                                              pro, epi, 0, st);
    }
    return launch_gemm_bits<AM, 4, 1>(L.qkv.bits, qt_of(L.qkv), R, 1, 0, 0, ADirect{nullptr, 0},
                                      pro, epi, 0, st);
  }

  // The large-tile GEMMs apply (bf16 activations, many rows, a tileable shape).
  bool big(int R, const AltxsQTensor& t) const {
    return AM == A_BF16 && R >= kBigRows && big_gemm_fits(qt_of(t));
  }

  char* slot_kv(const Group& G, int s) const {
    const int64_t esz = d->kv_bf16 ? 2 : 4;
    return G.kv + (int64_t)s * d->B * 2 * d->Hkv * d->max_len * HD * esz;
  }

  AltxsAttnArgs attn_args(const Group& G, int s) const {
    const WS& w = G.w;
    const AltxsLayer& L = d->layers[d->slots[s].layer];
    const int64_t esz = d->kv_bf16 ? 2 : 4;
    char* kv = slot_kv(G, s);
    AltxsAttnArgs a;
    memset(&a, 0, sizeof(a));
    a.B = G.nb; a.W = d->W; a.H = d->H; a.Hkv = d->Hkv; a.head_dim = HD; a.max_len = d->max_len;
    a.kv_bf16 = d->kv_bf16; a.y_bf16 = hb16; a.q = w.Q;
    a.k = kv; a.v = kv + (int64_t)d->Hkv * d->max_len * HD * esz;
    a.kv_seg_stride = 2ll * d->Hkv * d->max_len * HD; a.pos = G.pos;
    a.gate = (d->flags & ALTXS_F_SPARSE_GATE) ? w.GATE : nullptr;
    a.use_xsa = L.use_xsa; a.y = w.Y; a.err = d->err;
    a.flags = (AM == A_BF16 ? ALTXS_ATTN_OPS_BF16 : 0) | (xr(G) ? ALTXS_ATTN_XCD_ROWS : 0);
    a.kv_tail_end = d->kv_tail_end;
    return a;
  }

  bool fuse_o(const Group& G, int s) const { return out_proj_fused(d, s, G.nb * d->W); }
  OutFin out_fin(const AltxsLayer& L) const {
    OutFin f;
    f.osc = (const uint16_t*)L.o.scales; f.attn_scale = L.attn_scale; f.H = d->H; f.ks = pick_ks(L.o.K, kKsO);
    return f;
  }

  hipError_t attn(const Group& G, int s, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) const {
    const AltxsAttnArgs a = attn_args(G, s);
    hipError_t e;
    if (ev0 && (e = hipEventRecord(ev0, st)) != hipSuccess) return e;
    if (fuse_o(G, s)) {
      const AltxsQTensor& o = d->layers[d->slots[s].layer].o;
      if ((e = altxs_launch_attn_o(a, (const uint8_t*)o.codes, o.bits, d->D, G.w.OPART, st)) != hipSuccess)
        return e;
    } else if ((e = altxs_launch_attn(a, st)) != hipSuccess) {
      return e;
    }
    if (ev1 && (e = hipEventRecord(ev1, st)) != hipSuccess) return e;
    return hipSuccess;
  }

  // O, UP, DOWN of slot s (DOWN also forms slot s+1's inputs)
  hipError_t mlp(const Group& G, int s, hipStream_t st) const {
    const WS& w = G.w;
    const int R = G.nb * d->W;
    const int64_t Rp = align_up(R, 16), D = d->D;
    const AltxsSlot& S = d->slots[s];
    const AltxsLayer& L = d->layers[S.layer];
    const bool par = S.kind == ALTXS_SLOT_PAR;
    float* xin_slot = w.X0 + s * Rp * D;           // x or lane0 entering the slot
    const float* lane1_in = par ? (S.first_parallel ? xin_slot : w.X1 + s * Rp * D) : nullptr;
    float* base_s = w.XIN + (s & 1) * Rp * D;      // x_in (seq) / lane0 after skip (par)
    hipError_t e;
    const bool fo = fuse_o(G, s);
    if (!fo) {  // out-projection + attention residual
      EpiO epi{base_s, L.attn_scale, w.XOUT, d->D, par ? 1 : 0};
      if (big(R, L.o))
        e = launch_gemm_big4(kKsO, qt_big(L.o).bits, qt_big(L.o), R, (const uint16_t*)w.Y, epi, st);
      else
        // two K-slices (K = 512) on one 16-column block per task: twice the
        // workgroups of (2, 2) at half the size, same per-block arithmetic, so
        // the same bits (cfg3 0.669 -> 0.665 ms); the prologue-free epilogue
        // allows two-wave tasks
        e = pick_ks(L.o.K, kKsO) == 2
                ? launch_gemm_bits<AM, 1, 2>(L.o.bits, qt_of(L.o), R, 1, 0, 0, ADirect{w.Y, 0}, ProNone{}, epi,
                                             0, st, xr(G))
                : launch_gemm4<AM>(kKsO, L.o.bits, qt_of(L.o), R, ADirect{w.Y, 0}, ProNone{}, epi, 0, st, xr(G));
      if (e != hipSuccess) return e;
    }
    {  // MLP up + LeakyReLU(0.5)^2
      ProNorm pro{par ? lane1_in : w.XOUT, nullptr, 0, L.ln_scale, d->norm_eps, d->D};
      EpiUp epi{w.HB, d->F, hb16};
      if (fo && !par) {  // sequential slot: the out-projection finished in the prologue
        if constexpr (AM == A_BF16) {
          ProOutNorm po{out_fin(L), base_s, w.XOUT, L.ln_scale, d->norm_eps, d->D};
          po.of.part = w.OPART;
          e = launch_gemm4<AM>(kKsUp, L.up.bits, qt_of(L.up), R, ADirect{nullptr, 0}, po, epi, 0, st, xr(G));
        } else {
          e = hipErrorInvalidValue;
        }
      } else if (big(R, L.up) && band_norm_fits(qt_of(L.up))) {
        e = launch_gemm_band_norm4(kKsUp, qt_big(L.up).bits, qt_big(L.up), R, pro, epi, st);
      } else if (big(R, L.up)) {  // normalised rows in Y (the out-projection has read it)
        if ((e = launch_norm_rows(pro, R, d->D, (uint16_t*)w.Y, st)) != hipSuccess) return e;
        e = launch_gemm_big4(kKsUp, qt_big(L.up).bits, qt_big(L.up), R, (const uint16_t*)w.Y, epi, st);
      } else {
        e = launch_gemm4<AM == A_F32 ? A_F32S : AM>(kKsUp, L.up.bits, qt_of(L.up), R, ADirect{nullptr, 0},
                                                    pro, epi, 0, st, xr(G));
      }
      if (e != hipSuccess) return e;
    }
    {  // MLP down + residual / lanes
      auto fill = [&](auto& epi) {
        epi.xout = w.XOUT; epi.mlp_scale = L.mlp_scale;
        epi.out0 = w.X0 + (s + 1) * Rp * D; epi.out1 = w.X1 + (s + 1) * Rp * D;
        epi.lane0 = base_s; epi.lane1 = lane1_in; epi.pr = L.par_resid; epi.pp = L.par_post;
        epi.D = d->D; epi.parallel = par ? 1 : 0;
        if (s + 1 < d->n_slots) {  // the next slot's residual base and attention input
          const AltxsSlot& S1 = d->slots[s + 1];
          const bool par1 = S1.kind == ALTXS_SLOT_PAR;
          NextIn& nx = epi.next;
          nx.x0 = w.X0;
          nx.skip = S1.skip_src >= 0 ? w.X0 + (S1.skip_src + 1) * Rp * D : nullptr;
          nx.skip_w = S1.skip_src >= 0 ? d->skip_weights + (int64_t)S1.skip_idx * D : nullptr;
          nx.skip_g = (S1.skip_src >= 0 && (d->flags & ALTXS_F_SKIP_GATES) && d->skip_gates)
                          ? d->skip_gates + (int64_t)S1.skip_idx * D : nullptr;
          nx.mix = d->layers[S1.layer].resid_mix;
          nx.base = w.XIN + ((s + 1) & 1) * Rp * D;
          nx.attn = par1 ? w.QIN + ((s + 1) & 1) * Rp * D : nx.base;
          nx.parallel = par1 ? 1 : 0;
          nx.skip_self = S1.skip_src == s ? 1 : 0;
        }
      };
      if (fo && par) {  // parallel slot: the attention term from the out-projection's terms
        if constexpr (AM == A_BF16) {
          EpiDownT<true> epi;
          fill(epi);
          epi.ofin = out_fin(L);
          epi.ofin.part = w.OPART;
          e = launch_gemm4<AM>(kKsDown, L.down.bits, qt_of(L.down), R, ADirect{w.HB, 0}, ProNone{},
                               epi, 0, st, xr(G));
        } else {
          e = hipErrorInvalidValue;
        }
      } else {
        EpiDown epi;
        fill(epi);
        if (big(R, L.down))
          e = launch_gemm_big4(kKsDown, L.down.bits, qt_of(L.down), R, (const uint16_t*)w.HB, epi, st);
        else
          e = launch_gemm4<AM>(kKsDown, L.down.bits, qt_of(L.down), R, ADirect{w.HB, 0}, ProNone{},
                               epi, 0, st, xr(G));
      }
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }

  // final norm + LM head + softcap, softmax -> CDF, commit
  hipError_t head(const Group& G, hipStream_t st) const {
    const WS& w = G.w;
    const int R = G.nb * d->W;
    const int64_t Rp = align_up(R, 16), D = d->D;
    const bool fast_cdf = !(d->flags & ALTXS_F_RENORM) && d->V % 64 == 0;
    hipError_t e;
    // the one-row-per-workgroup CDF forms its row statistics itself; only the
    // chunked CDF (other vocabularies) reads the LM head's tile statistics
    const bool tile_stats = fast_cdf && G.cum && !altxs_cdf_rows_kernel(R, d->V);
    {
      const int n = d->n_slots, fm = final_mode(d);
      const float* xf = (fm == 2 ? w.X1 : w.X0) + n * Rp * D;
      ProNorm pro{xf, fm == 1 ? w.X1 + n * Rp * D : nullptr, fm == 1 ? 1 : 0, 1.0f, d->norm_eps, d->D};
      EpiLogits epi{G.logits, tile_stats ? w.STATS : nullptr, d->V,
                    (d->flags & ALTXS_F_ASYM_SOFTCAP) ? 1 : 0, d->logit_softcap, d->softcap_pn};
      if (big(R, d->emb) && band_norm_fits(qt_of(d->emb))) {
        e = launch_gemm_band_norm<4, 1>(d->emb.bits, qt_of(d->emb), R, pro, epi, st);
      } else if (big(R, d->emb)) {
        if ((e = launch_norm_rows(pro, R, d->D, (uint16_t*)w.Y, st)) != hipSuccess) return e;
        e = launch_gemm_big<4, 1>(d->emb.bits, qt_of(d->emb), R, (const uint16_t*)w.Y, epi, st);
      } else {
        e = launch_gemm_bits<AM == A_F32 ? A_F32S : AM, 4, 1>(d->emb.bits, qt_of(d->emb), R, 1, 0, 0,
                                                              ADirect{nullptr, 0}, pro, epi, kLmHeadColWgs, st);
      }
      if (e != hipSuccess) return e;
    }
    if (G.probs || G.cum) {
      if (fast_cdf && G.cum) {
        if ((e = altxs_launch_cdf_stats(G.logits, tile_stats ? w.STATS : nullptr, R, d->V, G.probs,
                                        G.cum, st, xr(G))) != hipSuccess)
          return e;
      } else {
        const int fl = (d->flags & ALTXS_F_RENORM) ? ALTXS_CDF_RENORM : 0;
        if ((e = altxs_launch_cdf(G.logits, R, d->V, fl, true, G.probs, G.cum, st)) != hipSuccess)
          return e;
      }
    }
    if (d->flags & ALTXS_F_COMMIT) {
      hipLaunchKernelGGL(commit_kernel, dim3(G.nb), dim3(256), 0, st, G.pos, G.prev_raw,
                         (const float*)G.cand_raw, G.nb, d->D, d->W);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return hipSuccess;
  }
};

// ---- persistent layer kernel -------------------------------------------------

bool persist_ok(const AltxsStepDesc* d) {
  for (int l = 0; l < d->n_layers; ++l) {  // the layer kernel decodes packed widths only
    const AltxsLayer& L = d->layers[l];
    if (L.qkv.bits > 6 || L.o.bits > 6 || L.up.bits > 6 || L.down.bits > 6) return false;
  }
  return d->kv_bf16 == ALTXS_KV_BF16 && d->kv_tail_end == 0 && 16 % d->W == 0 && !split_mode(d);
}
int64_t plan_slots_off() { return align_up((int64_t)sizeof(PersistArgs), 256); }
int64_t plan_bytes_of(const AltxsStepDesc* d) {
  return plan_slots_off() + (int64_t)d->n_slots * (int64_t)sizeof(SlotPlan);
}

// Field-by-field copies into the zeroed plan image: struct assignment would
// also copy padding bytes, and the image is compared byte-wise.
void put_qt(QT& q, const AltxsQTensor& t) {
  q.codes = (const uint8_t*)t.codes;
  q.scales = (const uint16_t*)t.scales;
  q.N = (int)t.N;
  q.K = (int)t.K;
  q.bits = t.bits;
}
void put_ws(WS& o, const WS& w) {
  o.X0 = w.X0; o.X1 = w.X1; o.XIN = w.XIN; o.QIN = w.QIN; o.XOUT = w.XOUT; o.Q = w.Q;
  o.GATE = w.GATE; o.Y = w.Y; o.HB = w.HB; o.STATS = w.STATS; o.SYNC = w.SYNC; o.nsync = w.nsync;
}

// The plan image (host bytes) of the single-group step whose device copy is at dev.
void fill_plan(const AltxsStepDesc* d, const Group& G, char* host, const char* dev) {
  memset(host, 0, (size_t)plan_bytes_of(d));
  PersistArgs& a = *(PersistArgs*)host;
  SlotPlan* sp = (SlotPlan*)(host + plan_slots_off());
  const int R = G.nb * d->W;
  const int64_t Rp = align_up(R, 16), D = d->D;
  a.plan = (const SlotPlan*)(dev + plan_slots_off());
  a.n_slots = d->n_slots; a.R = R; a.W = d->W; a.D = d->D; a.H = d->H; a.Hkv = d->Hkv;
  a.F = d->F; a.max_len = d->max_len; a.rd = d->rope_dims; a.gw = d->gate_window;
  a.flags = d->flags & ALTXS_F_SPARSE_GATE;  // the only flag the layer tasks read
  a.G = d->H / d->Hkv; a.eps = d->norm_eps; a.gate_scale = d->gate_scale;
  a.nrt = (int)(Rp / 16);
  const int ncol_o = 16 * (4 / pick_ks(d->D, kKsO)), ncol_d = 16 * (4 / pick_ks(d->F, kKsDown));
  a.n_task[ST_QKV] = (d->D + 2 * d->Hkv * HD + 63) / 64;
  a.n_task[ST_ATT] = 16 * d->Hkv;
  a.n_task[ST_O] = (d->D + ncol_o - 1) / ncol_o;
  a.n_task[ST_UP] = (d->F + ncol_o - 1) / ncol_o;
  a.n_task[ST_DOWN] = (d->D + ncol_d - 1) / ncol_d;
  a.pos = G.pos; a.kv = G.kv;
  a.slot_kv_bytes = (int64_t)d->B * 2 * d->Hkv * d->max_len * HD * 2;
  a.rope_cos = d->rope_cos; a.rope_sin = d->rope_sin;
  put_ws(a.w, G.w);
  a.done = G.w.SYNC + kTicketPad;
  a.ctr_stride = kCtrStride;
  a.err = d->err;
  a.ng = persist_gemm_workers();
  a.gblock = a.n_task[ST_O] + a.n_task[ST_UP] + a.n_task[ST_DOWN] + a.n_task[ST_QKV];
  a.n_gtask = a.gblock * (a.n_slots + 1) * a.nrt;
  a.n_atask = a.n_task[ST_ATT] * a.n_slots * a.nrt;
  a.role_ctr = G.w.SYNC;
  a.gticket = G.w.SYNC + 16;
  a.aticket = G.w.SYNC + 32;
  for (int s = 0; s < d->n_slots; ++s) {
    const AltxsSlot& S = d->slots[s];
    const AltxsLayer& L = d->layers[S.layer];
    SlotPlan& P = sp[s];
    put_qt(P.qkv, L.qkv); put_qt(P.o, L.o); put_qt(P.up, L.up); put_qt(P.down, L.down);
    P.resid_mix = L.resid_mix; P.attn_scale = L.attn_scale; P.mlp_scale = L.mlp_scale;
    P.q_gain = L.q_gain; P.gate_w = L.attn_gate_w; P.par_resid = L.par_resid;
    P.par_post = L.par_post; P.ln_scale = L.ln_scale; P.use_xsa = L.use_xsa;
    P.par = S.kind == ALTXS_SLOT_PAR ? 1 : 0;
    P.first_parallel = S.first_parallel;
    if (S.lora_q_a) {
      P.lqa = S.lora_q_a; P.lqb = S.lora_q_b; P.lva = S.lora_v_a; P.lvb = S.lora_v_b;
      P.lora_s = S.lora_scale; P.lora_rank = d->lora_rank;
    }
    P.has_next = s + 1 < d->n_slots ? 1 : 0;
    if (P.has_next) {
      const AltxsSlot& S1 = d->slots[s + 1];
      P.next_par = S1.kind == ALTXS_SLOT_PAR ? 1 : 0;
      P.next_skip_src = S1.skip_src;
      P.next_skip_self = S1.skip_src == s ? 1 : 0;
      P.next_mix = d->layers[S1.layer].resid_mix;
      P.next_skip_w = S1.skip_src >= 0 ? d->skip_weights + (int64_t)S1.skip_idx * D : nullptr;
      P.next_skip_g = (S1.skip_src >= 0 && (d->flags & ALTXS_F_SKIP_GATES) && d->skip_gates)
                          ? d->skip_gates + (int64_t)S1.skip_idx * D : nullptr;
    } else {
      P.next_skip_src = -1;
    }
  }
}

// embed -> one persistent launch for every slot -> head.
template <int AM>
hipError_t run_persist(const AltxsStepDesc* d, const Group& G, hipStream_t st) {
  StepRun<AM> run{d};
  hipError_t e;
  hipEvent_t* ev = (hipEvent_t*)d->attn_events;
  const PersistArgs& a = *(const PersistArgs*)d->plan_host;
  if ((e = run.embed(G, st)) != hipSuccess) return e;
  if (ev && (e = hipEventRecord(ev[0], st)) != hipSuccess) return e;
  if ((e = launch_persist(a, (const PersistArgs*)d->plan_dev, AM == A_BF16 ? 1 : 0,
                          pick_ks(d->D, kKsO), pick_ks(d->F, kKsDown), 0, st)) != hipSuccess)
    return e;
  if (ev && (e = hipEventRecord(ev[1], st)) != hipSuccess) return e;
  return run.head(G, st);
}

// One group on one stream.
template <int AM>
hipError_t run_single(const AltxsStepDesc* d, const Group& G, hipStream_t st) {
  StepRun<AM> run{d};
  hipError_t e;
  hipEvent_t* ev = (hipEvent_t*)d->attn_events;
  if ((e = run.embed(G, st)) != hipSuccess) return e;
  for (int s = 0; s < d->n_slots; ++s) {
    if ((e = run.qkv(G, s, st)) != hipSuccess) return e;
    if ((e = run.attn(G, s, st, ev ? ev[2 * s] : nullptr, ev ? ev[2 * s + 1] : nullptr)) != hipSuccess)
      return e;
    if ((e = run.mlp(G, s, st)) != hipSuccess) return e;
  }
  return run.head(G, st);
}

// Two segment groups on two streams, each group's whole step a chain of its
// own: the only cross-stream edges are the fork (group 1 starts once group
// 0's slot-0 QKV is done, so the two chains run about half a slot apart and
// one group's GEMM stages overlap the other's attention) and the join.  Every
// kernel computes a row from that row's inputs only, so the split changes no
// bits.  (Alternating the attention launches with two event edges per slot
// measured 0.82 ms on cfg3; this form 0.68 ms; one group 0.70 ms.)
template <int AM>
hipError_t run_split(const AltxsStepDesc* d, const Group (&G)[2], hipStream_t s0, hipStream_t s1) {
  StepRun<AM> run{d};
  hipEvent_t* sync = (hipEvent_t*)d->sync_events;  // [0] fork, [1] join
  hipEvent_t* ev = (hipEvent_t*)d->attn_events;    // timing hook: [(g*n + s)*2 + 0/1]
  const hipStream_t st[2] = {s0, s1};
  const int n = d->n_slots;
  const int fork = split_fork_stage();
  hipError_t e;
  for (int g = 0; g < 2; ++g) {
    if (g == 1 && (e = hipStreamWaitEvent(s1, sync[0], 0)) != hipSuccess) return e;
    if ((e = run.embed(G[g], st[g])) != hipSuccess) return e;
    for (int s = 0; s < n; ++s) {
      const bool fk = g == 0 && s == 0;
      const int k = (g * n + s) * 2;
      hipEvent_t e0 = ev ? ev[k] : nullptr, e1 = ev ? ev[k + 1] : nullptr;
      if ((e = run.qkv(G[g], s, st[g])) != hipSuccess) return e;
      if (fk && fork == 0 && (e = hipEventRecord(sync[0], s0)) != hipSuccess) return e;
      if ((e = run.attn(G[g], s, st[g], e0, e1)) != hipSuccess) return e;
      if (fk && fork == 1 && (e = hipEventRecord(sync[0], s0)) != hipSuccess) return e;
      if ((e = run.mlp(G[g], s, st[g])) != hipSuccess) return e;
      if (fk && fork >= 2 && (e = hipEventRecord(sync[0], s0)) != hipSuccess) return e;
    }
    if ((e = run.head(G[g], st[g])) != hipSuccess) return e;
  }
  if ((e = hipEventRecord(sync[1], s1)) != hipSuccess) return e;
  return hipStreamWaitEvent(s0, sync[1], 0);
}

}  // namespace

extern "C" int64_t altxs_step_workspace_bytes(const AltxsStepDesc* d) {
  if (!d) return -1;
  return ws_bytes_needed(d);
}

extern "C" int32_t altxs_step_fuses_out_proj(const AltxsStepDesc* d, int32_t slot) {
  if (!d || slot < 0 || slot >= d->n_slots || d->n_slots > ALTXS_MAX_SLOTS) return -1;
  const int nb0 = (d->B + 1) / 2;
  return out_proj_fused(d, slot, split_mode(d) ? nb0 : d->B * d->W) ? 1 : 0;
}

extern "C" int64_t altxs_step_plan_bytes(const AltxsStepDesc* d) {
  if (!d || d->n_slots < 1 || d->n_slots > ALTXS_MAX_SLOTS) return -1;
  return plan_bytes_of(d);
}

extern "C" int32_t altxs_step_plan_build(const AltxsStepDesc* d, void* plan_host, void* plan_dev,
                                         int64_t bytes, altxs_stream_t stream) {
  int rc = validate(d);
  if (rc) return rc;
  ALTXS_REQUIRE(plan_host && plan_dev, "altxs_step_plan_build: null plan buffer");
  ALTXS_REQUIRE(bytes >= plan_bytes_of(d), "altxs_step_plan_build: %lld bytes < %lld",
                (long long)bytes, (long long)plan_bytes_of(d));
  ALTXS_REQUIRE(persist_ok(d),
                "altxs_step_plan_build: the persistent kernel needs a tiled bf16 KV cache (no tail rows), W dividing 16 "
                "and one stream");
  const Group G = make_group(d, 0, d->B, (char*)d->ws);
  fill_plan(d, G, (char*)plan_host, (const char*)plan_dev);
  hipStream_t st = (hipStream_t)stream;
  ALTXS_CHECK_HIP(hipMemcpyAsync(plan_dev, plan_host, (size_t)plan_bytes_of(d), hipMemcpyHostToDevice, st));
  ALTXS_CHECK_HIP(hipStreamSynchronize(st));
  return ALTXS_OK;
}

extern "C" int32_t altxs_step(const AltxsStepDesc* d, altxs_stream_t stream) {
  int rc = validate(d);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (d->plan_dev) {
    ALTXS_REQUIRE(d->plan_host && d->plan_bytes >= plan_bytes_of(d),
                  "altxs_step: plan_dev needs plan_host and plan_bytes");
    ALTXS_REQUIRE(persist_ok(d),
                  "altxs_step: the persistent kernel needs a tiled bf16 KV cache (no tail rows), W dividing 16 and one stream");
    const Group G = make_group(d, 0, d->B, (char*)d->ws);
    static thread_local std::vector<char> img;
    img.resize((size_t)plan_bytes_of(d));
    fill_plan(d, G, img.data(), (const char*)d->plan_dev);
    ALTXS_REQUIRE(memcmp(img.data(), d->plan_host, img.size()) == 0,
                  "altxs_step: the plan was built for other pointers or shapes; rebuild it");
    e = d->act_bf16 ? run_persist<A_BF16>(d, G, st) : run_persist<A_F32>(d, G, st);
    ALTXS_CHECK_HIP(e);
    return ALTXS_OK;
  }
  if (split_mode(d)) {
    const int nb0 = (d->B + 1) / 2;
    Group G[2] = {make_group(d, 0, nb0, (char*)d->ws),
                  make_group(d, nb0, d->B - nb0, (char*)d->ws + carve(d, nb0, nullptr, nullptr))};
    hipStream_t s1 = (hipStream_t)d->aux_stream;
    e = d->act_bf16 ? run_split<A_BF16>(d, G, st, s1) : run_split<A_F32>(d, G, st, s1);
  } else {
    const Group G = make_group(d, 0, d->B, (char*)d->ws);
    e = d->act_bf16 ? run_single<A_BF16>(d, G, st) : run_single<A_F32>(d, G, st);
  }
  ALTXS_CHECK_HIP(e);
  return ALTXS_OK;
}

// ---- normalised-rows GEMM: y = (RMSNorm(x) * ln_scale) . W^T ----------------
// The step's LM-head prologue (ProNorm) with a plain store: the standalone form
// of logits_stage_rows (final RMS -> LM projection, ac_gemv.py:562-582).

extern "C" int32_t altxs_rms_qgemm(const AltxsQTensor* w, const float* x, int64_t rows, float ln_scale,
                                   float eps, int32_t act_bf16, float* y, altxs_stream_t stream) {
  ALTXS_REQUIRE((act_bf16 & ~(ALTXS_RMS_ROUND_ROW | ALTXS_RMS_ROUND_SCALE)) == 0,
                "altxs_rms_qgemm: unknown rounding flags 0x%x", act_bf16);
  ALTXS_REQUIRE(w && w->codes && (w->bits == 16 || w->bits == 32 || w->scales), "altxs_rms_qgemm: null tensor");
  ALTXS_REQUIRE(w->bits == 2 || w->bits == 3 || w->bits == 4 || w->bits == 6 || w->bits == 16 || w->bits == 32,
                "altxs_rms_qgemm: bits=%d", w->bits);
  ALTXS_REQUIRE(w->bits != 32 || !(act_bf16 & ALTXS_RMS_ROUND_ROW),
                "altxs_rms_qgemm: fp32 weights (bits 32) take an fp32 row");
  ALTXS_REQUIRE(w->N > 0 && w->N % 16 == 0 && w->N < (1 << 24), "altxs_rms_qgemm: N=%lld",
                (long long)w->N);
  ALTXS_REQUIRE(w->K == 256 || w->K == 512, "altxs_rms_qgemm: K=%lld must be 256 or 512",
                (long long)w->K);
  ALTXS_REQUIRE(((uintptr_t)w->codes & 15) == 0 && ((uintptr_t)w->scales & 7) == 0,
                "altxs_rms_qgemm: misaligned tensor");
  ALTXS_REQUIRE(x && y && ((uintptr_t)x & 15) == 0, "altxs_rms_qgemm: x must be 16-byte aligned");
  ALTXS_REQUIRE(rows >= 1 && rows <= (1 << 20), "altxs_rms_qgemm: rows=%lld", (long long)rows);
  ProNorm pro{x, nullptr, 0, ln_scale, eps, (int)w->K};
  pro.round_scale = (act_bf16 & ALTXS_RMS_ROUND_SCALE) ? 1 : 0;
  EpiStore epi{y, (int)w->N, 0};
  const QT q = qt_of(*w);
  hipStream_t st = (hipStream_t)stream;
  const hipError_t e =
      (act_bf16 & ALTXS_RMS_ROUND_ROW)
               ? launch_gemm_bits<A_BF16, 4, 1>(w->bits, q, (int)rows, 1, 0, 0, ADirect{nullptr, 0}, pro,
                                                  epi, 0, st)
               : launch_gemm_bits<A_F32, 4, 1>(w->bits, q, (int)rows, 1, 0, 0, ADirect{nullptr, 0}, pro,
                                                 epi, 0, st);
  ALTXS_CHECK_HIP(e);
  return ALTXS_OK;
}

// ---- allocation-free step: the workspace is a file-scope device array -------
//
// Each GPU that runs altxs_step_noalloc holds its own copy of `scratch` until
// the process ends.  Host code never passes the array's name to a kernel (on
// the host it is only a stand-in symbol); it passes the per-device address
// hipGetSymbolAddress returns, looked up once per device with that device
// current.

namespace {

__device__ __align__(256) char scratch[ALTXS_STEP_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];  // guarded by g_scratch_mu

int scratch_for_stream(hipStream_t st, void** out) {
  int cur = -1;
  ALTXS_CHECK_HIP(hipGetDevice(&cur));
  hipDevice_t dev = cur;
  if (st) ALTXS_CHECK_HIP(hipStreamGetDevice(st, &dev));
  ALTXS_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, "altxs_step_noalloc: device %d out of range",
                (int)dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    if (dev != cur) ALTXS_CHECK_HIP(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) ALTXS_CHECK_HIP(hipSetDevice(cur));
    ALTXS_CHECK_HIP(e);
    ALTXS_REQUIRE(p != nullptr, "altxs_step_noalloc: no scratch address on device %d", (int)dev);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ALTXS_OK;
}

}  // namespace

extern "C" int32_t altxs_step_noalloc(const AltxsStepDesc* d, altxs_stream_t stream) {
  ALTXS_REQUIRE(d, "altxs_step_noalloc: null descriptor");
  ALTXS_REQUIRE(!d->plan_dev,
                "altxs_step_noalloc: the persistent plan points at a caller workspace; use altxs_step");
  const int64_t need = ws_bytes_needed(d);
  ALTXS_REQUIRE(need <= (int64_t)ALTXS_STEP_SCRATCH_BYTES,
                "altxs_step_noalloc: this step needs %lld workspace bytes, more than the %lld-byte "
                "static scratch; use altxs_step with a caller workspace",
                (long long)need, (long long)ALTXS_STEP_SCRATCH_BYTES);
  void* ws = nullptr;
  int rc = scratch_for_stream((hipStream_t)stream, &ws);
  if (rc) return rc;
  AltxsStepDesc dd = *d;  // the caller's descriptor with the scratch as workspace
  dd.ws = ws;
  dd.ws_bytes = ALTXS_STEP_SCRATCH_BYTES;
  return altxs_step(&dd, stream);
}
