/*
 * altxs.h -- C-ABI of libaltxs_hip.so, the MI355X (gfx950) implementation of
 * the altxs per-symbol model step.
 *
 * All pointers are device pointers unless stated otherwise; sizes are element
 * counts.  Every entry point enqueues work on `stream` (a hipStream_t passed as
 * void*; NULL = the legacy default stream), never allocates, never synchronises
 * (except the set-up call altxs_step_plan_build, which waits for its copy),
 * and returns ALTXS_OK (0) or a negative ALTXS_ERR_* code.  The
 * message for the last failure on the calling thread is altxs_last_error().
 * Runtime values that live in device memory (positions, token ids) cannot be
 * checked on the host; kernels skip out-of-range accesses and OR a code into
 * the caller's device error word instead of faulting.
 *
 * Reference citations are path:line into altvectra/altxs.
 */
#ifndef ALTXS_H
#define ALTXS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ALTXS_ABI_VERSION 8

enum {
  ALTXS_OK = 0,
  ALTXS_ERR_ARG = -1,         /* bad shape / pointer / unsupported combination */
  ALTXS_ERR_HIP = -2,         /* a HIP runtime call failed */
  ALTXS_ERR_UNSUPPORTED = -3, /* feature not built */
};

/* dtype codes for activation inputs */
enum { ALTXS_F32 = 0, ALTXS_BF16 = 1, ALTXS_F16 = 2 };

typedef void *altxs_stream_t;

/* ABI version of the loaded library (== ALTXS_ABI_VERSION). */
int32_t altxs_abi_version(void);

/* Message for the last error returned on this thread ("" if none). */
const char *altxs_last_error(void);

/*
 * Packed mixed-bit weight tensor W[N, K]: symmetric group-64 quantisation
 * along K, w[n,k] = (code[n,k] - (2^bits - 1)/2) * scale[n, k/64], fp16 scales,
 * bits in {2,3,4,6} per tensor.  The math is the reference's "symmetric"
 * codebook mode (src/hyperflow_distillation/mixed_bit_delta.py:147-152,
 * 172-229) with the channel width set to a 64-wide group and b = 6 added.
 * Storage is the MFMA-tiled layout produced by altxs_amd.codec.pack_tiled:
 * 16-row x 256-column blocks; in each block every lane of a wave owns the
 * codes its v_mfma_f32_16x16x32 B operand needs, split into 4/2/1-bit planes
 * so each lane reads whole 16/8-byte words.  N % 16 == 0, K % 256 == 0.
 * Dense forms (no codes, scales unused): bits = 16 holds bf16 values in the
 * same tiled order (N*K*2 bytes); bits = 32 holds fp32 values exactly as three
 * bf16 planes hi + mid + lo (hi = bf16(w), mid = bf16(w - hi), lo = w - hi -
 * mid), the three 8 KB planes of each 16 x 256 block stored one after the
 * other (N*K*6 bytes), for the reference's fp32 compute mode; bits 32 needs
 * fp32 activations.
 */
typedef struct AltxsQTensor {
  const void *codes;  /* uint8 planes, N*K*bits/8 bytes */
  const void *scales; /* fp16, N*K/64 entries (tiled) */
  int64_t N, K;
  int32_t bits;
  int32_t reserved;
  /* Optional (NULL = none; packed widths 2/3/4/6 only): the same tensor
   * expanded by altxs_expand_codes.  In steps of at least 1024 rows (W-token
   * windows, prefill-style scoring) the QKV, out-projection and MLP-up GEMMs
   * read its values instead of decoding codes once per 64 rows: the same
   * operands, the same bits (other tensors' copies are not read). */
  const void *expanded;
} AltxsQTensor;

/*
 * probs[rows, V] (fp32) -> cum[rows, V+1] (uint32): f_i = max(1,
 * floor(double(p_i) * 1e6 + 0.5)) with two IEEE double roundings and no FMA,
 * cum_0 = 0, cum_{i+1} = cum_i + f_i.  Bit-exact with _scale_cum_np
 * (src/model/arithmetic_coder_lm.py:49-64) and the GPU coder's scale_p
 * (src/xsa_ttt/gpu_ac.py:38-42).  Requires V <= 65536.
 */
int32_t altxs_scale_cum(const float *probs, int64_t rows, int64_t V, uint32_t *cum,
                        altxs_stream_t stream);

/* The same tables from float64 probabilities (the reference's _scale_cum_np
 * converts its input to float64, arithmetic_coder_lm.py:58-60). */
int32_t altxs_scale_cum_f64(const double *probs, int64_t rows, int64_t V, uint32_t *cum,
                            altxs_stream_t stream);

#define ALTXS_CDF_RENORM 1 /* p /= sum(p) after the softmax, the sum in numpy's float32
                              order (pairwise blocks of 128, 8192-element chunks) as the
                              reference's _softmax_np computes it (compress.py:64-85);
                              a non-positive or non-finite sum gives the uniform row;
                              V <= 16384 */

/*
 * Deterministic softmax + CDF: probs = softmax(logits) in fp32 with a fixed
 * reduction order (independent of `rows`), then cum as altxs_scale_cum.
 * Replaces torch.softmax(state.logits, -1, out=probs_dev)
 * (src/xsa_ttt/incremental.py:603-605, 627-633) followed by _scale_cum_np.
 * probs or cum may be NULL.  Requires V <= 65536.
 */
int32_t altxs_softmax_cdf(const float *logits, int64_t rows, int64_t V, int32_t flags,
                          float *probs, uint32_t *cum, altxs_stream_t stream);

/* Dense fp32 copy of a packed tensor (bits in {2,3,4,6}): out[N, K].  Replaces
 * dequantize_channels (mixed_bit_delta.py:172-229) for the group-64 format. */
int32_t altxs_dequant(const AltxsQTensor *w, float *out, altxs_stream_t stream);

/* The expanded form of a packed tensor (bits in {2,3,4,6}): out holds the
 * bf16 values code - (2^bits - 1)/2 (exact), N*K*2 bytes, for
 * AltxsQTensor.expanded (scales stay the packed tensor's).  Per 16 x 256
 * block (8 KB), the 16-byte MFMA B operand of k-step s and lane l (the values
 * a bits-16 block keeps at lane l's bytes 16 s ..) sits at 16 (64 s + l).
 * No reference counterpart: a layout the large-row GEMMs read in place of
 * decoding codes. */
int32_t altxs_expand_codes(const AltxsQTensor *w, void *out, altxs_stream_t stream);

/*
 * y[rows, N] = x[rows, K] . W^T with the dequantisation fused into an MFMA
 * GEMM (fp32 accumulate).  x_dtype: ALTXS_F16 / ALTXS_BF16 (one MFMA pass) or
 * ALTXS_F32 (three-way bf16 split of x, fp32-faithful); bits 16 (dense bf16
 * weights in the tiled order, scales unused) takes fp32 or bf16 x.  Row results do not
 * depend on `rows` (batch-invariant).  Replaces gemv_rows(x, w, out)
 * (src/xsa_ttt/ac_gemv.py:391-420) and F.linear in _projection_linear
 * (src/xsa_ttt/model.py:93-111).
 */
int32_t altxs_qgemm(const AltxsQTensor *w, const void *x, int32_t x_dtype, int64_t rows,
                    float *y, altxs_stream_t stream);

/*
 * The same GEMM over `count` tensors of one shape and bit width laid out at a
 * fixed byte stride (codes_stride, scales_stride bytes) from w->codes /
 * w->scales; y is [count, rows, N].  One launch streams all of them; it is the
 * HBM microbenchmark form of altxs_qgemm (no reference counterpart).
 */
int32_t altxs_qgemm_stream(const AltxsQTensor *w, int64_t count, int64_t codes_stride,
                           int64_t scales_stride, const void *x, int32_t x_dtype,
                           int64_t rows, float *y, altxs_stream_t stream);

/*
 * y[rows, N] = x[rows, K] . W^T for 1 <= rows <= 4, each row on its own: the
 * row-independent GEMV of the reference's `_gemv_row_tiles` / gemv_rows
 * (src/xsa_ttt/ac_gemv.py:26-58, 391-425: one program per row and column
 * tile), on packed weights (bits in {2,3,4,6}) with fp16 or bf16 x.  VALU
 * arithmetic (each code decoded once into a 16-bit pair, one v_dot2 per pair
 * and row, fp32 accumulation, group centre taken out with the group's sum of
 * x), so its bits are not altxs_qgemm's; a row's result depends on that row
 * alone.  For the bandwidth-bound batch-1 regime: each weight is decoded once
 * for all rows and with ~1-2 VALU instructions.
 */
int32_t altxs_qgemv(const AltxsQTensor *w, const void *x, int32_t x_dtype, int64_t rows,
                    float *y, altxs_stream_t stream);

/* altxs_qgemv over `count` tensors at fixed byte strides (as
 * altxs_qgemm_stream); y is [count, rows, N]. */
int32_t altxs_qgemv_stream(const AltxsQTensor *w, int64_t count, int64_t codes_stride,
                           int64_t scales_stride, const void *x, int32_t x_dtype,
                           int64_t rows, float *y, altxs_stream_t stream);

/*
 * y[rows, N] = (RMSNorm(x[rows, K]) * ln_scale) . W^T: the step's normalised
 * prologue (x fp32, eps added to the mean square, one fixed reduction order
 * per row) in front of the dequant GEMM; bits in {2,3,4,6,16}, K in {256,
 * 512}.  act_bf16 holds rounding flags: ALTXS_RMS_ROUND_ROW rounds the
 * normalised row to bf16 for the MFMAs (a bf16 weight, the reference's
 * `.to(W.dtype)`), ALTXS_RMS_ROUND_SCALE first rounds the rsqrt factor to
 * bf16 (a bf16 source row: the reference's `.to(src.dtype)` of the scale);
 * 0 keeps the row fp32-faithful.  Replaces logits_stage_rows(src, weight,
 * logit_buf) (src/xsa_ttt/ac_gemv.py:312-359, 562-582).
 */
#define ALTXS_RMS_ROUND_ROW 1
#define ALTXS_RMS_ROUND_SCALE 2
int32_t altxs_rms_qgemm(const AltxsQTensor *w, const float *x, int64_t rows, float ln_scale,
                        float eps, int32_t act_bf16, float *y, altxs_stream_t stream);

/*
 * The stage-fused FFN of one slot over `win` rows, as three stream-ordered
 * launches: (1) hid = y . out_w^T; scaled = hid * a_sc; parallel: attn_s =
 * scaled, else xin += scaled.  (2) scr = leaky(RMS(src) * ln . up_w^T)^2
 * with leaky(v) = v >= 0 ? v : v / 2.  (3) hid = scr . down_w^T; mlp_s = hid
 * * m_sc; parallel: lane0 = pr0 lane0 + pp0 attn_s + pp2 mlp_s and lane1 =
 * pr1 lane1 + pp1 attn_s + pp3 mlp_s; else x = xin + mlp_s, also stored to
 * skips[skip_dst] when skip_dst >= 0.  Activations and parameters (a_sc,
 * m_sc, ln, pr, pp) share act_dtype (fp32 or bf16); each value is rounded to
 * it where the reference rounds (`.to(dtype)`, bf16 arithmetic).  Weights are
 * dense tiles (bits 16, or 32 with fp32 activations); d in {256, 512}, mlp a
 * multiple of 256 up to 8192; y and scr 16-byte aligned; hid and attn_s must
 * not alias y.  Replaces ffn_stage_rows(...) (src/xsa_ttt/ac_gemv.py:455-550;
 * stage kernels 89-310).
 */
typedef struct AltxsFfnStageArgs {
  int32_t win, d, mlp;
  int32_t act_dtype;  /* ALTXS_F32 or ALTXS_BF16 */
  int32_t parallel;   /* 1: parallel-lane slot (lane0/lane1/attn_s/pr/pp) */
  int32_t skip_dst;   /* sequential: skip buffer written with x, or -1 */
  float eps;          /* RMS epsilon of stage 2 */
  int32_t reserved;
  AltxsQTensor out_w; /* [d, d] */
  AltxsQTensor up_w;  /* [mlp, d] */
  AltxsQTensor down_w;/* [d, mlp] */
  const void *y;      /* [win, d] attention output */
  void *hid;          /* [win, d] out: stage 1's projection, then stage 3's */
  const void *a_sc;   /* [d] attn_scale */
  void *xin;          /* [win, d] sequential residual, updated by stage 1 */
  void *attn_s;       /* [win, d] parallel: scaled attention */
  const void *src;    /* [win, d] stage 2 input: xin (sequential) or lane1 */
  const void *ln;     /* [1] the layer's ln_scale_factor */
  void *scr;          /* [win, mlp] activation */
  const void *m_sc;   /* [d] mlp_scale */
  void *x;            /* [win, d] sequential: slot output */
  void *lane0;        /* [win, d] parallel lanes, updated in place */
  void *lane1;
  const void *pr;     /* [2] parallel_resid_lambdas of the layer */
  const void *pp;     /* [4] parallel_post_lambdas of the layer, [2, 2] row-major */
  void *skips;        /* [n_skips, win, d] */
} AltxsFfnStageArgs;
int32_t altxs_ffn_stage_rows(const AltxsFfnStageArgs *a, altxs_stream_t stream);

/*
 * gate[r, h] = 1 / (1 + exp(-(x[r, :gw] . w[h, :gw]))) in fp32, for r < rows,
 * h < H; x (row stride x_stride) and w share x_dtype (fp32 or bf16).  The
 * sparse-gate multiplier of the split attention's reduce step
 * (src/xsa_ttt/split_attn.py:291-303; w already carries the gate scale,
 * persistent_step.py:349-357), in the form altxs_decode_attn takes.
 */
int32_t altxs_attn_gate(const void *x, int32_t x_dtype, int64_t x_stride, const void *w, int32_t H,
                        int32_t gw, int32_t rows, float *gate, altxs_stream_t stream);

/*
 * KV cache layout.  Per (segment, kv head) the cache holds max_len keys of
 * head_dim = 64 in 64-key tiles (ALTXS_KV_TILE); max_len % 64 == 0.  The
 * kv_bf16 field of the descriptors selects one of three layouts:
 *   ALTXS_KV_F32 (0), fp32 cache: natural order, element (key, d) at key*64 + d.
 *   ALTXS_KV_BF16_NATURAL (2), bf16 cache in the same natural order: the
 *   reference's own packed layout k_pack[slot][kv_head][max_len][head_dim]
 *   (src/xsa_ttt/persistent_step.py:472-479), so a reference StaticKV can be a
 *   view of it.  Attention runs the MFMA kernel of the tiled layout on it
 *   (V tiles transposed through LDS): the same operands, the same bits.
 *   ALTXS_KV_BF16 (1), bf16 cache: each 4096-element tile is stored in MFMA operand order so one
 *   16-byte load per lane feeds v_mfma_f32_16x16x32_bf16.  For key kt = key % 64
 *   of tile key / 64 and dim d (tile base + offset):
 *     K: ((((kt>>4)*2 + (d>>5))*4 + ((d>>3)&3))*16 + (kt&15))*8 + (d&7)
 *     V: ((((kt>>5)*4 + (d>>4))*4 + ((kt>>2)&3))*16 + (d&15))*8
 *          + 4*((kt>>4)&1) + (kt&3)
 *   altxs_amd.codec.tile_kv() converts a natural [.., max_len, 64] tensor.
 */
#define ALTXS_KV_TILE 64
enum { ALTXS_KV_F32 = 0, ALTXS_KV_BF16 = 1, ALTXS_KV_BF16_NATURAL = 2 };

/*
 * Tail placement (kv_tail_end > 0, natural layouts only): the reference's
 * StaticState keeps a W-token window's K/V in the last W rows of its buffers
 * and commits them into the prefix afterwards (src/xsa_ttt/model.py:259-461:
 * StaticKV, commit_window; run_split_attn's tail_at_pos = False,
 * split_attn.py:341-425).  With kv_tail_end = E the window's token t has its
 * K/V in row E - W + t; query row t at position p = pos + t attends to the
 * prefix rows [0, pos) and then the window rows E - W .. E - W + t, in that
 * key order (the order of keys 0 .. p, so a committed row gives the same
 * result).  pos must not exceed E - W (flagged as ALTXS_EDEV_POS).
 * kv_tail_end = 0: the window's K/V sit at their own positions pos + t.
 */

/* AltxsAttnArgs.flags */
#define ALTXS_ATTN_OPS_BF16 1 /* bf16 cache: round q and the softmax weights to
                                 bf16 for the MFMA products (the reference's
                                 tl.dot arithmetic, split_attn.py:86-141);
                                 0 = fp32-faithful (3-part bf16 splits) */
#define ALTXS_ATTN_ROWS 2     /* bf16 cache, W > 1: one workgroup per row (the
                                 decode kernel) instead of the window kernel,
                                 which serves up to 64 rows of a segment per
                                 K/V read; both give the same bits */
#define ALTXS_ATTN_XCD_ROWS 4 /* one-row kernel, B*W % 64 == 0: rows in tiles
                                 of 8, tile t's workgroups on XCD t % 8 (the
                                 placement of the step's decode GEMMs, so each
                                 reads the rows the previous launch wrote from
                                 its own XCD's L2); same bits */

/*
 * Decode attention over a KV cache.  For row r = b*W + t the query sits at
 * position p = pos[b] + t and attends to keys [0, p] of segment b.  Keys are
 * scanned in fixed 64-key tiles (tile T by wave T % waves) and the per-wave
 * partials merged in wave order, so a row's result does not depend on B or W
 * (windows of a bf16 cache run up to 64 rows per workgroup with the same
 * per-row arithmetic; prefill_cache/_sdpa_with_past, model.py:679-700,
 * 1821-1947, is such a window starting at position 0).
 * Replaces run_split_attn (split_attn.py:341-425) and the eager
 * _static_window_attention (model.py:550-585).
 */
typedef struct AltxsAttnArgs {
  int32_t B, W, H, Hkv, head_dim, max_len;
  int32_t kv_bf16;  /* KV layout: ALTXS_KV_F32, ALTXS_KV_BF16 or ALTXS_KV_BF16_NATURAL */
  int32_t y_bf16;   /* output element type: 0 fp32, 1 bf16 */
  const float *q;   /* [B*W, H, head_dim] fp32 */
  const void *k;    /* [B, Hkv, max_len, head_dim] in the cache layout above,
                       seg stride kv_seg_stride elems; 16-byte aligned */
  const void *v;
  int64_t kv_seg_stride; /* elements between segments (both K and V); 0: every
                            segment reads the same cache (rows of one sequence
                            at positions pos[b]) */
  const int32_t *pos;    /* [B] */
  const float *gate;     /* [B*W, H] multiplier (sparse attention gate) or NULL */
  int32_t use_xsa;       /* subtract the current value direction (model.py:760-768) */
  int32_t flags;         /* ALTXS_ATTN_* */
  int32_t kv_tail_end;   /* 0, or tail placement (above; natural layouts) */
  int32_t reserved;
  void *y;               /* [B*W, H*head_dim] */
  int32_t *err;          /* device error word or NULL */
} AltxsAttnArgs;

int32_t altxs_decode_attn(const AltxsAttnArgs *a, altxs_stream_t stream);

/* ---- the whole per-symbol step ------------------------------------------ */

#define ALTXS_MAX_LAYERS 32
#define ALTXS_MAX_SLOTS 64

enum {
  ALTXS_F_SMEAR = 1 << 0,       /* SmearGate on the embedding (model.py:1559-1579) */
  ALTXS_F_SPARSE_GATE = 1 << 1, /* sparse attention gate (model.py:854-862) */
  ALTXS_F_SKIP_GATES = 1 << 2,  /* gated U-Net skips (model.py:1275-1291) */
  ALTXS_F_ASYM_SOFTCAP = 1 << 3,/* asymmetric tanh softcap (model.py:1478-1493) */
  ALTXS_F_COMMIT = 1 << 4,      /* after the step: pos += W, prev_raw = last raw */
  ALTXS_F_RENORM = 1 << 5,      /* renormalise probs before the CDF (ALTXS_CDF_RENORM; V <= 16384) */
  ALTXS_F_FINAL_ATTN = 1 << 6,  /* parallel_final_lane = "attn" (default mean) */
  ALTXS_F_FINAL_MLP = 1 << 7,   /* parallel_final_lane = "mlp" */
  ALTXS_F_FUSE_O = 1 << 8,      /* decode: form the out-projection inside the attention launch
                                 * and finish it where it is read (the same bits; slower on
                                 * the benchmark model, so off by default) */
};

enum { ALTXS_SLOT_SEQ = 0, ALTXS_SLOT_PAR = 1 };

typedef struct AltxsLayer {
  AltxsQTensor qkv;          /* [(H + 2*Hkv)*head_dim, D]: q rows, k rows, v rows */
  AltxsQTensor o;            /* [D, D] */
  AltxsQTensor up;           /* [F, D] */
  AltxsQTensor down;         /* [D, F] */
  const float *resid_mix;    /* [2, D], 16-byte aligned */
  const float *attn_scale;   /* [D], 16-byte aligned */
  const float *mlp_scale;    /* [D], 16-byte aligned */
  const float *q_gain;       /* [H] */
  const float *attn_gate_w;  /* [H, gate_window] or NULL */
  const float *par_resid;    /* [2] parallel_resid_lambdas[layer] or NULL */
  const float *par_post;     /* [2, 2] parallel_post_lambdas[layer] or NULL */
  float ln_scale;            /* 1/sqrt(layer+1) with ln_scale, else 1 */
  int32_t use_xsa;
  int32_t reserved;
} AltxsLayer;

typedef struct AltxsSlot {
  int32_t layer;
  int32_t kind;            /* ALTXS_SLOT_SEQ / ALTXS_SLOT_PAR */
  int32_t skip_idx;        /* decoder skip weight row, -1 = none */
  int32_t skip_src;        /* slot whose output is popped, -1 = none */
  int32_t first_parallel;  /* first parallel slot: both lanes start from x */
  /* Unmerged LoRA on this slot's q and v projections (rank = desc.lora_rank,
   * 1..16; all four NULL = none): q += s * (n A_q^T) B_q^T, v likewise, added
   * to the projection before QK-RMSNorm/RoPE (ttt_lora.py:53-55, 143-151;
   * per slot as the reference's q_loras[slot]).  fp16, row-major. */
  float lora_scale;          /* s = alpha/rank (or alpha/sqrt(rank) for rsLoRA) */
  const uint16_t *lora_q_a;  /* [rank, D] */
  const uint16_t *lora_q_b;  /* [H*head_dim, rank] */
  const uint16_t *lora_v_a;  /* [rank, D] */
  const uint16_t *lora_v_b;  /* [Hkv*head_dim, rank] */
} AltxsSlot;

typedef struct AltxsStepDesc {
  int32_t abi_version;
  int32_t B, W, D, H, Hkv, head_dim, F, V;
  int32_t n_layers, n_slots, max_len, gate_window, rope_dims, lora_rank;
  int32_t act_bf16; /* 0: fp32 activations (3-way split MFMA), 1: bf16 */
  int32_t kv_bf16;  /* KV layout: ALTXS_KV_F32, ALTXS_KV_BF16 or ALTXS_KV_BF16_NATURAL */
  int32_t kv_tail_end; /* 0, or tail placement of the window's K/V (above; natural
                          layouts, per-stage launches only) */
  int32_t flags;    /* ALTXS_F_* */
  float norm_eps, gate_scale, logit_softcap;
  AltxsLayer layers[ALTXS_MAX_LAYERS];
  AltxsSlot slots[ALTXS_MAX_SLOTS];
  AltxsQTensor emb;          /* tied embedding / LM head [V, D] */
  const float *skip_weights; /* [n_skip, D], 16-byte aligned */
  const float *skip_gates;   /* [n_skip, D] or NULL, 16-byte aligned */
  const float *smear_w;      /* [gate_window] */
  const float *smear_lambda; /* [1] */
  const float *softcap_pn;   /* [2] = (softcap_pos, softcap_neg) */
  const float *rope_cos;     /* [max_len, rope_dims/2] fp32 */
  const float *rope_sin;
  /* caller-owned state */
  const int32_t *tokens; /* [B, W] */
  int32_t *pos;          /* [B] window start position of each segment */
  float *prev_raw;       /* [B, D] raw embedding of each segment's previous token */
  float *cand_raw;       /* [B, D] raw embedding of the window's last token */
  void *kv;              /* [n_slots, B, 2, Hkv, max_len, head_dim], cache layout above */
  void *ws;              /* workspace, altxs_step_workspace_bytes() bytes */
  int64_t ws_bytes;
  float *logits;         /* [B*W, V] */
  float *probs;          /* [B*W, V] or NULL */
  uint32_t *cum;         /* [B*W, V+1] or NULL */
  int32_t *err;          /* [1] device error word */
  /* Optional timing hook: NULL, or hipEvent_t handles recorded right before and
   * after every attention launch (the dominant kernel) on the stream that runs
   * it: events 2s, 2s+1 for slot s (one group); (g*n_slots + s)*2 + {0,1} for
   * group g in split mode. */
  void **attn_events;
  /* Split mode (B >= 2): a second stream and at least 2 caller-created
   * events (hipEventDisableTiming; 2*n_slots + 2 are accepted).  Segments
   * [0, ceil(B/2)) run on `stream`, the rest on aux_stream, each group's step
   * one chain; the second starts after the first group's slot-0 QKV, so one
   * group's projections and MLP overlap the other group's KV streaming.
   * Results are bit-identical to the single-stream step.  NULL = one stream. */
  void *aux_stream;
  void **sync_events;
  /* Persistent layer kernel (single stream, bf16 KV, W dividing 16): a plan
   * built once by altxs_step_plan_build() for this descriptor's pointers and
   * shapes -- plan_dev on the device, plan_host its host image, both
   * altxs_step_plan_bytes() long.  Every slot of the step then runs in ONE
   * launch: workgroups take tasks (a GEMM column tile or an attention
   * (row, kv-head) pair of one 16-row tile) in dependency order, so one row
   * tile's projections and MLP run while other tiles' attention streams the
   * KV cache.  Bit-identical to the per-stage launches.  In this mode
   * attn_events 0 and 1 bracket the layer kernel.  NULL = per-stage launches. */
  void *plan_dev;
  const void *plan_host;
  int64_t plan_bytes;
} AltxsStepDesc;

/* Workspace bytes altxs_step needs for this descriptor (host-only). */
int64_t altxs_step_workspace_bytes(const AltxsStepDesc *d);

/* Whether altxs_step forms slot `slot`'s out-projection inside the attention
 * launch (per-head MFMA terms) and finishes it in the MLP-up prologue
 * (sequential slot) or the MLP-down epilogue (parallel slot) instead of a
 * launch of its own (host-only): 1 yes, 0 no, <0 bad arguments.  The
 * reference runs the out-projection as one stage of its fused step
 * (src/xsa_ttt/ac_gemv.py:89-310, persistent_step.py:777-811); here it is done
 * when d->flags has ALTXS_F_FUSE_O, for decode steps (W = 1) with bf16
 * activations, the tiled bf16 cache, MHA and a packed out-projection.  Either
 * way the results are the same bits. */
int32_t altxs_step_fuses_out_proj(const AltxsStepDesc *d, int32_t slot);

/* Bytes of the persistent-kernel plan for this descriptor (host-only; <0 on error). */
int64_t altxs_step_plan_bytes(const AltxsStepDesc *d);

/*
 * Build the persistent-kernel plan for d (its plan fields are ignored): the
 * per-slot weight pointers, parameters and workspace layout, written to
 * plan_host and copied to plan_dev on `stream` (the call waits for the copy).
 * A step whose descriptor no longer matches the plan fails with ALTXS_ERR_ARG.
 * The reference keeps the same stacked per-layer tables for its persistent
 * decode kernel (src/xsa_ttt/persistent_step.py:452-588).
 */
int32_t altxs_step_plan_build(const AltxsStepDesc *d, void *plan_host, void *plan_dev,
                              int64_t bytes, altxs_stream_t stream);

/*
 * One W-token step for B independent segments: embedding (+smear), every slot
 * (QKV + QK-RMS + RoPE + KV write, attention, out-projection + residual,
 * RMSNorm/MLP), final norm, LM head + softcap, softmax and integer CDFs.
 * K/V rows are written at pos[b] + t (or in the tail rows, kv_tail_end).
 * W = 1 is the decode row; W > 1 is the
 * teacher-forced encode window; per-row results are identical for the same
 * prefix.  Replaces try_persistent_extend(model, state)
 * (src/xsa_ttt/persistent_step.py:1081), try_mega_encode(model, state)
 * (src/xsa_ttt/mega_encode.py:1693) and GPT.static_extend
 * (src/xsa_ttt/model.py:1617-1781), plus the softmax that follows
 * (incremental.py:603-633).
 */
int32_t altxs_step(const AltxsStepDesc *d, altxs_stream_t stream);

/* Size of the static device scratch altxs_step_noalloc uses as its workspace:
 * 24 MiB, enough for decode rows of the cfg3 model up to B = 256. */
#define ALTXS_STEP_SCRATCH_BYTES (24ll << 20)

/*
 * altxs_step without a caller workspace: d->ws and d->ws_bytes are ignored and
 * the step's partial results (slot outputs, normalised rows, LM-head tile
 * statistics, counters) live in a file-scope device array of
 * ALTXS_STEP_SCRATCH_BYTES inside the library, one per GPU, held until the
 * process ends.  It calls no allocator, so callers that cannot allocate --
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc -- can run the step; the caller still passes every input and
 * output buffer.  Same results as altxs_step.  A step whose
 * altxs_step_workspace_bytes() exceeds ALTXS_STEP_SCRATCH_BYTES, or with a
 * persistent plan (d->plan_dev, built for a caller workspace), is rejected
 * with ALTXS_ERR_ARG.  All calls on one GPU share its scratch and each call
 * leaves its contents behind (the step's first kernel clears its counters):
 * calls that overlap on one GPU (two streams, or two host threads) race.
 * No counterpart in the reference.
 */
int32_t altxs_step_noalloc(const AltxsStepDesc *d, altxs_stream_t stream);

/*
 * Range coder (the 32-bit Witten-Neal-Cleary coder with E3 bits of
 * arithmetic_coder_lm.py:90-288; replaces GpuRangeCoder, gpu_ac.py:397-479,
 * and its one-thread kernels 84-218).  One stream per segment, state in device
 * memory; the tables are the integer CDF rows altxs_step writes (cum[V+1],
 * total = cum[V]).  Stream b's bytes live at buf + b*stride (MSB-first bits,
 * the reference's _pack_bits layout); framing (<u64 len><bytes> per segment,
 * incremental.py:1721-1722) is host work on the returned lengths.
 */
typedef struct AltxsCoderState {
  uint64_t low, high;
  uint64_t pending;  /* encoder: E3 bits owed */
  uint64_t value;    /* decoder: code value */
  int64_t nbits;     /* encoder: bits written; decoder: bits read */
  int64_t nbytes;    /* after altxs_range_finish: the stream's length; decoder: input length */
  uint32_t partial;  /* encoder: bits of the unfinished byte */
  int32_t err;       /* 1: output buffer full, 2: symbol or table invalid */
} AltxsCoderState;

/* Encoder start state for n streams. */
int32_t altxs_range_init(AltxsCoderState *st, int32_t n, altxs_stream_t stream);

/* Encode W symbols per stream: stream b codes syms[b*W + t] with table row
 * b*W + t of cum ([n*W, V+1] uint32), t = 0 .. W-1 in order (a decode row
 * is W = 1, an encode window W > 1).  Replaces encode_symbol (gpu_ac.py:431). */
int32_t altxs_range_encode(AltxsCoderState *st, int32_t n, int32_t W, const int32_t *syms,
                           const uint32_t *cum, int32_t V, uint8_t *buf, int64_t stride,
                           altxs_stream_t stream);

/* Flush every stream (final bits, last partial byte); st[b].nbytes = length.
 * Replaces finish (gpu_ac.py:443). */
int32_t altxs_range_finish(AltxsCoderState *st, int32_t n, uint8_t *buf, int64_t stride,
                           altxs_stream_t stream);

/* Decoder start: read the first 32 bits of each stream (nbytes[b] = its
 * length; bits past it read as 0).  Replaces begin_decode (gpu_ac.py:448). */
int32_t altxs_range_seed(AltxsCoderState *st, int32_t n, const uint8_t *buf, int64_t stride,
                         const int64_t *nbytes, altxs_stream_t stream);

/* Decode one symbol per stream from table row b of cum ([n, V+1]) and write
 * it to out[b*out_stride] -- e.g. the next step's token buffer, so decoding
 * needs no host round trip.  Replaces decode_symbol (gpu_ac.py:466). */
int32_t altxs_range_decode(AltxsCoderState *st, int32_t n, const uint32_t *cum, int32_t V,
                           const uint8_t *buf, int64_t stride, int32_t *out, int64_t out_stride,
                           altxs_stream_t stream);

/* ---- the shipped per-channel codec (dense runtime banks) -------------------
 *
 * The reference ships weights as Init(seed) + a per-channel mixed-bit delta
 * (src/hyperflow_distillation/mixed_bit_delta.py): every channel (a row, or
 * a column of the o / down banks, of `width` values) has 0/2/3/4 bits; the
 * codes of all channels of one width are packed together LSB first (3-bit:
 * 8 codes per 3 bytes, little endian); each width has its own codebook. At
 * runtime the banks are dense (model.py:1183-1245): in this library a dense
 * tensor is an AltxsQTensor with bits = 16 (bf16 values in the MFMA-tiled
 * order, no scales), which altxs_step accepts for every matrix. */
enum {
  ALTXS_CODEBOOK_LLOYD = 0,     /* codebook [n_b][2^b] fp16 levels per channel */
  ALTXS_CODEBOOK_SYMMETRIC = 1, /* codebook [n_b] fp16 scale: (c - (2^b-1)/2) * s */
  ALTXS_CODEBOOK_SHARED = 2,    /* shared [2^b] fp16 levels x codebook [n_b] fp16 scale */
  ALTXS_CODEBOOK_FP4 = 3,       /* 4-bit codes as FP4 E2M1 x codebook [n_b] fp16 scale */
  ALTXS_CODEBOOK_HYBRID = 4     /* 4-bit channels as FP4, 2/3-bit symmetric */
};

typedef struct AltxsCodecGroups {
  const uint8_t *packed[3];    /* index b - 2 (b = 2, 3, 4): the width's packed codes */
  const uint16_t *codebook[3]; /* fp16, per mode (above) */
  const uint16_t *shared[3];   /* ALTXS_CODEBOOK_SHARED: [2^b] fp16 levels, else NULL */
  int64_t n_codes[3];          /* codes held by packed[b - 2] (bounds every read) */
  int64_t n_book[3];           /* fp16 entries of codebook[b - 2] */
  int32_t mode;                /* ALTXS_CODEBOOK_* */
  int32_t reserved;
} AltxsCodecGroups;

/* Decode channels j = 0 .. n_channels-1: channel j has bits[j] (0: a dead
 * channel, all zero) and is the rank[j]-th channel of its width (its codes are
 * codes rank*width .. +width of that width's stream); value i of channel j goes
 * to out[j*stride_ch + i*stride_el] (fp32), so o / down channels can land as
 * columns. Replaces dequantize_channels + _from_channels
 * (mixed_bit_delta.py:116-229) for one bank part. A channel with a bad width,
 * or whose codes or codebook entries lie past the given counts, is written as
 * zeros and ORs 2 into *err (a caller-owned device int32). */
int32_t altxs_codec_decode(const AltxsCodecGroups *g, const uint8_t *bits, const int32_t *rank,
                           int64_t n_channels, int64_t width, float *out, int64_t stride_ch,
                           int64_t stride_el, int32_t *err, altxs_stream_t stream);

/* A dense bits = 16 tensor from fp32 rows: w = base + delta (base may be NULL;
 * fp32 add as apply_delta_to, train_hyperflow.py:8-19), rounded to bf16 (to
 * nearest even) and written in the MFMA-tiled order of AltxsQTensor (N % 16 ==
 * 0, K % 256 == 0; row r of base/delta at r*ld). tiled: N*K*2 bytes. */
int32_t altxs_pack_dense(const float *base, const float *delta, int64_t N, int64_t K, int64_t ld,
                         void *tiled, altxs_stream_t stream);

/* The same for a dense bits = 32 tensor: w = base + delta kept in fp32, as
 * the three exact bf16 planes (tiled: tiled_bytes >= N*K*6, checked).  The
 * reference's fp32 compute mode keeps its banks in fp32 (model.py:1183-1196). */
int32_t altxs_pack_dense32(const float *base, const float *delta, int64_t N, int64_t K, int64_t ld,
                           void *tiled, int64_t tiled_bytes, altxs_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* ALTXS_H */
