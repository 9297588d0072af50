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
#include <string.h>

#include "common.h"
#include "kernels.h"
#include "gemm.h"

using namespace altxs;

namespace {

constexpr int HD = 64;

// torch.lerp(start, end, w) (ATen's two-branch formula)
__device__ __forceinline__ float lerp_t(float start, float end, float w) {
  return (fabsf(w) < 0.5f) ? start + w * (end - start) : end - (end - start) * (1.f - w);
}
__device__ __forceinline__ float sigmoidf(float x) { return 1.f / (1.f + expf(-x)); }
// tanh(x) = sign(x) * (1 - 2 / (exp(2|x|) + 1)); absolute error ~1e-7.
__device__ __forceinline__ float tanh_fast(float x) {
  const float e = __expf(2.f * fabsf(x));
  return copysignf(1.f - 2.f * __builtin_amdgcn_rcpf(e + 1.f), x);
}

// ---- embedding (+ SmearGate) ------------------------------------------------

// Dequantise 8 consecutive weights [8*run, 8*run+8) of row n of a packed tensor.
template <int BITS>
__device__ void dequant_run(const QT& w, int n, int run, float (&out)[8]) {
  constexpr int P0 = Planes<BITS>::P0, P1 = Planes<BITS>::P1;
  constexpr float center = 0.5f * (float)((1 << BITS) - 1);
  const int KB = w.K >> 8;
  const int k0 = 8 * run, kb = k0 >> 8, kk = k0 & 255;
  const int s = kk >> 5, lg = (kk & 31) >> 3;
  const int L = (n & 15) + 16 * lg;
  const size_t bi = (size_t)(n >> 4) * KB + kb;
  const uint8_t* blk = w.codes + bi * (512 * BITS);
  uint32_t p0[2 * P0], p1[P1 > 0 ? 2 * P1 : 1];
  const uint32_t* a0 = (const uint32_t*)(blk + L * (8 * P0));
#pragma unroll
  for (int i = 0; i < 2 * P0; ++i) p0[i] = a0[i];
  if constexpr (P1 > 0) {
    const uint32_t* a1 = (const uint32_t*)(blk + 512 * P0 + L * (8 * P1));
#pragma unroll
    for (int i = 0; i < 2 * P1; ++i) p1[i] = a1[i];
  }
  uint32_t c[8];
  codes_step<BITS>(p0, p1, s, c);
  const float sc = __half2float(__ushort_as_half(w.scales[bi * 64 + (n & 15) * 4 + (kk >> 6)]));
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = ((float)c[i] - center) * sc;
}

__device__ void dequant_run_bits(int bits, const QT& w, int n, int run, float (&out)[8]) {
  switch (bits) {
    case 2: dequant_run<2>(w, n, run, out); break;
    case 3: dequant_run<3>(w, n, run, out); break;
    case 4: dequant_run<4>(w, n, run, out); break;
    default: dequant_run<6>(w, n, run, out); break;
  }
}

struct EmbedP {
  QT emb;
  int bits, V, D, W, gw, smear;
  float eps;
  const int32_t* tokens;
  const float* prev_raw;
  float* cand_raw;
  const float* smear_w;
  const float* smear_lambda;
  float* x0;  // [R, D]
  int32_t* err;
  int* sync;  // step counters, zeroed here (this is the step's first kernel)
  int nsync;
  const float* mix0;  // resid_mix of slot 0's layer [2, D]
  float* xin0;        // slot 0's x_in = m0*x0 + m1*x0 (sequential, no skip)
};

constexpr int MAX_RUNS = 4;  // D <= 64 lanes * 4 runs * 8 = 2048

__global__ __launch_bounds__(64) void embed_kernel(EmbedP a) {
  const int r = blockIdx.x, lane = threadIdx.x;
  if (r == 0)
    for (int i = lane; i < a.nsync; i += 64) a.sync[i] = 0;
  const int b = r / a.W, t = r % a.W;
  auto tok_at = [&](int tt) {
    int tk = a.tokens[(int64_t)b * a.W + tt];
    if (tk < 0 || tk >= a.V) {
      if (lane == 0) flag_err(a.err, ALTXS_EDEV_TOKEN);
      tk = tk < 0 ? 0 : a.V - 1;
    }
    return tk;
  };
  const int tok = tok_at(t);
  const int nruns = a.D / 8;
  float raw[MAX_RUNS][8], prev[MAX_RUNS][8];
#pragma unroll
  for (int j = 0; j < MAX_RUNS; ++j) {
    const int run = lane + 64 * j;
    if (run < nruns) dequant_run_bits(a.bits, a.emb, tok, run, raw[j]);
  }
  float x[MAX_RUNS][8];
  if (a.smear) {
    const int ptok = t > 0 ? tok_at(t - 1) : -1;
#pragma unroll
    for (int j = 0; j < MAX_RUNS; ++j) {
      const int run = lane + 64 * j;
      if (run >= nruns) continue;
      if (ptok >= 0) {
        dequant_run_bits(a.bits, a.emb, ptok, run, prev[j]);
      } else {
        const float* pr = a.prev_raw + (int64_t)b * a.D + 8 * run;
#pragma unroll
        for (int i = 0; i < 8; ++i) prev[j][i] = pr[i];
      }
    }
    // g = lambda * sigmoid(raw[:gw] . w_smear)
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < MAX_RUNS; ++j) {
      const int run = lane + 64 * j;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int k = 8 * run + i;
        if (run < nruns && k < a.gw) part += raw[j][i] * a.smear_w[k];
      }
    }
    const float gsum = wave_sum(part);
    const float g = a.smear_lambda[0] * sigmoidf(gsum);
#pragma unroll
    for (int j = 0; j < MAX_RUNS; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) x[j][i] = raw[j][i] + g * prev[j][i];
  } else {
#pragma unroll
    for (int j = 0; j < MAX_RUNS; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) x[j][i] = raw[j][i];
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < MAX_RUNS; ++j)
    if (lane + 64 * j < nruns)
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += x[j][i] * x[j][i];
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / (float)a.D + a.eps);
#pragma unroll
  for (int j = 0; j < MAX_RUNS; ++j) {
    const int run = lane + 64 * j;
    if (run >= nruns) continue;
    float* xo = a.x0 + (int64_t)r * a.D + 8 * run;
    float* xi = a.xin0 + (int64_t)r * a.D + 8 * run;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float v = x[j][i] * inv;
      xo[i] = v;
      xi[i] = a.mix0[8 * run + i] * v + a.mix0[a.D + 8 * run + i] * v;
    }
    if (t == a.W - 1) {
      float* co = a.cand_raw + (int64_t)b * a.D + 8 * run;
#pragma unroll
      for (int i = 0; i < 8; ++i) co[i] = raw[j][i];
    }
  }
}

// ---- prologues -------------------------------------------------------------
//
// 256 threads stage the 16-row A tile: 16 lanes per row, each lane owning the
// float4 chunks c = lane + 16*j of the row (D <= 512 -> j < 8).  All loads of
// a row are issued before any arithmetic; the row's RMS is a 16-lane butterfly.

constexpr int PTPR = 16;                  // prologue threads per row
constexpr int PMAXJ = 512 / 4 / PTPR;     // float4 chunks per lane (D <= 512)


// RMSNorm (* scale) of 16 rows of x staged as the A tile.  Inputs of the
// attention side (the QKV prologue) also carry the sparse attention gate
// (model.py:854-862): the task that owns column tile 0 (`first`) forms
// sigmoid(gate_scale * n[:gw] . W_gate[h]) for every head from the normalised
// row.  The final norm before the LM head may average the two parallel lanes.
struct ProNorm {
  static constexpr bool kStage = true;
  static constexpr size_t kScratch = 0;
  const float* x;
  const float* x2;  // second lane (final parallel "mean") or NULL
  int lane_mode;    // 0: x, 1: 0.5*(x + x2)
  float scale, eps;
  int D;
  const float* gate_w = nullptr;  // [H, gw] or NULL
  float* gate_out = nullptr;      // [R, H]
  float gate_scale = 0.f;
  int H = 0, gw = 0;
  template <int AM, int NT>
  __device__ void stage(void* As, void*, int m0, int R, int K, int, bool first) const {
    static_assert(NT == 16 * PTPR, "one row per 16 lanes, 16 rows per task");
    constexpr int HMAX = 8;  // D <= 512 -> H <= 8
    const int t = threadIdx.x, row = t / PTPR, li = t % PTPR;
    const int r = m0 + row;
    const int nch = D >> 2;
    f32x4 v[PMAXJ], v2[PMAXJ];
#pragma unroll
    for (int j = 0; j < PMAXJ; ++j) {
      const int c = li + PTPR * j;
      if (c < nch && r < R) {
        v[j] = *(const f32x4*)(x + (int64_t)r * D + 4 * c);
        if (lane_mode == 1) v2[j] = *(const f32x4*)(x2 + (int64_t)r * D + 4 * c);
      }
    }
    const bool gating = first && gate_w;
    float gwv[HMAX][4];
    if (gating) {  // gate of head h reads features [0, gw), gw <= 16: lanes 0-3, chunk 0
#pragma unroll
      for (int h = 0; h < HMAX; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          gwv[h][e] = (h < H && 4 * li + e < gw) ? gate_w[h * gw + 4 * li + e] : 0.f;
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < PMAXJ; ++j) {
      const int c = li + PTPR * j;
      if (c >= nch) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float y = r < R ? v[j][e] : 0.f;
        if (lane_mode == 1 && r < R) y = 0.5f * (v[j][e] + v2[j][e]);
        v[j][e] = y;
        ss += y * y;
      }
    }
    ss = row16_sum(ss);
    const float inv = r < R ? rsqrtf(ss / (float)D + eps) : 0.f;
    float n0[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < PMAXJ; ++j) {
      const int c = li + PTPR * j;
      if (c >= nch) continue;
      float n[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) n[e] = (v[j][e] * inv) * scale;
      if (j == 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) n0[e] = n[e];
      }
      a_store4<AM>(As, row, 4 * c, K, n);
    }
    if (gating) {
      float part[HMAX];
#pragma unroll
      for (int h = 0; h < HMAX; ++h) {
        part[h] = 0.f;
        if (li < 4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) part[h] += n0[e] * gwv[h][e];
        }
      }
#pragma unroll
      for (int h = 0; h < HMAX; ++h) part[h] = row16_sum(part[h]);
      if (li < H && r < R) {
        float dot = part[0];
#pragma unroll
        for (int h = 1; h < HMAX; ++h) dot = li == h ? part[h] : dot;
        gate_out[(int64_t)r * H + li] = sigmoidf(gate_scale * dot);
      }
    }
  }
};

// The next slot's inputs, formed elementwise where the current slot's output
// is produced (DOWN epilogue; the embedding for slot 0): decoder skip (lerp
// gate or add, model.py:1275-1291), then resid_mix with x0 (model.py:947-950,
// 1310-1316).  base = x_in (sequential) or lane0 after the skip (parallel) --
// the residual base the O/DOWN epilogues of that slot use; attn = the
// pre-RMSNorm attention input m0*base + m1*x0.
struct NextIn {
  const float* x0 = nullptr;
  const float* skip = nullptr;    // popped encoder output or NULL
  const float* skip_w = nullptr;  // [D]
  const float* skip_g = nullptr;  // [D] gate logits or NULL
  const float* mix = nullptr;     // next layer's resid_mix [2, D]
  float* base = nullptr;          // NULL: no next slot
  float* attn = nullptr;          // may equal base (sequential slot)
  int parallel = 0;
  int skip_self = 0;  // the popped encoder output is the value being produced here
  struct El { float x0, sk, sw, sg, m0, m1; };
  __device__ El load(int64_t idx, int c, int D) const {
    El e;
    e.x0 = x0[idx];
    e.m0 = mix[c];
    e.m1 = mix[D + c];
    e.sk = (skip && !skip_self) ? skip[idx] : 0.f;
    e.sw = skip ? skip_w[c] : 0.f;
    e.sg = skip_g ? skip_g[c] : 0.f;
    return e;
  }
  __device__ void put(int64_t idx, float x, const El& e) const {
    float bs = x;
    if (skip) {
      const float sc = e.sw * (skip_self ? x : e.sk);
      bs = skip_g ? lerp_t(sc, x, sigmoidf(e.sg)) : x + sc;
    }
    const float in = e.m0 * bs + e.m1 * e.x0;
    base[idx] = parallel ? bs : in;
    if (attn != base) attn[idx] = in;
  }
};

// ---- epilogues --------------------------------------------------------------

__device__ __forceinline__ int row_pos(const int32_t* pos, int W, int r) {
  return pos[r / W] + (r % W);
}

// One head (64 columns) per tile: QK-RMSNorm, RoPE, q_gain, KV-cache write.
struct EpiQKV {
  float* q;          // [R, H, 64]
  char* kv;          // this slot's cache: [B][2][Hkv][max_len][64]
  int kv_bf16, H, Hkv, W, max_len, rd;
  const int32_t* pos;
  const float* cosb;  // [max_len, rd/2]
  const float* sinb;
  const float* q_gain;
  float eps;
  int32_t* err;
  template <class Cfg> struct Pre {
    static constexpr int TPR = Cfg::THREADS / 16, CPT = 64 / TPR;
    int p;
    float cs[CPT], sn[CPT], gain;
  };
  template <class Cfg>
  __device__ Pre<Cfg> prefetch(int m0, int n0, int R, int) const {
    using P = Pre<Cfg>;
    static_assert(Cfg::NCOL == HD, "one head per column tile");
    P o;
    const int row = threadIdx.x / P::TPR, c0 = (threadIdx.x % P::TPR) * P::CPT;
    const int r = m0 + row;
    o.p = r < R ? row_pos(pos, W, r) : 0;
    const int nt = n0 / HD;
    o.gain = nt < H ? q_gain[nt] : 1.f;
    const int half = rd >> 1;
    const int pp = (o.p >= 0 && o.p < max_len) ? o.p : 0;
#pragma unroll
    for (int i = 0; i < P::CPT; ++i) {
      const int c = c0 + i;
      const int fi = c < half ? c : c - half;
      o.cs[i] = (c < rd && nt < H + Hkv) ? cosb[(int64_t)pp * half + fi] : 1.f;
      o.sn[i] = (c < rd && nt < H + Hkv) ? sinb[(int64_t)pp * half + fi] : 0.f;
    }
    return o;
  }
  template <class Cfg, class P>
  __device__ void apply(const float* C, const P& pre, const void*, int m0, int n0, int R, int) const {
    constexpr int TPR = P::TPR, CPT = P::CPT;
    const int row = threadIdx.x / TPR, li = threadIdx.x % TPR, c0 = li * CPT;
    const int r = m0 + row;
    const int nt = n0 / HD;
    const int kind = nt < H ? 0 : (nt < H + Hkv ? 1 : 2);
    const int head = kind == 0 ? nt : (kind == 1 ? nt - H : nt - H - Hkv);
    float v[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) v[i] = C[row * Cfg::CS + c0 + i];
    if (kind < 2) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < CPT; ++i) ss += v[i] * v[i];
      static_assert(TPR == 16, "a head's 64 columns are one 16-lane row");
      ss = row16_sum(ss);
      const float inv = rsqrtf(ss * (1.0f / HD) + eps);
#pragma unroll
      for (int i = 0; i < CPT; ++i) v[i] *= inv;
      // partner column c +- rd/2 lives (rd/2)/CPT lanes away
      const int off = (rd >> 1) / CPT;
      float pv[CPT];
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const float up = __shfl_down(v[i], off, WAVE);
        const float dn = __shfl_up(v[i], off, WAVE);
        pv[i] = (c0 < (rd >> 1)) ? up : dn;
      }
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int c = c0 + i;
        if (c < (rd >> 1)) v[i] = v[i] * pre.cs[i] + pv[i] * pre.sn[i];
        else if (c < rd) v[i] = pv[i] * -pre.sn[i] + v[i] * pre.cs[i];
      }
    }
    if (r >= R) return;
    const int p = pre.p;
    const bool pos_ok = p >= 0 && p < max_len;
    if (kind == 0) {
      float* qo = q + ((int64_t)r * H + head) * HD + c0;
#pragma unroll
      for (int i = 0; i < CPT; ++i) qo[i] = v[i] * pre.gain;
    } else if (pos_ok) {
      const int b = r / W;
      const int64_t head_base = (((int64_t)b * 2 + (kind == 2 ? 1 : 0)) * Hkv + head) * max_len * HD;
      if (kv_bf16) {  // tiled operand layout (kv_tile_k / kv_tile_v)
        uint16_t* tile = (uint16_t*)kv + head_base + (int64_t)(p / ALTXS_KV_TILE) * (ALTXS_KV_TILE * HD);
        const int kt = p % ALTXS_KV_TILE;
#pragma unroll
        for (int i = 0; i < CPT; ++i)
          tile[kind == 1 ? kv_tile_k(kt, c0 + i) : kv_tile_v(kt, c0 + i)] = f32_to_bf16(v[i]);
      } else {
        float* row = (float*)kv + head_base + (int64_t)p * HD + c0;
#pragma unroll
        for (int i = 0; i < CPT; ++i) row[i] = v[i];
      }
    } else if (li == 0) {
      flag_err(err, ALTXS_EDEV_POS);
    }
  }
};

// Elementwise epilogues: thread t handles tile elements t + THREADS*j.
template <class Cfg> struct EW {
  static constexpr int EPT = 16 * Cfg::NCOL / Cfg::THREADS;
  __device__ static int row(int j) { return (threadIdx.x + Cfg::THREADS * j) / Cfg::NCOL; }
  __device__ static int col(int j) { return (threadIdx.x + Cfg::THREADS * j) % Cfg::NCOL; }
};

struct EpiO {
  const float* xin;
  const float* attn_scale;
  float* xout;
  int D, parallel;
  template <class Cfg> struct Pre { float base[EW<Cfg>::EPT], sc[EW<Cfg>::EPT]; };
  template <class Cfg>
  __device__ Pre<Cfg> prefetch(int m0, int n0, int R, int) const {
    Pre<Cfg> o;
#pragma unroll
    for (int j = 0; j < EW<Cfg>::EPT; ++j) {
      const int r = m0 + EW<Cfg>::row(j), c = n0 + EW<Cfg>::col(j);
      const bool ok = r < R && c < D;
      o.base[j] = (ok && !parallel) ? xin[(int64_t)r * D + c] : 0.f;
      o.sc[j] = ok ? attn_scale[c] : 0.f;
    }
    return o;
  }
  template <class Cfg, class P>
  __device__ void apply(const float* C, const P& pre, const void*, int m0, int n0, int R, int) const {
#pragma unroll
    for (int j = 0; j < EW<Cfg>::EPT; ++j) {
      const int rr = EW<Cfg>::row(j), cc = EW<Cfg>::col(j);
      const int r = m0 + rr, c = n0 + cc;
      if (r >= R || c >= D) continue;
      const float a = pre.sc[j] * C[rr * Cfg::CS + cc];
      xout[(int64_t)r * D + c] = parallel ? a : pre.base[j] + a;
    }
  }
};

struct EpiUp {
  void* h;  // [R, F] fp32 or bf16
  int F, hb16;
  template <class Cfg> struct Pre {};
  template <class Cfg>
  __device__ Pre<Cfg> prefetch(int, int, int, int) const { return {}; }
  template <class Cfg, class P>
  __device__ void apply(const float* C, const P&, const void*, int m0, int n0, int R, int) const {
#pragma unroll
    for (int j = 0; j < EW<Cfg>::EPT; ++j) {
      const int rr = EW<Cfg>::row(j), cc = EW<Cfg>::col(j);
      const int r = m0 + rr, c = n0 + cc;
      if (r >= R || c >= F) continue;
      const float v = C[rr * Cfg::CS + cc];
      const float lr = v > 0.f ? v : 0.5f * v;
      const float o = lr * lr;
      const int64_t idx = (int64_t)r * F + c;
      if (hb16) ((uint16_t*)h)[idx] = f32_to_bf16(o);
      else ((float*)h)[idx] = o;
    }
  }
};

struct EpiDown {
  const float* xout;   // seq: x_out; par: attn term a
  const float* mlp_scale;
  float* out0;         // seq: slot output; par: lane0'
  float* out1;         // par: lane1'
  const float* lane0;  // par: lane0 after skip
  const float* lane1;  // par: lane1 input
  const float* pr;     // par: [2]
  const float* pp;     // par: [2, 2]
  int D, parallel;
  NextIn next;  // inputs of the following slot (next.base == NULL: none)
  template <class Cfg> struct Pre {
    float xo[EW<Cfg>::EPT], sc[EW<Cfg>::EPT], l0[EW<Cfg>::EPT], l1[EW<Cfg>::EPT];
    NextIn::El nx[EW<Cfg>::EPT];
  };
  template <class Cfg>
  __device__ Pre<Cfg> prefetch(int m0, int n0, int R, int) const {
    Pre<Cfg> o;
#pragma unroll
    for (int j = 0; j < EW<Cfg>::EPT; ++j) {
      const int r = m0 + EW<Cfg>::row(j), c = n0 + EW<Cfg>::col(j);
      const bool ok = r < R && c < D;
      const int64_t idx = (int64_t)r * D + c;
      o.xo[j] = ok ? xout[idx] : 0.f;
      o.sc[j] = ok ? mlp_scale[c] : 0.f;
      o.l0[j] = (ok && parallel) ? lane0[idx] : 0.f;
      o.l1[j] = (ok && parallel) ? lane1[idx] : 0.f;
      if (ok && next.base) o.nx[j] = next.load(idx, c, D);
    }
    return o;
  }
  template <class Cfg, class P>
  __device__ void apply(const float* C, const P& pre, const void*, int m0, int n0, int R, int) const {
#pragma unroll
    for (int j = 0; j < EW<Cfg>::EPT; ++j) {
      const int rr = EW<Cfg>::row(j), cc = EW<Cfg>::col(j);
      const int r = m0 + rr, c = n0 + cc;
      if (r >= R || c >= D) continue;
      const int64_t o = (int64_t)r * D + c;
      const float m = pre.sc[j] * C[rr * Cfg::CS + cc];
      float x;
      if (!parallel) {
        x = pre.xo[j] + m;
        out0[o] = x;
      } else {
        const float a = pre.xo[j];
        x = pr[0] * pre.l0[j] + pp[0] * a + pp[2] * m;
        out0[o] = x;
        out1[o] = pr[1] * pre.l1[j] + pp[1] * a + pp[3] * m;
      }
      if (next.base) next.put(o, x, pre.nx[j]);
    }
  }
};

// Softcapped logits, plus per (row, 64-column tile) softmax statistics
// (tile max m and sum of exp(l - m)) for the row-parallel CDF kernel.
struct EpiLogits {
  float* logits;
  float2* stats;  // [R][V/64] or NULL
  int V, asym;
  float cap;
  const float* cap_pn;
  template <class Cfg> struct Pre { float cp, cn, icp, icn; };
  template <class Cfg>
  __device__ Pre<Cfg> prefetch(int, int, int, int) const {
    Pre<Cfg> o;
    o.cp = asym ? cap_pn[0] : cap;
    o.cn = asym ? cap_pn[1] : cap;
    o.icp = 1.f / o.cp;
    o.icn = 1.f / o.cn;
    return o;
  }
  template <class Cfg, class P>
  __device__ void apply(const float* C, const P& pre, const void*, int m0, int n0, int R, int) const {
    static_assert(Cfg::NCOL == 64 && Cfg::THREADS == 256, "a wave holds one row of a 64-column tile");
    constexpr int EPT = EW<Cfg>::EPT;
    float v[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int rr = EW<Cfg>::row(j), cc = EW<Cfg>::col(j);
      const int r = m0 + rr, c = n0 + cc;
      v[j] = -INFINITY;
      if (r < R && c < V) {
        const float l = C[rr * Cfg::CS + cc];
        const bool pos = l >= 0.f;
        v[j] = (pos ? pre.cp : pre.cn) * tanh_fast(l * (pos ? pre.icp : pre.icn));
        logits[(int64_t)r * V + c] = v[j];
      }
    }
    if (stats) {  // wave w holds rows w + 4j of the tile, one column per lane
      float m[EPT], e[EPT];
#pragma unroll
      for (int j = 0; j < EPT; ++j) m[j] = wave_max(v[j]);
#pragma unroll
      for (int j = 0; j < EPT; ++j) e[j] = v[j] == -INFINITY ? 0.f : __expf(v[j] - m[j]);
#pragma unroll
      for (int j = 0; j < EPT; ++j) e[j] = wave_sum(e[j]);
      if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
          const int r = m0 + EW<Cfg>::row(j);
          if (r < R) stats[(int64_t)r * (V / 64) + n0 / 64] = make_float2(m[j], e[j]);
        }
      }
    }
  }
};

__global__ void commit_kernel(int32_t* pos, float* prev_raw, const float* cand_raw, int B, int D,
                              int W) {
  const int b = blockIdx.x;
  for (int k = threadIdx.x; k < D; k += blockDim.x)
    prev_raw[(int64_t)b * D + k] = cand_raw[(int64_t)b * D + k];
  if (threadIdx.x == 0) pos[b] += W;
}

// ---- host side --------------------------------------------------------------

struct WS {
  float *X0, *X1, *XIN, *QIN, *XOUT, *Q, *GATE;  // XIN, QIN: [2][Rp][D] (slot parity)
  void *Y, *HB;
  float2* STATS;
  int* SYNC;
  int nsync;
};

int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

// LM head: workgroups per 16-row tile (0 = one per 64-column tile).
constexpr int kLmHeadColWgs = 0;
// Preferred K-splits of the 4-wave GEMM stages (QKV and the LM head use
// (NB, KS) = (4, 1): one 64-column head tile per task).
constexpr int kKsO = 2, kKsUp = 2, kKsDown = 4;

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
  const int nsync = (int)(Rp / 16);
  char* sync = take(nsync * 4);
  if (w) {
    w->X0 = (float*)x0; w->X1 = (float*)x1; w->XIN = (float*)xin; w->QIN = (float*)qin;
    w->XOUT = (float*)xout;
    w->Q = (float*)q; w->GATE = (float*)gate; w->Y = y; w->HB = hb;
    w->STATS = (float2*)stats; w->SYNC = (int*)sync; w->nsync = nsync;
  }
  return off;
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
  return q;
}

int check_tensor(const AltxsQTensor& t, int64_t N, int64_t K, const char* what, int li) {
  ALTXS_REQUIRE(t.codes && t.scales, "altxs_step: layer %d %s: null tensor", li, what);
  ALTXS_REQUIRE(t.N == N && t.K == K, "altxs_step: layer %d %s: shape [%lld,%lld] != [%lld,%lld]",
                li, what, (long long)t.N, (long long)t.K, (long long)N, (long long)K);
  ALTXS_REQUIRE(t.bits == 2 || t.bits == 3 || t.bits == 4 || t.bits == 6,
                "altxs_step: layer %d %s: bits=%d", li, what, t.bits);
  ALTXS_REQUIRE(((uintptr_t)t.codes & 15) == 0 && ((uintptr_t)t.scales & 7) == 0,
                "altxs_step: layer %d %s: misaligned", li, what);
  return ALTXS_OK;
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
  ALTXS_REQUIRE(d->rope_dims >= 8 && d->rope_dims <= HD && d->rope_dims % 8 == 0,
                "altxs_step: rope_dims=%d", d->rope_dims);
  ALTXS_REQUIRE(d->gate_window >= 0 && d->gate_window <= d->D, "altxs_step: gate_window");
  ALTXS_REQUIRE(d->lora_rank == 0, "altxs_step: LoRA is not built in this version");
  ALTXS_REQUIRE(d->tokens && d->pos && d->prev_raw && d->cand_raw && d->kv && d->ws && d->logits &&
                    d->rope_cos && d->rope_sin && d->err,
                "altxs_step: null state/output pointer");
  ALTXS_REQUIRE(d->ws_bytes >= ws_bytes_needed(d), "altxs_step: workspace too small");
  if (d->aux_stream) ALTXS_REQUIRE(d->sync_events, "altxs_step: aux_stream needs sync_events");
  if (d->flags & ALTXS_F_SMEAR)
    ALTXS_REQUIRE(d->smear_w && d->smear_lambda, "altxs_step: smear params missing");
  if (d->flags & ALTXS_F_ASYM_SOFTCAP) ALTXS_REQUIRE(d->softcap_pn, "altxs_step: softcap_pn missing");
  const int kvd = d->Hkv * HD;
  for (int l = 0; l < d->n_layers; ++l) {
    const AltxsLayer& L = d->layers[l];
    int rc;
    if ((rc = check_tensor(L.qkv, d->D + 2 * kvd, d->D, "qkv", l))) return rc;
    if ((rc = check_tensor(L.o, d->D, d->D, "o", l))) return rc;
    if ((rc = check_tensor(L.up, d->F, d->D, "up", l))) return rc;
    if ((rc = check_tensor(L.down, d->D, d->F, "down", l))) return rc;
    ALTXS_REQUIRE(L.resid_mix && L.attn_scale && L.mlp_scale && L.q_gain,
                  "altxs_step: layer %d small params missing", l);
    if (d->flags & ALTXS_F_SPARSE_GATE)
      ALTXS_REQUIRE(L.attn_gate_w, "altxs_step: layer %d attn_gate_w missing", l);
  }
  int rc;
  if ((rc = check_tensor(d->emb, d->V, d->D, "emb", -1))) return rc;
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

  hipError_t embed(const Group& G, hipStream_t st) const {
    const WS& w = G.w;
    EmbedP p;
    p.emb = qt_of(d->emb); p.bits = d->emb.bits; p.V = d->V; p.D = d->D; p.W = d->W;
    p.gw = d->gate_window; p.smear = (d->flags & ALTXS_F_SMEAR) ? 1 : 0; p.eps = d->norm_eps;
    p.tokens = G.tokens; p.prev_raw = G.prev_raw; p.cand_raw = G.cand_raw;
    p.smear_w = d->smear_w; p.smear_lambda = d->smear_lambda; p.x0 = w.X0; p.err = d->err;
    p.sync = w.SYNC; p.nsync = w.nsync;
    p.mix0 = d->layers[d->slots[0].layer].resid_mix; p.xin0 = w.XIN;
    hipLaunchKernelGGL(embed_kernel, dim3(G.nb * d->W), dim3(64), 0, st, p);
    return hipGetLastError();
  }

  // QKV of slot s: RMSNorm * ln_scale of the attention input (+ sparse-gate multipliers)
  hipError_t qkv(const Group& G, int s, hipStream_t st) const {
    const WS& w = G.w;
    const int R = G.nb * d->W;
    const int64_t Rp = align_up(R, 16), D = d->D;
    const AltxsSlot& S = d->slots[s];
    const AltxsLayer& L = d->layers[S.layer];
    const bool par = S.kind == ALTXS_SLOT_PAR;
    const float* attn_in = par ? w.QIN + (s & 1) * Rp * D : w.XIN + (s & 1) * Rp * D;
    ProNorm pro{attn_in, nullptr, 0, L.ln_scale, d->norm_eps, d->D};
    pro.gate_w = (d->flags & ALTXS_F_SPARSE_GATE) ? L.attn_gate_w : nullptr;
    pro.gate_out = w.GATE; pro.gate_scale = d->gate_scale; pro.H = d->H; pro.gw = d->gate_window;
    EpiQKV epi;
    epi.q = w.Q; epi.kv = slot_kv(G, s); epi.kv_bf16 = d->kv_bf16; epi.H = d->H; epi.Hkv = d->Hkv;
    epi.W = d->W; epi.max_len = d->max_len; epi.rd = d->rope_dims; epi.pos = G.pos;
    epi.cosb = d->rope_cos; epi.sinb = d->rope_sin; epi.q_gain = L.q_gain; epi.eps = d->norm_eps;
    epi.err = d->err;
    return launch_gemm_bits<AM, 4, 1>(L.qkv.bits, qt_of(L.qkv), R, 1, 0, 0, ADirect{nullptr, 0},
                                      pro, epi, 0, st);
  }

  char* slot_kv(const Group& G, int s) const {
    const int64_t esz = d->kv_bf16 ? 2 : 4;
    return G.kv + (int64_t)s * d->B * 2 * d->Hkv * d->max_len * HD * esz;
  }

  hipError_t attn(const Group& G, int s, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) const {
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
    a.flags = AM == A_BF16 ? ALTXS_ATTN_OPS_BF16 : 0;
    hipError_t e;
    if (ev0 && (e = hipEventRecord(ev0, st)) != hipSuccess) return e;
    if ((e = altxs_launch_attn(a, st)) != hipSuccess) return e;
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
    {  // out-projection + attention residual
      EpiO epi{base_s, L.attn_scale, w.XOUT, d->D, par ? 1 : 0};
      if ((e = launch_gemm4<AM>(kKsO, L.o.bits, qt_of(L.o), R, ADirect{w.Y, 0}, ProNone{}, epi, 0,
                                st)) != hipSuccess)
        return e;
    }
    {  // MLP up + LeakyReLU(0.5)^2
      ProNorm pro{par ? lane1_in : w.XOUT, nullptr, 0, L.ln_scale, d->norm_eps, d->D};
      EpiUp epi{w.HB, d->F, hb16};
      if ((e = launch_gemm4<AM>(kKsUp, L.up.bits, qt_of(L.up), R, ADirect{nullptr, 0}, pro, epi, 0,
                                st)) != hipSuccess)
        return e;
    }
    {  // MLP down + residual / lanes
      EpiDown epi;
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
      if ((e = launch_gemm4<AM>(kKsDown, L.down.bits, qt_of(L.down), R, ADirect{w.HB, 0}, ProNone{},
                                epi, 0, st)) != hipSuccess)
        return e;
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
    {
      const int n = d->n_slots, fm = final_mode(d);
      const float* xf = (fm == 2 ? w.X1 : w.X0) + n * Rp * D;
      ProNorm pro{xf, fm == 1 ? w.X1 + n * Rp * D : nullptr, fm == 1 ? 1 : 0, 1.0f, d->norm_eps, d->D};
      EpiLogits epi{G.logits, fast_cdf ? w.STATS : nullptr, d->V,
                    (d->flags & ALTXS_F_ASYM_SOFTCAP) ? 1 : 0, d->logit_softcap, d->softcap_pn};
      if ((e = launch_gemm_bits<AM, 4, 1>(d->emb.bits, qt_of(d->emb), R, 1, 0, 0, ADirect{nullptr, 0},
                                          pro, epi, kLmHeadColWgs, st)) != hipSuccess)
        return e;
    }
    if (G.probs || G.cum) {
      if (fast_cdf && G.cum) {
        if ((e = altxs_launch_cdf_stats(G.logits, w.STATS, R, d->V, G.probs, G.cum, st)) != hipSuccess)
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

// Two segment groups on two streams.  Attention launches alternate
// A0 B0 A1 B1 ... (event dependencies), so each group's GEMM chain runs while
// the other group's attention streams the KV cache.  Every kernel computes a
// row from that row's inputs only, so the split changes no bits.
template <int AM>
hipError_t run_split(const AltxsStepDesc* d, const Group (&G)[2], hipStream_t s0, hipStream_t s1) {
  StepRun<AM> run{d};
  hipEvent_t* sync = (hipEvent_t*)d->sync_events;  // [0] fork, [1] join, [2 + 2s + g] attention done
  hipEvent_t* ev = (hipEvent_t*)d->attn_events;    // timing hook: [(g*n + s)*2 + 0/1]
  const hipStream_t st[2] = {s0, s1};
  const int n = d->n_slots;
  hipError_t e;
  if ((e = hipEventRecord(sync[0], s0)) != hipSuccess) return e;
  if ((e = hipStreamWaitEvent(s1, sync[0], 0)) != hipSuccess) return e;
  for (int g = 0; g < 2; ++g)
    if ((e = run.embed(G[g], st[g])) != hipSuccess) return e;
  for (int s = 0; s < n; ++s) {
    for (int g = 0; g < 2; ++g) {
      if ((e = run.qkv(G[g], s, st[g])) != hipSuccess) return e;
      // wait for the previous attention launch (B of slot s-1 before A of s; A of s before B of s)
      hipEvent_t prev = g == 0 ? (s > 0 ? sync[2 + 2 * (s - 1) + 1] : nullptr) : sync[2 + 2 * s];
      if (prev && (e = hipStreamWaitEvent(st[g], prev, 0)) != hipSuccess) return e;
      const int k = (g * n + s) * 2;
      if ((e = run.attn(G[g], s, st[g], ev ? ev[k] : nullptr, ev ? ev[k + 1] : nullptr)) != hipSuccess)
        return e;
      if ((e = hipEventRecord(sync[2 + 2 * s + g], st[g])) != hipSuccess) return e;
    }
    for (int g = 0; g < 2; ++g)
      if ((e = run.mlp(G[g], s, st[g])) != hipSuccess) return e;
  }
  for (int g = 0; g < 2; ++g)
    if ((e = run.head(G[g], st[g])) != hipSuccess) return e;
  if ((e = hipEventRecord(sync[1], s1)) != hipSuccess) return e;
  return hipStreamWaitEvent(s0, sync[1], 0);
}

}  // namespace

extern "C" int64_t altxs_step_workspace_bytes(const AltxsStepDesc* d) {
  if (!d) return -1;
  return ws_bytes_needed(d);
}

extern "C" int32_t altxs_step(const AltxsStepDesc* d, altxs_stream_t stream) {
  int rc = validate(d);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
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
