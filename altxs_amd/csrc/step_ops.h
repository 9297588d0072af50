// Device-side building blocks of the per-symbol step: the embedding kernel,
// the GEMM prologue/epilogue functors, the LM-head epilogue and the commit
// kernel.  Shared by the per-stage launches (step.hip) and the persistent
// layer kernel (persist.hip).
//
#pragma once
#include <string.h>

#include "common.h"
#include "gemm.h"
#include "persist.h"

namespace altxs_sk {
namespace {  // internal linkage: included by more than one translation unit

using namespace altxs;


constexpr int HD = 64;

// torch.lerp(start, end, w) (ATen's two-branch formula)
// Sums of two (three) products in one fixed rounding order: the earlier
// products rounded, the last one fused into an FMA over them.  Written out
// because the compiler, free to contract a*b + c*d either way, fuses a
// different product in different inlining contexts -- and every kernel that
// produces a value must round it alike (tiles, strips, persistent tasks).
__device__ __forceinline__ float dot2(float a, float b, float c, float d) {
  return __builtin_fmaf(c, d, a * b);
}
__device__ __forceinline__ float dot3(float a, float b, float c, float d, float e, float f) {
  return __builtin_fmaf(e, f, __builtin_fmaf(c, d, a * b));
}
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

// Dense bf16 rows (bits 16): the 8 values of run `run` of row n, one 16-byte load.
__device__ void dense_run(const QT& w, int n, int run, float (&out)[8]) {
  const int KB = w.K >> 8;
  const int k0 = 8 * run, kb = k0 >> 8, kk = k0 & 255;
  const int s = kk >> 5, lg = (kk & 31) >> 3;
  const int L = (n & 15) + 16 * lg;
  const size_t bi = (size_t)(n >> 4) * KB + kb;
  const u32x4 x = *((const u32x4*)(w.codes + bi * (512 * 16)) + L * 8 + s);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = bf16_lo(x[i]);
    out[2 * i + 1] = bf16_hi(x[i]);
  }
}

// Dense fp32 rows (bits 32): hi + mid + lo of the three bf16 planes (exact).
__device__ void dense32_run(const QT& w, int n, int run, float (&out)[8]) {
  const int KB = w.K >> 8;
  const int k0 = 8 * run, kb = k0 >> 8, kk = k0 & 255;
  const int s = kk >> 5, lg = (kk & 31) >> 3;
  const int L = (n & 15) + 16 * lg;
  const size_t plane0 = ((size_t)(n >> 4) * KB + kb) * 3;
  u32x4 x[3];
#pragma unroll
  for (int p = 0; p < 3; ++p) x[p] = *((const u32x4*)(w.codes + (plane0 + p) * (512 * 16)) + L * 8 + s);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = (bf16_lo(x[0][i]) + bf16_lo(x[1][i])) + bf16_lo(x[2][i]);
    out[2 * i + 1] = (bf16_hi(x[0][i]) + bf16_hi(x[1][i])) + bf16_hi(x[2][i]);
  }
}

__device__ void dequant_run_bits(int bits, const QT& w, int n, int run, float (&out)[8]) {
  switch (bits) {
    case 16: dense_run(w, n, run, out); break;
    case 32: dense32_run(w, n, run, out); break;
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
  int R;              // rows (B * W)
  int xcd_rows;       // one row per workgroup, R % 64 == 0: row tile t of 8 on XCD t % 8
};

constexpr int MAX_RUNS = 4;  // D <= 64 lanes * 4 runs * 8 = 2048

// One wave per row; a workgroup holds blockDim.x / 64 rows (only wave-level
// reductions, so the launch shape changes no bits).
__global__ __launch_bounds__(256) void embed_kernel(EmbedP a) {
  int r = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (a.xcd_rows) {
    int rt, j;
    xcd_row_split((int)blockIdx.x, a.R / 8, rt, j);
    r = 8 * rt + j;
  }
  if (r >= a.R) return;
  if (r == 0)
    for (int i = lane; i < a.nsync; i += 64) a.sync[i] = 0;
  const int b = r / a.W, t = r % a.W;
  const int nruns = a.D / 8;
  // Operands that do not depend on the token (resid_mix rows, smear weights
  // and lambda, the carried raw row) are loaded before the token, so they do
  // not add a memory round trip after the row's norm.
  f32x4 mx[MAX_RUNS][2][2];
  float sw[MAX_RUNS][8], prev[MAX_RUNS][8];
#pragma unroll
  for (int j = 0; j < MAX_RUNS; ++j) {
    const int run = lane + 64 * j;
    if (run >= nruns) continue;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      mx[j][0][h] = *((const f32x4*)(a.mix0 + 8 * run) + h);
      mx[j][1][h] = *((const f32x4*)(a.mix0 + a.D + 8 * run) + h);
    }
    if (a.smear) {
#pragma unroll
      for (int i = 0; i < 8; ++i) sw[j][i] = 8 * run + i < a.gw ? a.smear_w[8 * run + i] : 0.f;
      if (t == 0) {
        const float* pr = a.prev_raw + (int64_t)b * a.D + 8 * run;
#pragma unroll
        for (int i = 0; i < 8; ++i) prev[j][i] = pr[i];
      }
    }
  }
  const float lam = a.smear ? a.smear_lambda[0] : 0.f;
  auto tok_at = [&](int tt) {
    int tk = a.tokens[(int64_t)b * a.W + tt];
    if (tk < 0 || tk >= a.V) {
      if (lane == 0) flag_err(a.err, ALTXS_EDEV_TOKEN);
      tk = tk < 0 ? 0 : a.V - 1;
    }
    return tk;
  };
  const int tok = tok_at(t);
  float raw[MAX_RUNS][8];
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
      if (ptok >= 0) dequant_run_bits(a.bits, a.emb, ptok, run, prev[j]);
    }
    // g = lambda * sigmoid(raw[:gw] . w_smear)
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < MAX_RUNS; ++j) {
      const int run = lane + 64 * j;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int k = 8 * run + i;
        if (run < nruns && k < a.gw) part += raw[j][i] * sw[j][i];
      }
    }
    const float gsum = wave_sum(part);
    const float g = lam * sigmoidf(gsum);
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
    // 8 consecutive floats per lane (32-byte aligned: D % 8 == 0): vector accesses
    f32x4* xo = (f32x4*)(a.x0 + (int64_t)r * a.D + 8 * run);
    f32x4* xi = (f32x4*)(a.xin0 + (int64_t)r * a.D + 8 * run);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const f32x4 ma = mx[j][0][h], mb = mx[j][1][h];
      f32x4 vo, vi;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = x[j][4 * h + e] * inv;
        vo[e] = v;
        vi[e] = dot2(ma[e], v, mb[e], v);
      }
      xo[h] = vo;
      xi[h] = vi;
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
  int round_scale = 0;  // 1: the rsqrt factor rounded to bf16 before the products
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
    float inv = r < R ? rsqrtf(ss / (float)D + eps) : 0.f;
    if (round_scale) inv = round_bf16(inv);
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
  struct Out { float base, attn; };
  __device__ Out calc(float x, const El& e) const {
    float bs = x;
    if (skip) {
      const float sc = e.sw * (skip_self ? x : e.sk);
      bs = skip_g ? lerp_t(sc, x, sigmoidf(e.sg)) : x + sc;
    }
    const float in = dot2(e.m0, bs, e.m1, e.x0);
    return {parallel ? bs : in, in};
  }
  __device__ void put(int64_t idx, float x, const El& e) const {
    const Out o = calc(x, e);
    base[idx] = o.base;
    if (attn != base) attn[idx] = o.attn;
  }
};

// ---- per-element arithmetic of the O / UP / DOWN epilogues -----------------
// Shared by apply() (tiles of the 16-row tasks) and strip() (16 x 128 strips
// of the large-tile kernel), so both paths compile to the same operations.
__device__ __forceinline__ float o_el(float c, float sc, float base, int parallel) {
  const float a = sc * c;
  return parallel ? a : base + a;
}
__device__ __forceinline__ float up_el(float v) {
  const float lr = v > 0.f ? v : 0.5f * v;
  return lr * lr;
}
struct DownOut { float x, x1; };
__device__ __forceinline__ DownOut down_el(float c, float sc, float xo, float l0, float l1, int parallel,
                                           const float* pr, const float* pp) {
  const float m = sc * c;
  if (!parallel) return {xo + m, 0.f};
  return {dot3(pr[0], l0, pp[0], xo, pp[2], m), dot3(pr[1], l1, pp[1], xo, pp[3], m)};
}

// Strips (large-tile kernel, 256 threads): 16 rows x 128 columns, thread t
// on row t / 16, columns 8 (t % 16) .. +8 -- one sub-tile of the LDS C layout
// (16 x NCOL tiles, stride CS) -- with 16- and 32-byte vector accesses.
template <class Cfg>
__device__ __forceinline__ const float* strip_src(const float* Cst, int rr, int c8) {
  return Cst + (size_t)(c8 / Cfg::NCOL) * 16 * Cfg::CS + rr * Cfg::CS + c8 % Cfg::NCOL;
}
__device__ __forceinline__ void ld8(float (&v)[8], const float* p) {
  const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) { v[i] = a[i]; v[4 + i] = b[i]; }
}
__device__ __forceinline__ void st8(float* p, const float (&v)[8]) {
  *(f32x4*)p = f32x4{v[0], v[1], v[2], v[3]};
  *(f32x4*)(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
}

// ---- epilogues --------------------------------------------------------------

__device__ __forceinline__ int row_pos(const int32_t* pos, int W, int r) {
  return pos[r / W] + (r % W);
}

// One head (64 columns) per tile: QK-RMSNorm, RoPE, q_gain, KV-cache write.
struct EpiQKV {
  float* q;          // [R, H, 64]
  char* kv;          // this slot's cache: [B][2][Hkv][max_len][64]
  int kv_bf16, H, Hkv, W, max_len, rd;  // kv_bf16: ALTXS_KV_F32 / ALTXS_KV_BF16 / ALTXS_KV_BF16_NATURAL
  // natural layouts: window token t's K/V go to row kv_tail + t (the reference's
  // tail rows, model.py:259-461) instead of its position; -1 = at the position
  int kv_tail = -1;
  const int32_t* pos;
  const float* cosb;  // [max_len, rd/2]
  const float* sinb;
  const float* q_gain;
  float eps;
  int32_t* err;
  // Unmerged LoRA of the slot (ttt_lora.py:53-55): q/v += s * (n A^T) B^T,
  // n = the normalised input tile staged in LDS (bf16 or fp32: a_f32), D = K.
  const uint16_t *lqa = nullptr, *lqb = nullptr, *lva = nullptr, *lvb = nullptr;
  float lora_s = 0.f;
  int rank = 0, D = 0, a_f32 = 0;
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
  // t = n A^T for the 16 rows (one 16x16 MFMA tile over K = D, operands in
  // fp16: bf16 inputs convert exactly, fp32 inputs as two fp16 parts; A is
  // fp16), then v[c] += s * sum_j t[row][j] B[col][j] in fp32, j < rank <= 16.
  template <class Cfg, int CPT>
  __device__ void lora_add(float (&v)[CPT], const void* As, int kind, int head, int row,
                           int c0) const {
    __shared__ float lt[16][17];
    const uint16_t* A = kind == 0 ? lqa : lva;
    const uint16_t* Bm = kind == 0 ? lqb : lvb;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (wave == 0) {
      const int r = lane & 15, kq = 8 * (lane >> 4);
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int s = 0; s < D / 32; ++s) {
        const int k = 32 * s + kq;
        f16x8 a0, a1, b;
        if (a_f32) {
          const float* x = (const float*)As + r * lds_stride(D, A_F32) + k;
          const f32x4 lo = *(const f32x4*)x, hi = *(const f32x4*)(x + 4);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float f = i < 4 ? lo[i] : hi[i - 4];
            a0[i] = (_Float16)f;
            a1[i] = (_Float16)(f - (float)a0[i]);
          }
        } else {
          const u32x4 raw = *(const u32x4*)((const uint16_t*)As + r * lds_stride(D, A_BF16) + k);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            a0[2 * i] = (_Float16)bf16_lo(raw[i]);
            a0[2 * i + 1] = (_Float16)bf16_hi(raw[i]);
          }
        }
        if (r < rank) b = __builtin_bit_cast(f16x8, *(const u32x4*)(A + (int64_t)r * D + k));
        else b = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b, acc, 0, 0, 0);
        if (a_f32) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b, acc, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) lt[4 * (lane >> 4) + i][lane & 15] = acc[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const uint16_t* brow = Bm + (int64_t)(head * HD + c0 + i) * rank;
      float d = 0.f;
      for (int j = 0; j < rank; ++j) d += lt[row][j] * __half2float(__ushort_as_half(brow[j]));
      v[i] += lora_s * d;
    }
  }

  // Strips of the large-tile kernel (two heads of 16 rows): 8 threads per head
  // row, 8 consecutive columns each.  The RMS sum keeps apply()'s order: the
  // two 4-column partial sums of a thread are apply()'s lanes 2k and 2k + 1,
  // which its first butterfly step (XOR 1) adds; its remaining steps (XOR 2,
  // half-row mirror, row mirror over 16 lanes of 4 columns) pair the same
  // lanes as XOR 1, quad reversal and half-row mirror over these 8 threads.
  // The RoPE partner (rd / 2 columns away, a multiple of 8) is rd / 16
  // threads away.  Without LoRA, bf16 cache only.
  static constexpr bool kStrip = true;
  __device__ bool strip_ok() const {
    return rank == 0 && kv_bf16 == ALTXS_KV_BF16 && kv_tail < 0 && rd % 16 == 0 && rd <= HD;
  }
  template <class Cfg>
  __device__ void strip(const float* Cst, int r0, int n0, int R) const {
    const int rr = threadIdx.x >> 4, c8 = (threadIdx.x & 15) * 8, r = r0 + rr;
    const int cw = c8 % HD, nt = (n0 + c8) / HD;
    const int kind = nt < H ? 0 : (nt < H + Hkv ? 1 : 2);
    const int head = kind == 0 ? nt : (kind == 1 ? nt - H : nt - H - Hkv);
    const float* cs = strip_src<Cfg>(Cst, rr, c8);
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = cs[i];
    // every lane takes part in the DPP steps (rows past R included)
    const int p = r < R ? row_pos(pos, W, r) : 0;
    const bool pos_ok = p >= 0 && p < max_len;
    if (kind < 2) {
      float sa = 0.f, sb = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) sa += v[i] * v[i];
#pragma unroll
      for (int i = 4; i < 8; ++i) sb += v[i] * v[i];
      float ss = sa + sb;
      ss += dpp_f<DPP_XOR1>(ss);
      ss += dpp_f<0x1B>(ss);  // quad_perm [3, 2, 1, 0]
      ss += dpp_f<DPP_HALF_MIRROR>(ss);
      const float inv = rsqrtf(ss * (1.0f / HD) + eps);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] *= inv;
      const int half = rd >> 1, off = half / 8;
      const int pp = pos_ok ? p : 0;
      float pv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float up = __shfl_down(v[i], off, WAVE);
        const float dn = __shfl_up(v[i], off, WAVE);
        pv[i] = (cw < half) ? up : dn;
      }
      if (cw < rd) {
        const int fi = cw < half ? cw : cw - half;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float cs_ = cosb[(int64_t)pp * half + fi + i], sn_ = sinb[(int64_t)pp * half + fi + i];
          if (cw < half) v[i] = dot2(v[i], cs_, pv[i], sn_);
          else v[i] = dot2(pv[i], -sn_, v[i], cs_);
        }
      }
    }
    if (r >= R) return;
    if (kind == 0) {
      const float g = q_gain[nt];
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = v[i] * g;
      st8(q + ((int64_t)r * H + head) * HD + cw, o);
    } else if (pos_ok) {
      const int b = r / W;
      const int64_t head_base = (((int64_t)b * 2 + (kind == 2 ? 1 : 0)) * Hkv + head) * max_len * HD;
      uint16_t* tile = (uint16_t*)kv + head_base + (int64_t)(p / ALTXS_KV_TILE) * (ALTXS_KV_TILE * HD);
      const int kt = p % ALTXS_KV_TILE;
      if (kind == 1) {  // K: dims cw .. cw+7 are one 16-byte run of the tile
        u32x4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          w[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
        *(u32x4*)(tile + kv_tile_k(kt, cw)) = w;
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) tile[kv_tile_v(kt, cw + i)] = f32_to_bf16(v[i]);
      }
    } else if (cw == 0) {
      flag_err(err, ALTXS_EDEV_POS);
    }
  }

  template <class Cfg, class P>
  __device__ void apply(const float* C, const P& pre, const void* As, int m0, int n0, int R,
                        int) const {
    constexpr int TPR = P::TPR, CPT = P::CPT;
    const int row = threadIdx.x / TPR, li = threadIdx.x % TPR, c0 = li * CPT;
    const int r = m0 + row;
    const int nt = n0 / HD;
    const int kind = nt < H ? 0 : (nt < H + Hkv ? 1 : 2);
    const int head = kind == 0 ? nt : (kind == 1 ? nt - H : nt - H - Hkv);
    float v[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) v[i] = C[row * Cfg::CS + c0 + i];
    if (rank > 0 && kind != 1) lora_add<Cfg, CPT>(v, As, kind, head, row, c0);
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
        if (c < (rd >> 1)) v[i] = dot2(v[i], pre.cs[i], pv[i], pre.sn[i]);
        else if (c < rd) v[i] = dot2(pv[i], -pre.sn[i], v[i], pre.cs[i]);
      }
    }
    if (r >= R) return;
    const int p = pre.p;
    // the row the K/V go to: the position, or the window's tail row (whose
    // prefix [0, pos) must end at or before the tail)
    const int krow = kv_tail >= 0 ? kv_tail + r % W : p;
    const bool pos_ok = p >= 0 && p < max_len && (kv_tail < 0 || p - r % W <= kv_tail);
    static_assert(CPT == 4, "four consecutive columns per thread (16-byte q / K stores)");
    if (kind == 0) {  // q row: 16-byte aligned (c0 % 4 == 0)
      *(f32x4*)(q + ((int64_t)r * H + head) * HD + c0) =
          f32x4{v[0] * pre.gain, v[1] * pre.gain, v[2] * pre.gain, v[3] * pre.gain};
    } else if (pos_ok) {
      const int b = r / W;
      const int64_t head_base = (((int64_t)b * 2 + (kind == 2 ? 1 : 0)) * Hkv + head) * max_len * HD;
      if (kv_bf16 == ALTXS_KV_BF16_NATURAL) {  // natural order: 4 dims = one 8-byte store
        *(u32x2*)((uint16_t*)kv + head_base + (int64_t)krow * HD + c0) =
            u32x2{(uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                  (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16)};
      } else if (kv_bf16) {  // tiled operand layout (kv_tile_k / kv_tile_v)
        uint16_t* tile = (uint16_t*)kv + head_base + (int64_t)(krow / ALTXS_KV_TILE) * (ALTXS_KV_TILE * HD);
        const int kt = krow % ALTXS_KV_TILE;
        if (kind == 1) {  // K: dims c0 .. c0+3 are adjacent in the tile (one 8-byte store)
          *(u32x2*)(tile + kv_tile_k(kt, c0)) =
              u32x2{(uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                    (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16)};
        } else {
#pragma unroll
          for (int i = 0; i < CPT; ++i) tile[kv_tile_v(kt, c0 + i)] = f32_to_bf16(v[i]);
        }
      } else {
        *(f32x4*)((float*)kv + head_base + (int64_t)krow * HD + c0) = f32x4{v[0], v[1], v[2], v[3]};
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
      xout[(int64_t)r * D + c] = o_el(C[rr * Cfg::CS + cc], pre.sc[j], pre.base[j], parallel);
    }
  }
  static constexpr bool kStrip = true;
  __device__ bool strip_ok() const { return true; }
  template <class Cfg>
  __device__ void strip(const float* Cst, int r0, int n0, int R) const {
    const int rr = threadIdx.x >> 4, c8 = (threadIdx.x & 15) * 8, r = r0 + rr;
    if (r >= R) return;
    const float* cs = strip_src<Cfg>(Cst, rr, c8);
    const int64_t o = (int64_t)r * D + n0 + c8;
    float sc[8], base[8], out[8];
    ld8(sc, attn_scale + n0 + c8);
    if (!parallel) ld8(base, xin + o);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = o_el(cs[i], sc[i], parallel ? 0.f : base[i], parallel);
    st8(xout + o, out);
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
      const float o = up_el(C[rr * Cfg::CS + cc]);
      const int64_t idx = (int64_t)r * F + c;
      if (hb16) ((uint16_t*)h)[idx] = f32_to_bf16(o);
      else ((float*)h)[idx] = o;
    }
  }
  static constexpr bool kStrip = true;
  __device__ bool strip_ok() const { return true; }
  template <class Cfg>
  __device__ void strip(const float* Cst, int r0, int n0, int R) const {
    const int rr = threadIdx.x >> 4, c8 = (threadIdx.x & 15) * 8, r = r0 + rr;
    if (r >= R) return;
    const float* cs = strip_src<Cfg>(Cst, rr, c8);
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = up_el(cs[i]);
    const int64_t idx = (int64_t)r * F + n0 + c8;
    if (hb16) {
      u32x4 w;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = (uint32_t)f32_to_bf16(o[2 * i]) | ((uint32_t)f32_to_bf16(o[2 * i + 1]) << 16);
      *(u32x4*)((uint16_t*)h + idx) = w;
    } else {
      st8((float*)h + idx, o);
    }
  }
};

// The out-projection of a parallel slot, finished where its only reader is:
// the attention launch formed part[(r * H + h) * D + n], head h's MFMA sum
// for output column n (attn_mfma_task, OP); the GEMM (gemm_task on the packed
// tensor with scales osc, ks K-slices of H / ks heads) forms acc += scale(n, h)
// * t_h head by head from zero in each slice and adds the slices in order,
// and EpiO's o_el scales by attn_scale -- the same operations here give the
// value the separate launch stores in x_out.
struct OutFin {
  static constexpr int HMAX = 8;
  const float* part = nullptr;  // NULL: x_out comes from the out-projection launch
  const uint16_t* osc = nullptr;
  const float* attn_scale = nullptr;
  int H = 0, ks = 1;
  // loaded in a prologue, used after the k-loop: the scales stay fp16 pairs
  // as loaded (converted in value()), so nothing waits for them before it
  struct El { float t[HMAX], a; u32x2 s[HMAX / 4]; };
  __device__ El load(int r, int c, int D) const {
    El e;
    const int KB = H >> 2;
#pragma unroll
    for (int kb = 0; kb < HMAX / 4; ++kb)  // the column's four group scales of block kb
      e.s[kb] = *(const u32x2*)(osc + ((int64_t)(c >> 4) * KB + (kb < KB ? kb : 0)) * 64 + (c & 15) * 4);
#pragma unroll
    for (int h = 0; h < HMAX; ++h)
      if (h < H) e.t[h] = part[((int64_t)r * H + h) * D + c];
    e.a = attn_scale[c];
    return e;
  }
  __device__ float value(const El& e) const {
    const int hps = H / ks;
    float sum = 0.f, acc = 0.f;
#pragma unroll
    for (int h = 0; h < HMAX; ++h) {
      if (h < H) {
        const uint32_t w = e.s[h >> 2][(h & 3) >> 1];
        acc += ((h & 1) ? half_hi(w) : half_lo(w)) * e.t[h];
        if ((h + 1) % hps == 0) {  // end of a K-slice: slices added in order
          sum = h + 1 == hps ? acc : sum + acc;
          acc = 0.f;
        }
      }
    }
    return o_el(sum, e.a, 0.f, 1);
  }
};

// OF: a parallel slot whose out-projection the attention launch formed --
// the attention term comes from OutFin instead of x_out.
template <bool OF>
struct EpiDownT {
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
  OutFin ofin;  // OF: the out-projection's head terms
  template <class Cfg> struct Pre {
    float xo[EW<Cfg>::EPT], sc[EW<Cfg>::EPT], l0[EW<Cfg>::EPT], l1[EW<Cfg>::EPT];
    NextIn::El nx[EW<Cfg>::EPT];
    OutFin::El of[OF ? EW<Cfg>::EPT : 1];
  };
  template <class Cfg>
  __device__ Pre<Cfg> prefetch(int m0, int n0, int R, int) const {
    Pre<Cfg> o;
#pragma unroll
    for (int j = 0; j < EW<Cfg>::EPT; ++j) {
      const int r = m0 + EW<Cfg>::row(j), c = n0 + EW<Cfg>::col(j);
      const bool ok = r < R && c < D;
      const int64_t idx = (int64_t)r * D + c;
      if constexpr (OF) {
        if (ok) o.of[j] = ofin.load(r, c, D);
      } else {
        o.xo[j] = ok ? xout[idx] : 0.f;
      }
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
      float xo;
      if constexpr (OF) xo = ofin.value(pre.of[OF ? j : 0]);
      else xo = pre.xo[j];
      const DownOut y = down_el(C[rr * Cfg::CS + cc], pre.sc[j], xo, pre.l0[j], pre.l1[j], parallel, pr, pp);
      out0[o] = y.x;
      if (parallel) out1[o] = y.x1;
      if (next.base) next.put(o, y.x, pre.nx[j]);
    }
  }
  static constexpr bool kStrip = true;
  __device__ bool strip_ok() const { return !OF; }  // strips read x_out
  template <class Cfg>
  __device__ void strip(const float* Cst, int r0, int n0, int R) const {
    const int rr = threadIdx.x >> 4, c8 = (threadIdx.x & 15) * 8, r = r0 + rr;
    if (r >= R) return;
    const float* cs = strip_src<Cfg>(Cst, rr, c8);
    const int c = n0 + c8;
    const int64_t o = (int64_t)r * D + c;
    float sc[8], xo[8], l0[8], l1[8], x[8], x1[8];
    ld8(sc, mlp_scale + c);
    ld8(xo, xout + o);
    if (parallel) {
      ld8(l0, lane0 + o);
      ld8(l1, lane1 + o);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) l0[i] = l1[i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const DownOut y = down_el(cs[i], sc[i], xo[i], l0[i], l1[i], parallel, pr, pp);
      x[i] = y.x;
      x1[i] = y.x1;
    }
    st8(out0 + o, x);
    if (parallel) st8(out1 + o, x1);
    if (next.base) {  // the next slot's inputs (NextIn::load / put, eight at a time)
      float ex0[8], em0[8], em1[8], esk[8], esw[8], esg[8], ob[8], oa[8];
      ld8(ex0, next.x0 + o);
      ld8(em0, next.mix + c);
      ld8(em1, next.mix + D + c);
#pragma unroll
      for (int i = 0; i < 8; ++i) esk[i] = esw[i] = esg[i] = 0.f;
      if (next.skip && !next.skip_self) ld8(esk, next.skip + o);
      if (next.skip) ld8(esw, next.skip_w + c);
      if (next.skip_g) ld8(esg, next.skip_g + c);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const NextIn::Out q = next.calc(x[i], NextIn::El{ex0[i], esk[i], esw[i], esg[i], em0[i], em1[i]});
        ob[i] = q.base;
        oa[i] = q.attn;
      }
      st8(next.base + o, ob);
      if (next.attn != next.base) st8(next.attn + o, oa);
    }
  }
};
using EpiDown = EpiDownT<false>;

// The MLP-up prologue of a sequential slot whose out-projection terms the
// attention launch formed (attn_mfma_task, OP): every column task needs the
// slot's whole x_out rows for the RMS norm, so each forms them (OutFin's
// arithmetic, plus the residual base of EpiO) in LDS -- the first column task
// also stores them for the MLP-down epilogue -- and then normalises them with
// ProNorm's arithmetic and lane layout.
struct ProOutNorm {
  static constexpr bool kStage = true;
  static constexpr int XS = 512 + 4;  // LDS row stride of the staged x_out (floats)
  static constexpr size_t kScratch = (size_t)16 * XS * 4;
  static constexpr int HMAX = OutFin::HMAX;
  OutFin of;                // part, osc, attn_scale, H, ks
  const float* xin;         // residual base
  float* xout;              // [R, D], stored by the first column task
  float scale, eps;
  int D;
  // D = 256 or 512 (out_proj_fused): D / 4 column quads divide the NT threads
  // into NT / (D / 4) row groups that cover the task's 16 rows exactly
  template <int AM, int NT>
  __device__ void stage(void* As, void* scratch, int m0, int R, int K, int, bool first) const {
    static_assert(NT == 16 * PTPR, "one row per 16 lanes, 16 rows per task");
    float* xs = (float*)scratch;
    const int t = threadIdx.x;
    {  // x_out of the task's rows, four columns per thread
      const int nq = D >> 2, rgs = NT / nq, cq = t % nq, rg = t / nq;
      const int c0 = 4 * cq, KB = of.H >> 2, hps = of.H / of.ks, H = of.H;
      // 16 scales per block: columns c0 .. c0+3 x the block's four groups,
      // kept as loaded (fp16 pairs) until their first use, so that the first
      // rows' term loads are issued before anything waits for them
      u32x4 sraw[HMAX / 4][2];
#pragma unroll
      for (int kb = 0; kb < HMAX / 4; ++kb) {
        const int kbc = kb < KB ? kb : 0;
        const uint16_t* sp = of.osc + ((int64_t)(c0 >> 4) * KB + kbc) * 64 + (c0 & 15) * 4;
        sraw[kb][0] = *(const u32x4*)sp;
        sraw[kb][1] = *(const u32x4*)(sp + 8);
      }
      const f32x4 asc = *(const f32x4*)(of.attn_scale + c0);
      auto scl = [&](int h, int e) {  // scale of head h (block h / 4, group h % 4), column c0 + e
        const u32x4& w = sraw[h >> 2][e >> 1];
        const uint32_t v = w[2 * (e & 1) + ((h & 3) >> 1)];
        return (h & 1) ? half_hi(v) : half_lo(v);
      };
      for (int i0 = 0; i0 < 16 / rgs; i0 += 2) {
        if (m0 + rgs * i0 >= R) break;  // no row of this pair is below R in any thread
        f32x4 tv[2][HMAX], base[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {  // every load on every path (rows past R read row R - 1)
          const int r = m0 + rg + rgs * (i0 + u), rc = r < R ? r : R - 1;
#pragma unroll
          for (int h = 0; h < HMAX; ++h)
            if (h < H) tv[u][h] = *(const f32x4*)(of.part + ((int64_t)rc * H + h) * D + c0);
          base[u] = *(const f32x4*)(xin + (int64_t)rc * D + c0);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int row = rg + rgs * (i0 + u), r = m0 + row;
          if (r >= R) continue;
          float xo[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float sum = 0.f, acc = 0.f;
#pragma unroll
            for (int h = 0; h < HMAX; ++h) {
              if (h < H) {
                acc += scl(h, e) * tv[u][h][e];
                if ((h + 1) % hps == 0) {  // end of a K-slice: slices added in order
                  sum = h + 1 == hps ? acc : sum + acc;
                  acc = 0.f;
                }
              }
            }
            xo[e] = o_el(sum, asc[e], base[u][e], 0);
          }
          const f32x4 o = {xo[0], xo[1], xo[2], xo[3]};
          *(f32x4*)(xs + row * XS + c0) = o;
          if (first) *(f32x4*)(xout + (int64_t)r * D + c0) = o;
        }
      }
      __syncthreads();
    }
    // ProNorm (lane_mode 0, no gate, unrounded scale) on the staged rows
    const int row = t / PTPR, li = t % PTPR;
    const int r = m0 + row;
    const int nch = D >> 2;
    f32x4 v[PMAXJ];
#pragma unroll
    for (int j = 0; j < PMAXJ; ++j) {
      const int c = li + PTPR * j;
      if (c < nch && r < R) v[j] = *(const f32x4*)(xs + row * XS + 4 * c);
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < PMAXJ; ++j) {
      const int c = li + PTPR * j;
      if (c >= nch) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float y = r < R ? v[j][e] : 0.f;
        v[j][e] = y;
        ss += y * y;
      }
    }
    ss = row16_sum(ss);
    const float inv = r < R ? rsqrtf(ss / (float)D + eps) : 0.f;
#pragma unroll
    for (int j = 0; j < PMAXJ; ++j) {
      const int c = li + PTPR * j;
      if (c >= nch) continue;
      float n[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) n[e] = (v[j][e] * inv) * scale;
      a_store4<AM>(As, row, 4 * c, K, n);
    }
  }
};


__device__ __forceinline__ float softcap_el(float l, float cp, float cn, float icp, float icn) {
  const bool pos = l >= 0.f;
  return (pos ? cp : cn) * tanh_fast(l * (pos ? icp : icn));
}

// Softcapped logits, plus per (row, 64-column tile) softmax statistics
// (tile max m and sum of exp(l - m)) for the chunked CDF kernel.
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
        v[j] = softcap_el(C[rr * Cfg::CS + cc], pre.cp, pre.cn, pre.icp, pre.icn);
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
  // strips only without tile statistics (the one-row CDF kernel reads none)
  static constexpr bool kStrip = true;
  __device__ bool strip_ok() const { return stats == nullptr; }
  template <class Cfg>
  __device__ void strip(const float* Cst, int r0, int n0, int R) const {
    const int rr = threadIdx.x >> 4, c8 = (threadIdx.x & 15) * 8, r = r0 + rr;
    if (r >= R) return;
    const float* cs = strip_src<Cfg>(Cst, rr, c8);
    const Pre<Cfg> pre = prefetch<Cfg>(0, 0, 0, 0);
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = softcap_el(cs[i], pre.cp, pre.cn, pre.icp, pre.icn);
    st8(logits + (int64_t)r * V + n0 + c8, o);
  }
};

__global__ void commit_kernel(int32_t* pos, float* prev_raw, const float* cand_raw, int B, int D,
                              int W) {
  const int b = blockIdx.x;
  for (int k = threadIdx.x; k < D; k += blockDim.x)
    prev_raw[(int64_t)b * D + k] = cand_raw[(int64_t)b * D + k];
  if (threadIdx.x == 0) pos[b] += W;
}

}  // namespace
}  // namespace altxs_sk
