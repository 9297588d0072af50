// Stage-level entry points of the reference's stage-fused row path, run on the
// step's 16-row GEMM tasks:
//
//   altxs_ffn_stage_rows -- three stream-ordered launches: out-projection and
//     its rounded residual update; RMS, MLP up and the rounded leaky-square
//     activation; MLP down and the rounded residual / parallel-lane commit
//     (ffn_stage_rows, src/xsa_ttt/ac_gemv.py:455-550, with the stage kernels
//     _ffn_out_residual_rows 89-146, _ffn_up_activation_rows 148-200,
//     _ffn_down_commit_rows 202-310);
//   altxs_attn_gate -- the split attention's sparse-gate multiplier
//     sigmoid(x[:gate_n] . w_h) per (row, head) (_split_attn_reduce,
//     src/xsa_ttt/split_attn.py:291-303).
//
// Activations and the per-layer parameters (attn_scale, mlp_scale, ln,
// parallel lambdas) are all fp32 or all bf16, the reference workspace's dtype
// (persistent_step.py:307-398).  Every value the reference rounds to that
// dtype -- an explicit `.to(T.dtype.element_ty)` or bf16 tensor arithmetic --
// is rounded here at the same point; nothing is fused across such a point
// (fp contraction off).  The GEMM sums are fp32 over exact products of bf16
// values (fp32 weights: the three-plane split), one fixed order per column
// whatever the row count.
#include "common.h"
#include "gemm.h"

using namespace altxs;

namespace {

// A row-major activation or parameter buffer in the stage dtype.
struct ActP {
  void* p;
  int bf16;
  __device__ float ld(int64_t i) const {
    return bf16 ? bf16_to_f32(((const uint16_t*)p)[i]) : ((const float*)p)[i];
  }
  __device__ void st(int64_t i, float v) const {
    if (bf16) ((uint16_t*)p)[i] = f32_to_bf16(v);
    else ((float*)p)[i] = v;
  }
};
__device__ __forceinline__ float rnd(float v, int bf16) { return bf16 ? round_bf16(v) : v; }

// Stage 1 (ac_gemv.py:120-146): attn = acc -> hid; scaled = attn * a_sc;
// parallel: attn_s = scaled, else xin = xin + scaled.
struct EpiFfnOut {
  ActP hid, xin, attn_s, a_sc;
  int D, par, bf16;
  struct Pre {};
  template <class Cfg>
  __device__ Pre prefetch(int, int, int, int) const { return {}; }
  template <class Cfg, class P>
  __device__ void apply(const float* C, const P&, const void*, int m0, int n0, int R, int) const {
#pragma clang fp contract(off)
    for (int e = threadIdx.x; e < 16 * Cfg::NCOL; e += Cfg::THREADS) {
      const int r = e / Cfg::NCOL, c = e % Cfg::NCOL, row = m0 + r, col = n0 + c;
      if (row >= R || col >= D) continue;
      const int64_t i = (int64_t)row * D + col;
      const float attn = rnd(C[r * Cfg::CS + c], bf16);
      hid.st(i, attn);
      const float scaled = rnd(attn * a_sc.ld(col), bf16);
      if (par) attn_s.st(i, scaled);
      else xin.st(i, rnd(xin.ld(i) + scaled, bf16));
    }
  }
};

// Stage 2 prologue (ac_gemv.py:162-191): scale = rsqrt(mean(src^2) + eps) in
// the src dtype, then ((src * scale) * ln) in the src dtype, then the weight's
// dtype (the A tile: bf16 for bf16 weights).  One row per 16 lanes, 16 rows.
struct ProFfnNorm {
  static constexpr bool kStage = true;
  static constexpr size_t kScratch = 0;
  ActP src, ln;
  float eps;
  int D, bf16;
  template <int AM, int NT>
  __device__ void stage(void* As, void*, int m0, int R, int K, int, bool) const {
#pragma clang fp contract(off)
    constexpr int TPR = 16, MAXJ = 512 / 4 / TPR;  // D <= 512
    static_assert(NT == 16 * TPR, "one row per 16 lanes, 16 rows per task");
    const int t = threadIdx.x, row = t / TPR, li = t % TPR, r = m0 + row;
    const int nch = D >> 2;
    float v[MAXJ][4];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
      const int c = li + TPR * j;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[j][e] = (c < nch && r < R) ? src.ld((int64_t)r * D + 4 * c + e) : 0.f;
        ss += v[j][e] * v[j][e];
      }
    }
    ss = row16_sum(ss);
    const float scale = rnd(rsqrtf(ss / (float)D + eps), bf16);
    const float lnv = ln.ld(0);
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
      const int c = li + TPR * j;
      if (c >= nch) continue;
      float n[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) n[e] = r < R ? rnd(rnd(v[j][e] * scale, bf16) * lnv, bf16) : 0.f;
      a_store4<AM>(As, row, 4 * c, K, n);
    }
  }
};

// Stage 2 epilogue (ac_gemv.py:192-200): raw = acc; leaky = raw >= 0 ? raw :
// raw * 0.5; scr = leaky * leaky.
struct EpiFfnUp {
  ActP scr;
  int F, bf16;
  struct Pre {};
  template <class Cfg>
  __device__ Pre prefetch(int, int, int, int) const { return {}; }
  template <class Cfg, class P>
  __device__ void apply(const float* C, const P&, const void*, int m0, int n0, int R, int) const {
#pragma clang fp contract(off)
    for (int e = threadIdx.x; e < 16 * Cfg::NCOL; e += Cfg::THREADS) {
      const int r = e / Cfg::NCOL, c = e % Cfg::NCOL, row = m0 + r, col = n0 + c;
      if (row >= R || col >= F) continue;
      const float raw = rnd(C[r * Cfg::CS + c], bf16);
      const float neg = rnd(raw * 0.5f, bf16);
      const float leaky = raw >= 0.f ? raw : neg;
      scr.st((int64_t)row * F + col, rnd(leaky * leaky, bf16));
    }
  }
};

// Stage 3 epilogue (ac_gemv.py:244-310): mlp = acc -> hid; mlp_s = mlp *
// m_sc; parallel: lane0 = (pr0 l0 + pp0 a) + pp2 mlp_s, lane1 = (pr1 l1 +
// pp1 a) + pp3 mlp_s with a = attn_s, every product and sum rounded; else
// x = xin + mlp_s, also written to skips[skip_dst] when skip_dst >= 0.
struct EpiFfnDown {
  ActP hid, m_sc, xin, x, attn_s, lane0, lane1, pr, pp, skips;
  int D, win, par, skip_dst, bf16;
  struct Pre {};
  template <class Cfg>
  __device__ Pre prefetch(int, int, int, int) const { return {}; }
  template <class Cfg, class P>
  __device__ void apply(const float* C, const P&, const void*, int m0, int n0, int R, int) const {
#pragma clang fp contract(off)
    for (int e = threadIdx.x; e < 16 * Cfg::NCOL; e += Cfg::THREADS) {
      const int r = e / Cfg::NCOL, c = e % Cfg::NCOL, row = m0 + r, col = n0 + c;
      if (row >= R || col >= D) continue;
      const int64_t i = (int64_t)row * D + col;
      const float mlp = rnd(C[r * Cfg::CS + c], bf16);
      hid.st(i, mlp);
      const float mlp_s = rnd(mlp * m_sc.ld(col), bf16);
      if (par) {
        const float l0 = lane0.ld(i), l1 = lane1.ld(i), a = attn_s.ld(i);
        float n0 = rnd(rnd(pr.ld(0) * l0, bf16) + rnd(pp.ld(0) * a, bf16), bf16);
        n0 = rnd(n0 + rnd(pp.ld(2) * mlp_s, bf16), bf16);
        float n1 = rnd(rnd(pr.ld(1) * l1, bf16) + rnd(pp.ld(1) * a, bf16), bf16);
        n1 = rnd(n1 + rnd(pp.ld(3) * mlp_s, bf16), bf16);
        lane0.st(i, n0);
        lane1.st(i, n1);
      } else {
        const float upd = rnd(xin.ld(i) + mlp_s, bf16);
        x.st(i, upd);
        if (skip_dst >= 0) skips.st(((int64_t)skip_dst * win + row) * D + col, upd);
      }
    }
  }
};

QT qt_from(const AltxsQTensor& t) {
  QT q;
  q.codes = (const uint8_t*)t.codes;
  q.scales = (const uint16_t*)t.scales;
  q.N = (int)t.N;
  q.K = (int)t.K;
  q.bits = t.bits;
  return q;
}

// One stage on the (4 column blocks, whole K) tasks of 16 rows; dense bf16
// (bits 16) or fp32 (bits 32, fp32 A only) weights.
template <int AM, class Pro, class Epi>
hipError_t run_stage(const AltxsQTensor& w, int rows, const void* a, const Pro& pro, const Epi& epi,
                     hipStream_t s) {
  const QT q = qt_from(w);
  if (w.bits == 16) return launch_gemm<16, AM, 4, 1>(q, rows, 1, 0, 0, ADirect{a, 0}, pro, epi, 0, s);
  if constexpr (AM == A_F32) {
    if (w.bits == 32) return launch_gemm<32, AM, 4, 1>(q, rows, 1, 0, 0, ADirect{a, 0}, pro, epi, 0, s);
  }
  return hipErrorInvalidValue;
}

int check_dense(const AltxsQTensor& t, int64_t N, int64_t K, int act_bf16, const char* what) {
  ALTXS_REQUIRE(t.codes && ((uintptr_t)t.codes & 15) == 0,
                "altxs_ffn_stage_rows: %s: null or misaligned tensor", what);
  ALTXS_REQUIRE(t.bits == 16 || t.bits == 32, "altxs_ffn_stage_rows: %s: bits=%d (dense 16 or 32)", what,
                t.bits);
  ALTXS_REQUIRE(t.bits == 16 || !act_bf16,
                "altxs_ffn_stage_rows: %s: fp32 weights (bits 32) take fp32 activations", what);
  ALTXS_REQUIRE(t.N == N && t.K == K, "altxs_ffn_stage_rows: %s is [%lld, %lld], expected [%lld, %lld]",
                what, (long long)t.N, (long long)t.K, (long long)N, (long long)K);
  return ALTXS_OK;
}

__global__ __launch_bounds__(256) void attn_gate_kernel(ActP x, int64_t x_stride, ActP w, int H, int gw,
                                                        int rows, float* __restrict__ gate) {
#pragma clang fp contract(off)
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * H) return;
  const int r = i / H, h = i % H;
  float s = 0.f;
  for (int k = 0; k < gw; ++k) s += x.ld((int64_t)r * x_stride + k) * w.ld((int64_t)h * gw + k);
  gate[i] = 1.f / (1.f + expf(-s));
}

}  // namespace

extern "C" int32_t altxs_ffn_stage_rows(const AltxsFfnStageArgs* a, altxs_stream_t stream) {
  ALTXS_REQUIRE(a, "altxs_ffn_stage_rows: null arguments");
  ALTXS_REQUIRE(a->act_dtype == ALTXS_F32 || a->act_dtype == ALTXS_BF16,
                "altxs_ffn_stage_rows: act_dtype %d (fp32 or bf16)", a->act_dtype);
  const int b16 = a->act_dtype == ALTXS_BF16;
  const int64_t win = a->win, d = a->d, mlp = a->mlp;
  ALTXS_REQUIRE(win >= 1 && win <= (1 << 20), "altxs_ffn_stage_rows: win=%lld", (long long)win);
  ALTXS_REQUIRE((d == 256 || d == 512), "altxs_ffn_stage_rows: d=%lld (256 or 512)", (long long)d);
  ALTXS_REQUIRE(mlp >= 256 && mlp % 256 == 0 && mlp <= 8192,
                "altxs_ffn_stage_rows: mlp=%lld (a multiple of 256, <= 8192)", (long long)mlp);
  int rc = check_dense(a->out_w, d, d, b16, "out_w");
  if (rc) return rc;
  if ((rc = check_dense(a->up_w, mlp, d, b16, "up_w"))) return rc;
  if ((rc = check_dense(a->down_w, d, mlp, b16, "down_w"))) return rc;
  ALTXS_REQUIRE(a->y && a->hid && a->a_sc && a->src && a->scr && a->m_sc && a->ln,
                "altxs_ffn_stage_rows: null pointer");
  ALTXS_REQUIRE(((uintptr_t)a->y & 15) == 0 && ((uintptr_t)a->scr & 15) == 0,
                "altxs_ffn_stage_rows: y and scr must be 16-byte aligned");
  if (a->parallel) {
    ALTXS_REQUIRE(a->attn_s && a->lane0 && a->lane1 && a->pr && a->pp,
                  "altxs_ffn_stage_rows: parallel slot needs attn_s, lane0, lane1, pr, pp");
    ALTXS_REQUIRE(a->attn_s != a->y, "altxs_ffn_stage_rows: attn_s must not alias y");
  } else {
    ALTXS_REQUIRE(a->xin && a->x, "altxs_ffn_stage_rows: sequential slot needs xin and x");
    ALTXS_REQUIRE(a->skip_dst < 0 || a->skips, "altxs_ffn_stage_rows: skip_dst >= 0 needs skips");
  }
  ALTXS_REQUIRE(a->hid != a->y, "altxs_ffn_stage_rows: hid must not alias y");
  auto P = [&](const void* p) { return ActP{(void*)p, b16}; };
  hipStream_t s = (hipStream_t)stream;
  const int R = (int)win;

  EpiFfnOut e1{P(a->hid), P(a->xin), P(a->attn_s), P(a->a_sc), (int)d, a->parallel ? 1 : 0, b16};
  ALTXS_CHECK_HIP(b16 ? run_stage<A_BF16>(a->out_w, R, a->y, ProNone{}, e1, s)
                      : run_stage<A_F32>(a->out_w, R, a->y, ProNone{}, e1, s));

  ProFfnNorm pro{P(a->src), P(a->ln), a->eps, (int)d, b16};
  EpiFfnUp e2{P(a->scr), (int)mlp, b16};
  // the normalised row enters the MFMAs in the weight's dtype (ac_gemv.py:182)
  ALTXS_CHECK_HIP(a->up_w.bits == 16 ? run_stage<A_BF16>(a->up_w, R, nullptr, pro, e2, s)
                                     : run_stage<A_F32>(a->up_w, R, nullptr, pro, e2, s));

  EpiFfnDown e3{P(a->hid), P(a->m_sc), P(a->xin), P(a->x), P(a->attn_s), P(a->lane0), P(a->lane1),
                P(a->pr), P(a->pp), P(a->skips), (int)d, R, a->parallel ? 1 : 0,
                a->parallel ? -1 : a->skip_dst, b16};
  ALTXS_CHECK_HIP(b16 ? run_stage<A_BF16>(a->down_w, R, a->scr, ProNone{}, e3, s)
                      : run_stage<A_F32>(a->down_w, R, a->scr, ProNone{}, e3, s));
  return ALTXS_OK;
}

extern "C" int32_t altxs_attn_gate(const void* x, int32_t x_dtype, int64_t x_stride, const void* w,
                                   int32_t H, int32_t gw, int32_t rows, float* gate,
                                   altxs_stream_t stream) {
  ALTXS_REQUIRE(x && w && gate, "altxs_attn_gate: null pointer");
  ALTXS_REQUIRE(x_dtype == ALTXS_F32 || x_dtype == ALTXS_BF16, "altxs_attn_gate: x_dtype %d", x_dtype);
  ALTXS_REQUIRE(H >= 1 && H <= 256 && gw >= 1 && gw <= 4096 && rows >= 1 && rows <= (1 << 20) &&
                    x_stride >= gw,
                "altxs_attn_gate: H=%d gw=%d rows=%d x_stride=%lld", H, gw, rows, (long long)x_stride);
  const int b16 = x_dtype == ALTXS_BF16;
  const int n = rows * H;
  hipLaunchKernelGGL(attn_gate_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     ActP{(void*)x, b16}, x_stride, ActP{(void*)w, b16}, H, gw, rows, gate);
  ALTXS_CHECK_HIP(hipGetLastError());
  return ALTXS_OK;
}
