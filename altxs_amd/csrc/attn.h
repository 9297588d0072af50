// Decode attention device code shared by the standalone kernels (attn.hip)
// and the persistent layer kernel (step.hip).  See attn.hip for the design.
#pragma once
#include <type_traits>

#include "common.h"

#ifndef ALTXS_ATT_WAVES
#define ALTXS_ATT_WAVES 4  // waves per workgroup (tile T goes to wave T % waves)
#endif

namespace altxs_attn {

constexpr int ATT_WAVES = ALTXS_ATT_WAVES;
constexpr int ATT_THREADS = ATT_WAVES * WAVE;
constexpr int TILE = ALTXS_KV_TILE;
constexpr int HD = 64;

struct AttnP {
  int B, W, H, Hkv, max_len;
  const float* q;
  const void* k;
  const void* v;
  int64_t seg_stride;
  const int32_t* pos;
  const float* gate;
  int use_xsa;
  void* y;
  int32_t* err;
};

// Per-wave partial results, merged in wave order by the whole workgroup.
template <int G> struct MergeLds {
  float m[ATT_WAVES][G];
  float l[ATT_WAVES][G];
  float acc[ATT_WAVES][G][HD];
};

// Wave `wave` < G finishes query head g*G + wave: merge, XSA, gate, store.
// v_at(p, d) returns the current token's value entry.
template <int G, int YBF16, class VAt>
__device__ __forceinline__ void merge_and_store(const AttnP& a, const MergeLds<G>& sm, int r, int g,
                                                int p, int wave, int lane, VAt v_at) {
  if (wave >= G) return;
  const int j = wave, d = lane;
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < ATT_WAVES; ++w) M = fmaxf(M, sm.m[w][j]);
  float Ls = 0.f, Y = 0.f;
#pragma unroll
  for (int w = 0; w < ATT_WAVES; ++w) {
    const float mw = sm.m[w][j];
    if (mw == -INFINITY) continue;
    const float f = __expf(mw - M);
    Ls += sm.l[w][j] * f;
    Y += sm.acc[w][j][d] * f;
  }
  float y = Y / Ls;
  const int h = g * G + j;
  if (a.use_xsa) {
    const float vv = v_at(p, d);
    const float nrm = sqrtf(wave_sum(vv * vv));
    const float vn = vv / fmaxf(nrm, 1e-12f);
    const float dot = wave_sum(y * vn);
    y = y - dot * vn;
  }
  if (a.gate) y *= a.gate[(int64_t)r * a.H + h];
  const int64_t o = ((int64_t)r * a.H + h) * HD + d;
  if (YBF16) ((uint16_t*)a.y)[o] = f32_to_bf16(y);
  else ((float*)a.y)[o] = y;
}

__device__ __forceinline__ int clamp_pos(const AttnP& a, int b, int t) {
  int p = a.pos[b] + t;
  if (p < 0 || p >= a.max_len) {
    if (threadIdx.x == 0) flag_err(a.err, ALTXS_EDEV_POS);
    p = p < 0 ? 0 : a.max_len - 1;
  }
  return p;
}

// ---------------------------------------------------------------------------
// bf16 cache: MFMA kernel.
// ---------------------------------------------------------------------------

// bf16x8 from 8 floats, plus (optionally) the rounding residues as further parts.
template <int NP>
__device__ __forceinline__ void split_parts(const float (&x)[8], bf16x8 (&out)[NP]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float rem = x[i];
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const __bf16 h = (__bf16)rem;
      out[k][i] = h;
      rem -= (float)h;
    }
  }
}

// One (query row r, kv head g) of the bf16-cache attention: ATT_WAVES waves.
// PF = 1: each wave keeps its next tile's loads in flight while it computes the
// current one (two register buffers), for launches with one workgroup per CU;
// the arithmetic, and so the result, is the same for PF = 0 and 1.
template <int G, int NP, int YBF16, int PF = 0>
__device__ __forceinline__ void attn_mfma_task(const AttnP& a, int r, int g, MergeLds<G>& sm) {
  static_assert(TILE == 64, "the MFMA tiling below assumes 64-key tiles");
  const int b = r / a.W, t = r % a.W;
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  const int lg = lane >> 4, col = lane & 15;
  const int p = clamp_pos(a, b, t);
  const int nkeys = p + 1;
  const int ntiles = (nkeys + TILE - 1) / TILE;
  const uint16_t* kb = (const uint16_t*)a.k + (int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD;
  const uint16_t* vb = (const uint16_t*)a.v + (int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD;

  // q operand (B of the score MFMA): column col holds head col % G; k-step ks
  // covers dims 32*ks + 8*lg + [0, 8).  Scaled by 1/sqrt(64) (exact).
  bf16x8 qop[2][NP];
  {
    const float* qh = a.q + ((int64_t)r * a.H + g * G + (col % G)) * HD;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const f32x4 lo = *(const f32x4*)(qh + 32 * ks + 8 * lg);
      const f32x4 hi = *(const f32x4*)(qh + 32 * ks + 8 * lg + 4);
      float x[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) { x[i] = lo[i] * 0.125f; x[4 + i] = hi[i] * 0.125f; }
      split_parts<NP>(x, qop[ks]);
    }
  }
  float m_run = -INFINITY, l_part = 0.f;
  f32x4 acc[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto load = [&](u32x4 (&kr)[8], u32x4 (&vr)[8], int T) {
    const u32x4* kt = (const u32x4*)(kb + (int64_t)T * (TILE * HD)) + lane;
    const u32x4* vt = (const u32x4*)(vb + (int64_t)T * (TILE * HD)) + lane;
#pragma unroll
    for (int i = 0; i < 8; ++i) kr[i] = __builtin_nontemporal_load(kt + 64 * i);
#pragma unroll
    for (int i = 0; i < 8; ++i) vr[i] = __builtin_nontemporal_load(vt + 64 * i);
  };
  auto process = [&](const u32x4 (&kr)[8], const u32x4 (&vr)[8], int T) {
    // scores: S[blk] row 4*lg + i = key 16*blk + 4*lg + i, column col
    f32x4 S[4];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      S[blk] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 kop = __builtin_bit_cast(bf16x8, kr[2 * blk + ks]);
#pragma unroll
        for (int k = 0; k < NP; ++k)
          S[blk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qop[ks][k], S[blk], 0, 0, 0);
      }
    }
    const int k0 = T * TILE;
    float mt = -INFINITY;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (k0 + 16 * blk + 4 * lg + i >= nkeys) S[blk][i] = -INFINITY;
        mt = fmaxf(mt, S[blk][i]);
      }
    mt = rows_max(mt);
    const float m_new = fmaxf(m_run, mt);
    const float alpha = __expf(m_run - m_new);
    float ps = 0.f;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        S[blk][i] = __expf(S[blk][i] - m_new);
        ps += S[blk][i];
      }
    l_part = l_part * alpha + ps;
    m_run = m_new;
    // acc rows 4*lg + i hold head i % G; this lane's alpha is head col % G's.
    float al[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (G == 1) al[i] = alpha;
      else al[i] = __shfl(alpha, (lane & ~(G - 1)) | (i % G), WAVE);
    }
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[nb][i] *= al[i];
    // P x V: k-step s covers keys of blocks 2s and 2s+1 (this lane's own scores)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float pv[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) { pv[i] = S[2 * s][i]; pv[4 + i] = S[2 * s + 1][i]; }
      bf16x8 pop[NP];
      split_parts<NP>(pv, pop);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const bf16x8 vop = __builtin_bit_cast(bf16x8, vr[4 * s + nb]);
#pragma unroll
        for (int k = 0; k < NP; ++k)
          acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pop[k], vop, acc[nb], 0, 0, 0);
      }
    }
  };

  if constexpr (PF == 0) {
    for (int T = wave; T < ntiles; T += ATT_WAVES) {
      u32x4 kr[8], vr[8];
      load(kr, vr, T);
      process(kr, vr, T);
    }
  } else {
    // two buffers: A holds tiles wave + 2j*W, B tiles wave + (2j+1)*W
    u32x4 ka[8], va[8], kb2[8], vb2[8];
    int T = wave;
    if (T < ntiles) load(ka, va, T);
    for (; T < ntiles; T += 2 * ATT_WAVES) {
      const int T1 = T + ATT_WAVES, T2 = T + 2 * ATT_WAVES;
      if (T1 < ntiles) load(kb2, vb2, T1);
      process(ka, va, T);
      if (T2 < ntiles) load(ka, va, T2);
      if (T1 < ntiles) process(kb2, vb2, T1);
    }
  }
  // l: this lane's keys only; add the four lane groups (fixed butterfly).
  l_part = rows_sum(l_part);
  // acc row h (lane group 0, register h) is head h for h < G: dims 16*nb + col.
  if (lg == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) sm.acc[wave][h][16 * nb + col] = acc[nb][h];
  }
  if (lane < G) {
    sm.m[wave][lane] = m_run;
    sm.l[wave][lane] = l_part;
  }
  __syncthreads();
  merge_and_store<G, YBF16>(a, sm, r, g, p, wave, lane, [&](int pp, int d) {
    return bf16_to_f32(vb[(int64_t)(pp / TILE) * (TILE * HD) + kv_tile_v(pp % TILE, d)]);
  });
}

// ---------------------------------------------------------------------------
// bf16 cache, windows (W > 1): 16*NG consecutive query rows of one segment and
// one query head per workgroup, so each K/V tile is read once for all of them.
// Every query column performs exactly the decode task's arithmetic: the same
// MFMA operand placement for its scores and P x V, tile T on wave T mod 4, the
// same online softmax and the same wave-order merge.  Tiles past a query's
// own last key are fully masked for it; they leave its running state
// unchanged (alpha = 1, P = 0, and a wave that has seen no key keeps
// m = -inf), so a window row gives the bits of the decode row.
// ---------------------------------------------------------------------------

struct WinLds {
  float m[ATT_WAVES][16];
  float l[ATT_WAVES][16];
  float acc[ATT_WAVES][16][HD];
};

template <int NG, int NP, int YBF16>
__device__ __forceinline__ void attn_window_task(const AttnP& a, int b, int h, int t0, WinLds& sm) {
  static_assert(TILE == 64, "the MFMA tiling below assumes 64-key tiles");
  const int G = a.H / a.Hkv, g = h / G;
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  const int lg = lane >> 4, col = lane & 15;
  const uint16_t* kb = (const uint16_t*)a.k + (int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD;
  const uint16_t* vb = (const uint16_t*)a.v + (int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD;
  const int base = a.pos[b];
  // this lane's query column in each group: window index t, position p (-1: inactive)
  int pc[NG];
  bf16x8 qop[NG][2][NP];
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    const int t = t0 + 16 * gi + col;
    int p = -1;
    if (t < a.W) {
      p = base + t;
      if (p < 0 || p >= a.max_len) {
        flag_err(a.err, ALTXS_EDEV_POS);
        p = p < 0 ? 0 : a.max_len - 1;
      }
    }
    pc[gi] = p;
    const float* qh = a.q + ((int64_t)(b * a.W + (t < a.W ? t : 0)) * a.H + h) * HD;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      float x[8];
      if (t < a.W) {
        const f32x4 lo = *(const f32x4*)(qh + 32 * ks + 8 * lg);
        const f32x4 hi = *(const f32x4*)(qh + 32 * ks + 8 * lg + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) { x[i] = lo[i] * 0.125f; x[4 + i] = hi[i] * 0.125f; }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = 0.f;
      }
      split_parts<NP>(x, qop[gi][ks]);
    }
  }
  // keys to visit: up to the last active query of the workgroup (uniform)
  const int t_last = (t0 + 16 * NG < a.W ? t0 + 16 * NG : a.W) - 1;
  int p_last = base + t_last;
  p_last = p_last < 0 ? 0 : (p_last >= a.max_len ? a.max_len - 1 : p_last);
  const int ntiles = (p_last + TILE) / TILE;

  float m_run[NG], l_part[NG];
  f32x4 acc[NG][4];
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    m_run[gi] = -INFINITY;
    l_part[gi] = 0.f;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[gi][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // tile T of the K and V caches -> registers (one 16-byte load per lane each).
  // Ordinary (temporal) loads: every query block of this (segment, head) reads
  // the same tiles, and they are meant to stay in L2 between the blocks.
  auto load_t = [&](u32x4 (&kr)[8], u32x4 (&vr)[8], int T) {
    const u32x4* kt = (const u32x4*)(kb + (int64_t)T * (TILE * HD)) + lane;
    const u32x4* vt = (const u32x4*)(vb + (int64_t)T * (TILE * HD)) + lane;
#pragma unroll
    for (int i = 0; i < 8; ++i) kr[i] = kt[64 * i];
#pragma unroll
    for (int i = 0; i < 8; ++i) vr[i] = vt[64 * i];
  };
  // MASK = false: a tile whose keys all precede every query of the workgroup
  // (no key is masked for any of them, so skipping the mask changes nothing)
  auto tile = [&](const u32x4 (&kr)[8], const u32x4 (&vr)[8], int T, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int k0 = T * TILE;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      f32x4 S[4];
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        S[blk] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const bf16x8 kop = __builtin_bit_cast(bf16x8, kr[2 * blk + ks]);
#pragma unroll
          for (int k = 0; k < NP; ++k)
            S[blk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qop[gi][ks][k], S[blk], 0, 0, 0);
        }
      }
      float mt = -INFINITY;
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (MASK && k0 + 16 * blk + 4 * lg + i > pc[gi]) S[blk][i] = -INFINITY;
          mt = fmaxf(mt, S[blk][i]);
        }
      mt = rows_max(mt);
      const float m_new = fmaxf(m_run[gi], mt);
      // A query with no key seen yet (m_new = -inf) subtracts 0 instead: its
      // scores give exp(-inf) = 0 and alpha = 0, which leaves its state (l = 0,
      // acc = 0) exactly as alpha = 1 and P = 0 would.
      const float mu = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __expf(m_run[gi] - mu);
      float ps = 0.f;
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          S[blk][i] = __expf(S[blk][i] - mu);
          ps += S[blk][i];
        }
      l_part[gi] = l_part[gi] * alpha + ps;
      m_run[gi] = m_new;
      // acc row 4*lg + i is query column 4*lg + i: its alpha lives on that lane
      float al[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * lg + i, WAVE);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[gi][nb][i] *= al[i];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float pv[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) { pv[i] = S[2 * s][i]; pv[4 + i] = S[2 * s + 1][i]; }
        bf16x8 pop[NP];
        split_parts<NP>(pv, pop);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          const bf16x8 vop = __builtin_bit_cast(bf16x8, vr[4 * s + nb]);
#pragma unroll
          for (int k = 0; k < NP; ++k)
            acc[gi][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pop[k], vop, acc[gi][nb], 0, 0, 0);
        }
      }
    }
  };
  // Tiles T = wave, wave + 4, ... in order, one tile in registers at a time:
  // that keeps NG = 2 at 164 VGPRs, three waves per SIMD, whose interleaving
  // hides the load latency far better than a second register buffer at one
  // wave per SIMD (288 VGPRs; cfg4: 0.93 vs 2.1 ms per slot).
  // Tiles below the diagonal of every query first, without the mask (two
  // loops rather than a branch in one: the branch costs the third wave).
  int t_first = t0 + 16 * NG <= a.W ? base + t0 : -1;  // lowest query position, all active
  t_first = t_first >= a.max_len ? -1 : t_first;
  const int nfull = t_first < 0 ? 0 : (t_first + 1) / TILE;  // tiles 0 .. nfull-1 unmasked
  int T = wave;
  for (; T < nfull; T += ATT_WAVES) {
    u32x4 kr[8], vr[8];
    load_t(kr, vr, T);
    tile(kr, vr, T, std::false_type{});
  }
  for (; T < ntiles; T += ATT_WAVES) {
    u32x4 kr[8], vr[8];
    load_t(kr, vr, T);
    tile(kr, vr, T, std::true_type{});
  }
  // merge and store, one group of 16 queries at a time (wave w: queries w, w+4, ...)
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    const float lsum = rows_sum(l_part[gi]);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) sm.acc[wave][4 * lg + i][16 * nb + col] = acc[gi][nb][i];
    if (lane < 16) {
      sm.m[wave][lane] = m_run[gi];
      sm.l[wave][lane] = lsum;
    }
    __syncthreads();
    for (int q = wave; q < 16; q += ATT_WAVES) {
      const int t = t0 + 16 * gi + q;
      if (t >= a.W) continue;
      const int r = b * a.W + t;
      int p = base + t;
      p = p < 0 ? 0 : (p >= a.max_len ? a.max_len - 1 : p);
      const int d = lane;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < ATT_WAVES; ++w) M = fmaxf(M, sm.m[w][q]);
      float Ls = 0.f, Y = 0.f;
#pragma unroll
      for (int w = 0; w < ATT_WAVES; ++w) {
        const float mw = sm.m[w][q];
        if (mw == -INFINITY) continue;
        const float f = __expf(mw - M);
        Ls += sm.l[w][q] * f;
        Y += sm.acc[w][q][d] * f;
      }
      float y = Y / Ls;
      if (a.use_xsa) {
        const float vv = bf16_to_f32(vb[(int64_t)(p / TILE) * (TILE * HD) + kv_tile_v(p % TILE, d)]);
        const float nrm = sqrtf(wave_sum(vv * vv));
        const float vn = vv / fmaxf(nrm, 1e-12f);
        const float dot = wave_sum(y * vn);
        y = y - dot * vn;
      }
      if (a.gate) y *= a.gate[(int64_t)r * a.H + h];
      const int64_t o = ((int64_t)r * a.H + h) * HD + d;
      if (YBF16) ((uint16_t*)a.y)[o] = f32_to_bf16(y);
      else ((float*)a.y)[o] = y;
    }
    __syncthreads();
  }
}

}  // namespace altxs_attn
