// Decode / window attention over the KV cache (one query row at a time).
//
// Workgroup = ATT_WAVES waves for one (query row r, kv head g); it serves the
// G = H/Hkv query heads of that group so each K/V byte is read once.  Keys
// [0, p] (p = pos[b] + t) are cut into fixed 64-key tiles from position 0;
// tile T goes to wave T % ATT_WAVES, so at any moment the waves of a
// workgroup read neighbouring tiles (a few long DRAM streams instead of one
// per wave).  Each wave keeps an online softmax (fp32) over its tiles; the
// per-wave partials (m, l, acc[64]) are merged in wave order through LDS.
// Everything depends only on p, never on the batch or window size, so a row
// gives the same bits as a decode row (W = 1) and inside an encode window.
//
// bf16 cache (attn_mfma_kernel): both products run on v_mfma_f32_16x16x32_bf16
// the way the reference's split-prefix kernel uses tl.dot
// (src/xsa_ttt/split_attn.py:55-152): q padded to 16 MFMA columns (column n
// holds head n % G), scores = K-tile x q, then P x V with P the exp'd scores.
// The K and V tiles are stored pre-swizzled (kv_tile_index below) so that every
// lane's MFMA operand is one 16-byte load and a wave's load instruction reads
// 1 KB of consecutive bytes.  Operand precision:
//   * OPS_BF16: q and P rounded to bf16 (the reference's production arithmetic);
//   * fp32-faithful: q split into three bf16 parts and P into three, each part
//     multiplied separately (sum of parts reproduces fp32 to ~2^-24).
// fp32 cache (attn_valu_kernel): plain fp32 FMAs on the natural [key][64] layout.
//
// Epilogue: XSA (subtract the projection onto the current value direction,
// src/xsa_ttt/model.py:760-768), the sparse attention gate multiplier, store.
#include "common.h"
#include "kernels.h"

#ifndef ALTXS_ATT_WAVES
#define ALTXS_ATT_WAVES 4  // waves per workgroup (tile T goes to wave T % waves)
#endif

namespace {

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

template <int G, int NP, int YBF16>
__global__ __launch_bounds__(ATT_THREADS) void attn_mfma_kernel(AttnP a) {
  static_assert(TILE == 64, "the MFMA tiling below assumes 64-key tiles");
  __shared__ MergeLds<G> sm;
  const int r = blockIdx.x / a.Hkv, g = blockIdx.x % a.Hkv;
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

  for (int T = wave; T < ntiles; T += ATT_WAVES) {
    const u32x4* kt = (const u32x4*)(kb + (int64_t)T * (TILE * HD)) + lane;
    const u32x4* vt = (const u32x4*)(vb + (int64_t)T * (TILE * HD)) + lane;
    u32x4 kr[8], vr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) kr[i] = __builtin_nontemporal_load(kt + 64 * i);
#pragma unroll
    for (int i = 0; i < 8; ++i) vr[i] = __builtin_nontemporal_load(vt + 64 * i);
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
// fp32 cache: VALU kernel on the natural [key][64] layout.
// ---------------------------------------------------------------------------

// Lanes: LPK = 16 lanes share a key (4 dims each); KPI = 4 keys per load.
constexpr int V_EPL = 4, V_LPK = HD / V_EPL, V_KPI = WAVE / V_LPK, V_NI = TILE / V_KPI;

// v[0..N) partial sums over LPK lanes -> lane keeps the full sum of index lane%LPK.
template <int N, int LPK>
__device__ __forceinline__ float transpose_reduce(float (&v)[N], int lane) {
  static_assert(N == LPK, "one value per lane after the reduction");
#pragma unroll
  for (int step = LPK / 2, half = N / 2; step >= 1; step >>= 1, half >>= 1) {
    const bool up = (lane & step) != 0;
#pragma unroll
    for (int j = 0; j < half; ++j) {
      const float send = up ? v[j] : v[j + half];
      const float keep = up ? v[j + half] : v[j];
      v[j] = keep + __shfl_xor(send, step, WAVE);
    }
  }
  return v[0];
}

template <int G, int YBF16>
__global__ __launch_bounds__(ATT_THREADS) void attn_valu_kernel(AttnP a) {
  __shared__ MergeLds<G> sm;
  const int r = blockIdx.x / a.Hkv, g = blockIdx.x % a.Hkv;
  const int b = r / a.W, t = r % a.W;
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  const int p = clamp_pos(a, b, t);
  const int nkeys = p + 1;
  const int ntiles = (nkeys + TILE - 1) / TILE;
  const float* kb = (const float*)a.k + (int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD;
  const float* vb = (const float*)a.v + (int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD;
  const int dslice = V_EPL * (lane % V_LPK);
  const int ksub = lane / V_LPK;
  float qv[G][V_EPL];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const float* qh = a.q + ((int64_t)r * a.H + g * G + j) * HD + dslice;
#pragma unroll
    for (int e = 0; e < V_EPL; ++e) qv[j][e] = qh[e] * 0.125f;
  }
  float m_run[G], l_run[G], acc[G][V_EPL];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    m_run[j] = -INFINITY;
    l_run[j] = 0.f;
#pragma unroll
    for (int e = 0; e < V_EPL; ++e) acc[j][e] = 0.f;
  }
  for (int T = wave; T < ntiles; T += ATT_WAVES) {
    const int k0 = T * TILE;
    f32x4 kr[V_NI], vr[V_NI];
#pragma unroll
    for (int i = 0; i < V_NI; ++i)
      kr[i] = __builtin_nontemporal_load((const f32x4*)(kb + (int64_t)(k0 + V_KPI * i + ksub) * HD + dslice));
#pragma unroll
    for (int i = 0; i < V_NI; ++i)
      vr[i] = __builtin_nontemporal_load((const f32x4*)(vb + (int64_t)(k0 + V_KPI * i + ksub) * HD + dslice));
    const int my_key = k0 + V_KPI * (lane % V_LPK) + ksub;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      float s[V_NI];
#pragma unroll
      for (int i = 0; i < V_NI; ++i) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < V_EPL; ++e) d += qv[j][e] * kr[i][e];
        s[i] = d;
      }
      float sc = transpose_reduce<V_NI, V_LPK>(s, lane);
      if (my_key >= nkeys) sc = -INFINITY;
      const float m_new = fmaxf(m_run[j], wave_max(sc));
      const float alpha = __expf(m_run[j] - m_new);
      const float pl = __expf(sc - m_new);
      l_run[j] = l_run[j] * alpha + pl;
#pragma unroll
      for (int e = 0; e < V_EPL; ++e) acc[j][e] *= alpha;
#pragma unroll
      for (int i = 0; i < V_NI; ++i) {
        const float pk = __shfl(pl, (lane & ~(V_LPK - 1)) | i, WAVE);
#pragma unroll
        for (int e = 0; e < V_EPL; ++e) acc[j][e] += pk * vr[i][e];
      }
      m_run[j] = m_new;
    }
  }
#pragma unroll
  for (int j = 0; j < G; ++j) {
#pragma unroll
    for (int e = 0; e < V_EPL; ++e) {
#pragma unroll
      for (int msk = V_LPK; msk < WAVE; msk <<= 1) acc[j][e] += __shfl_xor(acc[j][e], msk, WAVE);
    }
    const float lsum = wave_sum(l_run[j]);
    if (lane < V_LPK) {
#pragma unroll
      for (int e = 0; e < V_EPL; ++e) sm.acc[wave][j][dslice + e] = acc[j][e];
    }
    if (lane == 0) {
      sm.m[wave][j] = m_run[j];
      sm.l[wave][j] = lsum;
    }
  }
  __syncthreads();
  merge_and_store<G, YBF16>(a, sm, r, g, p, wave, lane,
                            [&](int pp, int d) { return vb[(int64_t)pp * HD + d]; });
}

template <int YBF16>
hipError_t launch_y(const AttnP& p, int group, bool kv_bf16, bool ops_bf16, hipStream_t s) {
  dim3 grid((unsigned)(p.B * p.W * p.Hkv)), block(ATT_THREADS);
#define ATT_GO(K) \
  do { hipLaunchKernelGGL(K, grid, block, 0, s, p); return hipGetLastError(); } while (0)
  if (kv_bf16) {
    if (ops_bf16) {
      if (group == 1) ATT_GO((attn_mfma_kernel<1, 1, YBF16>));
      if (group == 2) ATT_GO((attn_mfma_kernel<2, 1, YBF16>));
      if (group == 4) ATT_GO((attn_mfma_kernel<4, 1, YBF16>));
    } else {
      if (group == 1) ATT_GO((attn_mfma_kernel<1, 3, YBF16>));
      if (group == 2) ATT_GO((attn_mfma_kernel<2, 3, YBF16>));
      if (group == 4) ATT_GO((attn_mfma_kernel<4, 3, YBF16>));
    }
  } else {
    if (group == 1) ATT_GO((attn_valu_kernel<1, YBF16>));
    if (group == 2) ATT_GO((attn_valu_kernel<2, YBF16>));
    if (group == 4) ATT_GO((attn_valu_kernel<4, YBF16>));
  }
#undef ATT_GO
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t altxs_launch_attn(const AltxsAttnArgs& a, hipStream_t s) {
  AttnP p;
  p.B = a.B; p.W = a.W; p.H = a.H; p.Hkv = a.Hkv; p.max_len = a.max_len;
  p.q = a.q; p.k = a.k; p.v = a.v; p.seg_stride = a.kv_seg_stride;
  p.pos = a.pos; p.gate = a.gate; p.use_xsa = a.use_xsa; p.y = a.y; p.err = a.err;
  const int group = a.H / a.Hkv;
  const bool ops_bf16 = (a.flags & ALTXS_ATTN_OPS_BF16) != 0;
  return a.y_bf16 ? launch_y<1>(p, group, a.kv_bf16 != 0, ops_bf16, s)
                  : launch_y<0>(p, group, a.kv_bf16 != 0, ops_bf16, s);
}

extern "C" int32_t altxs_decode_attn(const AltxsAttnArgs* a, altxs_stream_t stream) {
  ALTXS_REQUIRE(a && a->q && a->k && a->v && a->pos && a->y, "altxs_decode_attn: null pointer");
  ALTXS_REQUIRE(a->head_dim == HD, "altxs_decode_attn: head_dim=%d (only 64 is built)", a->head_dim);
  ALTXS_REQUIRE(a->B >= 1 && a->W >= 1 && (int64_t)a->B * a->W * a->Hkv < (1ll << 31),
                "altxs_decode_attn: bad B/W");
  ALTXS_REQUIRE(a->Hkv >= 1 && a->H % a->Hkv == 0, "altxs_decode_attn: H %% Hkv != 0");
  const int group = a->H / a->Hkv;
  ALTXS_REQUIRE(group == 1 || group == 2 || group == 4,
                "altxs_decode_attn: H/Hkv=%d not in {1,2,4}", group);
  ALTXS_REQUIRE(a->max_len >= TILE && a->max_len % TILE == 0,
                "altxs_decode_attn: max_len=%d must be a positive multiple of %d", a->max_len, TILE);
  ALTXS_REQUIRE(a->kv_seg_stride >= (int64_t)a->Hkv * a->max_len * HD,
                "altxs_decode_attn: kv_seg_stride too small");
  ALTXS_REQUIRE((a->flags & ~ALTXS_ATTN_OPS_BF16) == 0, "altxs_decode_attn: unknown flags 0x%x",
                a->flags);
  ALTXS_REQUIRE(((uintptr_t)a->k & 15) == 0 && ((uintptr_t)a->v & 15) == 0 && ((uintptr_t)a->q & 15) == 0,
                "altxs_decode_attn: q, k and v must be 16-byte aligned");
  ALTXS_CHECK_HIP(altxs_launch_attn(*a, (hipStream_t)stream));
  return ALTXS_OK;
}
