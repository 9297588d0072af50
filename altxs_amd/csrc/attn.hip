// Decode / window attention over the KV cache (one query row at a time).
//
// Workgroup = 8 waves for one (query row r, kv head g); it serves the
// H/Hkv query heads of that group so each K/V byte is read once.  Keys
// [0, p] (p = pos[b] + t) are cut into fixed 256-key chunks; chunk c goes to
// wave c % 8, which walks it in 64-key tiles:
//   * K tile: every lane issues 16-byte loads; LPK lanes share a key (each
//     holds 16 bytes of it), so a wave reads 1 KB of consecutive keys per load.
//   * partial q.k dots are transpose-reduced across those LPK lanes so each
//     of the 64 lanes ends up owning the full score of one key.
//   * online softmax per wave (fp32): tile max by wave butterfly; per-lane
//     partial sums; the accumulator holds the lane's 16-byte dim slice.
//   * V tile: same load pattern; each lane fetches the probability of the key
//     it holds a V slice of with one ds_bpermute.
// The 8 per-wave partials (m, l, acc[64]) are merged in wave order through
// LDS.  Everything depends only on p, never on the batch or window size.
// Epilogue: XSA (subtract the projection onto the current value direction,
// src/xsa_ttt/model.py:760-768), the sparse attention gate multiplier, store.
#include "common.h"
#include "kernels.h"

// Build-time knobs (the defaults are the measured best on MI355X).
#ifndef ALTXS_ATT_WAVES
#define ALTXS_ATT_WAVES 8      // waves per workgroup (chunk c goes to wave c % waves)
#endif
#ifndef ALTXS_ATT_PREFETCH
#define ALTXS_ATT_PREFETCH 1   // load the next K/V tile while computing the current one
#endif
#ifndef ALTXS_ATT_NT
#define ALTXS_ATT_NT 1         // non-temporal (streaming) K/V loads
#endif
#ifndef ALTXS_ATT_MINW
#define ALTXS_ATT_MINW 1       // min waves per SIMD the register allocation must allow
#endif

namespace {

__device__ __forceinline__ u32x4 kv_load(const u32x4* p) {
#if ALTXS_ATT_NT
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}

constexpr int ATT_WAVES = ALTXS_ATT_WAVES;
constexpr int ATT_THREADS = ATT_WAVES * WAVE;
constexpr int CHUNK = 256;
constexpr int TILE = 64;
constexpr int HD = 64;

template <int KVBF16> struct KVL;
template <> struct KVL<1> {  // bf16: 8 elements per 16-byte load
  static constexpr int EPL = 8, LPK = HD / EPL, KPI = WAVE / LPK, NI = TILE / KPI;
};
template <> struct KVL<0> {  // fp32: 4 elements per 16-byte load
  static constexpr int EPL = 4, LPK = HD / EPL, KPI = WAVE / LPK, NI = TILE / KPI;
};

template <int KVBF16>
__device__ __forceinline__ void unpack16(const u32x4& w, float (&x)[KVL<KVBF16>::EPL]) {
  if constexpr (KVBF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = bf16_lo(w[i]);
      x[2 * i + 1] = bf16_hi(w[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = __uint_as_float(w[i]);
  }
}

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

template <int KVBF16, int GROUP, int YBF16>
__global__ __launch_bounds__(ATT_THREADS, ALTXS_ATT_MINW) void attn_kernel(AttnP a) {
  using L = KVL<KVBF16>;
  constexpr int EPL = L::EPL, LPK = L::LPK, KPI = L::KPI, NI = L::NI;
  constexpr int ESZ = KVBF16 ? 2 : 4;
  __shared__ float sm_m[ATT_WAVES][GROUP];
  __shared__ float sm_l[ATT_WAVES][GROUP];
  __shared__ float sm_acc[ATT_WAVES][GROUP][HD];

  const int r = blockIdx.x / a.Hkv, g = blockIdx.x % a.Hkv;
  const int b = r / a.W, t = r % a.W;
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  int p = a.pos[b] + t;
  if (p < 0 || p >= a.max_len) {
    if (threadIdx.x == 0) flag_err(a.err, ALTXS_EDEV_POS);
    p = p < 0 ? 0 : a.max_len - 1;
  }
  const int nkeys = p + 1;
  const int nchunks = (nkeys + CHUNK - 1) / CHUNK;
  const char* kb = (const char*)a.k + ((int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD) * ESZ;
  const char* vb = (const char*)a.v + ((int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD) * ESZ;

  const int dslice = EPL * (lane % LPK);  // this lane's dims within a key
  const int ksub = lane / LPK;            // key offset within a load group
  float qv[GROUP][EPL];
#pragma unroll
  for (int j = 0; j < GROUP; ++j) {
    const float* qh = a.q + ((int64_t)r * a.H + g * GROUP + j) * HD + dslice;
#pragma unroll
    for (int e = 0; e < EPL; ++e) qv[j][e] = qh[e] * 0.125f;  // 1/sqrt(64), exact
  }
  float m_run[GROUP], l_run[GROUP], acc[GROUP][EPL];
#pragma unroll
  for (int j = 0; j < GROUP; ++j) {
    m_run[j] = -INFINITY;
    l_run[j] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[j][e] = 0.f;
  }

  // The wave's tiles, in order: chunks c = wave, wave + ATT_WAVES, ...; within
  // a chunk, 64-key tiles while k0 < nkeys.  Rows [k0, k0+64) are inside the
  // cache because max_len is a multiple of 256.
  auto load_tile = [&](u32x4 (&kr)[NI], u32x4 (&vr)[NI], int k0) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int64_t off = ((int64_t)(k0 + KPI * i + ksub) * HD + dslice) * ESZ;
      kr[i] = kv_load((const u32x4*)(kb + off));
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int64_t off = ((int64_t)(k0 + KPI * i + ksub) * HD + dslice) * ESZ;
      vr[i] = kv_load((const u32x4*)(vb + off));
    }
  };
  auto process_tile = [&](const u32x4 (&kr)[NI], const u32x4 (&vr)[NI], int k0) {
    const int my_key = k0 + KPI * (lane % LPK) + ksub;
#pragma unroll
    for (int j = 0; j < GROUP; ++j) {
      float s[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        float kx[EPL];
        unpack16<KVBF16>(kr[i], kx);
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) d += qv[j][e] * kx[e];
        s[i] = d;
      }
      float sc = transpose_reduce<NI, LPK>(s, lane);
      if (my_key >= nkeys) sc = -INFINITY;
      const float m_new = fmaxf(m_run[j], wave_max(sc));
      const float alpha = __expf(m_run[j] - m_new);
      const float pl = __expf(sc - m_new);
      l_run[j] = l_run[j] * alpha + pl;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[j][e] *= alpha;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const float pk = __shfl(pl, (lane & ~(LPK - 1)) | i, WAVE);
        float vx[EPL];
        unpack16<KVBF16>(vr[i], vx);
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[j][e] += pk * vx[e];
      }
      m_run[j] = m_new;
    }
  };
  // next tile after (c, tt) in this wave's order; false when none is left
  auto advance = [&](int& c, int& tt) {
    ++tt;
    if (tt == CHUNK / TILE || c * CHUNK + tt * TILE >= nkeys) {
      c += ATT_WAVES;
      tt = 0;
    }
    return c < nchunks;
  };
  int c = wave, tt = 0;
  bool have = c < nchunks;
  u32x4 k0r[NI], v0r[NI];
  if (have) load_tile(k0r, v0r, c * CHUNK);
#if ALTXS_ATT_PREFETCH
  u32x4 k1r[NI], v1r[NI];
  while (have) {  // two tiles per trip: ping-pong register buffers
    int c1 = c, t1 = tt;
    const bool have1 = advance(c1, t1);
    if (have1) load_tile(k1r, v1r, c1 * CHUNK + t1 * TILE);
    process_tile(k0r, v0r, c * CHUNK + tt * TILE);
    if (!have1) break;
    c = c1; tt = t1;
    int c2 = c, t2 = tt;
    have = advance(c2, t2);
    if (have) load_tile(k0r, v0r, c2 * CHUNK + t2 * TILE);
    process_tile(k1r, v1r, c * CHUNK + tt * TILE);
    c = c2; tt = t2;
  }
#else
  while (have) {
    process_tile(k0r, v0r, c * CHUNK + tt * TILE);
    have = advance(c, tt);
    if (have) load_tile(k0r, v0r, c * CHUNK + tt * TILE);
  }
#endif
  // Combine the lanes that share a dim slice (fixed butterfly), then publish.
#pragma unroll
  for (int j = 0; j < GROUP; ++j) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
#pragma unroll
      for (int msk = LPK; msk < WAVE; msk <<= 1) acc[j][e] += __shfl_xor(acc[j][e], msk, WAVE);
    }
    const float lsum = wave_sum(l_run[j]);
    if (lane < LPK) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) sm_acc[wave][j][dslice + e] = acc[j][e];
    }
    if (lane == 0) {
      sm_m[wave][j] = m_run[j];
      sm_l[wave][j] = lsum;
    }
  }
  __syncthreads();
  // Merge the wave partials in wave order: wave j finishes query head j.
  if (wave < GROUP) {
    const int j = wave, d = lane;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) M = fmaxf(M, sm_m[w][j]);
    float Ls = 0.f, Y = 0.f;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) {
      const float mw = sm_m[w][j];
      if (mw == -INFINITY) continue;
      const float f = __expf(mw - M);
      Ls += sm_l[w][j] * f;
      Y += sm_acc[w][j][d] * f;
    }
    float y = Y / Ls;
    const int h = g * GROUP + j;
    if (a.use_xsa) {
      const char* vc = vb + ((int64_t)p * HD + d) * ESZ;
      const float vv = KVBF16 ? bf16_to_f32(*(const uint16_t*)vc) : *(const float*)vc;
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
}

template <int KVBF16, int YBF16>
hipError_t launch_group(const AttnP& p, int group, hipStream_t s) {
  dim3 grid((unsigned)(p.B * p.W * p.Hkv)), block(ATT_THREADS);
  switch (group) {
    case 1: hipLaunchKernelGGL((attn_kernel<KVBF16, 1, YBF16>), grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL((attn_kernel<KVBF16, 2, YBF16>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL((attn_kernel<KVBF16, 4, YBF16>), grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t altxs_launch_attn(const AltxsAttnArgs& a, hipStream_t s) {
  AttnP p;
  p.B = a.B; p.W = a.W; p.H = a.H; p.Hkv = a.Hkv; p.max_len = a.max_len;
  p.q = a.q; p.k = a.k; p.v = a.v; p.seg_stride = a.kv_seg_stride;
  p.pos = a.pos; p.gate = a.gate; p.use_xsa = a.use_xsa; p.y = a.y; p.err = a.err;
  const int group = a.H / a.Hkv;
  if (a.kv_bf16) return a.y_bf16 ? launch_group<1, 1>(p, group, s) : launch_group<1, 0>(p, group, s);
  return a.y_bf16 ? launch_group<0, 1>(p, group, s) : launch_group<0, 0>(p, group, s);
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
  ALTXS_REQUIRE(a->max_len >= CHUNK && a->max_len % CHUNK == 0,
                "altxs_decode_attn: max_len=%d must be a positive multiple of %d", a->max_len, CHUNK);
  ALTXS_REQUIRE(a->kv_seg_stride >= (int64_t)a->Hkv * a->max_len * HD,
                "altxs_decode_attn: kv_seg_stride too small");
  ALTXS_CHECK_HIP(altxs_launch_attn(*a, (hipStream_t)stream));
  return ALTXS_OK;
}
