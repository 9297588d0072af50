// Deterministic softmax -> integer CDF (the frequency tables the range coder
// consumes).  One workgroup of 1024 threads per row; thread t owns the
// contiguous elements [t*EPT, t*EPT + EPT).  Every floating-point reduction
// runs in a fixed order that depends only on V, so a row's tables are the same
// whatever the number of rows in the launch (encode windows vs decode rows).
//
// Count rule (src/model/arithmetic_coder_lm.py:49-64, gpu_ac.py:38-42):
//   f = max(1, floor(double(p) * 1e6 + 0.5))   -- two IEEE double roundings
#include "common.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace {

constexpr int CDF_THREADS = 1024;
constexpr int CDF_WAVES = CDF_THREADS / WAVE;
// Renormalised rows stage the row in LDS for numpy's summation order (64 KB).
constexpr int kRenormMaxV = 16384;

__device__ __forceinline__ uint32_t scale_count(float p) {
  double t = __dmul_rn((double)p, 1000000.0);
  t = __dadd_rn(t, 0.5);
  double f = floor(t);
  if (!(f >= 1.0)) return 1u;  // max(1, .); NaN maps to 1 as numpy's int cast + max does
  if (f >= 4294967295.0) return 0xffffffffu;
  return (uint32_t)f;
}

// The same rule on a float64 probability (the reference converts every row to
// float64 first, arithmetic_coder_lm.py:58-60; an fp32 value converts exactly).
__device__ __forceinline__ uint32_t scale_count64(double p) {
  double t = __dmul_rn(p, 1000000.0);
  t = __dadd_rn(t, 0.5);
  double f = floor(t);
  if (!(f >= 1.0)) return 1u;
  if (f >= 4294967295.0) return 0xffffffffu;
  return (uint32_t)f;
}

// Fixed-order block reductions over 16 waves.
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x / WAVE, l = threadIdx.x % WAVE;
  if (l == 0) red[w] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int i = 1; i < CDF_WAVES; ++i) m = fmaxf(m, red[i]);
  __syncthreads();
  return m;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x / WAVE, l = threadIdx.x % WAVE;
  if (l == 0) red[w] = v;
  __syncthreads();
  float s = red[0];
#pragma unroll
  for (int i = 1; i < CDF_WAVES; ++i) s += red[i];
  __syncthreads();
  return s;
}

// Exclusive block scan of one uint32 per thread (exact integer arithmetic).
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* wred) {
  const int w = threadIdx.x / WAVE, l = threadIdx.x % WAVE;
  uint32_t incl = v;
#pragma unroll
  for (int d = 1; d < WAVE; d <<= 1) {
    uint32_t o = __shfl_up(incl, d, WAVE);
    if (l >= d) incl += o;
  }
  if (l == WAVE - 1) wred[w] = incl;
  __syncthreads();
  uint32_t base = 0;
  for (int i = 0; i < w; ++i) base += wred[i];
  __syncthreads();
  return base + incl - v;
}

// numpy's float32 add-reduce of a contiguous row, which the reference's
// renormalisation uses (``p /= float(p.sum())``, compress.py:64-85): the row
// is summed in chunks of NPY_BUFSIZE = 8192 elements, accumulated in order
// from 0, each chunk by numpy's pairwise_sum -- blocks of at most 128
// elements summed into 8 interleaved accumulators combined as
// ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)) plus the tail in order, larger ranges
// split at half the length rounded down to a multiple of 8, the two halves
// added.  One thread, from LDS (the row is summed once per context reset).
constexpr int kNpyBuf = 8192, kNpyBlock = 128;

__device__ float np_leaf_sum(const float* a, int n) {
  if (n < 8) {
    float r = 0.f;
    for (int i = 0; i < n; ++i) r += a[i];
    return r;
  }
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = a[j];
  int i = 8;
  for (; i < n - (n % 8); i += 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] += a[i + j];
  }
  float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (; i < n; ++i) res += a[i];
  return res;
}

__device__ float np_pairwise_sum(const float* a, int n) {
  struct Frame { int off, n, stage; float left; };
  Frame st[16];  // depth <= log2(8192 / 128) + 1
  int sp = 0;
  float ret = 0.f;
  st[sp++] = Frame{0, n, 0, 0.f};
  while (sp > 0) {
    Frame& f = st[sp - 1];
    if (f.n <= kNpyBlock) {
      ret = np_leaf_sum(a + f.off, f.n);
      --sp;
      continue;
    }
    const int n2 = f.n / 2 - (f.n / 2) % 8;
    if (f.stage == 0) {
      f.stage = 1;
      st[sp++] = Frame{f.off, n2, 0, 0.f};
    } else if (f.stage == 1) {
      f.left = ret;
      f.stage = 2;
      st[sp++] = Frame{f.off + n2, f.n - n2, 0, 0.f};
    } else {
      ret = f.left + ret;
      --sp;
    }
  }
  return ret;
}

__device__ float np_sum(const float* a, int n) {
  float acc = 0.f;
  for (int k = 0; k < n; k += kNpyBuf) acc += np_pairwise_sum(a + k, n - k < kNpyBuf ? n - k : kNpyBuf);
  return acc;
}

template <int EPT, bool FROM_LOGITS>
__global__ __launch_bounds__(CDF_THREADS) void cdf_kernel(const float* __restrict__ in,
                                                           int V, int flags,
                                                           float* __restrict__ probs,
                                                           uint32_t* __restrict__ cum) {
  __shared__ float red[CDF_WAVES];
  __shared__ uint32_t wred[CDF_WAVES];
  extern __shared__ float row_lds[];  // [V] with ALTXS_CDF_RENORM
  const int64_t row = blockIdx.x;
  const float* x = in + row * (int64_t)V;
  const int base = threadIdx.x * EPT;
  float v[EPT];
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int j = base + i;
    v[i] = (j < V) ? x[j] : 0.f;
  }
  if (FROM_LOGITS) {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < EPT; ++i)
      if (base + i < V) m = fmaxf(m, v[i]);
    m = block_max(m, red);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      v[i] = (base + i < V) ? expf(v[i] - m) : 0.f;
      s += v[i];
    }
    s = block_sum(s, red);
#pragma unroll
    for (int i = 0; i < EPT; ++i) v[i] = v[i] / s;
    if (flags & ALTXS_CDF_RENORM) {  // p /= float(p.sum()) with numpy's sum (compress.py:78-83)
#pragma unroll
      for (int i = 0; i < EPT; ++i)
        if (base + i < V) row_lds[base + i] = v[i];
      __syncthreads();
      if (threadIdx.x == 0) red[0] = np_sum(row_lds, V);
      __syncthreads();
      const float s2 = red[0];
      if (!(s2 > 0.f) || s2 == INFINITY) {  // non-positive or non-finite sum: the uniform row
        const float u = 1.0f / (float)V;
#pragma unroll
        for (int i = 0; i < EPT; ++i) v[i] = u;
      } else {
#pragma unroll
        for (int i = 0; i < EPT; ++i) v[i] = v[i] / s2;
      }
    }
    if (probs) {
      float* po = probs + row * (int64_t)V;
#pragma unroll
      for (int i = 0; i < EPT; ++i)
        if (base + i < V) po[base + i] = v[i];
    }
  }
  if (!cum) return;
  uint32_t f[EPT];
  uint32_t tot = 0;
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    f[i] = (base + i < V) ? scale_count(v[i]) : 0u;
    tot += f[i];
  }
  uint32_t run = block_excl_scan(tot, wred);
  uint32_t* co = cum + row * (int64_t)(V + 1);
  if (threadIdx.x == 0) co[0] = 0u;
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    run += f[i];
    if (base + i < V) co[base + i + 1] = run;
  }
}

// float64 probability rows -> CDF rows (one 1024-thread workgroup per row).
template <int EPT>
__global__ __launch_bounds__(CDF_THREADS) void cdf_f64_kernel(const double* __restrict__ in, int V,
                                                               uint32_t* __restrict__ cum) {
  __shared__ uint32_t wred[CDF_WAVES];
  const int64_t row = blockIdx.x;
  const double* x = in + row * (int64_t)V;
  const int base = threadIdx.x * EPT;
  uint32_t f[EPT];
  uint32_t tot = 0;
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    f[i] = (base + i < V) ? scale_count64(x[base + i]) : 0u;
    tot += f[i];
  }
  uint32_t run = block_excl_scan(tot, wred);
  uint32_t* co = cum + row * (int64_t)(V + 1);
  if (threadIdx.x == 0) co[0] = 0u;
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    run += f[i];
    if (base + i < V) co[base + i + 1] = run;
  }
}

// ---- row-parallel softmax -> CDF ---------------------------------------------
//
// Chunked form (vocabularies the one-row kernel below does not tile): the LM
// head leaves, for every (row, 64-column tile), the tile max m_t and
// s_t = sum exp(l - m_t).  Workgroup (chunk c, row) first forms the row's
// M = max m_t and S = sum s_t * exp(m_t - M) in a fixed order (identical in
// every workgroup of the row), then p_i = exp(l_i - M) * (1 / S).  Its CDF offset is
// the exact integer sum of the counts of all elements before the chunk, which
// it recomputes itself (integer sums do not depend on order), so no workgroup
// waits for another.  Its own chunk is scanned and stored.

constexpr int CH_THREADS = 1024;
constexpr int CH_WAVES = CH_THREADS / WAVE;

__device__ __forceinline__ float block_max_n(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x / WAVE, l = threadIdx.x % WAVE;
  if (l == 0) red[w] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int i = 1; i < CH_WAVES; ++i) m = fmaxf(m, red[i]);
  __syncthreads();
  return m;
}

__device__ __forceinline__ float block_sum_n(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x / WAVE, l = threadIdx.x % WAVE;
  if (l == 0) red[w] = v;
  __syncthreads();
  float s = red[0];
#pragma unroll
  for (int i = 1; i < CH_WAVES; ++i) s += red[i];
  __syncthreads();
  return s;
}

__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t* wred) {
  v = wave_sum_u32(v);
  const int w = threadIdx.x / WAVE, l = threadIdx.x % WAVE;
  if (l == 0) wred[w] = v;
  __syncthreads();
  uint32_t s = 0;
#pragma unroll
  for (int i = 0; i < CH_WAVES; ++i) s += wred[i];
  __syncthreads();
  return s;
}

template <int EPT>
__global__ __launch_bounds__(CH_THREADS) void cdf_chunk_kernel(const float* __restrict__ logits,
                                                                const float2* __restrict__ stats,
                                                                int V, int chunk,
                                                                float* __restrict__ probs,
                                                                uint32_t* __restrict__ cum) {
  __shared__ float red[CH_WAVES];
  __shared__ uint32_t wred[CH_WAVES];
  const int64_t row = blockIdx.y;
  const int c0 = blockIdx.x * chunk;
  const int t = threadIdx.x;
  const float* x = logits + row * (int64_t)V;
  const int ntile = V / 64;
  const float2* st = stats + row * (int64_t)ntile;
  // this thread's chunk elements (issued first)
  float v[EPT];
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int i = c0 + t * EPT + k;
    v[k] = i < c0 + chunk ? x[i] : 0.f;
  }
  // M, S over the tiles (fixed order: thread-strided, wave butterfly, waves in order)
  float mt = -INFINITY;
  for (int i = t; i < ntile; i += CH_THREADS) mt = fmaxf(mt, st[i].x);
  const float M = block_max_n(mt, red);
  float sp = 0.f;
  for (int i = t; i < ntile; i += CH_THREADS) {
    const float2 q = st[i];
    sp += q.y * __expf(q.x - M);
  }
  const float S = block_sum_n(sp, red);
  const float iS = 1.f / S;
  // CDF offset: counts of every element before the chunk (exact integers)
  uint32_t before = 0;
  for (int i = t; i < c0; i += CH_THREADS) before += scale_count(__expf(x[i] - M) * iS);
  const uint32_t offset = block_sum_u32(before, wred);
  // own chunk
  uint32_t f[EPT];
  uint32_t tot = 0;
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int i = c0 + t * EPT + k;
    const float p = __expf(v[k] - M) * iS;
    if (probs && i < c0 + chunk) probs[row * (int64_t)V + i] = p;
    f[k] = i < c0 + chunk ? scale_count(p) : 0u;
    tot += f[k];
  }
  uint32_t run = offset + block_excl_scan(tot, wred);
  uint32_t* co = cum + row * (int64_t)(V + 1);
  if (c0 == 0 && t == 0) co[0] = 0u;
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int i = c0 + t * EPT + k;
    run += f[k];
    if (i < c0 + chunk) co[i + 1] = run;
  }
}

// Inclusive scan over the 64 lanes of a wave (exact integers): DPP row shifts
// inside each 16-lane row (a lane whose source is across the row edge reads
// 0), then the totals of the rows before it.
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  v += dpp_u<0x111>(v);  // row_shr:1
  v += dpp_u<0x112>(v);  // row_shr:2
  v += dpp_u<0x114>(v);  // row_shr:4
  v += dpp_u<0x118>(v);  // row_shr:8
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 15);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 31);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 47);
  const int rw = (threadIdx.x % WAVE) >> 4;
  return v + (rw > 0 ? r0 : 0u) + (rw > 1 ? r1 : 0u) + (rw > 2 ? r2 : 0u);
}

// One workgroup per row, the row in registers: wave w holds the 64-column
// tiles w, w + 16, ... (TPW of them), column c of a tile on lane c.  The row
// max M and S = sum exp(l - M) come from the registers in one fixed order
// (each lane over its tiles in order, then the wave's DPP tree, then the 16
// waves in order), so a row's probabilities and table depend on its logits
// alone, whatever launch produced them; each exponential serves both S and
// the row's probability p = exp(l - M) / S (one exponential per element).  The
// table is the exact integer prefix (in-tile wave scans plus the exclusive
// prefix of the tile totals).  Loads and stores are 64 consecutive words per
// wave instruction; LDS holds only the reductions and tile totals.
template <int TPW>
__global__ __launch_bounds__(CH_THREADS) void cdf_row_kernel(const float* __restrict__ logits, int V,
                                                              float* __restrict__ probs,
                                                              uint32_t* __restrict__ cum,
                                                              int xcd_rows) {
  constexpr int NT = CH_WAVES * TPW;  // tiles of the row (V / 64, host check)
  static_assert(NT <= 4 * WAVE, "one wave forms the prefix of the tile totals");
  __shared__ float red[CH_WAVES];
  __shared__ uint32_t tex[NT];
  int64_t row = blockIdx.x;
  if (xcd_rows) {  // row tile rt of 8 rows on XCD rt % 8
    int rt, j;
    xcd_row_split((int)blockIdx.x, (int)(gridDim.x / 8), rt, j);
    row = 8 * rt + j;
  }
  const int t = threadIdx.x, w = t / WAVE, l = t % WAVE;
  const float* x = logits + row * (int64_t)V;
  float v[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) v[j] = x[64 * (w + CH_WAVES * j) + l];
  float mt = v[0];
#pragma unroll
  for (int j = 1; j < TPW; ++j) mt = fmaxf(mt, v[j]);
  const float M = block_max_n(mt, red);
  float sp = 0.f;
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    v[j] = __expf(v[j] - M);
    sp += v[j];
  }
  const float S = block_sum_n(sp, red);
  const float iS = 1.f / S;
  uint32_t inc[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const float p = v[j] * iS;
    if (probs) probs[row * (int64_t)V + 64 * (w + CH_WAVES * j) + l] = p;
    inc[j] = wave_incl_scan_u32(scale_count(p));
    if (l == WAVE - 1) tex[w + CH_WAVES * j] = inc[j];
  }
  __syncthreads();
  if (w == 0) {  // tile totals -> exclusive prefix, tiles 4l .. 4l+3 on lane l
    uint32_t a[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] = 4 * l + k < NT ? tex[4 * l + k] : 0u;
    const uint32_t s4 = a[0] + a[1] + a[2] + a[3];
    uint32_t run = wave_incl_scan_u32(s4) - s4;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (4 * l + k < NT) tex[4 * l + k] = run;
      run += a[k];
    }
  }
  __syncthreads();
  uint32_t* co = cum + row * (int64_t)(V + 1);
  if (t == 0) co[0] = 0u;
#pragma unroll
  for (int j = 0; j < TPW; ++j) co[1 + 64 * (w + CH_WAVES * j) + l] = tex[w + CH_WAVES * j] + inc[j];
}

template <bool FROM_LOGITS>
hipError_t launch_cdf(const float* in, int64_t rows, int V, int flags, float* probs,
                      uint32_t* cum, hipStream_t s) {
  const int ept = (V + CDF_THREADS - 1) / CDF_THREADS;
  dim3 grid((unsigned)rows), block(CDF_THREADS);
  const bool renorm = FROM_LOGITS && (flags & ALTXS_CDF_RENORM);
  if (renorm && V > kRenormMaxV) return hipErrorInvalidValue;
  const size_t lds = renorm ? (size_t)V * sizeof(float) : 0;
#define CDF_CASE(E)                                                                     \
  if (ept <= E) {                                                                       \
    hipLaunchKernelGGL((cdf_kernel<E, FROM_LOGITS>), grid, block, lds, s, in, V, flags, \
                       probs, cum);                                                     \
    return hipGetLastError();                                                           \
  }
  CDF_CASE(1) CDF_CASE(2) CDF_CASE(4) CDF_CASE(8) CDF_CASE(16) CDF_CASE(32) CDF_CASE(64)
#undef CDF_CASE
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t altxs_launch_cdf(const float* in, int64_t rows, int V, int flags, bool from_logits,
                            float* probs, uint32_t* cum, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  return from_logits ? launch_cdf<true>(in, rows, V, flags, probs, cum, s)
                     : launch_cdf<false>(in, rows, V, flags, probs, cum, s);
}

// The row kernel serves every launch whose vocabulary it tiles (V a multiple
// of 4096 up to 16384); cfg3's 64 decode rows take 8.0 us with it against
// 12.2 us in the chunk kernel (8 chunks per row, each recounting the counts
// before it), which remains for other vocabularies.
bool altxs_cdf_rows_kernel(int64_t rows, int V) {
  return rows >= 1 && V >= 4096 && V <= 16 * CH_THREADS && V % (4 * CH_THREADS) == 0;
}

hipError_t altxs_launch_cdf_stats(const float* logits, const float2* stats, int64_t rows, int V,
                                  float* probs, uint32_t* cum, hipStream_t s, bool xcd_rows) {
  if (rows <= 0) return hipSuccess;
  if (V % 64) return hipErrorInvalidValue;
  if (altxs_cdf_rows_kernel(rows, V)) {
    // one workgroup per row, the statistics from its own registers (the tile
    // statistics are not read)
    const dim3 grid((unsigned)rows), block(CH_THREADS);
    const int xr = (xcd_rows && rows % 64 == 0) ? 1 : 0;
    switch (V / (64 * CH_WAVES)) {  // tiles per wave
      case 4: hipLaunchKernelGGL(cdf_row_kernel<4>, grid, block, 0, s, logits, V, probs, cum, xr); break;
      case 8: hipLaunchKernelGGL(cdf_row_kernel<8>, grid, block, 0, s, logits, V, probs, cum, xr); break;
      case 12: hipLaunchKernelGGL(cdf_row_kernel<12>, grid, block, 0, s, logits, V, probs, cum, xr); break;
      case 16: hipLaunchKernelGGL(cdf_row_kernel<16>, grid, block, 0, s, logits, V, probs, cum, xr); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  if (!stats) return hipErrorInvalidValue;
  const int chunk = V < 2048 ? V : 2048;
  if (V % chunk) return hipErrorInvalidValue;
  dim3 grid((unsigned)(V / chunk), (unsigned)rows), block(CH_THREADS);
  if (chunk > CH_THREADS)
    hipLaunchKernelGGL(cdf_chunk_kernel<2>, grid, block, 0, s, logits, stats, V, chunk, probs, cum);
  else
    hipLaunchKernelGGL(cdf_chunk_kernel<1>, grid, block, 0, s, logits, stats, V, chunk, probs, cum);
  return hipGetLastError();
}

extern "C" int32_t altxs_scale_cum(const float* probs, int64_t rows, int64_t V, uint32_t* cum,
                                   altxs_stream_t stream) {
  ALTXS_REQUIRE(probs && cum, "altxs_scale_cum: null pointer");
  ALTXS_REQUIRE(V >= 1 && V <= 65536, "altxs_scale_cum: V=%lld outside [1, 65536]", (long long)V);
  ALTXS_REQUIRE(rows >= 0 && rows < (1ll << 31), "altxs_scale_cum: bad rows");
  ALTXS_CHECK_HIP(altxs_launch_cdf(probs, rows, (int)V, 0, false, nullptr, cum,
                                   (hipStream_t)stream));
  return ALTXS_OK;
}

extern "C" int32_t altxs_scale_cum_f64(const double* probs, int64_t rows, int64_t V, uint32_t* cum,
                                       altxs_stream_t stream) {
  ALTXS_REQUIRE(probs && cum, "altxs_scale_cum_f64: null pointer");
  ALTXS_REQUIRE(V >= 1 && V <= 65536, "altxs_scale_cum_f64: V=%lld outside [1, 65536]", (long long)V);
  ALTXS_REQUIRE(rows >= 0 && rows < (1ll << 31), "altxs_scale_cum_f64: bad rows");
  if (rows == 0) return ALTXS_OK;
  const int ept = (int)((V + CDF_THREADS - 1) / CDF_THREADS);
  const dim3 grid((unsigned)rows), block(CDF_THREADS);
  hipStream_t s = (hipStream_t)stream;
#define F64_CASE(E)                                                                                \
  if (ept <= E) {                                                                                  \
    hipLaunchKernelGGL(cdf_f64_kernel<E>, grid, block, 0, s, probs, (int)V, cum);                  \
    ALTXS_CHECK_HIP(hipGetLastError());                                                            \
    return ALTXS_OK;                                                                               \
  }
  F64_CASE(1) F64_CASE(2) F64_CASE(4) F64_CASE(8) F64_CASE(16) F64_CASE(32) F64_CASE(64)
#undef F64_CASE
  return ALTXS_ERR_ARG;
}

extern "C" int32_t altxs_softmax_cdf(const float* logits, int64_t rows, int64_t V, int32_t flags,
                                     float* probs, uint32_t* cum, altxs_stream_t stream) {
  ALTXS_REQUIRE(logits, "altxs_softmax_cdf: null logits");
  ALTXS_REQUIRE(V >= 1 && V <= 65536, "altxs_softmax_cdf: V=%lld outside [1, 65536]",
                (long long)V);
  ALTXS_REQUIRE(!(flags & ALTXS_CDF_RENORM) || V <= kRenormMaxV,
                "altxs_softmax_cdf: renormalised rows need V <= %d", kRenormMaxV);
  ALTXS_REQUIRE(rows >= 0 && rows < (1ll << 31), "altxs_softmax_cdf: bad rows");
  ALTXS_CHECK_HIP(altxs_launch_cdf(logits, rows, (int)V, flags, true, probs, cum,
                                   (hipStream_t)stream));
  return ALTXS_OK;
}
