// Dequant-fused MFMA GEMM: Y[r, n] = sum_k A[r, k] * W[n, k], W packed as
// symmetric group-64 codes with fp16 scales (see include/altxs.h, AltxsQTensor).
//
// Tiling.  A workgroup owns one 16-row M tile and NB 16-column n-blocks; its
// NB*KS waves split the work as (n-block, K-slice): wave w computes n-block
// w % NB over the K-slice w / NB.  Every wave issues the loads of its weight
// blocks (16 rows x 256 k each, <= 2 in flight) before anything else, so the
// HBM latency overlaps the activation prologue.  In the tiled layout lane l of
// a wave owns the 64 codes of row (l % 16) at k = 32*s + 8*(l / 16) + i
// (s, i < 8) -- exactly the B operand of v_mfma_f32_16x16x32_{bf16,f16} for the
// block's eight k-steps -- so a block arrives as one or two 16-byte loads per
// lane.  Codes become (c - (2^b-1)/2), exact in bf16/fp16; each 64-wide group's
// fp32 partial is scaled by its fp16 scale.
//
// A operand: either staged in LDS by a prologue functor (RMSNorm, residual
// mixes and skips fused there) or, for plain inputs, loaded by each lane
// straight into MFMA registers.
//
// Reduction and determinism.  Inside a wave: the MFMA's fixed internal order,
// then groups in increasing k.  Across the KS K-slices: partial tiles go to LDS
// and are added in slice order.  The order depends only on K and the kernel's
// (NB, KS), never on the number of rows, so results are bit-identical for any
// batch or window size.
//
// Epilogue: a tile functor.  Epi::prefetch() runs first (issue loads of
// residuals, positions, RoPE tables early); Epi::apply() gets the reduced
// 16 x (16*NB) fp32 tile in LDS and runs on all threads.
#pragma once
#include <type_traits>

#include "common.h"

namespace altxs {

template <int BITS> struct Planes;
template <> struct Planes<2> { static constexpr int P0 = 2, P1 = 0; };
template <> struct Planes<3> { static constexpr int P0 = 2, P1 = 1; };
template <> struct Planes<4> { static constexpr int P0 = 4, P1 = 0; };
template <> struct Planes<6> { static constexpr int P0 = 4, P1 = 2; };

// A-operand modes
enum AMode : int { A_F32 = 0, A_BF16 = 1, A_F16 = 2 };

struct QT {
  const uint8_t* codes;
  const uint16_t* scales;
  int N, K;
};

__host__ __device__ constexpr int lds_stride(int K, int am) { return K + (am == A_F32 ? 4 : 8); }
__host__ __device__ constexpr int a_esz(int am) { return am == A_F32 ? 4 : 2; }

// Store one fp32 activation value into an LDS A tile in the mode's format.
template <int AM>
__device__ __forceinline__ void a_store(void* As, int row, int col, int K, float v) {
  if constexpr (AM == A_F32) {
    ((float*)As)[row * lds_stride(K, AM) + col] = v;
  } else if constexpr (AM == A_BF16) {
    ((uint16_t*)As)[row * lds_stride(K, AM) + col] = f32_to_bf16(v);
  } else {
    _Float16 h = (_Float16)v;
    ((uint16_t*)As)[row * lds_stride(K, AM) + col] = __builtin_bit_cast(uint16_t, h);
  }
}

// Store four consecutive fp32 values (col % 4 == 0).
template <int AM>
__device__ __forceinline__ void a_store4(void* As, int row, int col, int K, const float (&v)[4]) {
  if constexpr (AM == A_F32) {
    f32x4 o = {v[0], v[1], v[2], v[3]};
    *(f32x4*)((float*)As + row * lds_stride(K, AM) + col) = o;
  } else {
    uint16_t h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (AM == A_BF16) h[i] = f32_to_bf16(v[i]);
      else h[i] = __builtin_bit_cast(uint16_t, (_Float16)v[i]);
    }
    u32x2 o = {(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
    *(u32x2*)((uint16_t*)As + row * lds_stride(K, AM) + col) = o;
  }
}

// Extract the 8 codes of k-step s (0..7) from a lane's planes.
template <int BITS>
__device__ __forceinline__ void codes_step(const uint32_t* p0, const uint32_t* p1, int s,
                                           uint32_t (&c)[8]) {
  constexpr int P0 = Planes<BITS>::P0, P1 = Planes<BITS>::P1;
  uint32_t w0, sh0;
  if constexpr (P0 == 4) { w0 = p0[s]; sh0 = 0; }
  else { w0 = p0[s >> 1]; sh0 = 16 * (s & 1); }
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = (w0 >> (sh0 + P0 * i)) & ((1u << P0) - 1u);
  if constexpr (P1 == 1) {
    const uint32_t w1 = p1[s >> 2];
    const uint32_t sh1 = 8 * (s & 3);
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] |= ((w1 >> (sh1 + i)) & 1u) << P0;
  } else if constexpr (P1 == 2) {
    const uint32_t w1 = p1[s >> 1];
    const uint32_t sh1 = 16 * (s & 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] |= ((w1 >> (sh1 + 2 * i)) & 3u) << P0;
  }
}

template <int BITS>
__device__ __forceinline__ bf16x8 b_op_bf16(const uint32_t* p0, const uint32_t* p1, int s) {
  constexpr float center = 0.5f * (float)((1 << BITS) - 1);
  uint32_t c[8];
  codes_step<BITS>(p0, p1, s, c);
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (__bf16)((float)c[i] - center);
  return r;
}

template <int BITS>
__device__ __forceinline__ f16x8 b_op_f16(const uint32_t* p0, const uint32_t* p1, int s) {
  constexpr float center = 0.5f * (float)((1 << BITS) - 1);
  uint32_t c[8];
  codes_step<BITS>(p0, p1, s, c);
  f16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (_Float16)((float)c[i] - center);
  return r;
}

// One weight block (plus, for direct A, the lane's A slice of that block).
template <int BITS, int AM, bool ADIRECT>
struct Blk {
  static constexpr int P0 = Planes<BITS>::P0, P1 = Planes<BITS>::P1;
  static constexpr int AW = ADIRECT ? (AM == A_F32 ? 16 : 8) : 1;  // u32x4 per block
  uint32_t p0[2 * P0];
  uint32_t p1[P1 > 0 ? 2 * P1 : 1];
  uint32_t sc[2];
  u32x4 a[AW];
};

// Direct A source: x[batch][R][K] of element type AM (fp32 / bf16 / fp16).
struct ADirect {
  const void* x;
  int64_t batch_stride;  // elements
};

template <int BITS, int AM, bool ADIRECT>
__device__ __forceinline__ void load_blk(Blk<BITS, AM, ADIRECT>& b, const QT& w, int nb, int kb,
                                         int lane, const ADirect& ad, int m0, int R, int batch) {
  constexpr int P0 = Planes<BITS>::P0, P1 = Planes<BITS>::P1;
  const int KB = w.K >> 8;
  const size_t bi = (size_t)nb * KB + kb;
  const uint8_t* blk = w.codes + bi * (512 * BITS);
  const uint8_t* a0 = blk + lane * (8 * P0);
  if constexpr (P0 == 4) {
    const u32x4 x = *(const u32x4*)a0;
    const u32x4 y = *(const u32x4*)(a0 + 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) { b.p0[i] = x[i]; b.p0[4 + i] = y[i]; }
  } else {
    const u32x4 x = *(const u32x4*)a0;
#pragma unroll
    for (int i = 0; i < 4; ++i) b.p0[i] = x[i];
  }
  if constexpr (P1 == 1) {
    const u32x2 x = *(const u32x2*)(blk + 512 * P0 + lane * 8);
    b.p1[0] = x[0]; b.p1[1] = x[1];
  } else if constexpr (P1 == 2) {
    const u32x4 x = *(const u32x4*)(blk + 512 * P0 + lane * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) b.p1[i] = x[i];
  }
  const u32x2 sv = *(const u32x2*)(w.scales + bi * 64 + (lane & 15) * 4);
  b.sc[0] = sv[0]; b.sc[1] = sv[1];
  if constexpr (ADIRECT) {
    const int r = m0 + (lane & 15);
    const int kc = kb * 256 + 8 * (lane >> 4);
    if (r < R) {
      if constexpr (AM == A_F32) {
        const float* xr = (const float*)ad.x + batch * ad.batch_stride + (int64_t)r * w.K + kc;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          b.a[2 * s] = *(const u32x4*)(xr + 32 * s);
          b.a[2 * s + 1] = *(const u32x4*)(xr + 32 * s + 4);
        }
      } else {
        const uint16_t* xr = (const uint16_t*)ad.x + batch * ad.batch_stride + (int64_t)r * w.K + kc;
#pragma unroll
        for (int s = 0; s < 8; ++s) b.a[s] = *(const u32x4*)(xr + 32 * s);
      }
    } else {
#pragma unroll
      for (int i = 0; i < Blk<BITS, AM, ADIRECT>::AW; ++i) b.a[i] = u32x4{0, 0, 0, 0};
    }
  }
}

__device__ __forceinline__ float half_lo(uint32_t v) {
  return __half2float(__ushort_as_half((uint16_t)(v & 0xffffu)));
}
__device__ __forceinline__ float half_hi(uint32_t v) {
  return __half2float(__ushort_as_half((uint16_t)(v >> 16)));
}

// fp32 x[8] -> three bf16x8 parts whose sum reproduces x to ~2^-27.
__device__ __forceinline__ void split3(const float (&x)[8], bf16x8& a0, bf16x8& a1, bf16x8& a2) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const __bf16 h0 = (__bf16)x[i];
    const float r1 = x[i] - (float)h0;
    const __bf16 h1 = (__bf16)r1;
    const float r2 = r1 - (float)h1;
    a0[i] = h0;
    a1[i] = h1;
    a2[i] = (__bf16)r2;
  }
}

// acc += W-block . A-slice (one 16x256 block, 8 MFMA k-steps).
template <int BITS, int AM, bool ADIRECT>
__device__ __forceinline__ void compute_blk(const Blk<BITS, AM, ADIRECT>& b, const void* As, int K,
                                            int kb, int lane, f32x4& acc) {
  const float scale[4] = {half_lo(b.sc[0]), half_hi(b.sc[0]), half_lo(b.sc[1]), half_hi(b.sc[1])};
  const int row = lane & 15;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) {
      const int s = 2 * g + ss;
      const int kc = kb * 256 + 32 * s + 8 * (lane >> 4);
      if constexpr (AM == A_F32) {
        float x[8];
        if constexpr (ADIRECT) {
          const u32x4 lo = b.a[2 * s], hi = b.a[2 * s + 1];
#pragma unroll
          for (int i = 0; i < 4; ++i) { x[i] = __uint_as_float(lo[i]); x[4 + i] = __uint_as_float(hi[i]); }
        } else {
          const float* a = (const float*)As + row * lds_stride(K, AM) + kc;
          const f32x4 lo = *(const f32x4*)a, hi = *(const f32x4*)(a + 4);
#pragma unroll
          for (int i = 0; i < 4; ++i) { x[i] = lo[i]; x[4 + i] = hi[i]; }
        }
        bf16x8 a0, a1, a2;
        split3(x, a0, a1, a2);
        const bf16x8 bo = b_op_bf16<BITS>(b.p0, b.p1, s);
        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bo, t, 0, 0, 0);
        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bo, t, 0, 0, 0);
        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, bo, t, 0, 0, 0);
      } else {
        u32x4 araw;
        if constexpr (ADIRECT) araw = b.a[s];
        else araw = *(const u32x4*)((const uint16_t*)As + row * lds_stride(K, AM) + kc);
        if constexpr (AM == A_BF16) {
          const bf16x8 bo = b_op_bf16<BITS>(b.p0, b.p1, s);
          t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, araw), bo, t, 0, 0, 0);
        } else {
          const f16x8 bo = b_op_f16<BITS>(b.p0, b.p1, s);
          t = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, araw), bo, t, 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] += scale[g] * t[i];
  }
}

// Prologue that stages nothing (A comes straight from global memory).
struct ProNone {
  static constexpr bool kStage = false;
  template <int AM, int NT>
  __device__ void stage(void*, int, int, int, int) const {}
};

template <int NB, int KS>
struct TileCfg {
  static constexpr int WAVES = NB * KS;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int NCOL = 16 * NB;
  static constexpr int CS = NCOL + 1;  // padded C tile stride (floats)
};

// LDS layout: [A tile (if staged)] [C partial tiles: KS x 16 x CS floats]
template <int NB, int KS>
__host__ __device__ constexpr size_t c_tile_bytes() {
  return (size_t)KS * 16 * TileCfg<NB, KS>::CS * 4;
}

template <int BITS, int AM, int NB, int KS, class Pro, class Epi>
__global__ __launch_bounds__(64 * NB * KS) void qgemm_kernel(
    QT w, int R, int64_t codes_stride, int64_t scales_stride, ADirect ad, Pro pro, Epi epi) {
  using Cfg = TileCfg<NB, KS>;
  constexpr bool STAGE = Pro::kStage;
  constexpr bool ADIRECT = !STAGE;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int batch = blockIdx.z;
  QT wb = w;
  wb.codes += batch * codes_stride;
  wb.scales += batch * scales_stride;
  const int m0 = blockIdx.y * 16;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nbi = wave % NB, ks = wave / NB;
  const int nb = blockIdx.x * NB + nbi;
  const bool active = nb * 16 < w.N;
  const int KB = w.K >> 8;
  const int kb0 = ks * (KB / KS), kb1 = kb0 + KB / KS;  // host guarantees KB % KS == 0
  void* As = smem;
  float* Cp = (float*)(smem + (STAGE ? (size_t)16 * lds_stride(w.K, AM) * a_esz(AM) : 0));

  const auto pre = epi.template prefetch<Cfg>(m0, R, batch);
  Blk<BITS, AM, ADIRECT> b0, b1;
  if (active) {
    if (kb0 < kb1) load_blk(b0, wb, nb, kb0, lane, ad, m0, R, batch);
    if (kb0 + 1 < kb1) load_blk(b1, wb, nb, kb0 + 1, lane, ad, m0, R, batch);
  }
  if constexpr (STAGE) {
    pro.template stage<AM, Cfg::THREADS>(As, m0, R, w.K, batch);
    __syncthreads();
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (active) {
    for (int kb = kb0; kb < kb1; kb += 2) {
      compute_blk(b0, As, w.K, kb, lane, acc);
      if (kb + 2 < kb1) load_blk(b0, wb, nb, kb + 2, lane, ad, m0, R, batch);
      if (kb + 1 < kb1) {
        compute_blk(b1, As, w.K, kb + 1, lane, acc);
        if (kb + 3 < kb1) load_blk(b1, wb, nb, kb + 3, lane, ad, m0, R, batch);
      }
    }
  }
  // partial tile of this wave -> LDS slice ks (MFMA layout: rows 4*(l/16)+i, col l%16)
  {
    float* C = Cp + (size_t)ks * 16 * Cfg::CS;
    const int col = nbi * 16 + (lane & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) C[(4 * (lane >> 4) + i) * Cfg::CS + col] = acc[i];
  }
  __syncthreads();
  if constexpr (KS > 1) {  // fixed-order reduction of the K-slices into slice 0
    for (int e = threadIdx.x; e < 16 * Cfg::NCOL; e += Cfg::THREADS) {
      const int r = e / Cfg::NCOL, c = e % Cfg::NCOL;
      float s = Cp[r * Cfg::CS + c];
#pragma unroll
      for (int k = 1; k < KS; ++k) s += Cp[(size_t)k * 16 * Cfg::CS + r * Cfg::CS + c];
      Cp[r * Cfg::CS + c] = s;
    }
    __syncthreads();
  }
  epi.template apply<Cfg>(Cp, pre, m0, blockIdx.x * Cfg::NCOL, R, batch);
}

// ---- generic epilogue: y[batch][r][n] = acc -----------------------------------
struct EpiStore {
  float* y;
  int N;
  int64_t y_batch_stride;
  struct Pre {};
  template <class Cfg>
  __device__ Pre prefetch(int, int, int) const { return {}; }
  template <class Cfg, class P>
  __device__ void apply(const float* C, const P&, int m0, int n0, int R, int batch) const {
    for (int e = threadIdx.x; e < 16 * Cfg::NCOL; e += Cfg::THREADS) {
      const int r = e / Cfg::NCOL, c = e % Cfg::NCOL;
      if (m0 + r < R && n0 + c < N)
        y[batch * y_batch_stride + (int64_t)(m0 + r) * N + n0 + c] = C[r * Cfg::CS + c];
    }
  }
};

// Launch helper: sets the dynamic LDS limit once per instantiation.
template <int BITS, int AM, int NB, int KS, class Pro, class Epi>
hipError_t launch_qgemm(const QT& w, int R, int batch, int64_t codes_stride,
                        int64_t scales_stride, const ADirect& ad, const Pro& pro, const Epi& epi,
                        hipStream_t s) {
  auto kfn = qgemm_kernel<BITS, AM, NB, KS, Pro, Epi>;
  const size_t lds = (Pro::kStage ? (size_t)16 * lds_stride(w.K, AM) * a_esz(AM) : 0) +
                     c_tile_bytes<NB, KS>();
  static size_t configured = 0;
  if (lds > 65536 && lds > configured) {
    hipError_t e = hipFuncSetAttribute((const void*)kfn,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    configured = lds;
  }
  dim3 grid((unsigned)((w.N + 16 * NB - 1) / (16 * NB)), (unsigned)((R + 15) / 16), (unsigned)batch);
  hipLaunchKernelGGL(kfn, grid, dim3(TileCfg<NB, KS>::THREADS), lds, s, w, R, codes_stride,
                     scales_stride, ad, pro, epi);
  return hipGetLastError();
}

// Dispatch on the runtime bit width and K-split.  KS is the largest of
// {4, 2, 1} that is <= ks_max and divides K/256.
template <int AM, int NB, int KSMAX, class Pro, class Epi>
hipError_t launch_qgemm_rt(int bits, const QT& w, int R, int batch, int64_t codes_stride,
                           int64_t scales_stride, const ADirect& ad, const Pro& pro,
                           const Epi& epi, hipStream_t s) {
  const int KB = w.K >> 8;
  auto go = [&](auto ks_tag) -> hipError_t {
    constexpr int KS = decltype(ks_tag)::value;
    switch (bits) {
      case 2: return launch_qgemm<2, AM, NB, KS>(w, R, batch, codes_stride, scales_stride, ad, pro, epi, s);
      case 3: return launch_qgemm<3, AM, NB, KS>(w, R, batch, codes_stride, scales_stride, ad, pro, epi, s);
      case 4: return launch_qgemm<4, AM, NB, KS>(w, R, batch, codes_stride, scales_stride, ad, pro, epi, s);
      case 6: return launch_qgemm<6, AM, NB, KS>(w, R, batch, codes_stride, scales_stride, ad, pro, epi, s);
      default: return hipErrorInvalidValue;
    }
  };
  if constexpr (KSMAX >= 4) {
    if (KB % 4 == 0) return go(std::integral_constant<int, 4>{});
  }
  if constexpr (KSMAX >= 2) {
    if (KB % 2 == 0) return go(std::integral_constant<int, 2>{});
  }
  return go(std::integral_constant<int, 1>{});
}

}  // namespace altxs
