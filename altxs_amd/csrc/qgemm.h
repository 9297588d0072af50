// Dequant-fused MFMA GEMM: Y[r, n] = sum_k A[r, k] * W[n, k], W packed as
// symmetric group-64 codes with fp16 scales (see include/altxs.h, AltxsQTensor).
//
// Workgroup = 4 waves; it owns one 16-row M tile (one MFMA row block) and 64
// output columns (one 16-column MFMA block per wave).  A (the activations) is
// staged once in LDS by a prologue functor -- which is where RMSNorm, residual
// mixes and skips are fused -- and each wave streams its 16 weight rows
// straight from HBM in the tiled layout: per 16x256 block, lane l owns the 64
// codes of row (l % 16) at k = 32*s + 8*(l / 16) + i (s = 0..7, i = 0..7),
// i.e. exactly the B operand of v_mfma_f32_16x16x32_{bf16,f16} for the eight
// k-steps, so one or two 16-byte loads per lane fetch a whole block with no
// shuffles.  Codes become (c - (2^b-1)/2), which is exact in bf16/fp16; the
// per-group fp16 scale is applied to the fp32 partial of each 64-wide group.
//
// Determinism: each output element's reduction order depends only on K (the
// MFMA's fixed internal order inside a group, then groups in increasing k), so
// results are bit-identical for any number of rows and any grid.
#pragma once
#include "common.h"

namespace altxs {

// bits -> (low plane bits, high plane bits)
template <int BITS> struct Planes;
template <> struct Planes<2> { static constexpr int P0 = 2, P1 = 0; };
template <> struct Planes<3> { static constexpr int P0 = 2, P1 = 1; };
template <> struct Planes<4> { static constexpr int P0 = 4, P1 = 0; };
template <> struct Planes<6> { static constexpr int P0 = 4, P1 = 2; };

// A-operand modes
enum AMode : int { A_F32 = 0, A_BF16 = 1, A_F16 = 2 };

template <int AM> struct AElem;
template <> struct AElem<A_F32> { using T = float; static constexpr int PAD = 4; };
template <> struct AElem<A_BF16> { using T = uint16_t; static constexpr int PAD = 8; };
template <> struct AElem<A_F16> { using T = uint16_t; static constexpr int PAD = 8; };

struct QT {
  const uint8_t* codes;
  const uint16_t* scales;
  int N, K;
};

__host__ __device__ constexpr int lds_stride(int K, int am) {
  return K + (am == A_F32 ? 4 : 8);
}
inline size_t lds_bytes(int K, int am) {
  return (size_t)16 * lds_stride(K, am) * (am == A_F32 ? 4 : 2);
}

// Store one fp32 activation value into the LDS A tile in the mode's format.
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

// MFMA over one k-step (32 columns of A starting at `col`) into t.
template <int BITS, int AM>
__device__ __forceinline__ void mfma_kstep(const void* As, int K, int col, int lane,
                                           const uint32_t* p0, const uint32_t* p1, int s,
                                           f32x4& t) {
  const int row = lane & 15;
  const int kc = col + 8 * (lane >> 4);
  if constexpr (AM == A_F32) {
    const float* a = (const float*)As + row * lds_stride(K, AM) + kc;
    const f32x4 lo = *(const f32x4*)a;
    const f32x4 hi = *(const f32x4*)(a + 4);
    float x[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    bf16x8 a0, a1, a2;
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
    const bf16x8 b = b_op_bf16<BITS>(p0, p1, s);
    t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b, t, 0, 0, 0);
    t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b, t, 0, 0, 0);
    t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b, t, 0, 0, 0);
  } else if constexpr (AM == A_BF16) {
    const bf16x8 a = *(const bf16x8*)((const uint16_t*)As + row * lds_stride(K, AM) + kc);
    const bf16x8 b = b_op_bf16<BITS>(p0, p1, s);
    t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, t, 0, 0, 0);
  } else {
    const f16x8 a = *(const f16x8*)((const uint16_t*)As + row * lds_stride(K, AM) + kc);
    const f16x8 b = b_op_f16<BITS>(p0, p1, s);
    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, t, 0, 0, 0);
  }
}

// Per-lane load of one 16x256 block's planes and scales.
template <int BITS>
__device__ __forceinline__ void load_block(const uint8_t* blk, const uint16_t* sc, int lane,
                                           uint32_t* p0, uint32_t* p1, float* scale) {
  constexpr int P0 = Planes<BITS>::P0, P1 = Planes<BITS>::P1;
  const uint8_t* a0 = blk + lane * (8 * P0);
  if constexpr (P0 == 4) {
    const u32x4 x = *(const u32x4*)a0;
    const u32x4 y = *(const u32x4*)(a0 + 16);
    p0[0] = x[0]; p0[1] = x[1]; p0[2] = x[2]; p0[3] = x[3];
    p0[4] = y[0]; p0[5] = y[1]; p0[6] = y[2]; p0[7] = y[3];
  } else {
    const u32x4 x = *(const u32x4*)a0;
    p0[0] = x[0]; p0[1] = x[1]; p0[2] = x[2]; p0[3] = x[3];
  }
  if constexpr (P1 > 0) {
    const uint8_t* a1 = blk + 512 * P0 + lane * (8 * P1);
    if constexpr (P1 == 1) {
      const u32x2 x = *(const u32x2*)a1;
      p1[0] = x[0]; p1[1] = x[1];
    } else {
      const u32x4 x = *(const u32x4*)a1;
      p1[0] = x[0]; p1[1] = x[1]; p1[2] = x[2]; p1[3] = x[3];
    }
  }
  const u32x2 sv = *(const u32x2*)(sc + (lane & 15) * 4);
  scale[0] = __half2float(__ushort_as_half((uint16_t)(sv[0] & 0xffffu)));
  scale[1] = __half2float(__ushort_as_half((uint16_t)(sv[0] >> 16)));
  scale[2] = __half2float(__ushort_as_half((uint16_t)(sv[1] & 0xffffu)));
  scale[3] = __half2float(__ushort_as_half((uint16_t)(sv[1] >> 16)));
}

// The GEMM main loop for one wave: 16 rows (LDS) x 16 weight rows (block nb).
template <int BITS, int AM>
__device__ __forceinline__ f32x4 qgemm_wave(const QT& w, const void* As, int nb, int lane) {
  constexpr int P0 = Planes<BITS>::P0, P1 = Planes<BITS>::P1;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const int KB = w.K >> 8;
  const uint8_t* blk = w.codes + (size_t)nb * KB * (512 * BITS);
  const uint16_t* sc = w.scales + (size_t)nb * KB * 64;
  uint32_t p0[2 * P0], p1[P1 > 0 ? 2 * P1 : 1];
  float scale[4];
  load_block<BITS>(blk, sc, lane, p0, p1, scale);
  for (int kb = 0; kb < KB; ++kb) {
    uint32_t q0[2 * P0], q1[P1 > 0 ? 2 * P1 : 1];
    float qs[4];
    if (kb + 1 < KB)
      load_block<BITS>(blk + (size_t)(kb + 1) * (512 * BITS), sc + (kb + 1) * 64, lane, q0, q1,
                       qs);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      f32x4 t = {0.f, 0.f, 0.f, 0.f};
      mfma_kstep<BITS, AM>(As, w.K, kb * 256 + 64 * g, lane, p0, p1, 2 * g, t);
      mfma_kstep<BITS, AM>(As, w.K, kb * 256 + 64 * g + 32, lane, p0, p1, 2 * g + 1, t);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] += scale[g] * t[i];
    }
    if (kb + 1 < KB) {
#pragma unroll
      for (int i = 0; i < 2 * P0; ++i) p0[i] = q0[i];
      if constexpr (P1 > 0) {
#pragma unroll
        for (int i = 0; i < 2 * P1; ++i) p1[i] = q1[i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) scale[i] = qs[i];
    }
  }
  return acc;
}

// Generic kernel: grid (ceil(N/64), ceil(R/16), batch), 256 threads.
// Pro: void stage<AM>(void* As, int m0, int R, int K, int batch) const  (all threads)
// Epi: void operator()(const f32x4& acc, int m0, int nb, int lane, int wave,
//                      unsigned char* smem, int R, int batch) const     (all threads)
template <int BITS, int AM, class Pro, class Epi>
__global__ __launch_bounds__(256) void qgemm_kernel(QT w, int R, int64_t codes_stride,
                                                    int64_t scales_stride, Pro pro, Epi epi) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int batch = blockIdx.z;
  QT wb = w;
  wb.codes += batch * codes_stride;
  wb.scales += batch * scales_stride;
  const int m0 = blockIdx.y * 16;
  pro.template stage<AM>((void*)smem, m0, R, w.K, batch);
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nb = blockIdx.x * 4 + wave;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (nb * 16 < w.N) acc = qgemm_wave<BITS, AM>(wb, smem, nb, lane);
  epi(acc, m0, nb, lane, wave, smem, R, batch);
}

// ---- generic prologue / epilogue -----------------------------------------

// Copy rows [m0, m0+16) of x[R, K] (element type given by xdt) into LDS.
struct ProLoad {
  const void* x;
  int xdt;           // ALTXS_F32 / ALTXS_BF16 / ALTXS_F16
  int64_t x_batch_stride;  // elements between batches (0 = shared)
  template <int AM>
  __device__ void stage(void* As, int m0, int R, int K, int batch) const {
    for (int e = threadIdx.x; e < 16 * K; e += 256) {
      const int row = e / K, col = e % K;  // K is a multiple of 256
      const int r = m0 + row;
      float v = 0.f;
      if (r < R) {
        const int64_t idx = batch * x_batch_stride + (int64_t)r * K + col;
        if (xdt == ALTXS_F32) v = ((const float*)x)[idx];
        else if (xdt == ALTXS_BF16) v = bf16_to_f32(((const uint16_t*)x)[idx]);
        else v = __half2float(__ushort_as_half(((const uint16_t*)x)[idx]));
      }
      a_store<AM>(As, row, col, K, v);
    }
  }
};

// y[batch][r][n] = acc (fp32), rows < R only.
struct EpiStore {
  float* y;
  int N;
  int64_t y_batch_stride;
  __device__ void operator()(const f32x4& acc, int m0, int nb, int lane, int, unsigned char*,
                             int R, int batch) const {
    const int col = nb * 16 + (lane & 15);
    if (col >= N) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = m0 + 4 * (lane >> 4) + i;
      if (r < R) y[batch * y_batch_stride + (int64_t)r * N + col] = acc[i];
    }
  }
};

// Launch helper: sets the dynamic LDS limit once per instantiation.
template <int BITS, int AM, class Pro, class Epi>
hipError_t launch_qgemm(const QT& w, int R, int batch, int64_t codes_stride,
                        int64_t scales_stride, const Pro& pro, const Epi& epi, hipStream_t s) {
  auto kfn = qgemm_kernel<BITS, AM, Pro, Epi>;
  const size_t lds = lds_bytes(w.K, AM);
  static size_t configured = 0;
  if (lds > 65536 && lds > configured) {
    hipError_t e = hipFuncSetAttribute((const void*)kfn,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    configured = lds;
  }
  dim3 grid((unsigned)((w.N + 63) / 64), (unsigned)((R + 15) / 16), (unsigned)batch);
  hipLaunchKernelGGL(kfn, grid, dim3(256), lds, s, w, R, codes_stride, scales_stride, pro, epi);
  return hipGetLastError();
}

// Dispatch on the runtime bit width.
template <int AM, class Pro, class Epi>
hipError_t launch_qgemm_bits(int bits, const QT& w, int R, int batch, int64_t codes_stride,
                             int64_t scales_stride, const Pro& pro, const Epi& epi,
                             hipStream_t s) {
  switch (bits) {
    case 2: return launch_qgemm<2, AM>(w, R, batch, codes_stride, scales_stride, pro, epi, s);
    case 3: return launch_qgemm<3, AM>(w, R, batch, codes_stride, scales_stride, pro, epi, s);
    case 4: return launch_qgemm<4, AM>(w, R, batch, codes_stride, scales_stride, pro, epi, s);
    case 6: return launch_qgemm<6, AM>(w, R, batch, codes_stride, scales_stride, pro, epi, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace altxs
