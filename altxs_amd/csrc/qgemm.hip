// Standalone C-ABI for the packed-weight kernels: dense dequantisation (test
// and interop path), the fused dequant GEMM/GEMV, and its multi-tensor
// streaming form used to measure HBM throughput over many distinct matrices.
#include "common.h"
#include "gemm.h"

using namespace altxs;

namespace {

// One wave per 16x256 block: lane l expands its 64 codes.
template <int BITS>
__global__ __launch_bounds__(64) void dequant_kernel(QT w, float* __restrict__ out) {
  constexpr float center = 0.5f * (float)((1 << BITS) - 1);
  const int KB = w.K >> 8;
  const int nb = blockIdx.x / KB, kb = blockIdx.x % KB;
  const int lane = threadIdx.x;
  Blk<BITS, A_BF16, false> b;
  load_blk(b, w, nb, kb, lane, ADirect{nullptr, 0}, 0, 0, 0);
  const float scale[4] = {half_lo(b.sc[0]), half_hi(b.sc[0]), half_lo(b.sc[1]), half_hi(b.sc[1])};
  const int n = nb * 16 + (lane & 15);
  float* row = out + (size_t)n * w.K + kb * 256 + 8 * (lane >> 4);
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    uint32_t c[8];
    codes_step<BITS>(b.p0, b.p1, s, c);
#pragma unroll
    for (int i = 0; i < 8; ++i) row[32 * s + i] = ((float)c[i] - center) * scale[s >> 1];
  }
}

// One wave per 16x256 block: lane l writes the bf16 B operands of its eight
// k-steps (the packed path's b_op_bf16, so the very values its MFMAs see),
// k-step s at 16-byte slot 64 s + l of the block.
template <int BITS>
__global__ __launch_bounds__(64) void expand_kernel(QT w, u32x4* __restrict__ out) {
  const int lane = threadIdx.x;
  const int KB = w.K >> 8;
  const int nb = blockIdx.x / KB, kb = blockIdx.x % KB;
  Blk<BITS, A_BF16, false> b;
  load_w(b, w, nb, kb, lane);
  u32x4* o = out + (size_t)blockIdx.x * 512 + lane;  // 8 KB per block
#pragma unroll
  for (int s = 0; s < 8; ++s) o[64 * s] = __builtin_bit_cast(u32x4, b_op_bf16<BITS>(b.p0, b.p1, s, BITS));
}

int check_qt(const AltxsQTensor* w, const char* who, bool dense_ok) {
  ALTXS_REQUIRE(w && w->codes && (w->scales || w->bits == 16 || w->bits == 32), "%s: null tensor", who);
  ALTXS_REQUIRE(w->bits == 2 || w->bits == 3 || w->bits == 4 || w->bits == 6 ||
                    (dense_ok && (w->bits == 16 || w->bits == 32)),
                "%s: bits=%d not in {2,3,4,6%s}", who, w->bits, dense_ok ? ",16,32" : "");
  ALTXS_REQUIRE(w->N > 0 && w->N % 16 == 0 && w->N < (1 << 24),
                "%s: N=%lld must be a positive multiple of 16", who, (long long)w->N);
  ALTXS_REQUIRE(w->K > 0 && w->K % 256 == 0 && w->K <= 8192,
                "%s: K=%lld must be a positive multiple of 256 (<= 8192)", who, (long long)w->K);
  ALTXS_REQUIRE(((uintptr_t)w->codes & 15) == 0 && ((uintptr_t)w->scales & 7) == 0,
                "%s: codes must be 16-byte and scales 8-byte aligned", who);
  return ALTXS_OK;
}

QT to_qt(const AltxsQTensor* w) {
  QT q;
  q.codes = (const uint8_t*)w->codes;
  q.scales = (const uint16_t*)w->scales;
  q.N = (int)w->N;
  q.K = (int)w->K;
  q.bits = w->bits;
  return q;
}

template <int AM>
hipError_t run_gemm(const AltxsQTensor* w, int64_t count, int64_t cs, int64_t ss, const void* x,
                    int64_t rows, float* y, hipStream_t s) {
  QT q = to_qt(w);
  EpiStore epi{y, q.N, rows * q.N};
  // Every launch shape uses (NB, KS) = (4, 1) -- each wave a 16-column block
  // over the whole K, groups in increasing k -- so a row's result does not
  // depend on the number of rows or matrices.  16-row tiles, one workgroup
  // per 64 columns: B = 1 streams 2.3-4.1 TB/s over >= 2 GB of 2..6-bit
  // matrices (the K-split shapes (2,2), (1,4), (2,4), (4,2) reached 1.5-2.6
  // TB/s).  With 16-bit x and more rows, 64 x 128 tiles decode each weight
  // once per 64 rows instead of once per 16 (bit-identical); they are used
  // when the launch still fills the chip (>= 256 workgroups), so a single
  // small GEMM keeps the wider 16-row grid.
  if constexpr (AM != A_F32) {
    const int64_t big_wgs = count * (w->N / BIG_N) * ((rows + BIG_M - 1) / BIG_M);
    // (the large tiles read A rows by 16-byte global->LDS DMA: aligned rows only)
    if (rows > 16 && w->N % BIG_N == 0 && w->bits <= 6 && big_wgs >= 256 && ((uintptr_t)x & 15) == 0 &&
        w->K % 8 == 0) {
      const uint16_t* A = (const uint16_t*)x;
      const int R = (int)rows, C = (int)count;
      switch (w->bits) {
        case 2: return launch_gemm_big_t<2, 4, 1, EpiStore, AM>(q, R, A, epi, s, C, cs, ss);
        case 3: return launch_gemm_big_t<3, 4, 1, EpiStore, AM>(q, R, A, epi, s, C, cs, ss);
        case 4: return launch_gemm_big_t<4, 4, 1, EpiStore, AM>(q, R, A, epi, s, C, cs, ss);
        case 6: return launch_gemm_big_t<6, 4, 1, EpiStore, AM>(q, R, A, epi, s, C, cs, ss);
        default: break;
      }
    }
  }
  return launch_gemm_bits<AM, 4, 1>(w->bits, q, (int)rows, (int)count, cs, ss, ADirect{x, 0},
                                    ProNone{}, epi, 0, s);
}

int32_t gemm_common(const AltxsQTensor* w, int64_t count, int64_t cs, int64_t ss, const void* x,
                    int32_t xdt, int64_t rows, float* y, altxs_stream_t stream, const char* who) {
  int rc = check_qt(w, who, true);
  if (rc) return rc;
  ALTXS_REQUIRE(x && y, "%s: null x/y", who);
  ALTXS_REQUIRE(w->bits != 16 || xdt != ALTXS_F16, "%s: dense bf16 weights take fp32 or bf16 x", who);
  ALTXS_REQUIRE(w->bits != 32 || xdt == ALTXS_F32, "%s: dense fp32 weights take fp32 x", who);
  ALTXS_REQUIRE(((uintptr_t)x & 15) == 0, "%s: x must be 16-byte aligned", who);
  ALTXS_REQUIRE(rows >= 1 && rows <= (1 << 20), "%s: rows=%lld out of range", who, (long long)rows);
  ALTXS_REQUIRE(count >= 1 && count <= 65535, "%s: count=%lld out of range", who, (long long)count);
  ALTXS_REQUIRE(xdt == ALTXS_F32 || xdt == ALTXS_BF16 || xdt == ALTXS_F16, "%s: bad x dtype %d",
                who, xdt);
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (xdt == ALTXS_F32) e = run_gemm<A_F32>(w, count, cs, ss, x, rows, y, s);
  else if (xdt == ALTXS_BF16) e = run_gemm<A_BF16>(w, count, cs, ss, x, rows, y, s);
  else e = run_gemm<A_F16>(w, count, cs, ss, x, rows, y, s);
  ALTXS_CHECK_HIP(e);
  return ALTXS_OK;
}

}  // namespace

extern "C" int32_t altxs_dequant(const AltxsQTensor* w, float* out, altxs_stream_t stream) {
  int rc = check_qt(w, "altxs_dequant", false);
  if (rc) return rc;
  ALTXS_REQUIRE(out, "altxs_dequant: null out");
  QT q = to_qt(w);
  dim3 grid((unsigned)((q.N / 16) * (q.K / 256))), block(64);
  hipStream_t s = (hipStream_t)stream;
  switch (w->bits) {
    case 2: hipLaunchKernelGGL(dequant_kernel<2>, grid, block, 0, s, q, out); break;
    case 3: hipLaunchKernelGGL(dequant_kernel<3>, grid, block, 0, s, q, out); break;
    case 4: hipLaunchKernelGGL(dequant_kernel<4>, grid, block, 0, s, q, out); break;
    case 6: hipLaunchKernelGGL(dequant_kernel<6>, grid, block, 0, s, q, out); break;
  }
  ALTXS_CHECK_HIP(hipGetLastError());
  return ALTXS_OK;
}

extern "C" int32_t altxs_expand_codes(const AltxsQTensor* w, void* out, altxs_stream_t stream) {
  int rc = check_qt(w, "altxs_expand_codes", false);
  if (rc) return rc;
  ALTXS_REQUIRE(out && ((uintptr_t)out & 15) == 0, "altxs_expand_codes: out must be 16-byte aligned");
  QT q = to_qt(w);
  dim3 grid((unsigned)((q.N / 16) * (q.K / 256))), block(64);
  hipStream_t s = (hipStream_t)stream;
  switch (w->bits) {
    case 2: hipLaunchKernelGGL(expand_kernel<2>, grid, block, 0, s, q, (u32x4*)out); break;
    case 3: hipLaunchKernelGGL(expand_kernel<3>, grid, block, 0, s, q, (u32x4*)out); break;
    case 4: hipLaunchKernelGGL(expand_kernel<4>, grid, block, 0, s, q, (u32x4*)out); break;
    case 6: hipLaunchKernelGGL(expand_kernel<6>, grid, block, 0, s, q, (u32x4*)out); break;
  }
  ALTXS_CHECK_HIP(hipGetLastError());
  return ALTXS_OK;
}

extern "C" int32_t altxs_qgemm(const AltxsQTensor* w, const void* x, int32_t x_dtype, int64_t rows,
                               float* y, altxs_stream_t stream) {
  return gemm_common(w, 1, 0, 0, x, x_dtype, rows, y, stream, "altxs_qgemm");
}

extern "C" int32_t altxs_qgemm_stream(const AltxsQTensor* w, int64_t count, int64_t codes_stride,
                                      int64_t scales_stride, const void* x, int32_t x_dtype,
                                      int64_t rows, float* y, altxs_stream_t stream) {
  ALTXS_REQUIRE(w, "altxs_qgemm_stream: null tensor");
  ALTXS_REQUIRE(codes_stride >= w->N * w->K * w->bits / 8 && scales_stride >= w->N * w->K / 64 * 2 &&
                    scales_stride % 8 == 0 && codes_stride % 16 == 0,
                "altxs_qgemm_stream: strides smaller than one tensor or misaligned");
  return gemm_common(w, count, codes_stride, scales_stride / 2, x, x_dtype, rows, y, stream,
                     "altxs_qgemm_stream");
}
