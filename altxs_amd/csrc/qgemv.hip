// Row-independent GEMV on packed group-64 weights for a few rows (1..4):
// y[r, n] = sum_k x[r, k] * W[n, k], VALU arithmetic (v_dot2 of 16-bit
// pairs, fp32 accumulation), the form of the reference's per-row GEMV
// (src/xsa_ttt/ac_gemv.py:26-58 `_gemv_row_tiles`, gemv_rows 391-425: one
// program per (row, column tile), "independent rows -- not an M=W GEMM").
//
// Why a second arithmetic.  altxs_qgemm feeds v_mfma_f32_16x16x32 tiles of
// 16 rows; with one row, 15 of them are empty and the cost per weight is the
// code decoding into MFMA operands (~3.3 VALU instructions per weight and
// lane).  Here each weight is decoded once into a 16-bit pair operand and
// used by one v_dot2 per row, ~1-2 instructions per weight, so the kernel
// streams the packed bytes at HBM rate.  Its bits differ from altxs_qgemm's
// (another summation order); they depend only on the row.
//
// Layout: the MFMA-tiled blocks of include/altxs.h as they are (no second
// packing).  Lane l of a wave owns column n = 16 nb + (l % 16) of block
// (nb, kb) and the k-slice 8 (l / 16) + [0, 8) of every 32-wide k-step, so
// one wave walks one 16-column block over the whole K (kb ascending) and the
// four lane groups are added at the end in a fixed butterfly.
//
// Operands.  A code c becomes a 16-bit value with c in its low bits and no
// shift: for fp16 x the fp16 denormal c * 2^-24 (exact; products and sums in
// fp32 stay normal), for bf16 x the bf16 value 128 + c (exact for c < 128).
// The centre and the offset are taken out per 64-wide group with the group's
// sum of x: for group g of a lane slice
//   sum_k (c_k - z) x_k = U * a_g - (U * o + z) * S_g,   a_g = sum dot2(op, x)
// (U = 2^24, o = 0 for fp16; U = 1, o = 128 for bf16; z = (2^b - 1) / 2),
// and y = U * sum_g scale_g * (-C_g + a_g), the dot2 chain of group g started
// at -C_g, with C_g = (o + z / U) * S_g formed once per launch when x is
// staged (fp32, fixed order); the factor U is applied to the final sum
// (exact).  Each pair's two codes come out of the planes with one
// mask (plus a shift, and for 3/6 bits one more masked merge of the high
// bits); the x pairs are staged in LDS in the matching order, so a lane reads
// them with two 16-byte LDS loads per group and row (every lane of a lane
// group reads the same address: a broadcast).
#include "common.h"
#include "gemm.h"

using namespace altxs;

namespace {

constexpr int kGvWaves = 4, kGvThreads = 64 * kGvWaves;

// x format: 0 = fp16 (denormal code operands), 1 = bf16 (codes + 128)
template <int XB> struct GvFmt;
template <> struct GvFmt<0> {
  static constexpr uint32_t kOr = 0u;
  static constexpr float kU = 16777216.f;  // 2^24
  static constexpr float kOff = 0.f;
  __device__ static float dot2(uint32_t a, uint32_t b, float c) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
  }
  __device__ static float to_f32(uint16_t v) { return (float)__builtin_bit_cast(_Float16, v); }
};
template <> struct GvFmt<1> {
  static constexpr uint32_t kOr = 0x43004300u;  // bf16 128 in both halves
  static constexpr float kU = 1.f;
  static constexpr float kOff = 128.f;
  __device__ static float dot2(uint32_t a, uint32_t b, float c) {
    typedef short s2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(s2, a), __builtin_bit_cast(s2, b), c,
                                           false);
  }
  __device__ static float to_f32(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }
};

// Pair order.  Widths 4 and 6 pair codes j and j + 4 of one k-step: dword
// 4 ss + j of group g holds (k-step 2g + ss, code j | code j + 4).  Widths 2
// and 3 pair code i of the group's two k-steps: dword i holds (k-step 2g,
// code i | k-step 2g + 1, code i).  k of (k-step s, code i) in the block is
// 32 s + 8 lg + i.
template <int BITS>
__host__ __device__ constexpr bool gv_pairs_in_step() { return BITS == 4 || BITS == 6; }

__device__ __forceinline__ void gv_pair_k(bool in_step, int g, int lg, int d, int& klo, int& khi) {
  if (in_step) {
    const int s = 2 * g + (d >> 2), j = d & 3;
    klo = 32 * s + 8 * lg + j;
    khi = klo + 4;
  } else {
    klo = 64 * g + 8 * lg + d;
    khi = klo + 32;
  }
}

// bit i of x -> bit 2 (i < 8; the 16-bit half above moves along)
template <int I, int TO>
__device__ __forceinline__ uint32_t gv_move(uint32_t x) {
  if constexpr (I > TO) return x >> (I - TO);
  else if constexpr (I < TO) return x << (TO - I);
  else return x;
}

// The 8 operand dwords of group g of this lane's block.
template <int BITS, int XB>
__device__ __forceinline__ void gv_decode(const uint32_t* p0, const uint32_t* p1, int g, uint32_t (&d)[8]) {
  constexpr uint32_t OR = GvFmt<XB>::kOr;
  if constexpr (BITS == 4 || BITS == 6) {
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) {
      const uint32_t w = p0[2 * g + ss];
      d[4 * ss + 0] = (w & 0x000F000Fu) | OR;
      d[4 * ss + 1] = ((w >> 4) & 0x000F000Fu) | OR;
      d[4 * ss + 2] = ((w >> 8) & 0x000F000Fu) | OR;
      d[4 * ss + 3] = ((w >> 12) & 0x000F000Fu) | OR;
      if constexpr (BITS == 6) {
        // high two bits of code i at 16 ss + 2 i of p1[g]: bytes -> halves
        const uint32_t h = __builtin_amdgcn_perm(p1[g], p1[g], ss ? 0x0C030C02u : 0x0C010C00u);
        d[4 * ss + 0] |= gv_move<0, 4>(h) & 0x00300030u;
        d[4 * ss + 1] |= gv_move<2, 4>(h) & 0x00300030u;
        d[4 * ss + 2] |= h & 0x00300030u;
        d[4 * ss + 3] |= gv_move<6, 4>(h) & 0x00300030u;
      }
    }
  } else {
    const uint32_t w = p0[g];  // k-step 2g in the low half, 2g + 1 in the high half
    uint32_t h = 0;
    if constexpr (BITS == 3)  // third bits: byte 2 (g & 1) (+ 1) of p1[g >> 1] -> halves
      h = __builtin_amdgcn_perm(p1[g >> 1], p1[g >> 1], (g & 1) ? 0x0C030C02u : 0x0C010C00u);
#define GV_PAIR(I)                                                          \
  do {                                                                      \
    d[I] = ((w >> (2 * I)) & 0x00030003u) | OR;                             \
    if constexpr (BITS == 3) d[I] |= gv_move<I, 2>(h) & 0x00040004u;        \
  } while (0)
    GV_PAIR(0); GV_PAIR(1); GV_PAIR(2); GV_PAIR(3);
    GV_PAIR(4); GV_PAIR(5); GV_PAIR(6); GV_PAIR(7);
#undef GV_PAIR
  }
}

template <int BITS>
__host__ __device__ constexpr float gv_center() { return 0.5f * (float)((1 << BITS) - 1); }

// LDS: pairs[r][kb][g][lg][8] (dwords), then corr[r][kb][g][lg] (floats).
__host__ __device__ constexpr size_t gv_lds_bytes(int R, int K) {
  return (size_t)R * K * 2 + (size_t)R * (K / 64) * 4 * 4;
}

// Stage the R rows of x (16-bit values) in pair order and form the group
// corrections C = (o + z / U) * S (S summed over the slice's 16 values in
// dword order, low half first).
template <int BITS, int XB, int R>
__device__ void gv_stage(const uint16_t* __restrict__ x, int K, uint32_t* pairs, float* corr) {
  const int KB = K >> 8;
  const int ndw = R * KB * 4 * 4 * 8;
  for (int e = threadIdx.x; e < ndw; e += kGvThreads) {
    const int d = e & 7, lg = (e >> 3) & 3, g = (e >> 5) & 3, kb = (e >> 7) % KB, r = (e >> 7) / KB;
    int klo, khi;
    gv_pair_k(gv_pairs_in_step<BITS>(), g, lg, d, klo, khi);
    const uint16_t* xr = x + (int64_t)r * K + kb * 256;
    pairs[e] = (uint32_t)xr[klo] | ((uint32_t)xr[khi] << 16);
  }
  __syncthreads();
  constexpr float zc = GvFmt<XB>::kOff + gv_center<BITS>() / GvFmt<XB>::kU;
  const int nc = R * KB * 16;
  for (int e = threadIdx.x; e < nc; e += kGvThreads) {
    const uint32_t* p = pairs + 8 * e;
    float s = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      s += GvFmt<XB>::to_f32((uint16_t)(p[d] & 0xFFFFu));
      s += GvFmt<XB>::to_f32((uint16_t)(p[d] >> 16));
    }
    corr[e] = zc * s;
  }
  __syncthreads();
}

// A wave's work: whole tasks (task = matrix x column block) wave_id,
// wave_id + nwaves, ..., each the blocks kb = 0 .. KB-1 of one column block
// (consecutive in memory).  Item j of the wave is block j % KB of its task
// j / KB.  A cursor holds an item's (task, kb, matrix, column block) and is
// advanced without divisions; every field is wave-uniform (scalar).
struct GvItems {
  int KB;         // blocks along K
  uint32_t nblk;  // column blocks per matrix
  uint32_t ntasks;  // matrices x column blocks (< 2^31, checked by the host)
};

struct GvPos {
  uint32_t task, mat, nb;
  int kb;
};

template <int BITS>
__device__ __forceinline__ void gv_load(Blk<BITS, A_F16, false>& b, const QT& w, int64_t cs, int64_t ss,
                                        const GvPos& c, int lane) {
  QT wm = w;
  wm.codes += (int64_t)c.mat * cs;
  wm.scales += (int64_t)c.mat * ss;
  load_w(b, wm, (int)c.nb, c.kb, lane);
}

template <int BITS, int XB, int R>
__global__ __launch_bounds__(kGvThreads) void qgemv_kernel(QT w, int64_t cs, int64_t ss, GvItems it,
                                                            const uint16_t* __restrict__ x,
                                                            float* __restrict__ y, int64_t y_mat_stride) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  uint32_t* pairs = (uint32_t*)smem;
  float* corr = (float*)(smem + (size_t)R * w.K * 2);
  const int lane = threadIdx.x & 63, lg = lane >> 4;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t wave_id = blockIdx.x * kGvWaves + wave, nwaves = gridDim.x * kGvWaves;
  const int KB = it.KB;
  const uint32_t dq = nwaves / it.nblk, dr = nwaves - dq * it.nblk;  // a task stride in (matrix, block)
  auto advance = [&](GvPos& c, int n) {  // n items on
    c.kb += n;
    while (c.kb >= KB) {
      c.kb -= KB;
      c.task += nwaves;
      c.mat += dq;
      c.nb += dr;
      if (c.nb >= it.nblk) {
        c.nb -= it.nblk;
        ++c.mat;
      }
    }
  };
  // D blocks in flight per wave (rotating buffers): the narrow widths move
  // fewer bytes per block, so they keep more blocks in flight
  constexpr int D = BITS <= 3 ? 4 : 2;
  Blk<BITS, A_F16, false> b[D];
  GvPos c[D];
  c[0].task = wave_id;
  c[0].mat = wave_id / it.nblk;
  c[0].nb = wave_id - c[0].mat * it.nblk;
  c[0].kb = 0;
#pragma unroll
  for (int u = 1; u < D; ++u) {
    c[u] = c[u - 1];
    advance(c[u], 1);
  }
#pragma unroll
  for (int u = 0; u < D; ++u)  // weights fly while x is staged
    if (c[u].task < it.ntasks) gv_load(b[u], w, cs, ss, c[u], lane);
  gv_stage<BITS, XB, R>(x, w.K, pairs, corr);

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  auto compute = [&](const Blk<BITS, A_F16, false>& b, const GvPos& cu) {
    const int kb = cu.kb;
    const float scale[4] = {half_lo(b.sc[0]), half_hi(b.sc[0]), half_lo(b.sc[1]), half_hi(b.sc[1])};
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint32_t d[8];
      gv_decode<BITS, XB>(b.p0, b.p1, g, d);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int slot = ((r * KB + kb) * 4 + g) * 4 + lg;
        const u32x4 xa = *(const u32x4*)(pairs + 8 * slot);
        const u32x4 xb = *(const u32x4*)(pairs + 8 * slot + 4);
        float a = -corr[slot];  // the chain starts at -C_g
        a = GvFmt<XB>::dot2(d[0], xa[0], a);
        a = GvFmt<XB>::dot2(d[1], xa[1], a);
        a = GvFmt<XB>::dot2(d[2], xa[2], a);
        a = GvFmt<XB>::dot2(d[3], xa[3], a);
        a = GvFmt<XB>::dot2(d[4], xb[0], a);
        a = GvFmt<XB>::dot2(d[5], xb[1], a);
        a = GvFmt<XB>::dot2(d[6], xb[2], a);
        a = GvFmt<XB>::dot2(d[7], xb[3], a);
        acc[r] = __builtin_fmaf(scale[g], a, acc[r]);
      }
    }
    if (kb == KB - 1) {  // task done: add the four lane groups, store
      const uint32_t mat = cu.mat;
      const int n = (int)cu.nb * 16 + (lane & 15);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float v = acc[r];
        v += __shfl_xor(v, 16, 64);
        v += __shfl_xor(v, 32, 64);
        if (lg == 0) y[(int64_t)mat * y_mat_stride + (int64_t)r * w.N + n] = v * GvFmt<XB>::kU;
        acc[r] = 0.f;
      }
    }
  };
  // item j + u sits in buffer u; the items of a wave end together (tasks are
  // taken in order), so the first missing one ends the loop
  for (;;) {
    bool done = false;
#pragma unroll
    for (int u = 0; u < D; ++u) {
      if (!done) {
        if (c[u].task >= it.ntasks) {
          done = true;
        } else {
          compute(b[u], c[u]);
          advance(c[u], D);
          if (c[u].task < it.ntasks) gv_load(b[u], w, cs, ss, c[u], lane);
        }
      }
    }
    if (done) break;
  }
}

template <int BITS, int XB, int R>
hipError_t launch_gv(const QT& q, int64_t count, int64_t cs, int64_t ss, const uint16_t* x, float* y,
                     int64_t rows, hipStream_t s) {
  auto kfn = qgemv_kernel<BITS, XB, R>;
  const size_t lds = gv_lds_bytes(R, q.K);
  static bool attr_set = false;  // one instantiation, one attribute (set before the first launch)
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)gv_lds_bytes(4, 8192));
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  GvItems it;
  it.KB = q.K >> 8;
  it.nblk = (uint32_t)(q.N / 16);
  it.ntasks = (uint32_t)(count * (q.N / 16));
  // one wave per task up to 2048 workgroups (8 per CU); beyond that each
  // wave walks several tasks (x is staged once per workgroup)
  const int64_t wgs = ((int64_t)it.ntasks + kGvWaves - 1) / kGvWaves;
  const unsigned grid = (unsigned)(wgs < 2048 ? wgs : 2048);
  hipLaunchKernelGGL(kfn, dim3(grid), dim3(kGvThreads), lds, s, q, cs, ss, it, x, y, rows * q.N);
  return hipGetLastError();
}

template <int XB>
hipError_t gv_bits_rows(const QT& q, int64_t count, int64_t cs, int64_t ss, const uint16_t* x, float* y,
                        int64_t rows, hipStream_t s) {
#define GV_R(B)                                                                      \
  switch (rows) {                                                                    \
    case 1: return launch_gv<B, XB, 1>(q, count, cs, ss, x, y, rows, s);             \
    case 2: return launch_gv<B, XB, 2>(q, count, cs, ss, x, y, rows, s);             \
    case 3: return launch_gv<B, XB, 3>(q, count, cs, ss, x, y, rows, s);             \
    default: return launch_gv<B, XB, 4>(q, count, cs, ss, x, y, rows, s);            \
  }
  switch (q.bits) {
    case 2: GV_R(2)
    case 3: GV_R(3)
    case 4: GV_R(4)
    case 6: GV_R(6)
  }
#undef GV_R
  return hipErrorInvalidValue;
}

int32_t gemv_common(const AltxsQTensor* w, int64_t count, int64_t cs, int64_t ss, const void* x, int32_t xdt,
                    int64_t rows, float* y, altxs_stream_t stream, const char* who) {
  ALTXS_REQUIRE(w && w->codes && w->scales, "%s: null tensor", who);
  ALTXS_REQUIRE(w->bits == 2 || w->bits == 3 || w->bits == 4 || w->bits == 6, "%s: bits=%d not in {2,3,4,6}",
                who, w->bits);
  ALTXS_REQUIRE(w->N > 0 && w->N % 16 == 0 && w->N < (1 << 24), "%s: N=%lld must be a positive multiple of 16",
                who, (long long)w->N);
  ALTXS_REQUIRE(w->K > 0 && w->K % 256 == 0 && w->K <= 8192,
                "%s: K=%lld must be a positive multiple of 256 (<= 8192)", who, (long long)w->K);
  ALTXS_REQUIRE(((uintptr_t)w->codes & 15) == 0 && ((uintptr_t)w->scales & 7) == 0,
                "%s: codes must be 16-byte and scales 8-byte aligned", who);
  ALTXS_REQUIRE(x && y, "%s: null x/y", who);
  ALTXS_REQUIRE(xdt == ALTXS_F16 || xdt == ALTXS_BF16, "%s: x must be fp16 or bf16 (x_dtype %d)", who, xdt);
  ALTXS_REQUIRE(((uintptr_t)x & 3) == 0, "%s: x must be 4-byte aligned", who);
  ALTXS_REQUIRE(rows >= 1 && rows <= 4, "%s: rows=%lld not in 1..4 (altxs_qgemm takes more)", who,
                (long long)rows);
  ALTXS_REQUIRE(count >= 1 && count * (w->N / 16) < (1ll << 31), "%s: count=%lld out of range", who,
                (long long)count);
  QT q;
  q.codes = (const uint8_t*)w->codes;
  q.scales = (const uint16_t*)w->scales;
  q.N = (int)w->N;
  q.K = (int)w->K;
  q.bits = w->bits;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = xdt == ALTXS_F16 ? gv_bits_rows<0>(q, count, cs, ss, (const uint16_t*)x, y, rows, s)
                                  : gv_bits_rows<1>(q, count, cs, ss, (const uint16_t*)x, y, rows, s);
  ALTXS_CHECK_HIP(e);
  return ALTXS_OK;
}

}  // namespace

extern "C" int32_t altxs_qgemv(const AltxsQTensor* w, const void* x, int32_t x_dtype, int64_t rows, float* y,
                               altxs_stream_t stream) {
  return gemv_common(w, 1, 0, 0, x, x_dtype, rows, y, stream, "altxs_qgemv");
}

extern "C" int32_t altxs_qgemv_stream(const AltxsQTensor* w, int64_t count, int64_t codes_stride,
                                      int64_t scales_stride, const void* x, int32_t x_dtype, int64_t rows,
                                      float* y, altxs_stream_t stream) {
  ALTXS_REQUIRE(w, "altxs_qgemv_stream: null tensor");
  ALTXS_REQUIRE(codes_stride >= w->N * w->K * w->bits / 8 && scales_stride >= w->N * w->K / 64 * 2 &&
                    scales_stride % 8 == 0 && codes_stride % 16 == 0,
                "altxs_qgemv_stream: strides smaller than one tensor or misaligned");
  return gemv_common(w, count, codes_stride, scales_stride / 2, x, x_dtype, rows, y, stream,
                     "altxs_qgemv_stream");
}
