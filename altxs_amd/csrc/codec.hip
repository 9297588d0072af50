// The reference's shipped weight codec on the device: per-channel mixed-bit
// deltas (src/hyperflow_distillation/mixed_bit_delta.py) decoded into dense
// fp32 rows/columns, and dense rows (Init + delta) rounded to bf16 and laid
// out in the MFMA-tiled order the GEMMs read (AltxsQTensor, bits = 16).
//
// Decode arithmetic, per channel of width b and rank r, value i:
//   code  = bits [b*(r*width + i), +b) of the width's stream, LSB first; for
//           b = 3 the stream is 24-bit little-endian words of 8 codes
//           (unpack_codes, mixed_bit_delta.py:96-113)
//   lloyd     : value = float(codebook[r][code])                      (fp16 levels)
//   symmetric : value = (code - (2^b-1)/2) * float(scale[r])          (_symmetric_levels 147-152)
//   shared    : value = float(shared[code]) * float(scale[r])
//   fp4       : value = E2M1[code] * float(scale[r])                  (_fp4_e2m1_table 155-166)
// each a single fp32 rounding at most, as the numpy reference computes it.
#include "common.h"

namespace {

struct DecodeArgs {
  AltxsCodecGroups g;
  const uint8_t* bits;
  const int32_t* rank;
  int64_t n, width, stride_ch, stride_el;
  float* out;
  int32_t* err;
};

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// E2M1: sign bit 3, exponent bits 2-1, mantissa bit 0; e = 0 is subnormal (0.5 * m).
__device__ __forceinline__ float e2m1(uint32_t c) {
  const float m = (float)(c & 1u);
  const uint32_t e = (c >> 1) & 3u;
  const float mag = e == 0 ? 0.5f * m : (1.f + 0.5f * m) * (float)(1u << (e - 1));
  return (c & 8u) ? -mag : mag;
}

__device__ __forceinline__ uint32_t code_at(const uint8_t* p, int b, int64_t a) {
  if (b == 3) {  // 8 codes per 3-byte word
    const int64_t w = a >> 3;
    const uint32_t v = (uint32_t)p[3 * w] | ((uint32_t)p[3 * w + 1] << 8) | ((uint32_t)p[3 * w + 2] << 16);
    return (v >> (3 * (a & 7))) & 7u;
  }
  const int64_t bit = a * b;
  return ((uint32_t)p[bit >> 3] >> (bit & 7)) & ((1u << b) - 1u);
}

// grid: (ceil(width / 256), n channels); one value per thread
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
  const int64_t j = blockIdx.y;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.width) return;
  const int b = a.bits[j];
  float v = 0.f;
  bool bad = false;
  if (b != 0) {
    const int r = a.rank[j];
    const int gi = b - 2;
    const int64_t code_idx = (int64_t)r * a.width + i;
    bad = b < 2 || b > 4 || r < 0 || code_idx >= a.g.n_codes[gi < 0 ? 0 : gi > 2 ? 2 : gi];
    if (!bad) {
      const uint32_t c = code_at(a.g.packed[gi], b, code_idx);
      const uint16_t* cb = a.g.codebook[gi];
      int mode = a.g.mode;
      if (mode == ALTXS_CODEBOOK_HYBRID) mode = b == 4 ? ALTXS_CODEBOOK_FP4 : ALTXS_CODEBOOK_SYMMETRIC;
      if (mode == ALTXS_CODEBOOK_LLOYD) {
        const int64_t e = (int64_t)r * (1 << b) + c;
        bad = e >= a.g.n_book[gi];
        if (!bad) v = h2f(cb[e]);
      } else {
        bad = r >= a.g.n_book[gi] || (mode == ALTXS_CODEBOOK_SHARED && !a.g.shared[gi]) ||
              (mode == ALTXS_CODEBOOK_FP4 && b != 4);
        if (!bad) {
          const float s = h2f(cb[r]);
          if (mode == ALTXS_CODEBOOK_SYMMETRIC) v = ((float)c - 0.5f * (float)((1 << b) - 1)) * s;
          else if (mode == ALTXS_CODEBOOK_SHARED) v = h2f(a.g.shared[gi][c]) * s;
          else v = e2m1(c) * s;
        }
      }
    }
  }
  if (bad) {
    v = 0.f;
    flag_err(a.err, ALTXS_EDEV_TOKEN);
  }
  a.out[j * a.stride_ch + i * a.stride_el] = v;
}

// One 16-row x 256-column block per workgroup (256 threads): thread t packs
// lane t / 4's k-steps 2*(t % 4) and 2*(t % 4) + 1 (16 values, 32 bytes).
__global__ __launch_bounds__(256) void pack_dense_kernel(const float* base, const float* delta,
                                                         int64_t K, int64_t ld, uint8_t* tiled) {
  const int64_t KB = K >> 8;
  const int64_t blk = blockIdx.x;
  const int64_t nb = blk / KB, kb = blk % KB;
  const int lane = threadIdx.x >> 2, sp = threadIdx.x & 3;
  const int64_t row = nb * 16 + (lane & 15);
  uint32_t wv[8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int s = 2 * sp + h;
    const int64_t col = kb * 256 + 32 * s + 8 * (lane >> 4);
    const float* d = delta + row * ld + col;
    const float* bs = base ? base + row * ld + col : nullptr;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float x0 = d[2 * q], x1 = d[2 * q + 1];
      if (bs) { x0 = bs[2 * q] + x0; x1 = bs[2 * q + 1] + x1; }
      wv[4 * h + q] = (uint32_t)f32_to_bf16(x0) | ((uint32_t)f32_to_bf16(x1) << 16);
    }
  }
  u32x4* dst = (u32x4*)(tiled + blk * 8192 + lane * 128 + sp * 32);
  dst[0] = u32x4{wv[0], wv[1], wv[2], wv[3]};
  dst[1] = u32x4{wv[4], wv[5], wv[6], wv[7]};
}

// The same blocks for fp32 weights (bits 32): three bf16 planes hi, mid, lo of
// w = base + delta (hi = bf16(w), mid = bf16(w - hi), lo = bf16(w - hi - mid)
// = w - hi - mid exactly), plane p of block blk at (3 * blk + p) * 8192.
__global__ __launch_bounds__(256) void pack_dense32_kernel(const float* base, const float* delta,
                                                           int64_t K, int64_t ld, uint8_t* tiled) {
  const int64_t KB = K >> 8;
  const int64_t blk = blockIdx.x;
  const int64_t nb = blk / KB, kb = blk % KB;
  const int lane = threadIdx.x >> 2, sp = threadIdx.x & 3;
  const int64_t row = nb * 16 + (lane & 15);
  uint32_t wv[3][8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int s = 2 * sp + h;
    const int64_t col = kb * 256 + 32 * s + 8 * (lane >> 4);
    const float* d = delta + row * ld + col;
    const float* bs = base ? base + row * ld + col : nullptr;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint16_t part[3][2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        float x = d[2 * q + e];
        if (bs) x = bs[2 * q + e] + x;
        const uint16_t hi = f32_to_bf16(x);
        const float r1 = x - bf16_to_f32(hi);
        const uint16_t mid = f32_to_bf16(r1);
        const float r2 = r1 - bf16_to_f32(mid);
        part[0][e] = hi;
        part[1][e] = mid;
        part[2][e] = f32_to_bf16(r2);
      }
#pragma unroll
      for (int p = 0; p < 3; ++p) wv[p][4 * h + q] = (uint32_t)part[p][0] | ((uint32_t)part[p][1] << 16);
    }
  }
#pragma unroll
  for (int p = 0; p < 3; ++p) {
    u32x4* dst = (u32x4*)(tiled + (blk * 3 + p) * 8192 + lane * 128 + sp * 32);
    dst[0] = u32x4{wv[p][0], wv[p][1], wv[p][2], wv[p][3]};
    dst[1] = u32x4{wv[p][4], wv[p][5], wv[p][6], wv[p][7]};
  }
}

}  // namespace

extern "C" int32_t altxs_codec_decode(const AltxsCodecGroups* g, const uint8_t* bits,
                                      const int32_t* rank, int64_t n_channels, int64_t width,
                                      float* out, int64_t stride_ch, int64_t stride_el,
                                      int32_t* err, altxs_stream_t stream) {
  ALTXS_REQUIRE(g && bits && rank && out && err, "altxs_codec_decode: null pointer");
  ALTXS_REQUIRE(g->mode >= ALTXS_CODEBOOK_LLOYD && g->mode <= ALTXS_CODEBOOK_HYBRID,
                "altxs_codec_decode: mode %d", g->mode);
  ALTXS_REQUIRE(n_channels >= 0 && n_channels <= 65535 && width >= 1 && width <= (1 << 20),
                "altxs_codec_decode: n_channels=%lld width=%lld", (long long)n_channels,
                (long long)width);
  for (int b = 0; b < 3; ++b)
    ALTXS_REQUIRE(g->n_codes[b] == 0 || (g->packed[b] && g->codebook[b]),
                  "altxs_codec_decode: %d-bit group has codes but no data", b + 2);
  if (n_channels == 0) return ALTXS_OK;
  DecodeArgs a;
  a.g = *g; a.bits = bits; a.rank = rank; a.n = n_channels; a.width = width;
  a.stride_ch = stride_ch; a.stride_el = stride_el; a.out = out; a.err = err;
  hipLaunchKernelGGL(decode_kernel, dim3((unsigned)((width + 255) / 256), (unsigned)n_channels),
                     dim3(256), 0, (hipStream_t)stream, a);
  ALTXS_CHECK_HIP(hipGetLastError());
  return ALTXS_OK;
}

extern "C" int32_t altxs_pack_dense32(const float* base, const float* delta, int64_t N, int64_t K,
                                      int64_t ld, void* tiled, int64_t tiled_bytes,
                                      altxs_stream_t stream) {
  ALTXS_REQUIRE(delta && tiled, "altxs_pack_dense32: null pointer");
  ALTXS_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 256 == 0 && ld >= K && ld % 2 == 0,
                "altxs_pack_dense32: N=%lld K=%lld ld=%lld", (long long)N, (long long)K,
                (long long)ld);
  ALTXS_REQUIRE(tiled_bytes >= N * K * 6, "altxs_pack_dense32: tiled holds %lld bytes, %lld needed",
                (long long)tiled_bytes, (long long)(N * K * 6));
  ALTXS_REQUIRE(((uintptr_t)tiled & 15) == 0 && ((uintptr_t)delta & 7) == 0 &&
                    ((uintptr_t)base & 7) == 0,
                "altxs_pack_dense32: misaligned");
  hipLaunchKernelGGL(pack_dense32_kernel, dim3((unsigned)(N / 16 * (K / 256))), dim3(256), 0,
                     (hipStream_t)stream, base, delta, K, ld, (uint8_t*)tiled);
  ALTXS_CHECK_HIP(hipGetLastError());
  return ALTXS_OK;
}

extern "C" int32_t altxs_pack_dense(const float* base, const float* delta, int64_t N, int64_t K,
                                    int64_t ld, void* tiled, altxs_stream_t stream) {
  ALTXS_REQUIRE(delta && tiled, "altxs_pack_dense: null pointer");
  ALTXS_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 256 == 0 && ld >= K && ld % 2 == 0,
                "altxs_pack_dense: N=%lld K=%lld ld=%lld", (long long)N, (long long)K,
                (long long)ld);
  ALTXS_REQUIRE(((uintptr_t)tiled & 15) == 0 && ((uintptr_t)delta & 7) == 0 &&
                    ((uintptr_t)base & 7) == 0,
                "altxs_pack_dense: misaligned");
  hipLaunchKernelGGL(pack_dense_kernel, dim3((unsigned)(N / 16 * (K / 256))), dim3(256), 0,
                     (hipStream_t)stream, base, delta, K, ld, (uint8_t*)tiled);
  ALTXS_CHECK_HIP(hipGetLastError());
  return ALTXS_OK;
}
