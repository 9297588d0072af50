// Dequant-fused MFMA GEMM: Y[r, n] = sum_k A[r, k] * W[n, k], W packed as
// symmetric group-64 codes with fp16 scales (include/altxs.h, AltxsQTensor).
//
// The unit of work is a *task*: one 16-row tile (rows m0 .. m0+15) and a
// strided list of column tiles nt = nt0, nt0 + nstep, ... (16*NB columns
// each).  A task runs on one workgroup of NB*KS waves; wave w computes
// n-block w % NB of the current column tile over K-slice w / NB.  Tasks are
// placed by a kernel (one per workgroup, or several per workgroup when a
// persistent team walks a stage), so the same code serves every launch shape.
//
// Per column tile every wave issues the loads of its first two weight blocks
// (16 rows x 256 k each) before anything else -- for the first tile even
// before the A prologue -- so HBM latency overlaps the activation work.  In the
// tiled layout lane l of a wave owns the 64 codes of row (l % 16) at
// k = 32*s + 8*(l / 16) + i (s, i < 8) -- exactly the B operand of
// v_mfma_f32_16x16x32_{bf16,f16} for the block's eight k-steps -- so a block
// arrives as one or two 16-byte loads per lane.  Codes become (c - (2^b-1)/2),
// exact in bf16/fp16; each 64-wide group's fp32 partial is scaled by its fp16
// scale.
//
// A operand: staged once per task in LDS by a prologue functor (RMSNorm,
// residual mixes and skips fused there) or, for plain inputs, loaded by each
// lane straight into MFMA registers.
//
// Reduction and determinism.  Inside a wave: the MFMA's fixed internal order,
// then groups in increasing k.  Across the KS K-slices: partial tiles go to LDS
// and are added in slice order.  The order depends only on K and (NB, KS),
// never on the number of rows or on how tasks are placed, so results are
// bit-identical for any batch, window size or launch shape.
//
// Epilogue: a functor.  Epi::prefetch() runs before the MFMAs (issue loads of
// residuals, positions, RoPE tables early); Epi::apply() gets the reduced
// 16 x (16*NB) fp32 tile in LDS and runs on all threads.
#pragma once
#include <type_traits>

#include "common.h"

namespace altxs {

// BITS == 0 selects the run-time bit-width specialisation: one code path that
// decodes any width with uniform selects (used where one kernel serves tensors
// of several widths); it feeds the MFMAs exactly the operands of BITS = b.
template <int BITS> struct Planes;
template <> struct Planes<0> { static constexpr int P0 = 4, P1 = 2; };  // storage maxima
template <> struct Planes<2> { static constexpr int P0 = 2, P1 = 0; };
template <> struct Planes<3> { static constexpr int P0 = 2, P1 = 1; };
template <> struct Planes<4> { static constexpr int P0 = 4, P1 = 0; };
template <> struct Planes<6> { static constexpr int P0 = 4, P1 = 2; };
// BITS == 16: dense bf16 weights in the same tiled order (no codes, no scales):
// a lane's 64 values of a block are 32 words, k-step s in words 4s..4s+3.
template <> struct Planes<16> { static constexpr int P0 = 16, P1 = 0; };
// BITS == 32: dense fp32 weights as three bf16 planes w = hi + mid + lo
// (hi = bf16(w), mid = bf16(w - hi), lo = w - hi - mid, which is a bf16 value:
// the split is exact), each plane a bits-16 block, the three planes of a
// block stored one after the other.  The GEMM walks *virtual* blocks
// v = 3 * kb + plane: one plane in registers at a time, the A slice of block
// kb applied to each.
template <> struct Planes<32> { static constexpr int P0 = 16, P1 = 0; };
// BITS == kExpBits (8; internal, not a C-ABI width): the expanded form of a
// packed tensor -- the bf16 values (code - centre), exact, N*K*2 bytes written
// by altxs_expand_codes -- with the packed tensor's group scales.  Each 16 x
// 256 block is stored k-step-major: k-step s's 1 KB holds lane l's 16-byte B
// operand at 16 l, so one wave load reads 1 KB of consecutive bytes.  The MFMAs see exactly the operands the packed path
// builds from the codes, so results are the same bits; the large-tile kernels
// read them straight into B operands instead of decoding codes once per 64
// rows (the decode is most of their VALU work).
constexpr int kExpBits = 8;
template <> struct Planes<8> { static constexpr int P0 = 16, P1 = 0; };
// virtual blocks per 16 x 256 block of weights
template <int BITS> __host__ __device__ constexpr int vpb() { return BITS == 32 ? 3 : 1; }

// A-operand modes
// A_F32S: fp32 rows staged (by a prologue) as their three bf16 parts --
// split3's hi, mid and lo, each a plane of K + 8 elements inside the row -- so
// the k-loop reads the MFMA operands that A_F32 forms in the loop, without
// splitting them again in every wave.  The same operands: the same bits.
enum AMode : int { A_F32 = 0, A_BF16 = 1, A_F16 = 2, A_F32S = 3 };

struct QT {
  const uint8_t* codes;
  const uint16_t* scales;
  int N, K;
  int bits;  // read only by the run-time-width specialisation (BITS == 0)
};

__host__ __device__ constexpr int lds_stride(int K, int am) {
  return am == A_F32 ? K + 4 : am == A_F32S ? 3 * (K + 8) : K + 8;
}
__host__ __device__ constexpr int a_esz(int am) { return am == A_F32 ? 4 : 2; }

// Store four consecutive fp32 values (col % 4 == 0) into an LDS A tile.
template <int AM>
__device__ __forceinline__ void a_store4(void* As, int row, int col, int K, const float (&v)[4]) {
  if constexpr (AM == A_F32) {
    f32x4 o = {v[0], v[1], v[2], v[3]};
    *(f32x4*)((float*)As + row * lds_stride(K, AM) + col) = o;
  } else if constexpr (AM == A_F32S) {  // split3 (below) of each value, one plane per part
    // (the residuals from the rounded values, as split3 sees them after an
    // fp32 store: no product of the caller's may fuse into them)
#pragma clang fp contract(off)
    uint16_t h[3][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const __bf16 h0 = (__bf16)v[i];
      const float r1 = v[i] - (float)h0;
      const __bf16 h1 = (__bf16)r1;
      const float r2 = r1 - (float)h1;
      h[0][i] = __builtin_bit_cast(uint16_t, h0);
      h[1][i] = __builtin_bit_cast(uint16_t, h1);
      h[2][i] = __builtin_bit_cast(uint16_t, (__bf16)r2);
    }
    uint16_t* base = (uint16_t*)As + row * lds_stride(K, AM) + col;
#pragma unroll
    for (int p = 0; p < 3; ++p)
      *(u32x2*)(base + p * (K + 8)) =
          u32x2{(uint32_t)h[p][0] | ((uint32_t)h[p][1] << 16), (uint32_t)h[p][2] | ((uint32_t)h[p][3] << 16)};
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

// Run-time width (BITS == 0).  A block is loaded in its stored layout and, once
// its data is in registers, rewritten in place into the 6-bit layout: p0[s]
// holds the low nibbles of k-step s (code i at bits 4i), p1[s >> 1] the two
// high bits (code i at bits 16 (s & 1) + 2i).  Codes of 2 and 3 bits fit in a
// nibble, so their p1 is zero.  Every index is a compile-time constant and the
// only branch is on the (uniform) width, so nothing goes to scratch.
__device__ __forceinline__ uint32_t spread2to4(uint32_t x) {  // 8 fields of 2 bits -> nibbles
  x = (x | (x << 8)) & 0x00FF00FFu;
  x = (x | (x << 4)) & 0x0F0F0F0Fu;
  return (x | (x << 2)) & 0x33333333u;
}
__device__ __forceinline__ uint32_t spread1to4(uint32_t x) {  // 8 bits -> bit i at 4i
  x = (x | (x << 12)) & 0x000F000Fu;
  x = (x | (x << 6)) & 0x03030303u;
  return (x | (x << 3)) & 0x11111111u;
}
__device__ __forceinline__ void planes_to6(int bits, uint32_t (&p0)[8], uint32_t (&p1)[4]) {
  if (bits <= 3) {
    uint32_t t[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) t[s] = spread2to4((p0[s >> 1] >> (16 * (s & 1))) & 0xFFFFu);
    if (bits == 3) {
#pragma unroll
      for (int s = 0; s < 8; ++s) t[s] |= spread1to4((p1[s >> 2] >> (8 * (s & 3))) & 0xFFu) << 2;
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) p0[s] = t[s];
  }
  if (bits != 6) {
#pragma unroll
    for (int i = 0; i < 4; ++i) p1[i] = 0u;
  }
}

template <int BITS>
__device__ __forceinline__ float code_center(int bits) {
  if constexpr (BITS == 0) return 0.5f * (float)((1 << bits) - 1);
  else if constexpr (BITS <= 8) return 0.5f * (float)((1 << BITS) - 1);
  else return 0.f;  // dense widths carry values, not codes
}

// 2- and 3-bit codes by table: every value c - center is exact in bf16, so a
// byte table of the bf16 bits, read with v_perm_b32, gives the operand with
// the same bits as the conversion below at about half the VALU work.
// lut_bytes<BITS, F16>(hi, half): byte i = low (hi = 0) or high byte of
// bf16(c - center) (fp16 with F16) for c = 4 * half + i (folded to constants).
template <int BITS, bool F16 = false>
__device__ __forceinline__ uint32_t lut_bytes(int hi, int half) {
  uint32_t w = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v = (float)(4 * half + i) - 0.5f * (float)((1 << BITS) - 1);
    // exact in either format: at most 3 mantissa bits
    const uint32_t b = F16 ? (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v)
                           : __builtin_bit_cast(uint32_t, v) >> 16;
    w |= ((hi ? b >> 8 : b) & 0xFFu) << (8 * i);
  }
  return w;
}
// 2-bit fields i = 0..3 (bits 2i, 2i+1 of x < 256) -> byte i
__device__ __forceinline__ uint32_t spread2to8(uint32_t x) {
  x = (x | (x << 12)) & 0x000F000Fu;
  return (x | (x << 6)) & 0x03030303u;
}
// bits i = 0..3 of x < 16 -> bit 0 of byte i
__device__ __forceinline__ uint32_t spread1to8(uint32_t x) {
  x = (x | (x << 14)) & 0x00030003u;
  return (x | (x << 7)) & 0x01010101u;
}
// Four codes (one per byte of c4) -> two words of bf16 (fp16 with F16) pairs.
template <int BITS, bool F16 = false>
__device__ __forceinline__ void lut4(uint32_t c4, uint32_t& w01, uint32_t& w23) {
  // v_perm_b32: byte selector k < 4 takes byte k of the second source, 4..7
  // byte k - 4 of the first
  const uint32_t lo = __builtin_amdgcn_perm(lut_bytes<BITS, F16>(0, 1), lut_bytes<BITS, F16>(0, 0), c4);
  const uint32_t hi = __builtin_amdgcn_perm(lut_bytes<BITS, F16>(1, 1), lut_bytes<BITS, F16>(1, 0), c4);
  w01 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // lo0 hi0 lo1 hi1
  w23 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // lo2 hi2 lo3 hi3
}

// (float) of byte M of x.  The compiler folds the byte masks of the 4-bit
// path below into per-field extracts and then converts from byte 0 only; the
// instruction itself reads any byte in place.
template <int M>
__device__ __forceinline__ float ubyte_f32(uint32_t x) {
  float r;
  if constexpr (M == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(x));
  else if constexpr (M == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(x));
  else if constexpr (M == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(x));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(x));
  return r;
}

// B operand of k-step s: codes - center.  BITS == 0 expects the 6-bit layout
// (planes_to6 already applied).
template <int BITS>
__device__ __forceinline__ bf16x8 b_op_bf16(const uint32_t* p0, const uint32_t* p1, int s, int bits) {
  if constexpr (BITS == 16 || BITS == 32 || BITS == kExpBits)
    return __builtin_bit_cast(bf16x8, u32x4{p0[4 * s], p0[4 * s + 1], p0[4 * s + 2], p0[4 * s + 3]});
  if constexpr (BITS == 2 || BITS == 3) {
    static_assert(Planes<BITS>::P0 == 2, "2-bit low plane: k-step s is bits 16 (s & 1) + 2i of p0[s >> 1]");
    const uint32_t f0 = (p0[s >> 1] >> (16 * (s & 1))) & 0xFFFFu;
    uint32_t ca = spread2to8(f0 & 0xFFu), cb = spread2to8(f0 >> 8);
    if constexpr (BITS == 3) {  // third bit: bit 8 (s & 3) + i of p1[s >> 2]
      const uint32_t f1 = (p1[s >> 2] >> (8 * (s & 3))) & 0xFFu;
      ca |= spread1to8(f1 & 0xFu) << 2;
      cb |= spread1to8(f1 >> 4) << 2;
    }
    uint32_t r0, r1, r2, r3;
    lut4<BITS>(ca, r0, r1);
    lut4<BITS>(cb, r2, r3);
    return __builtin_bit_cast(bf16x8, u32x4{r0, r1, r2, r3});
  }
  if constexpr (BITS == 4) {
    // nibbles -> bytes: byte m of ca / cb holds code 2m / 2m + 1, which the
    // byte conversions (v_cvt_f32_ubyte0..3) read in place; the arithmetic is
    // the generic path's ((float)c - center, rounded to bf16)
    const uint32_t w = p0[s];
    const uint32_t ca = w & 0x0F0F0F0Fu, cb = (w >> 4) & 0x0F0F0F0Fu;
    bf16x8 r;
    r[0] = (__bf16)(ubyte_f32<0>(ca) - 7.5f);
    r[1] = (__bf16)(ubyte_f32<0>(cb) - 7.5f);
    r[2] = (__bf16)(ubyte_f32<1>(ca) - 7.5f);
    r[3] = (__bf16)(ubyte_f32<1>(cb) - 7.5f);
    r[4] = (__bf16)(ubyte_f32<2>(ca) - 7.5f);
    r[5] = (__bf16)(ubyte_f32<2>(cb) - 7.5f);
    r[6] = (__bf16)(ubyte_f32<3>(ca) - 7.5f);
    r[7] = (__bf16)(ubyte_f32<3>(cb) - 7.5f);
    return r;
  }
  const float center = code_center<BITS>(bits);
  uint32_t c[8];
  codes_step<BITS == 0 ? 6 : BITS>(p0, p1, s, c);
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (__bf16)((float)c[i] - center);
  return r;
}

template <int BITS>
__device__ __forceinline__ f16x8 b_op_f16(const uint32_t* p0, const uint32_t* p1, int s, int bits) {
  static_assert(BITS != 16 && BITS != kExpBits, "bf16 weight values take bf16 or fp32 activations");
  if constexpr (BITS == 2 || BITS == 3) {  // the bf16 path's byte table, with fp16 bytes
    const uint32_t f0 = (p0[s >> 1] >> (16 * (s & 1))) & 0xFFFFu;
    uint32_t ca = spread2to8(f0 & 0xFFu), cb = spread2to8(f0 >> 8);
    if constexpr (BITS == 3) {
      const uint32_t f1 = (p1[s >> 2] >> (8 * (s & 3))) & 0xFFu;
      ca |= spread1to8(f1 & 0xFu) << 2;
      cb |= spread1to8(f1 >> 4) << 2;
    }
    uint32_t r0, r1, r2, r3;
    lut4<BITS, true>(ca, r0, r1);
    lut4<BITS, true>(cb, r2, r3);
    return __builtin_bit_cast(f16x8, u32x4{r0, r1, r2, r3});
  }
  if constexpr (BITS == 4) {
    // fp16 0x4C00 | (c << 6) is exactly 16 + c (the mantissa step at 16 is
    // 1/64), and (16 + c) - 23.5 = c - 7.5 exactly: the generic path's value.
    // Byte j of t / u holds code 2j / 2j + 1 of the k-step.
    typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
    const uint32_t w = p0[s];
    const uint32_t t = w & 0x0F0F0F0Fu, u = (w >> 4) & 0x0F0F0F0Fu;
    const f16x2 off = {(_Float16)-23.5f, (_Float16)-23.5f};
    uint32_t r[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // bytes [t_j, 0, u_j, 0]: code 2j in bits 0-3, code 2j + 1 in bits 16-19
      const uint32_t sel = (uint32_t)j | (0x0Cu << 8) | ((uint32_t)(4 + j) << 16) | (0x0Cu << 24);
      const uint32_t m = (__builtin_amdgcn_perm(u, t, sel) << 6) | 0x4C004C00u;
      r[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, m) + off);
    }
    return __builtin_bit_cast(f16x8, u32x4{r[0], r[1], r[2], r[3]});
  }
  const float center = code_center<BITS>(bits);
  uint32_t c[8];
  codes_step<BITS == 0 ? 6 : BITS>(p0, p1, s, c);
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

// Weight codes + scales of block (nb, kb) for this lane (BITS == 32: kb is the
// virtual block 3 * block + plane).
template <int BITS, int AM, bool ADIRECT>
__device__ __forceinline__ void load_w(Blk<BITS, AM, ADIRECT>& b, const QT& w, int nb, int kb,
                                       int lane) {
  const int KB = w.K >> 8;
  const size_t bi = (size_t)nb * KB + kb;
  if constexpr (BITS == 32) {
    const size_t plane = (size_t)(nb * KB) * 3 + kb;  // (block, plane) in storage order
    const u32x4* a0 = (const u32x4*)(w.codes + plane * (512 * 16)) + lane * 8;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const u32x4 x = a0[v];
#pragma unroll
      for (int i = 0; i < 4; ++i) b.p0[4 * v + i] = x[i];
    }
    b.sc[0] = b.sc[1] = 0u;
  } else if constexpr (BITS == 0) {
    // every element is defined on every path (whole-vector phis), so the block
    // stays in registers; the branches are on the uniform width only
    const int nbits = w.bits;
    const bool wide = nbits >= 4;
    const uint8_t* blk = w.codes + bi * (512 * nbits);
    const uint8_t* a0 = blk + lane * (wide ? 32 : 16);
    const uint8_t* a1 = blk + 512 * (wide ? 4 : 2);
    const u32x4 x = *(const u32x4*)a0;
    u32x4 y = {0u, 0u, 0u, 0u}, z = {0u, 0u, 0u, 0u};
    if (wide) y = *(const u32x4*)(a0 + 16);
    if (nbits == 6) {
      z = *(const u32x4*)(a1 + lane * 16);
    } else if (nbits == 3) {
      const u32x2 t = *(const u32x2*)(a1 + lane * 8);
      z = u32x4{t[0], t[1], 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) { b.p0[i] = x[i]; b.p0[4 + i] = y[i]; b.p1[i] = z[i]; }
    const u32x2 sv = *(const u32x2*)(w.scales + bi * 64 + (lane & 15) * 4);
    b.sc[0] = sv[0]; b.sc[1] = sv[1];
  } else if constexpr (BITS == 16 || BITS == kExpBits) {
    // bits 16: lane-major (a lane's 128 bytes together); expanded: k-step-major
    const u32x4* a0 = (const u32x4*)(w.codes + bi * (512 * 16)) + (BITS == 16 ? lane * 8 : lane);
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const u32x4 x = a0[BITS == 16 ? v : 64 * v];
#pragma unroll
      for (int i = 0; i < 4; ++i) b.p0[4 * v + i] = x[i];
    }
    if constexpr (BITS == kExpBits) {
      const u32x2 sv = *(const u32x2*)(w.scales + bi * 64 + (lane & 15) * 4);
      b.sc[0] = sv[0]; b.sc[1] = sv[1];
    } else {
      b.sc[0] = b.sc[1] = 0u;
    }
  } else {
    constexpr int P0 = Planes<BITS>::P0, P1 = Planes<BITS>::P1;
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
  }
}

// The lane's slice of the A rows for block column kb (direct A only).
template <int BITS, int AM, bool ADIRECT>
__device__ __forceinline__ void load_a(Blk<BITS, AM, ADIRECT>& b, const QT& w, int kb, int lane,
                                       const ADirect& ad, int m0, int R, int batch) {
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

// Virtual block kb (= the weight block for every width but 32).
template <int BITS, int AM, bool ADIRECT>
__device__ __forceinline__ void load_blk(Blk<BITS, AM, ADIRECT>& b, const QT& w, int nb, int kb,
                                         int lane, const ADirect& ad, int m0, int R, int batch) {
  load_w(b, w, nb, kb, lane);
  load_a(b, w, kb / vpb<BITS>(), lane, ad, m0, R, batch);
}

// Dependency hook of a task: runs after the first tile's weight loads are
// issued and before anything that reads activations.  NoWait for kernels
// whose inputs were produced by earlier launches.
struct NoWait {
  __device__ void operator()() const {}
};

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

// acc += W-block . A-slice (one 16x256 block, 8 MFMA k-steps; BITS == 32: one
// plane of virtual block vb, applied to the A slice of block vb / 3).
template <int BITS, int AM, bool ADIRECT>
__device__ __forceinline__ void compute_blk(const Blk<BITS, AM, ADIRECT>& b, const void* As, int K,
                                            int vb, int lane, f32x4& acc, int bits = BITS) {
  const int kb = vb / vpb<BITS>();
  float scale[4] = {half_lo(b.sc[0]), half_hi(b.sc[0]), half_lo(b.sc[1]), half_hi(b.sc[1])};
  if constexpr (BITS == 16 || BITS == 32) scale[0] = scale[1] = scale[2] = scale[3] = 1.f;  // dense: acc += t
  const int row = lane & 15;
  constexpr int P0 = Planes<BITS>::P0, P1 = Planes<BITS>::P1;
  uint32_t q0[2 * P0], q1[P1 > 0 ? 2 * P1 : 1];
#pragma unroll
  for (int i = 0; i < 2 * P0; ++i) q0[i] = b.p0[i];
#pragma unroll
  for (int i = 0; i < (P1 > 0 ? 2 * P1 : 1); ++i) q1[i] = b.p1[i];
  if constexpr (BITS == 0) planes_to6(bits, q0, q1);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) {
      const int s = 2 * g + ss;
      const int kc = kb * 256 + 32 * s + 8 * (lane >> 4);
      if constexpr (AM == A_F32 || AM == A_F32S) {
        bf16x8 a0, a1, a2;
        if constexpr (AM == A_F32S) {
          static_assert(!ADIRECT, "pre-split rows are staged by a prologue");
          const uint16_t* a = (const uint16_t*)As + row * lds_stride(K, AM) + kc;
          a0 = __builtin_bit_cast(bf16x8, *(const u32x4*)a);
          a1 = __builtin_bit_cast(bf16x8, *(const u32x4*)(a + (K + 8)));
          a2 = __builtin_bit_cast(bf16x8, *(const u32x4*)(a + 2 * (K + 8)));
        } else {
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
          split3(x, a0, a1, a2);
        }
        const bf16x8 bo = b_op_bf16<BITS>(q0, q1, s, bits);
        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bo, t, 0, 0, 0);
        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bo, t, 0, 0, 0);
        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, bo, t, 0, 0, 0);
      } else {
        u32x4 araw;
        if constexpr (ADIRECT) araw = b.a[s];
        else araw = *(const u32x4*)((const uint16_t*)As + row * lds_stride(K, AM) + kc);
        if constexpr (AM == A_BF16) {
          const bf16x8 bo = b_op_bf16<BITS>(q0, q1, s, bits);
          t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, araw), bo, t, 0, 0, 0);
        } else {
          const f16x8 bo = b_op_f16<BITS>(q0, q1, s, bits);
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
  static constexpr size_t kScratch = 0;
  template <int AM, int NT>
  __device__ void stage(void*, void*, int, int, int, int, bool) const {}
};

template <int NB, int KS>
struct TileCfg {
  static constexpr int WAVES = NB * KS;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int NCOL = 16 * NB;
  static constexpr int CS = NCOL + 1;  // padded C tile stride (floats)
};

// LDS of a task: [A tile (if staged)] [C partial tiles: KS x 16 x CS floats]
// [prologue scratch].
template <int AM, int NB, int KS, class Pro>
__host__ __device__ constexpr size_t task_lds_bytes(int K) {
  return (Pro::kStage ? (size_t)16 * lds_stride(K, AM) * a_esz(AM) : 0) +
         (size_t)KS * 16 * TileCfg<NB, KS>::CS * 4 + Pro::kScratch;
}

// One task: rows [m0, m0+16) x column tiles nt0, nt0 + nstep, ... < ntiles.
template <int BITS, int AM, int NB, int KS, class Pro, class Epi, class Wait = NoWait>
__device__ __forceinline__ void gemm_task(const QT& w, int R, int m0, int nt0, int nstep,
                                          const ADirect& ad, const Pro& pro, const Epi& epi,
                                          unsigned char* smem, int batch = 0,
                                          const Wait& wait = Wait{}) {
  using Cfg = TileCfg<NB, KS>;
  constexpr bool STAGE = Pro::kStage;
  constexpr bool ADIRECT = !STAGE;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nbi = wave % NB, ks = wave / NB;
  const int ntiles = (w.N + Cfg::NCOL - 1) / Cfg::NCOL;
  const int KB = w.K >> 8;
  // virtual blocks (weight blocks, or planes of blocks for BITS == 32) of this K-slice
  const int kb0 = ks * (KB / KS) * vpb<BITS>(), kb1 = kb0 + KB / KS * vpb<BITS>();  // host: KB % KS == 0
  void* As = smem;
  const size_t a_bytes = STAGE ? (size_t)16 * lds_stride(w.K, AM) * a_esz(AM) : 0;
  float* Cp = (float*)(smem + a_bytes);
  void* scratch = smem + a_bytes + (size_t)KS * 16 * Cfg::CS * 4;

  Blk<BITS, AM, ADIRECT> b0, b1;
  auto issue_w = [&](int nt) {
    const int nb = nt * NB + nbi;
    if (nb * 16 < w.N) {
      if (kb0 < kb1) load_w(b0, w, nb, kb0, lane);
      if (kb0 + 1 < kb1) load_w(b1, w, nb, kb0 + 1, lane);
    }
  };
  auto issue_a = [&](int nt) {
    if constexpr (ADIRECT) {
      if ((nt * NB + nbi) * 16 < w.N) {
        if (kb0 < kb1) load_a(b0, w, kb0 / vpb<BITS>(), lane, ad, m0, R, batch);
        if (kb0 + 1 < kb1) load_a(b1, w, (kb0 + 1) / vpb<BITS>(), lane, ad, m0, R, batch);
      }
    }
  };
  auto issue = [&](int nt) { issue_w(nt); issue_a(nt); };
  if (nt0 < ntiles) issue_w(nt0);
  wait();
  if (nt0 < ntiles) issue_a(nt0);
  if constexpr (STAGE) {
    pro.template stage<AM, Cfg::THREADS>(As, scratch, m0, R, w.K, batch, nt0 == 0);
    __syncthreads();
  }
  for (int nt = nt0; nt < ntiles; nt += nstep) {
    const int n0 = nt * Cfg::NCOL;
    const int nb = nt * NB + nbi;
    const bool active = nb * 16 < w.N;
    const auto pre = epi.template prefetch<Cfg>(m0, n0, R, batch);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (active) {
      for (int kb = kb0; kb < kb1; kb += 2) {
        compute_blk(b0, As, w.K, kb, lane, acc, w.bits);
        if (kb + 2 < kb1) load_blk(b0, w, nb, kb + 2, lane, ad, m0, R, batch);
        if (kb + 1 < kb1) {
          compute_blk(b1, As, w.K, kb + 1, lane, acc, w.bits);
          if (kb + 3 < kb1) load_blk(b1, w, nb, kb + 3, lane, ad, m0, R, batch);
        }
      }
    }
    if (nt + nstep < ntiles) issue(nt + nstep);  // next tile's weights fly during the epilogue
    {  // partial tile of this wave -> LDS slice ks (MFMA layout: rows 4*(l/16)+i, col l%16)
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
    epi.template apply<Cfg>(Cp, pre, As, m0, n0, R, batch);
    __syncthreads();  // Cp (and As for epilogues that read it) are reused by the next tile
  }
}

// ---- generic epilogue: y[batch][r][n] = acc -----------------------------------
struct EpiStore {
  float* y;
  int N;
  int64_t y_batch_stride;
  struct Pre {};
  template <class Cfg>
  __device__ Pre prefetch(int, int, int, int) const { return {}; }
  template <class Cfg, class P>
  __device__ void apply(const float* C, const P&, const void*, int m0, int n0, int R, int batch) const {
    for (int e = threadIdx.x; e < 16 * Cfg::NCOL; e += Cfg::THREADS) {
      const int r = e / Cfg::NCOL, c = e % Cfg::NCOL;
      if (m0 + r < R && n0 + c < N)
        y[batch * y_batch_stride + (int64_t)(m0 + r) * N + n0 + c] = C[r * Cfg::CS + c];
    }
  }
};

// A grid of tasks: blockIdx.y = row tile, blockIdx.x = first column tile,
// stride gridDim.x; blockIdx.z = batch (tensors at fixed strides).
template <int BITS, int AM, int NB, int KS, class Pro, class Epi>
__global__ __launch_bounds__(64 * NB * KS) void gemm_kernel(QT w, int R, int64_t codes_stride,
                                                            int64_t scales_stride, ADirect ad,
                                                            Pro pro, Epi epi, int rows8) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int batch = blockIdx.z;
  QT wb = w;
  wb.codes += batch * codes_stride;
  wb.scales += batch * scales_stride;
  int cx = blockIdx.x, ry = blockIdx.y, m0, rows = R;
  if (rows8) {
    // decode launches: 8-row tiles (rows m0 .. m0+7 of a 16-row task; the
    // rest are bounds-masked like rows past R), tile t on XCD t % 8
    xcd_row_split(blockIdx.x + gridDim.x * blockIdx.y, gridDim.y, ry, cx);
    m0 = 8 * ry;
    rows = R < m0 + 8 ? R : m0 + 8;
  } else {
    // Workgroups are dealt to the 8 XCDs round-robin by linear id.  When the
    // column-task count is a multiple of 8, renumber so that every row tile of
    // a column task lands on the same XCD: its weights then come into that
    // XCD's L2 once instead of once per row tile.
    if (gridDim.x % 8 == 0) {
      const int bid = blockIdx.x + gridDim.x * blockIdx.y;
      const int rest = bid / 8;
      ry = rest % gridDim.y;
      cx = (rest / gridDim.y) * 8 + bid % 8;
    }
    m0 = 16 * ry;
  }
  gemm_task<BITS, AM, NB, KS>(wb, rows, m0, cx, gridDim.x, ad, pro, epi, smem, batch);
}

// Launch helper: column tiles are spread over `col_wgs` workgroups per row tile
// (0 = one workgroup per column tile).  rows8: decode placement (8-row tiles,
// tile t on XCD t % 8; R % 64 == 0, batch 1).  Sets the dynamic LDS limit once
// per instantiation.
template <int BITS, int AM, int NB, int KS, class Pro, class Epi>
hipError_t launch_gemm(const QT& w, int R, int batch, int64_t codes_stride, int64_t scales_stride,
                       const ADirect& ad, const Pro& pro, const Epi& epi, int col_wgs,
                       hipStream_t s, bool rows8 = false) {
  if (rows8 && (R % 64 != 0 || batch != 1)) return hipErrorInvalidValue;
  auto kfn = gemm_kernel<BITS, AM, NB, KS, Pro, Epi>;
  const size_t lds = task_lds_bytes<AM, NB, KS, Pro>(w.K);
  static size_t configured = 0;
  if (lds > 65536 && lds > configured) {
    hipError_t e = hipFuncSetAttribute((const void*)kfn,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    configured = lds;
  }
  const int ntiles = (w.N + 16 * NB - 1) / (16 * NB);
  const int cw = (col_wgs <= 0 || col_wgs > ntiles) ? ntiles : col_wgs;
  dim3 grid((unsigned)cw, (unsigned)(rows8 ? R / 8 : (R + 15) / 16), (unsigned)batch);
  hipLaunchKernelGGL(kfn, grid, dim3(TileCfg<NB, KS>::THREADS), lds, s, w, R, codes_stride,
                     scales_stride, ad, pro, epi, rows8 ? 1 : 0);
  return hipGetLastError();
}

// Dispatch on the runtime bit width.
template <int AM, int NB, int KS, class Pro, class Epi>
hipError_t launch_gemm_bits(int bits, const QT& w, int R, int batch, int64_t codes_stride,
                            int64_t scales_stride, const ADirect& ad, const Pro& pro,
                            const Epi& epi, int col_wgs, hipStream_t s, bool rows8 = false) {
  switch (bits) {
    case 2: return launch_gemm<2, AM, NB, KS>(w, R, batch, codes_stride, scales_stride, ad, pro, epi, col_wgs, s, rows8);
    case 3: return launch_gemm<3, AM, NB, KS>(w, R, batch, codes_stride, scales_stride, ad, pro, epi, col_wgs, s, rows8);
    case 4: return launch_gemm<4, AM, NB, KS>(w, R, batch, codes_stride, scales_stride, ad, pro, epi, col_wgs, s, rows8);
    case 6: return launch_gemm<6, AM, NB, KS>(w, R, batch, codes_stride, scales_stride, ad, pro, epi, col_wgs, s, rows8);
    case 16:
      if constexpr (AM != A_F16)
        return launch_gemm<16, AM, NB, KS>(w, R, batch, codes_stride, scales_stride, ad, pro, epi, col_wgs, s, rows8);
      return hipErrorInvalidValue;
    case 32:  // fp32 dense weights: the fp32-activation path only
      if constexpr (AM == A_F32 || AM == A_F32S)
        return launch_gemm<32, AM, NB, KS>(w, R, batch, codes_stride, scales_stride, ad, pro, epi, col_wgs, s, rows8);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

// 4-wave task shapes: (NB, KS) in {(4,1), (2,2), (1,4)}.  The K-split is the
// largest KS <= ks_max that divides K/256 (a property of the tensor, so every
// launch shape of a stage uses the same reduction order).
__host__ __device__ constexpr int pick_ks(int K, int ks_max) {
  return (ks_max >= 4 && (K >> 8) % 4 == 0) ? 4 : (ks_max >= 2 && (K >> 8) % 2 == 0) ? 2 : 1;
}

template <int AM, class Pro, class Epi>
hipError_t launch_gemm4(int ks_max, int bits, const QT& w, int R, const ADirect& ad,
                        const Pro& pro, const Epi& epi, int col_wgs, hipStream_t s,
                        bool rows8 = false) {
  switch (pick_ks(w.K, ks_max)) {
    case 4: return launch_gemm_bits<AM, 1, 4>(bits, w, R, 1, 0, 0, ad, pro, epi, col_wgs, s, rows8);
    case 2: return launch_gemm_bits<AM, 2, 2>(bits, w, R, 1, 0, 0, ad, pro, epi, col_wgs, s, rows8);
    default: return launch_gemm_bits<AM, 4, 1>(bits, w, R, 1, 0, 0, ad, pro, epi, col_wgs, s, rows8);
  }
}

// ---------------------------------------------------------------------------
// Large-tile variant for launches with many rows (encode windows, chunk
// scoring).  The 16-row tasks above decode every weight block once per 16
// rows, which makes thousands of row tiles VALU-bound on the code unpacking.
// Here a workgroup owns BIG_M = 64 rows x BIG_N = 128 columns: the A rows
// (bf16, already normalised by norm_rows_kernel where the stage has a
// prologue) pass through LDS one 256-wide k-block at a time, and each wave
// decodes its two 16-column weight blocks once per k-step and applies them
// to all four 16-row blocks.  Two workgroups share a CU: the kernel is bound
// by latency (weight decode, LDS reads, the scaled accumulation), and the
// second workgroup's waves hide it; 128-row tiles at one workgroup per CU
// ran 1.3-1.4x slower, 32-row tiles decode each weight block too often.
//
// Bit-identical to gemm_task for the same (NB, KS): every 16x16 output block
// sees the same MFMA sequence (k-steps in order, one group of two k-steps per
// fp16 scale, acc += scale * t), each K-slice of K/KS starts from zero, the
// slices are added in slice order, and the epilogue runs on 16 x (16*NB)
// tiles laid out exactly as gemm_task leaves them in LDS.
// ---------------------------------------------------------------------------
constexpr int BIG_M = 64, BIG_N = 128;
// A k-block in LDS: 64 rows x 256 bf16 (512 B a row, no padding), the 16-byte
// chunk c of row r stored at chunk position c ^ (r & 15): the 16 rows an MFMA
// A-operand read touches at one k then fall on 16 different bank groups.
__device__ __forceinline__ int big_a_off(int r, int c) { return r * 256 + ((c ^ (r & 15)) << 3); }

// Epilogues that also offer strip<Cfg>(strip C tile, r0, n0, R) -- the same
// per-element arithmetic over a 16 x BIG_N strip, used when strip_ok() -- set
// kStrip.
template <class E, class = void> struct epi_has_strip : std::false_type {};
template <class E>
struct epi_has_strip<E, std::void_t<decltype(E::kStrip)>> : std::integral_constant<bool, E::kStrip> {};

template <int NB, int KS>
__host__ __device__ constexpr size_t big_lds_bytes() {
  using Cfg = TileCfg<NB, KS>;
  const size_t a = (size_t)2 * BIG_M * 256 * 2;  // two A k-block buffers
  const size_t c = (size_t)(BIG_M / 16) * (BIG_N / Cfg::NCOL) * 16 * Cfg::CS * 4;
  return a > c ? a : c;
}

// AM: A_BF16 (bf16 rows, bf16 MFMAs) or A_F16 (fp16 rows, fp16 MFMAs; the
// operands are the same exact values).  blockIdx.z = batch: tensors at fixed
// code / scale strides, A shared, the epilogue told the batch index.
template <int BITS, int NB, int KS, class Epi, int AM = A_BF16>
// Two workgroups per CU (at most 256 VGPRs a lane): the 4 x 2 accumulator
// blocks per wave, their K-slice totals, the next k-block's weights and A rows
// in flight.
__global__ __launch_bounds__(256, 2) void gemm_big_kernel(QT w, int R, const uint16_t* __restrict__ A,
                                                          Epi epi, int64_t codes_stride,
                                                          int64_t scales_stride) {
  static_assert(AM == A_BF16 || AM == A_F16, "16-bit A rows");
  using Cfg = TileCfg<NB, KS>;
  const int batch = blockIdx.z;
  w.codes += batch * codes_stride;
  w.scales += batch * scales_stride;
  static_assert(Cfg::THREADS == 256, "the epilogues run on four waves");
  constexpr int MB = BIG_M / 16, NSUB = BIG_N / Cfg::NCOL;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  uint16_t* As = (uint16_t*)smem;
  float* Cs = (float*)smem;  // reused for the output tiles after the K loop
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // Workgroups are dealt to the 8 XCDs round-robin by linear id.  Here the A
  // rows are the large operand (the weights of a stage are a few hundred KB),
  // so every column tile of a row tile goes to one XCD, consecutively: the
  // tile's rows then enter that XCD's L2 once for all column tiles.
  int cx = blockIdx.x, ry = blockIdx.y;
  if (gridDim.y % 8 == 0) {
    const int bid = blockIdx.x + gridDim.x * blockIdx.y;
    const int j = bid / 8;
    ry = bid % 8 + 8 * (j / gridDim.x);
    cx = j % gridDim.x;
  }
  const int m0 = ry * BIG_M, n0 = cx * BIG_N;
  const int KB = w.K >> 8, KBS = KB / KS;
  const int nb0 = (n0 >> 4) + 2 * wave;  // this wave's two 16-column weight blocks

  f32x4 acc[MB][2], tot[MB][2];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = tot[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  constexpr bool EXP = BITS == kExpBits;
  static_assert(!EXP || AM == A_BF16, "expanded codes are bf16 values");
  Blk<EXP ? 4 : BITS, A_BF16, false> wb[2], wn[2];
  // expanded codes: B operands stream from memory one group ahead through a
  // ring of two register slots (group g of every k-block in slot g % 2; a
  // deeper ring spills here, next to the K-slice totals)
  constexpr int NSLOT = 2, PF = 1;
  u32x4 eb[EXP ? NSLOT : 1][2][2];  // [slot][j][ss]
  uint32_t esc[2][2], escn[2][2];   // [j]: this / the next k-block's group scales
  auto load_grp = [&](int slot, int kb, int g) {
    if constexpr (EXP) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const u32x4* p = (const u32x4*)(w.codes + ((size_t)(nb0 + j) * KB + kb) * 8192) + lane;
        eb[slot][j][0] = p[64 * (2 * g)];
        eb[slot][j][1] = p[64 * (2 * g + 1)];
      }
    }
  };
  auto load_sc = [&](uint32_t (&d)[2][2], int kb) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const u32x2 sv = *(const u32x2*)(w.scales + ((size_t)(nb0 + j) * KB + kb) * 64 + (lane & 15) * 4);
      d[j][0] = sv[0];
      d[j][1] = sv[1];
    }
  };
  if constexpr (EXP) {
    load_sc(esc, 0);
#pragma unroll
    for (int g = 0; g < PF; ++g) load_grp(g, 0, g);
  } else {
    load_w(wb[0], w, nb0, 0, lane);
    load_w(wb[1], w, nb0 + 1, 0, lane);
  }

  // A rows m0.. of k-block kb into LDS buffer kb & 1 by global->LDS DMA: one
  // instruction moves two rows (lane i: row 2q + i / 32, its LDS chunk i % 32
  // holding global chunk (i % 32) ^ (row & 15)); rows past R are left out
  auto dma_a_blk = [&](int kb) {
    uint16_t* buf = As + (kb & 1) * (BIG_M * 256);
    const int half = lane >> 5, ch = lane & 31;
#pragma unroll
    for (int q = 0; q < BIG_M / 8; ++q) {
      const int r = wave * (BIG_M / 4) + 2 * q + half;
      if (m0 + r < R)
        __builtin_amdgcn_global_load_lds(
            (const __attribute__((address_space(1))) void*)(A + (int64_t)(m0 + r) * w.K + kb * 256 +
                                                           ((ch ^ (r & 15)) << 3)),
            (__attribute__((address_space(3))) void*)(buf + (wave * (BIG_M / 4) + 2 * q) * 256), 16, 0, 0);
    }
  };
  dma_a_blk(0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  for (int kb = 0; kb < KB; ++kb) {
    if (kb + 1 < KB) {  // next k-block's A rows and weights fly during this one's MFMAs
      dma_a_blk(kb + 1);
      if constexpr (EXP) {
        load_sc(escn, kb + 1);
      } else {
        load_w(wn[0], w, nb0, kb + 1, lane);
        load_w(wn[1], w, nb0 + 1, kb + 1, lane);
      }
    }
    const uint16_t* Ab = As + (kb & 1) * (BIG_M * 256);
    float scale[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t s0 = EXP ? esc[j][0] : wb[j].sc[0], s1 = EXP ? esc[j][1] : wb[j].sc[1];
      scale[j][0] = half_lo(s0); scale[j][1] = half_hi(s0);
      scale[j][2] = half_lo(s1); scale[j][3] = half_hi(s1);
    }
    using BOp = std::conditional_t<AM == A_F16, f16x8, bf16x8>;
    auto mfma = [](u32x4 a, BOp b, f32x4 c) {
      if constexpr (AM == A_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), b, c, 0, 0, 0);
      else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), b, c, 0, 0, 0);
    };
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      BOp bo[2][2];
      if constexpr (EXP) {
        // group g + PF of this k-block, or group g + PF - 4 of the next one
        if (g + PF < 4) load_grp((g + PF) % NSLOT, kb, g + PF);
        else if (kb + 1 < KB) load_grp((g + PF) % NSLOT, kb + 1, g + PF - 4);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int ss = 0; ss < 2; ++ss) bo[j][ss] = __builtin_bit_cast(BOp, eb[g % NSLOT][j][ss]);
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int ss = 0; ss < 2; ++ss) {
            if constexpr (AM == A_F16) bo[j][ss] = b_op_f16<BITS>(wb[j].p0, wb[j].p1, 2 * g + ss, BITS);
            else bo[j][ss] = b_op_bf16<BITS>(wb[j].p0, wb[j].p1, 2 * g + ss, BITS);
          }
      }
      // the 2*MB independent MFMA chains of the group first, then the scaled
      // accumulation (the same per-block arithmetic as compute_blk; issuing the
      // chains back to back keeps the matrix pipe busy instead of waiting on
      // each chain's result)
      // all of the group's A operands first (one LDS wait), then the MFMAs
      u32x4 ar[2][MB];
#pragma unroll
      for (int ss = 0; ss < 2; ++ss)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          ar[ss][mb] = *(const u32x4*)(Ab + big_a_off(mb * 16 + (lane & 15), 8 * g + 4 * ss + (lane >> 4)));
      f32x4 t[MB][2];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          t[mb][j] = mfma(ar[0][mb], bo[j][0], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          t[mb][j] = mfma(ar[1][mb], bo[j][1], t[mb][j]);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[mb][j][i] += scale[j][g] * t[mb][j][i];
    }
    {  // (also for KS == 1: the compiler schedules the loop far worse without it)
      if ((kb + 1) % KBS == 0) {  // end of a K-slice: add it to the slices before (in order)
        const bool first = kb + 1 == KBS;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i) tot[mb][j][i] = first ? acc[mb][j][i] : tot[mb][j][i] + acc[mb][j][i];
            acc[mb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
      }
    }
    // the next k-block's rows have landed and every wave is done with this one's
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (kb + 1 < KB) {
      if constexpr (EXP) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          esc[j][0] = escn[j][0];
          esc[j][1] = escn[j][1];
        }
      } else {
        wb[0] = wn[0];
        wb[1] = wn[1];
      }
    }
  }
  // (the last barrier above also frees As for the output tiles)
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = 32 * wave + 16 * j + (lane & 15);  // column inside the workgroup tile
      float* C = Cs + (size_t)(mb * NSUB + col / Cfg::NCOL) * 16 * Cfg::CS;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        C[(4 * (lane >> 4) + i) * Cfg::CS + col % Cfg::NCOL] = tot[mb][j][i];
    }
  __syncthreads();
  if constexpr (epi_has_strip<Epi>::value) {  // whole 16 x 128 strips, vector accesses
    if (epi.strip_ok()) {  // uniform
      for (int mb = 0; mb < MB; ++mb) {
        const int r0 = m0 + 16 * mb;
        if (r0 >= R) break;  // uniform
        epi.template strip<Cfg>(Cs + (size_t)mb * NSUB * 16 * Cfg::CS, r0, n0, R);
      }
      return;
    }
  }
  for (int mb = 0; mb < MB; ++mb) {
    const int r0 = m0 + 16 * mb;
    if (r0 >= R) break;  // uniform
    using P = decltype(epi.template prefetch<Cfg>(0, 0, 0, 0));
    P pre[NSUB];
#pragma unroll
    for (int c = 0; c < NSUB; ++c) pre[c] = epi.template prefetch<Cfg>(r0, n0 + c * Cfg::NCOL, R, batch);
#pragma unroll
    for (int c = 0; c < NSUB; ++c)
      epi.template apply<Cfg>(Cs + (size_t)(mb * NSUB + c) * 16 * Cfg::CS, pre[c], nullptr, r0,
                              n0 + c * Cfg::NCOL, R, batch);
  }
}

// ---------------------------------------------------------------------------
// Row-band variant for K = 512 (every stage but the MLP down-projection): the
// workgroup's 64 A rows stay in LDS for the whole launch -- one 1 KB
// global->LDS DMA per row, no register staging, no barrier inside the k-loop
// -- and the workgroup walks column tiles ct = cx, cx + gridDim.x, ... of the
// same rows, so a row band is read from L2/HBM once per workgroup instead of
// once per column tile.  The weights of the next (column tile, k-block) are
// loaded while the current one computes, across tile boundaries.  The
// epilogue runs one 16-row strip at a time through a small LDS strip (the A
// band must stay), which keeps two workgroups per CU.  Stages with a prologue
// (Pro = ProNorm: QKV, MLP up, LM head) normalise the band's rows themselves
// with the 16-row tasks' stage() instead of reading rows a separate launch
// normalised.
//
// The MFMA sequence of every 16x16 output block is gemm_big_kernel's (and so
// gemm_task's): same k-steps in the same order, acc += scale * t per 64-wide
// group, K-slices of K/KS from zero added in order, and each strip is laid
// out in LDS exactly as gemm_big_kernel lays out that strip.
// ---------------------------------------------------------------------------
constexpr int BAND_K = 512, BAND_AST = BAND_K + 8;  // A row stride in LDS: 1040 B

template <int NB, int KS>
__host__ __device__ constexpr size_t band_lds_bytes() {
  using Cfg = TileCfg<NB, KS>;
  return (size_t)BIG_M * BAND_AST * 2 + (size_t)(BIG_N / Cfg::NCOL) * 16 * Cfg::CS * 4;
}

template <int BITS, int NB, int KS, class Epi, int AM = A_BF16, class Pro = ProNone>
__global__ __launch_bounds__(256, 2) void gemm_band_kernel(QT w, int R, const uint16_t* __restrict__ A,
                                                           Epi epi, int64_t codes_stride,
                                                           int64_t scales_stride, Pro pro) {
  static_assert(AM == A_BF16 || AM == A_F16, "16-bit A rows");
  using Cfg = TileCfg<NB, KS>;
  static_assert(Cfg::THREADS == 256, "the epilogues run on four waves");
  constexpr int MB = BIG_M / 16, NSUB = BIG_N / Cfg::NCOL, KB = BAND_K / 256, KBS = KB / KS;
  const int batch = blockIdx.z;
  w.codes += batch * codes_stride;
  w.scales += batch * scales_stride;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  uint16_t* As = (uint16_t*)smem;
  float* Cs = (float*)(smem + (size_t)BIG_M * BAND_AST * 2);  // one 16-row strip
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // every column group of a row band on one XCD, consecutively (as in
  // gemm_big_kernel): the band enters that XCD's L2 once
  int cx = blockIdx.x, ry = blockIdx.y;
  if (gridDim.y % 8 == 0) {
    const int bid = blockIdx.x + gridDim.x * blockIdx.y;
    const int j = bid / 8;
    ry = bid % 8 + 8 * (j / gridDim.x);
    cx = j % gridDim.x;
  }
  const int m0 = ry * BIG_M, NT = w.N / BIG_N, GX = gridDim.x;
  auto nblk = [&](int ct) { return ct * (BIG_N / 16) + 2 * wave; };  // this wave's first weight block
  // the first column tile's weights fly while the band arrives
  constexpr bool EXP = BITS == kExpBits;
  static_assert(!EXP || AM == A_BF16, "expanded codes are bf16 values");
  using WBlk = Blk<EXP ? 4 : BITS, A_BF16, false>;
  WBlk wt[EXP ? 1 : KB][2];  // a column tile's weights, both k-blocks (packed codes)
  auto load_tile_w = [&](WBlk(&d)[EXP ? 1 : KB][2], int ct) {
    if constexpr (!EXP) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        load_w(d[kb][0], w, nblk(ct), kb, lane);
        load_w(d[kb][1], w, nblk(ct) + 1, kb, lane);
      }
    }
  };
  // Expanded codes: a tile's eight groups (k-block kb, group g: q = 4 kb + g)
  // of B operands stream from memory PF groups ahead through a ring of NSLOT
  // register slots (slot q % NSLOT); the next tile's scales and first groups
  // are issued in the epilogue, as the packed weights are.
  constexpr int GPT = KB * 4, NSLOT = 4, PF = 3;
  u32x4 eb[EXP ? NSLOT : 1][2][2];  // [slot][j][ss]
  uint32_t esc[EXP ? KB : 1][2][2];   // [kb][j]: the group scales (fp16 pairs)
  auto load_grp = [&](int slot, int ct, int q) {
    if constexpr (EXP) {
      const int kb = q / 4, g = q % 4;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const u32x4* p = (const u32x4*)(w.codes + ((size_t)(nblk(ct) + j) * KB + kb) * 8192) + lane;
        eb[slot][j][0] = p[64 * (2 * g)];
        eb[slot][j][1] = p[64 * (2 * g + 1)];
      }
    }
  };
  auto load_scales = [&](int ct) {
    if constexpr (EXP) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const u32x2 sv = *(const u32x2*)(w.scales + ((size_t)(nblk(ct) + j) * KB + kb) * 64 + (lane & 15) * 4);
          esc[kb][j][0] = sv[0];
          esc[kb][j][1] = sv[1];
        }
    }
  };
  load_tile_w(wt, cx);
  if constexpr (EXP) {
    load_scales(cx);
#pragma unroll
    for (int q = 0; q < PF; ++q) load_grp(q, cx, q);
  }

  if constexpr (Pro::kStage) {
    // the stage's prologue in place of a separate row-normalisation launch:
    // stage() over the band's four 16-row strips (strip i at As + 16 i
    // BAND_AST, BAND_AST being stage()'s row stride for K = 512), so the band
    // holds the rows norm_rows_kernel would have written; side outputs
    // (sparse-gate logits) from the first column group only.  The first
    // column tile's weights are already in flight.  (Two strips' loads issued
    // before their arithmetic measured no faster; with the early weight loads
    // they spill.)
    static_assert(Pro::kScratch == 0, "no prologue scratch in the band's LDS");
    static_assert(BAND_AST == lds_stride(BAND_K, A_BF16), "stage() row stride");
#pragma unroll
    for (int i = 0; i < BIG_M / 16; ++i)
      pro.template stage<AM, 256>(As + (size_t)i * 16 * BAND_AST, nullptr, m0 + 16 * i, R, BAND_K, batch,
                                  cx == 0);
    __syncthreads();
  } else {
    // the band: row r of the tile at As + r * BAND_AST, lane l bringing k = 8l .. 8l+7
#pragma unroll 4
    for (int i = 0; i < BIG_M / 4; ++i) {
      const int r = wave * (BIG_M / 4) + i;
      if (m0 + r < R)
        __builtin_amdgcn_global_load_lds(
            (const __attribute__((address_space(1))) void*)(A + (int64_t)(m0 + r) * BAND_K + lane * 8),
            (__attribute__((address_space(3))) void*)(As + r * BAND_AST), 16, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  using BOp = std::conditional_t<AM == A_F16, f16x8, bf16x8>;
  auto mfma = [](u32x4 a, BOp b, f32x4 c) {
    if constexpr (AM == A_F16)
      return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), b, c, 0, 0, 0);
    else
      return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), b, c, 0, 0, 0);
  };
  for (int ct = cx; ct < NT; ct += GX) {
    const int n0 = ct * BIG_N;
    f32x4 acc[MB][2], tot[MB][2];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = tot[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const WBlk(&wb)[2] = wt[EXP ? 0 : kb];
      float scale[2][4];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t s0 = EXP ? esc[EXP ? kb : 0][j][0] : wb[j].sc[0];
        const uint32_t s1 = EXP ? esc[EXP ? kb : 0][j][1] : wb[j].sc[1];
        scale[j][0] = half_lo(s0); scale[j][1] = half_hi(s0);
        scale[j][2] = half_lo(s1); scale[j][3] = half_hi(s1);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        BOp bo[2][2];
        if constexpr (EXP) {
          const int q = 4 * kb + g, qn = q + PF;
          if (qn < GPT) load_grp(qn % NSLOT, ct, qn);  // (the next tile's first groups: in the epilogue)
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int ss = 0; ss < 2; ++ss) bo[j][ss] = __builtin_bit_cast(BOp, eb[q % NSLOT][j][ss]);
        } else {
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int ss = 0; ss < 2; ++ss) {
              if constexpr (AM == A_F16) bo[j][ss] = b_op_f16<BITS>(wb[j].p0, wb[j].p1, 2 * g + ss, BITS);
              else bo[j][ss] = b_op_bf16<BITS>(wb[j].p0, wb[j].p1, 2 * g + ss, BITS);
            }
        }
        f32x4 t[MB][2];
#pragma unroll
        for (int ss = 0; ss < 2; ++ss) {
          u32x4 ar[MB];
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
            ar[mb] = *(const u32x4*)(As + (mb * 16 + (lane & 15)) * BAND_AST + kb * 256 + 64 * g +
                                     32 * ss + 8 * (lane >> 4));
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int j = 0; j < 2; ++j)
              t[mb][j] = mfma(ar[mb], bo[j][ss], ss ? t[mb][j] : f32x4{0.f, 0.f, 0.f, 0.f});
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[mb][j][i] += scale[j][g] * t[mb][j][i];
      }
      if (KS > 1 && (kb + 1) % KBS == 0) {  // end of a K-slice: add it to the slices before (in order)
        const bool first = kb + 1 == KBS;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i) tot[mb][j][i] = first ? acc[mb][j][i] : tot[mb][j][i] + acc[mb][j][i];
            acc[mb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
      }
    }
    // epilogue: one 16 x 128 strip at a time (one copy of the epilogue code;
    // the accumulator blocks stay in registers through static indices)
#pragma unroll 1
    for (int mb = 0; mb < MB; ++mb) {
      const int r0 = m0 + 16 * mb;
#pragma unroll
      for (int q = 0; q < MB; ++q) {
        if (q != mb) continue;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int col = 32 * wave + 16 * j + (lane & 15);
          float* C = Cs + (size_t)(col / Cfg::NCOL) * 16 * Cfg::CS;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            C[(4 * (lane >> 4) + i) * Cfg::CS + col % Cfg::NCOL] = KS > 1 ? tot[q][j][i] : acc[q][j][i];
        }
      }
      __syncthreads();
      // the next column tile's weights fly during the epilogue (issued behind
      // the barrier so they do not compete with this tile's operands)
      if (mb == 0 && ct + GX < NT) {
        load_tile_w(wt, ct + GX);
        load_scales(ct + GX);
        if constexpr (EXP) {
#pragma unroll
          for (int q = 0; q < PF; ++q) load_grp(q, ct + GX, q);
        }
      }
      if (r0 < R) {  // uniform
        bool done = false;
        if constexpr (epi_has_strip<Epi>::value) {
          if (epi.strip_ok()) {  // uniform
            epi.template strip<Cfg>(Cs, r0, n0, R);
            done = true;
          }
        }
        if (!done) {
          using P = decltype(epi.template prefetch<Cfg>(0, 0, 0, 0));
          P pre[NSUB];
#pragma unroll
          for (int c = 0; c < NSUB; ++c) pre[c] = epi.template prefetch<Cfg>(r0, n0 + c * Cfg::NCOL, R, batch);
#pragma unroll
          for (int c = 0; c < NSUB; ++c)
            epi.template apply<Cfg>(Cs + (size_t)c * 16 * Cfg::CS, pre[c], nullptr, r0, n0 + c * Cfg::NCOL, R,
                                    batch);
        }
      }
      __syncthreads();
    }
  }
}

// Column groups per row band: enough workgroups to fill the chip several times
// over (two per CU), then as many column tiles per workgroup as that allows.
inline int band_col_groups(int R, int N, int batch) {
  const int bands = ((R + BIG_M - 1) / BIG_M) * batch, nt = N / BIG_N;
  const int want = (4096 + bands - 1) / bands;
  return want < 1 ? 1 : (want > nt ? nt : want);
}

template <int BITS, int NB, int KS, class Epi, int AM = A_BF16, class Pro = ProNone>
hipError_t launch_gemm_band_t(const QT& w, int R, const uint16_t* A, const Epi& epi, hipStream_t s,
                              int batch, int64_t codes_stride, int64_t scales_stride,
                              const Pro& pro = Pro{}) {
  auto kfn = gemm_band_kernel<BITS, NB, KS, Epi, AM, Pro>;
  constexpr size_t lds = band_lds_bytes<NB, KS>();
  static bool configured = false;
  if (!configured) {
    hipError_t e = hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
    configured = true;
  }
  dim3 grid((unsigned)band_col_groups(R, w.N, batch), (unsigned)((R + BIG_M - 1) / BIG_M), (unsigned)batch);
  hipLaunchKernelGGL(kfn, grid, dim3(256), lds, s, w, R, A, epi, codes_stride, scales_stride, pro);
  return hipGetLastError();
}

template <int BITS, int NB, int KS, class Epi, int AM = A_BF16>
hipError_t launch_gemm_big_t(const QT& w, int R, const uint16_t* A, const Epi& epi, hipStream_t s,
                             int batch = 1, int64_t codes_stride = 0, int64_t scales_stride = 0) {
  // A rows come by 16-byte global->LDS DMA: 16-byte aligned rows only
  if (((uintptr_t)A & 15) != 0) return hipErrorInvalidValue;
  // K = 512: the row-band kernel (same bits)
  if constexpr ((BAND_K / 256) % KS == 0) {
    if (w.K == BAND_K)
      return launch_gemm_band_t<BITS, NB, KS, Epi, AM>(w, R, A, epi, s, batch, codes_stride, scales_stride);
  }
  auto kfn = gemm_big_kernel<BITS, NB, KS, Epi, AM>;
  constexpr size_t lds = big_lds_bytes<NB, KS>();
  static bool configured = false;
  if (!configured) {
    hipError_t e = hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
    configured = true;
  }
  dim3 grid((unsigned)(w.N / BIG_N), (unsigned)((R + BIG_M - 1) / BIG_M), (unsigned)batch);
  hipLaunchKernelGGL(kfn, grid, dim3(256), lds, s, w, R, A, epi, codes_stride, scales_stride);
  return hipGetLastError();
}

// Usable for a tensor when its shape fits the tiling (else use gemm_task).
inline bool big_gemm_fits(const QT& w) {
  return (w.bits <= 6 || w.bits == kExpBits) && w.N % BIG_N == 0 && w.K % 256 == 0;
}

// (NB, KS) must be the 16-row path's choice for this tensor (pick_ks).
template <int NB, int KS, class Epi>
hipError_t launch_gemm_big(int bits, const QT& w, int R, const uint16_t* A, const Epi& epi,
                           hipStream_t s) {
  switch (bits) {
    case 2: return launch_gemm_big_t<2, NB, KS>(w, R, A, epi, s);
    case 3: return launch_gemm_big_t<3, NB, KS>(w, R, A, epi, s);
    case 4: return launch_gemm_big_t<4, NB, KS>(w, R, A, epi, s);
    case 6: return launch_gemm_big_t<6, NB, KS>(w, R, A, epi, s);
    case kExpBits: return launch_gemm_big_t<kExpBits, NB, KS>(w, R, A, epi, s);
    default: return hipErrorInvalidValue;
  }
}

template <class Epi>
hipError_t launch_gemm_big4(int ks_max, int bits, const QT& w, int R, const uint16_t* A,
                            const Epi& epi, hipStream_t s) {
  switch (pick_ks(w.K, ks_max)) {
    case 4: return launch_gemm_big<1, 4>(bits, w, R, A, epi, s);
    case 2: return launch_gemm_big<2, 2>(bits, w, R, A, epi, s);
    default: return launch_gemm_big<4, 1>(bits, w, R, A, epi, s);
  }
}

// K = 512 stages with a prologue (QKV, MLP up, LM head): the row-band kernel
// runs the prologue itself (same rows, same bits as norm_rows_kernel followed
// by the band kernel on them).  (NB, KS) as launch_gemm_big.
inline bool band_norm_fits(const QT& w) { return big_gemm_fits(w) && w.K == BAND_K; }
template <int NB, int KS, class Pro, class Epi>
hipError_t launch_gemm_band_norm(int bits, const QT& w, int R, const Pro& pro, const Epi& epi,
                                 hipStream_t s) {
  static_assert((BAND_K / 256) % KS == 0, "K-slices of the band");
  if (w.K != BAND_K) return hipErrorInvalidValue;
  switch (bits) {
    case 2: return launch_gemm_band_t<2, NB, KS, Epi, A_BF16, Pro>(w, R, nullptr, epi, s, 1, 0, 0, pro);
    case 3: return launch_gemm_band_t<3, NB, KS, Epi, A_BF16, Pro>(w, R, nullptr, epi, s, 1, 0, 0, pro);
    case 4: return launch_gemm_band_t<4, NB, KS, Epi, A_BF16, Pro>(w, R, nullptr, epi, s, 1, 0, 0, pro);
    case 6: return launch_gemm_band_t<6, NB, KS, Epi, A_BF16, Pro>(w, R, nullptr, epi, s, 1, 0, 0, pro);
    case kExpBits:
      return launch_gemm_band_t<kExpBits, NB, KS, Epi, A_BF16, Pro>(w, R, nullptr, epi, s, 1, 0, 0, pro);
    default: return hipErrorInvalidValue;
  }
}
template <class Pro, class Epi>
hipError_t launch_gemm_band_norm4(int ks_max, int bits, const QT& w, int R, const Pro& pro, const Epi& epi,
                                  hipStream_t s) {
  switch (pick_ks(w.K, ks_max)) {
    case 2: return launch_gemm_band_norm<2, 2>(bits, w, R, pro, epi, s);
    case 1: return launch_gemm_band_norm<4, 1>(bits, w, R, pro, epi, s);
    default: return hipErrorInvalidValue;  // K = 512 allows at most two K-slices
  }
}

// The prologue of a 16-row task, run on its own: rows [16*blockIdx.x, +16)
// normalised exactly as gemm_task stages them (and the same side outputs,
// e.g. sparse-gate logits), stored as bf16 rows of K for gemm_big_kernel.
template <class Pro>
__global__ __launch_bounds__(256) void norm_rows_kernel(Pro pro, int R, int K, uint16_t* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int m0 = blockIdx.x * 16;
  pro.template stage<A_BF16, 256>(smem, smem + (size_t)16 * lds_stride(K, A_BF16) * 2, m0, R, K, 0, true);
  __syncthreads();
  const uint16_t* As = (const uint16_t*)smem;
  const int n8 = K / 8;
  for (int c = threadIdx.x; c < 16 * n8; c += 256) {
    const int r = c / n8, k8 = (c % n8) * 8;
    if (m0 + r < R) *(u32x4*)(out + (int64_t)(m0 + r) * K + k8) = *(const u32x4*)(As + r * lds_stride(K, A_BF16) + k8);
  }
}

template <class Pro>
hipError_t launch_norm_rows(const Pro& pro, int R, int K, uint16_t* out, hipStream_t s) {
  const size_t lds = (size_t)16 * lds_stride(K, A_BF16) * 2 + Pro::kScratch;
  hipLaunchKernelGGL(norm_rows_kernel<Pro>, dim3((unsigned)((R + 15) / 16)), dim3(256), lds, s, pro, R,
                     K, out);
  return hipGetLastError();
}

}  // namespace altxs
