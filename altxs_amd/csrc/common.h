// Shared device helpers for the altxs HIP kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/altxs.h"

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

#define WAVE 64

// ---- bf16 <-> fp32 (bf16 stored as raw uint16) -----------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  // round-to-nearest-even via the hardware conversion (v_cvt_pk_bf16_f32)
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(uint16_t, b);
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// ---- bf16 KV cache tile layout (include/altxs.h, ALTXS_KV_TILE) -------------
// Offset of (key kt of a 64-key tile, dim d) inside the tile's 4096 elements.
// K: the A operand of the score MFMA (lane 16g + r: key r of a 16-key block,
//    dims 32*ks + 8*g + [0, 8)).
// V: the B operand of the P x V MFMA (lane 16g + c: dim 16*nb + c, keys
//    16*(2s + jb) + 4*g + jr for j = 4*jb + jr in [0, 8)).
__host__ __device__ __forceinline__ int kv_tile_k(int kt, int d) {
  return ((((kt >> 4) * 2 + (d >> 5)) * 4 + ((d >> 3) & 3)) * 16 + (kt & 15)) * 8 + (d & 7);
}
__host__ __device__ __forceinline__ int kv_tile_v(int kt, int d) {
  return ((((kt >> 5) * 4 + (d >> 4)) * 4 + ((kt >> 2) & 3)) * 16 + (d & 15)) * 8 +
         4 * ((kt >> 4) & 1) + (kt & 3);
}

// ---- wave reductions (fixed order: deterministic, every lane gets the result)
// Inside a 16-lane row: DPP quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror,
// row_mirror -- each step pairs every lane with a distinct partner, and a
// commutative op gives both the same bits; no LDS traffic.  The four row
// results are then read with v_readlane and combined as (r0 op r1) op (r2 op r3).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}
enum : int { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140 };

__device__ __forceinline__ float lane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<DPP_XOR1>(v);
  v += dpp_f<DPP_XOR2>(v);
  v += dpp_f<DPP_HALF_MIRROR>(v);
  v += dpp_f<DPP_MIRROR>(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<DPP_XOR1>(v));
  v = fmaxf(v, dpp_f<DPP_XOR2>(v));
  v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
  v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  v += dpp_u<DPP_XOR1>(v);
  v += dpp_u<DPP_XOR2>(v);
  v += dpp_u<DPP_HALF_MIRROR>(v);
  v += dpp_u<DPP_MIRROR>(v);
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 0) + (uint32_t)__builtin_amdgcn_readlane((int)v, 16) +
         (uint32_t)__builtin_amdgcn_readlane((int)v, 32) + (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
}
// Combine lanes c, c+16, c+32, c+48 (same position in each row): lane l adds
// (or maxes) lane l ^ 16, then lane l ^ 32.  gfx950's v_permlane16_swap /
// v_permlane32_swap (VALU, no LDS round trip) with both operands = v leave
// {v[l], v[l ^ 16]} (resp. ^ 32) in the two results, in one order or the
// other; + and max are commutative, so every lane gets the bits of the
// shuffle form v + v[l ^ 16].
__device__ __forceinline__ float rows_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ float rows_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
// The same pairs through the LDS crossbar (ds_bpermute), hence the same bits.
// The decode attention's tile loop (memory-bound, two waves per SIMD) runs
// ~0.5% faster with these than with the lane swaps.
__device__ __forceinline__ float rows_sum_ds(float v) {
  v += __shfl_xor(v, 16, WAVE);
  return v + __shfl_xor(v, 32, WAVE);
}
__device__ __forceinline__ float rows_max_ds(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, WAVE));
  return fmaxf(v, __shfl_xor(v, 32, WAVE));
}

// ---- row-local XCD placement of decode launches -----------------------------
// Workgroups are dealt to the 8 XCDs round-robin by linear id, and the count
// continues across launches, so in a chain of launches whose sizes are all
// multiples of 8 workgroup id i of every launch lands on XCD (i + c) % 8 for
// one c.  Decode launches (rows in tiles of 8, ntiles % 8 == 0) number their
// workgroups so that every piece of row tile t runs with id % 8 == t % 8: a
// stage then reads the rows the previous stage wrote from its own XCD's L2
// (a dependent launch that reads another XCD's output measured ~1.3 us slower
// per edge).  id -> (tile, j), j < per_tile; a bijection.
__host__ __device__ __forceinline__ void xcd_row_split(int id, int ntiles, int& tile, int& j) {
  const int q = ntiles / 8, b = id / 8;
  tile = id % 8 + 8 * (b % q);
  j = b / q;
}

// ---- device error word ------------------------------------------------------
// Kernels never fault on bad runtime values (positions, token ids): they skip
// the access and OR a code into *err, which the host reads when it syncs.
enum : int32_t {
  ALTXS_EDEV_POS = 1,    // position >= max_len (KV write/read skipped)
  ALTXS_EDEV_TOKEN = 2,  // token id outside [0, V) (clamped)
  ALTXS_EDEV_SPIN = 4,   // a persistent-kernel wait gave up (results invalid, kernel exited)
};
__device__ __forceinline__ void flag_err(int32_t* err, int32_t code) {
  if (err) atomicOr(err, code);
}

// ---- host-side error plumbing ----------------------------------------------
void altxs_set_error(const char* fmt, ...);
#define ALTXS_CHECK_HIP(expr)                                                   \
  do {                                                                          \
    hipError_t e_ = (expr);                                                     \
    if (e_ != hipSuccess) {                                                     \
      altxs_set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_),    \
                      __FILE__, __LINE__);                                      \
      return ALTXS_ERR_HIP;                                                     \
    }                                                                           \
  } while (0)
#define ALTXS_REQUIRE(cond, ...)                                                \
  do {                                                                          \
    if (!(cond)) {                                                              \
      altxs_set_error(__VA_ARGS__);                                             \
      return ALTXS_ERR_ARG;                                                     \
    }                                                                           \
  } while (0)
