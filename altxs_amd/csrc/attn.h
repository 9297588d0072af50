// Decode attention device code shared by the standalone kernels (attn.hip)
// and the persistent layer kernel (step.hip).  See attn.hip for the design.
#pragma once
#include <type_traits>

#include "common.h"
#include "gemm.h"

#ifndef ALTXS_ATT_WAVES
#define ALTXS_ATT_WAVES 4  // waves per workgroup (tile T goes to wave T % waves)
#endif

namespace altxs_attn {

constexpr int ATT_WAVES = ALTXS_ATT_WAVES;
// The gate multiplier of launches without the sparse gate (read like a gate entry).
static __device__ const float kNoGate = 1.f;
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
  int xcd_rows;  // one-row kernel: rows in tiles of 8, tile t on XCD t % 8
  int kv_tail = -1;  // natural layouts: first row of the window's K/V (-1: at pos + t)
  int helpers = 0;   // small MHA decode launches: prefetch workgroups per (row, kv head)
  // Out-projection terms (attn_mfma_task with OP = 1): o_part[(r * H + h) *
  // o_n + n] is the sum over head h's 64 features of row r's output y times
  // the codes of column n of the out-projection (o_codes, o_bits: its packed
  // tiled tensor, K = H * 64), before the column's group scale.
  const uint8_t* o_codes = nullptr;
  float* o_part = nullptr;
  int o_bits = 0, o_n = 0;
};

// Row of the cache that holds key j of a query of segment b whose window starts
// at pb (tail placement: keys pb .. p live in the rows from a.kv_tail on).
// Keys past the query's own position keep their own row (read, then masked).
__device__ __forceinline__ int key_row(const AttnP& a, int j, int pb, int p) {
  return (a.kv_tail >= 0 && j >= pb && j <= p) ? a.kv_tail + (j - pb) : j;
}

// Per-wave partial results, merged in wave order by the whole workgroup.
template <int G> struct alignas(16) MergeLds {
  float m[ATT_WAVES][G];
  float l[ATT_WAVES][G];
  float acc[ATT_WAVES][G][HD];
};

// What the last step of a query row reads besides the partials: the current
// token's value entries (XSA) and the row's gate multiplier.
template <int NK>
struct RowExtras {
  float vv[NK];
  float gv;
};
template <int NK, class VAt>
__device__ __forceinline__ RowExtras<NK> row_extras(const AttnP& a, int r, int h, int p, int c, VAt v_at) {
  RowExtras<NK> e;
#pragma unroll
  for (int k = 0; k < NK; ++k) e.vv[k] = a.use_xsa ? v_at(p, c + 16 * k) : 0.f;
  e.gv = a.gate ? a.gate[(int64_t)r * a.H + h] : 1.f;
  return e;
}

// Sum over the 64 dims of a row of per-dim values x (layouts of finish_query):
// (x[c] + x[c+16]) + (x[c+32] + x[c+48]) for each c, then the 16 of these
// through the DPP butterfly.  NK = 4 forms the bracket in-lane, NK = 1 with
// the lane swaps of rows_sum; every add pairs the same two values, so both
// give the same bits, in every lane (rows_sum_ds: rows_sum's pairs).
template <int NK>
__device__ __forceinline__ float row_dims_sum(const float (&x)[NK]) {
#pragma clang fp contract(off)
  if constexpr (NK == 4) return row16_sum((x[0] + x[1]) + (x[2] + x[3]));
  else return row16_sum(rows_sum_ds(x[0]));
}

// The last step of one query row (row r, query head h): merge the per-wave
// partials in wave order, XSA, gate, store.  Two layouts with the same
// arithmetic, so window rows get the bits of decode rows:
//   NK = 4: the 16 lanes of one wave row, lane c holding dims c + 16k (k < 4)
//           -- a wave finishes four rows at once and shares every per-row
//           scalar (exponentials, norms, divisions' set-up) among them;
//   NK = 1: a whole wave, lane c holding dim c (decode: one row per wave).
// Contraction is off here: products are rounded before they are summed (the
// compiler would otherwise fuse a product into the in-lane sum of one layout
// and not into the cross-lane sum of the other), and the FMAs are explicit.
// Wave w's partials: m[w * ms], l[w * ms], acc[w * as + d].
template <int NK, int YBF16>
__device__ __forceinline__ void finish_query(const AttnP& a, const float* m, const float* l, int ms,
                                             const float* acc, int as, int r, int h, int c,
                                             const RowExtras<NK>& e, uint16_t* ylds = nullptr) {
#pragma clang fp contract(off)
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < ATT_WAVES; ++w) M = fmaxf(M, m[w * ms]);
  float Ls = 0.f, y[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) y[k] = 0.f;
#pragma unroll
  for (int w = 0; w < ATT_WAVES; ++w) {
    const float mw = m[w * ms];
    if (mw == -INFINITY) continue;  // uniform over the row
    const float f = __expf(mw - M);
    Ls = __builtin_fmaf(l[w * ms], f, Ls);
#pragma unroll
    for (int k = 0; k < NK; ++k) y[k] = __builtin_fmaf(acc[w * as + c + 16 * k], f, y[k]);
  }
#pragma unroll
  for (int k = 0; k < NK; ++k) y[k] = y[k] / Ls;
  if (a.use_xsa) {  // y -= (y . v^) v^ with v^ = v / max(|v|, 1e-12), v the current token's value
    float sq[NK], vn[NK], yv[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) sq[k] = e.vv[k] * e.vv[k];
    const float nrm = fmaxf(sqrtf(row_dims_sum<NK>(sq)), 1e-12f);
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      vn[k] = e.vv[k] / nrm;
      yv[k] = y[k] * vn[k];
    }
    const float dot = row_dims_sum<NK>(yv);
#pragma unroll
    for (int k = 0; k < NK; ++k) y[k] = __builtin_fmaf(-dot, vn[k], y[k]);
  }
  if (a.gate) {
#pragma unroll
    for (int k = 0; k < NK; ++k) y[k] *= e.gv;
  }
  const int64_t o = ((int64_t)r * a.H + h) * HD + c;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    if (YBF16) {
      const uint16_t yb = f32_to_bf16(y[k]);
      ((uint16_t*)a.y)[o + 16 * k] = yb;
      if (ylds) ylds[c + 16 * k] = yb;
    } else {
      ((float*)a.y)[o + 16 * k] = y[k];
    }
  }
}

// Decode (and the fp32-cache kernel): wave j < G finishes query head j of the
// kv head, one dim per lane.  v_at(p, d) returns the current token's value entry.
template <int G, int YBF16, class VAt>
__device__ __forceinline__ void merge_and_store(const AttnP& a, const MergeLds<G>& sm, int r, int g,
                                                int p, int wave, int lane, VAt v_at) {
  static_assert(G <= ATT_WAVES, "one wave per query head of the group");
  if (wave >= G) return;
  const RowExtras<1> e = row_extras<1>(a, r, g * G + wave, p, lane, v_at);
  finish_query<1, YBF16>(a, &sm.m[0][wave], &sm.l[0][wave], G, &sm.acc[0][wave][0], G * HD, r,
                         g * G + wave, lane, e);
}
// The same with the extras read beforehand (the bf16 kernel loads them at its
// start, so the finish step waits on no memory).
template <int G, int YBF16>
__device__ __forceinline__ void merge_and_store(const AttnP& a, const MergeLds<G>& sm, int r, int g,
                                                int wave, int lane, const RowExtras<1>& e,
                                                uint16_t* ylds = nullptr) {
  static_assert(G <= ATT_WAVES, "one wave per query head of the group");
  if (wave >= G) return;
  finish_query<1, YBF16>(a, &sm.m[0][wave], &sm.l[0][wave], G, &sm.acc[0][wave][0], G * HD, r,
                         g * G + wave, lane, e, ylds);
}

__device__ __forceinline__ int clamp_pos(const AttnP& a, int b, int t, int pos_b) {
  int p = pos_b + t;
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

// Natural-order bf16 cache (NAT = 1): a wave stages each V tile in LDS as
// stored, rows of kVstRow elements (64 dims + 8 padding), and reads its V
// operands back transposed (ds_read_b64_tr_b16).
constexpr int kVstRow = HD + 8;

// One (query row r, kv head g) of the bf16-cache attention: ATT_WAVES waves.
// PF = 1: each wave keeps its next tile's loads in flight while it computes the
// current one (two register buffers), for launches with one workgroup per CU;
// the arithmetic, and so the result, is the same for PF = 0 and 1.
// NAT = 1: the cache in the natural [key][64] order (ALTXS_KV_BF16_NATURAL,
// with the tail placement of AttnP::kv_tail): the K operand of a lane is 16
// consecutive bytes of one key there as well; the V operand (8 keys of one
// dim) comes from the wave's LDS copy of the tile (vst: ATT_WAVES x 64 x
// kVstRow elements) by two transposed reads.  The MFMAs see the operands of the tiled layout, so both
// layouts give the same bits for the same cache values.
//
// OP = the out-projection's code width (2, 3, 4 or 6; 0: none), for MHA
// decode rows on the tiled cache with bf16 operands: the tail also forms this
// head's terms of the out-projection (AttnP::o_part), so the out-projection
// needs no launch of its own.  The GEMM (gemm_task, K-slices of 256 features
// = four heads) computes, per output column n, t_h = the MFMA sum over head
// h's features (two k-steps from zero) and then acc += scale * t_h head by
// head; here the same two MFMAs run on the same operands -- the row's bf16 y
// in every MFMA row, the column's codes as the B operand -- so t_h has the
// GEMM's bits, and the reader applies the scales in the GEMM's order
// (OutFin).  ys: 64 bf16 of LDS for the row.
template <int G, int NP, int YBF16, int PF = 0, int NAT = 0, int OP = 0>
__device__ __forceinline__ void attn_mfma_task(const AttnP& a, int r, int g, MergeLds<G>& sm,
                                               uint16_t* vst = nullptr, uint16_t* ys = nullptr) {
  static_assert(OP == 0 || OP == 2 || OP == 3 || OP == 4 || OP == 6, "out-projection width");
  static_assert(!OP || (G == 1 && NP == 1 && YBF16 && !NAT), "out-projection terms: MHA, bf16, tiled");
  static_assert(TILE == 64, "the MFMA tiling below assumes 64-key tiles");
  const int b = r / a.W, t = r % a.W;
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  const int lg = lane >> 4, col = lane & 15;
  const uint16_t* kb = (const uint16_t*)a.k + (int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD;
  const uint16_t* vb = (const uint16_t*)a.v + (int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD;
  int nat_pb = 0, nat_p = 0;  // NAT: the window's first position and the query's (key_row)
  auto load = [&](u32x4 (&kr)[8], u32x4 (&vr)[8], int T) {
    if constexpr (NAT) {
      // K operand kr[2 blk + ks]: key 16 blk + (lane & 15), dims 32 ks + 8 lg .. +8
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        const int64_t row = key_row(a, T * TILE + 16 * blk + col, nat_pb, nat_p);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          kr[2 * blk + ks] = __builtin_nontemporal_load((const u32x4*)(kb + row * HD + 32 * ks + 8 * lg));
      }
      // V rows as stored: vr[i] = key 8 i + (lane >> 3), dims 8 (lane & 7) .. +8
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t row = key_row(a, T * TILE + 8 * i + (lane >> 3), nat_pb, nat_p);
        vr[i] = __builtin_nontemporal_load((const u32x4*)(vb + row * HD + 8 * (lane & 7)));
      }
    } else {
      const u32x4* kt = (const u32x4*)(kb + (int64_t)T * (TILE * HD)) + lane;
      const u32x4* vt = (const u32x4*)(vb + (int64_t)T * (TILE * HD)) + lane;
#pragma unroll
      for (int i = 0; i < 8; ++i) kr[i] = __builtin_nontemporal_load(kt + 64 * i);
#pragma unroll
      for (int i = 0; i < 8; ++i) vr[i] = __builtin_nontemporal_load(vt + 64 * i);
    }
  };
  // Every workgroup of a decode launch starts (and ends) at the same time, so
  // a memory round trip after the last tile costs the whole launch: the
  // finish step's extras (the current value for XSA, the gate) are read here,
  // after the position and the q row, and kept raw until the finish step (the
  // load counter retires in order, so a use right after their loads would wait
  // for everything older).  Same values, same arithmetic; cfg3 0.675 -> 0.670
  // ms.  (Also issuing each wave's first tile before the q row: with the tile
  // buffer carried around the tile loop the rows came out wrong whenever a
  // row had more than two keys, cause not found; with the first tile peeled
  // into a buffer of its own the rows are right but the step is slower,
  // 0.693 against 0.668 ms.  Neither is in the build.)
  // NAT: one row per workgroup, so its position is uniform (scalar), and so
  // are the tile loop's bounds
  int p_raw = a.pos[b];
  if (NAT) p_raw = __builtin_amdgcn_readfirstlane(p_raw);
  f32x4 qraw[2][2];
  {
    const float* qh = a.q + ((int64_t)r * a.H + g * G + (col % G)) * HD;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      qraw[ks][0] = *(const f32x4*)(qh + 32 * ks + 8 * lg);
      qraw[ks][1] = *(const f32x4*)(qh + 32 * ks + 8 * lg + 4);
    }
  }
  if (NAT && a.kv_tail >= 0 && p_raw > a.kv_tail) {  // the prefix would run into the window rows
    if (threadIdx.x == 0) flag_err(a.err, ALTXS_EDEV_POS);
    p_raw = a.kv_tail;
  }
  const int p = clamp_pos(a, b, t, p_raw);
  nat_pb = p_raw;
  nat_p = p;
  const int nkeys = p + 1;
  const int ntiles = (nkeys + TILE - 1) / TILE;
  // unconditional loads (a load on one path only would leave the compiler
  // unsure how many are in flight, and it would then wait for all of them);
  // waves past G read a valid word they do not use
  const int hx = g * G + (wave < G ? wave : G - 1);
  const uint16_t v_raw = NAT ? vb[(int64_t)key_row(a, p, nat_pb, nat_p) * HD + lane]
                             : vb[(int64_t)(p / TILE) * (TILE * HD) + kv_tile_v(p % TILE, lane)];
  const float g_raw = *(a.gate ? a.gate + (int64_t)r * a.H + hx : &kNoGate);
  // OP: this lane's out-projection codes, loaded now and used in the tail.
  // Column block nb = wave + ATT_WAVES q of weight block (nb, h / 4), k-steps
  // 2 (h % 4) and 2 (h % 4) + 1: the low plane's word(s) of those steps and
  // the word of the high plane that holds them (6 and 3 bits).  Every load is
  // issued on every path (a column block past o_n reads block 0).
  constexpr int kOpQ = 512 / (16 * ATT_WAVES);  // o_n <= 512
  uint32_t ow[OP ? kOpQ : 1][3];
  if constexpr (OP) {
    constexpr bool wide = OP >= 4;
    const int KB = (a.H * HD) >> 8, kb = g >> 2, gq = g & 3;
    const int off0 = wide ? lane * 32 + 8 * gq : lane * 16 + 4 * gq;
    const int off1 = wide ? off0 + 4 : off0;
    const int off2 = OP == 6 ? 512 * 4 + lane * 16 + 4 * gq
                     : OP == 3 ? 512 * 2 + lane * 8 + 4 * (gq >> 1) : off0;
#pragma unroll
    for (int qi = 0; qi < kOpQ; ++qi) {
      const int nb = wave + ATT_WAVES * qi;
      const uint8_t* blk = a.o_codes + ((int64_t)(16 * nb < a.o_n ? nb : 0) * KB + kb) * (512 * OP);
      ow[qi][0] = *(const uint32_t*)(blk + off0);
      ow[qi][1] = *(const uint32_t*)(blk + off1);
      ow[qi][2] = *(const uint32_t*)(blk + off2);
    }
  }

  // q operand (B of the score MFMA): column col holds head col % G; k-step ks
  // covers dims 32*ks + 8*lg + [0, 8).  Scaled by 1/sqrt(64) (exact).
  bf16x8 qop[2][NP];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const f32x4 lo = qraw[ks][0], hi = qraw[ks][1];
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) { x[i] = lo[i] * 0.125f; x[4 + i] = hi[i] * 0.125f; }
    split_parts<NP>(x, qop[ks]);
  }
  float m_run = -INFINITY, l_part = 0.f;
  f32x4 acc[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto process = [&](const u32x4 (&kr)[8], const u32x4 (&vr)[8], int T) {
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
    mt = rows_max_ds(mt);
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
    l_part = __builtin_fmaf(l_part, alpha, ps);
    m_run = m_new;
    // (P x V)^T = V^T x P^T: acc[nb] row 4*lg + i is dim 16*nb + 4*lg + i,
    // column col is head col % G -- this lane's own alpha.
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[nb][i] *= alpha;
    // k-step s covers keys of blocks 2s and 2s+1 (this lane's own scores); the
    // V register of a lane is its A operand (dims x keys) as it is the B operand
    // of P x V, and the P operand likewise
    u32x4 vnat[NAT ? 8 : 1];
    if constexpr (NAT) {
      // the wave's tile into LDS as stored, then lane (lg, col)'s operand of
      // (k-step s, dim block nb): dim 16 nb + col of keys 32 s + 16 jb + 4 lg + jr
      // at element 4 jb + jr (the tiled layout's order)
      uint16_t* vw = vst + wave * (TILE * kVstRow);
#pragma unroll
      for (int i = 0; i < 8; ++i) *(u32x4*)(vw + (8 * i + (lane >> 3)) * kVstRow + 8 * (lane & 7)) = vr[i];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // ds_read_b64_tr_b16: lane i of a 16-lane group receives element i & 3 of
      // the 8-byte chunks that lanes (i >> 2) + 4 j of the group address, j =
      // 0..3.  Lane m of group lg addresses key 32 s + 16 jb + 4 lg + (m >> 2),
      // dims 16 nb + 4 (m & 3) .. +3, so lane (lg, col) gets dim 16 nb + col of
      // keys 32 s + 16 jb + 4 lg + j: operand elements 4 jb + j, in order.
      typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;
      const __attribute__((address_space(3))) uint16_t* vl = (const __attribute__((address_space(3))) uint16_t*)vw;
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          u32x2 h[2];
#pragma unroll
          for (int jb = 0; jb < 2; ++jb) {
            const int key = 32 * s + 16 * jb + 4 * lg + (col >> 2), dim = 16 * nb + 4 * (col & 3);
            h[jb] = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                           (__attribute__((address_space(3))) bf16x4_t*)(vl + key * kVstRow + dim)));
          }
          vnat[4 * s + nb] = u32x4{h[0][0], h[0][1], h[1][0], h[1][1]};
        }
      // every lane's reads are done before the next tile is stored over them
      __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float pv[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) { pv[i] = S[2 * s][i]; pv[4 + i] = S[2 * s + 1][i]; }
      bf16x8 pop[NP];
      split_parts<NP>(pv, pop);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const bf16x8 vop = __builtin_bit_cast(bf16x8, NAT ? vnat[NAT ? 4 * s + nb : 0] : vr[4 * s + nb]);
#pragma unroll
        for (int k = 0; k < NP; ++k)
          acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[k], acc[nb], 0, 0, 0);
      }
    }
  };

  if constexpr (PF == 0) {
    for (int T = wave; T < ntiles; T += ATT_WAVES) {
      u32x4 kr[8], vr[8];
      load(kr, vr, T);
      process(kr, vr, T);
    }
  } else {
    // two buffers: A holds tiles wave + 2j*W, B tiles wave + (2j+1)*W.  NAT:
    // the loads are unconditional (a tile past the end re-reads the last one),
    // so the compiler knows how many are in flight and waits for the computed
    // tile's loads only (B = 1: 19.6 -> 17.1 us); the tiled form keeps its
    // conditional loads, which measured faster there (9.0 against 9.9 us).
    u32x4 ka[8], va[8], kb2[8], vb2[8];
    int T = wave;
    if (T < ntiles) load(ka, va, T);
    for (; T < ntiles; T += 2 * ATT_WAVES) {
      const int T1 = T + ATT_WAVES, T2 = T + 2 * ATT_WAVES;
      if (NAT) load(kb2, vb2, T1 < ntiles ? T1 : ntiles - 1);
      else if (T1 < ntiles) load(kb2, vb2, T1);
      process(ka, va, T);
      if (NAT) load(ka, va, T2 < ntiles ? T2 : ntiles - 1);
      else if (T2 < ntiles) load(ka, va, T2);
      if (T1 < ntiles) process(kb2, vb2, T1);
    }
  }
  // l: this lane's keys only; add the four lane groups (fixed butterfly).
  l_part = rows_sum_ds(l_part);
  // column h < G is head h: dims 16*nb + 4*lg + i in acc[nb][i]
  if (col < G) {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) *(f32x4*)&sm.acc[wave][col][16 * nb + 4 * lg] = acc[nb];
  }
  if (lane < G) {
    sm.m[wave][lane] = m_run;
    sm.l[wave][lane] = l_part;
  }
  __syncthreads();
  RowExtras<1> ex;
  ex.vv[0] = a.use_xsa ? bf16_to_f32(v_raw) : 0.f;
  ex.gv = g_raw;
  merge_and_store<G, YBF16>(a, sm, r, g, wave, lane, ex, OP ? ys : nullptr);
  if constexpr (OP) {
    __syncthreads();  // the row's bf16 y is in ys
    const int gq = g & 3;
    // A operand of k-step ss: features 32 ss + 8 lg .. +8 of the head, the
    // same in all 16 MFMA rows (so every row of t is the row's sum)
    bf16x8 ya[2];
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) ya[ss] = __builtin_bit_cast(bf16x8, *(const u32x4*)(ys + 32 * ss + 8 * lg));
    float* dst = a.o_part + ((int64_t)r * a.H + g) * a.o_n;
#pragma unroll
    for (int qi = 0; qi < kOpQ; ++qi) {
      const int nb = wave + ATT_WAVES * qi;
      if (16 * nb >= a.o_n) break;
      // the steps' words where b_op_bf16<OP> reads k-steps 0 and 1: low-plane
      // word(s) at p0[0] (and p0[1]), the high-plane word at p1[0] (3 bits:
      // shifted so that the steps' bytes are its bytes 0 and 1)
      uint32_t q0[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u}, q1[4] = {0u, 0u, 0u, 0u};
      q0[0] = ow[qi][0];
      if constexpr (OP >= 4) q0[1] = ow[qi][1];
      if constexpr (OP == 6) q1[0] = ow[qi][2];
      if constexpr (OP == 3) q1[0] = ow[qi][2] >> (16 * (gq & 1));
      f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ss = 0; ss < 2; ++ss)
        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ya[ss], altxs::b_op_bf16<OP>(q0, q1, ss, OP), t, 0, 0, 0);
      if (lane < 16) dst[16 * nb + lane] = t[0];  // row 0, column lane of the block
    }
  }
}

// ---------------------------------------------------------------------------
// bf16 cache, windows (W > 1): 16*NG consecutive query rows of one segment and
// one query head per workgroup, so each K/V tile is read once for all of them.
// Every query column performs exactly the decode task's arithmetic: the same
// MFMA operand placement for its scores and P x V, tile T on wave T mod 4, the
// same online softmax and the same wave-order merge.  Tiles past a query's
// own last key are fully masked for it; they leave its running state
// unchanged (alpha = 1, P = 0, and a wave that has seen no key keeps
// m = -inf), so a window row gives the bits of the decode row.
// ---------------------------------------------------------------------------

struct alignas(16) WinLds {
  float m[ATT_WAVES][16];
  float l[ATT_WAVES][16];
  float acc[ATT_WAVES][16][HD + 4];  // rows padded: a wave's 16 query rows on distinct banks
};

template <int NG, int NP, int YBF16>
__device__ __forceinline__ void attn_window_task(const AttnP& a, int b, int h, int t0, WinLds& sm) {
  static_assert(TILE == 64, "the MFMA tiling below assumes 64-key tiles");
  const int G = a.H / a.Hkv, g = h / G;
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  const int lg = lane >> 4, col = lane & 15;
  const uint16_t* kb = (const uint16_t*)a.k + (int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD;
  const uint16_t* vb = (const uint16_t*)a.v + (int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD;
  const int base = a.pos[b];
  // this lane's query column in each group: window index t, position p (-1: inactive)
  int pc[NG];
  bf16x8 qop[NG][2][NP];
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    const int t = t0 + 16 * gi + col;
    int p = -1;
    if (t < a.W) {
      p = base + t;
      if (p < 0 || p >= a.max_len) {
        flag_err(a.err, ALTXS_EDEV_POS);
        p = p < 0 ? 0 : a.max_len - 1;
      }
    }
    pc[gi] = p;
    const float* qh = a.q + ((int64_t)(b * a.W + (t < a.W ? t : 0)) * a.H + h) * HD;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      float x[8];
      if (t < a.W) {
        const f32x4 lo = *(const f32x4*)(qh + 32 * ks + 8 * lg);
        const f32x4 hi = *(const f32x4*)(qh + 32 * ks + 8 * lg + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) { x[i] = lo[i] * 0.125f; x[4 + i] = hi[i] * 0.125f; }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = 0.f;
      }
      split_parts<NP>(x, qop[gi][ks]);
    }
  }
  // keys to visit: up to the last active query of the workgroup (uniform)
  const int t_last = (t0 + 16 * NG < a.W ? t0 + 16 * NG : a.W) - 1;
  int p_last = base + t_last;
  p_last = p_last < 0 ? 0 : (p_last >= a.max_len ? a.max_len - 1 : p_last);
  const int ntiles = (p_last + TILE) / TILE;

  float m_run[NG], l_part[NG];
  f32x4 acc[NG][4];
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    m_run[gi] = -INFINITY;
    l_part[gi] = 0.f;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[gi][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // tile T of the K and V caches -> registers (one 16-byte load per lane each).
  // Ordinary (temporal) loads: every query block of this (segment, head) reads
  // the same tiles, and they are meant to stay in L2 between the blocks.
  auto load_t = [&](u32x4 (&kr)[8], u32x4 (&vr)[8], int T) {
    const u32x4* kt = (const u32x4*)(kb + (int64_t)T * (TILE * HD)) + lane;
    const u32x4* vt = (const u32x4*)(vb + (int64_t)T * (TILE * HD)) + lane;
#pragma unroll
    for (int i = 0; i < 8; ++i) kr[i] = kt[64 * i];
#pragma unroll
    for (int i = 0; i < 8; ++i) vr[i] = vt[64 * i];
  };
  // MASK = false: a tile whose keys all precede every query of the workgroup
  // (no key is masked for any of them, so skipping the mask changes nothing)
  auto tile = [&](const u32x4 (&kr)[8], const u32x4 (&vr)[8], int T, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int k0 = T * TILE;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      f32x4 S[4];
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        S[blk] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const bf16x8 kop = __builtin_bit_cast(bf16x8, kr[2 * blk + ks]);
#pragma unroll
          for (int k = 0; k < NP; ++k)
            S[blk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qop[gi][ks][k], S[blk], 0, 0, 0);
        }
      }
      float mt = -INFINITY;
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (MASK && k0 + 16 * blk + 4 * lg + i > pc[gi]) S[blk][i] = -INFINITY;
          mt = fmaxf(mt, S[blk][i]);
        }
      mt = rows_max(mt);
      const float m_new = fmaxf(m_run[gi], mt);
      // A query with no key seen yet (m_new = -inf) subtracts 0 instead: its
      // scores give exp(-inf) = 0 and alpha = 0, which leaves its state (l = 0,
      // acc = 0) exactly as alpha = 1 and P = 0 would.
      const float mu = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __expf(m_run[gi] - mu);
      float ps = 0.f;
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          S[blk][i] = __expf(S[blk][i] - mu);
          ps += S[blk][i];
        }
      l_part[gi] = __builtin_fmaf(l_part[gi], alpha, ps);
      m_run[gi] = m_new;
      // acc[gi][nb] = (P x V)^T: row 4*lg + i is dim 16*nb + 4*lg + i, column
      // col is this lane's query
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[gi][nb][i] *= alpha;
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
            acc[gi][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[k], acc[gi][nb], 0, 0, 0);
        }
      }
    }
  };
  // Tiles T = wave, wave + 4, ... in order, one tile in registers at a time:
  // that keeps NG = 2 at 152 VGPRs, three waves per SIMD, whose interleaving
  // hides the load latency far better than a second register buffer at one
  // wave per SIMD (288 VGPRs; cfg4: 0.93 vs 2.1 ms per slot).
  // Tiles below the diagonal of every query first, without the mask (two
  // loops rather than a branch in one: the branch costs the third wave).
  int t_first = t0 + 16 * NG <= a.W ? base + t0 : -1;  // lowest query position, all active
  t_first = t_first >= a.max_len ? -1 : t_first;
  const int nfull = t_first < 0 ? 0 : (t_first + 1) / TILE;  // tiles 0 .. nfull-1 unmasked
  int T = wave;
  for (; T < nfull; T += ATT_WAVES) {
    u32x4 kr[8], vr[8];
    load_t(kr, vr, T);
    tile(kr, vr, T, std::false_type{});
  }
  for (; T < ntiles; T += ATT_WAVES) {
    u32x4 kr[8], vr[8];
    load_t(kr, vr, T);
    tile(kr, vr, T, std::true_type{});
  }
  // merge and store, one group of 16 queries at a time; wave w finishes
  // queries 4w .. 4w+3 (one per wave row), then 4w + 4*ATT_WAVES ...
  auto v_at = [&](int pp, int d) {
    return bf16_to_f32(vb[(int64_t)(pp / TILE) * (TILE * HD) + kv_tile_v(pp % TILE, d)]);
  };
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    const float lsum = rows_sum(l_part[gi]);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) *(f32x4*)&sm.acc[wave][col][16 * nb + 4 * lg] = acc[gi][nb];
    if (lane < 16) {
      sm.m[wave][lane] = m_run[gi];
      sm.l[wave][lane] = lsum;
    }
    __syncthreads();
    for (int q = 4 * wave + lg; q < 16; q += 4 * ATT_WAVES) {
      const int t = t0 + 16 * gi + q;
      if (t < a.W) {
        int p = base + t;
        p = p < 0 ? 0 : (p >= a.max_len ? a.max_len - 1 : p);
        const RowExtras<4> rx = row_extras<4>(a, b * a.W + t, h, p, col, v_at);
        finish_query<4, YBF16>(a, &sm.m[0][q], &sm.l[0][q], 16, &sm.acc[0][q][0], 16 * (HD + 4),
                               b * a.W + t, h, col, rx);
      }
    }
    __syncthreads();
  }
}

}  // namespace altxs_attn
