// Decode / window attention over the KV cache (one query row at a time).
//
// Workgroup = ATT_WAVES waves for one (query row r, kv head g); it serves the
// G = H/Hkv query heads of that group so each K/V byte is read once.  Keys
// [0, p] (p = pos[b] + t) are cut into fixed 64-key tiles from position 0;
// tile T goes to wave T % ATT_WAVES, so at any moment the waves of a
// workgroup read neighbouring tiles (a few long DRAM streams instead of one
// per wave).  Each wave keeps an online softmax (fp32) over its tiles; the
// per-wave partials (m, l, acc[64]) are merged in wave order through LDS.
// Everything depends only on p, never on the batch or window size, so a row
// gives the same bits as a decode row (W = 1) and inside an encode window.
//
// bf16 cache (attn_mfma_kernel): both products run on v_mfma_f32_16x16x32_bf16
// the way the reference's split-prefix kernel uses tl.dot
// (src/xsa_ttt/split_attn.py:55-152): q padded to 16 MFMA columns (column n
// holds head n % G), scores = K-tile x q, then (P x V)^T = V^T x P^T with P the
// exp'd scores (the output column is the query, so each lane rescales its
// accumulator by its own query's alpha, with no cross-lane shuffle).
// The K and V tiles are stored pre-swizzled (kv_tile_index below) so that every
// lane's MFMA operand is one 16-byte load and a wave's load instruction reads
// 1 KB of consecutive bytes.  The natural-order bf16 cache (the reference's
// own k_pack layout) runs the same kernel with K operands read in place and
// each V tile staged through LDS (attn_mfma_task, NAT): the same operands,
// the same bits.  Operand precision:
//   * OPS_BF16: q and P rounded to bf16 (the reference's production arithmetic);
//   * fp32-faithful: q split into three bf16 parts and P into three, each part
//     multiplied separately (sum of parts reproduces fp32 to ~2^-24).
// fp32 cache (attn_valu_kernel): plain fp32 FMAs on the natural [key][64] layout.
//
// Epilogue: XSA (subtract the projection onto the current value direction,
// src/xsa_ttt/model.py:760-768), the sparse attention gate multiplier, store.
#include "attn.h"
#include "common.h"
#include "kernels.h"

using namespace altxs_attn;

#ifndef ALTXS_ATT_PF
#define ALTXS_ATT_PF 0  // 1: each wave keeps its next tile's loads in flight
#endif

namespace {

// Decode launches with fewer (row, kv head) workgroups than this take the
// two-tiles-in-flight MHA variant (the chip has 256 CUs), with prefetch
// workgroups beside them (attn_prefetch_task).
constexpr unsigned kAttnSmallGrid = 256;

// Prefetch workgroup h (of a.helpers) of (row, kv head) pair c in a small
// decode launch: it touches one word of every 128-byte line of the pair's K
// and V tiles h, h + helpers, ... (both halves of the workgroup interleave
// tiles), all loads in flight at once, so the lines are in the L2 before the
// pair's compute waves reach them.  Pair c's compute workgroup has id c and
// helper h id (h + 1) * pairs + c; workgroups are dealt to the 8 XCDs
// round-robin by id, so with pairs % 8 == 0 both share an XCD and its L2
// (otherwise the lines still come from the memory-side cache).  Reads only:
// the results are the compute workgroups' alone.
// ESZ: bytes per cache element (2: bf16, tiled or natural; 4: fp32).  In
// every layout tile T of a (segment, kv head) is TILE x HD consecutive
// elements (keys 64T .. 64T + 63); with a tail placement the window's rows
// are not prefetched (one row per query at W = 1).
template <int ESZ>
__device__ __forceinline__ void attn_prefetch_task(const AttnP& a, int c, int h) {
  constexpr int kLines = TILE * HD * ESZ / 128;  // 128-byte lines per K (or V) tile
  constexpr int kGroups = ATT_THREADS / (2 * kLines);  // tiles one pass touches
  static_assert(kGroups >= 1 && ATT_THREADS % (2 * kLines) == 0, "one K and one V tile per thread group");
  const int r = c / a.Hkv, g = c % a.Hkv, b = r / a.W;
  int p = a.pos[b] + r % a.W;
  p = p < 0 ? 0 : (p >= a.max_len ? a.max_len - 1 : p);  // the compute task flags it
  const int ntiles = p / TILE + 1;
  const int grp = threadIdx.x / (2 * kLines), li = threadIdx.x % (2 * kLines);
  const int64_t off = ((int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD) * ESZ;
  const char* base = (const char*)(li < kLines ? a.k : a.v) + off + (li % kLines) * 128;
  const int step = kGroups * a.helpers;
  uint32_t acc = 0;
  for (int T0 = h + a.helpers * grp; T0 < ntiles; T0 += 8 * step) {
    uint32_t x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {  // unconditional: a tile past the end re-reads the last one
      const int T = min(T0 + u * step, ntiles - 1);
      x[u] = *(const uint32_t*)(base + (int64_t)T * (TILE * HD * ESZ));
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += x[u];
  }
  asm volatile("" ::"v"(acc));  // keeps the loads
}

// Helpers per (row, kv head) pair of a launch of `pairs` workgroups (0: none).
inline int attn_helpers(unsigned pairs) {
  return pairs < kAttnSmallGrid ? (int)(kAttnSmallGrid / pairs < 16 ? kAttnSmallGrid / pairs : 16) : 0;
}

template <int G, int NP, int YBF16, int PF, int NAT = 0, int OP = 0>
__global__ __launch_bounds__(ATT_THREADS) void attn_mfma_kernel(AttnP a) {
  __shared__ MergeLds<G> sm;
  __shared__ __attribute__((aligned(16))) uint16_t vst[NAT ? ATT_WAVES * TILE * kVstRow : 8];
  __shared__ __attribute__((aligned(16))) uint16_t ys[OP ? HD : 8];
  if constexpr ((G == 1 && PF == 1) || NAT) {
    const int pairs = a.B * a.W * a.Hkv;
    if (a.helpers > 0 && (int)blockIdx.x >= pairs) {
      const int id = blockIdx.x - pairs;
      attn_prefetch_task<2>(a, id % pairs, id / pairs);
      return;
    }
  }
  int r = blockIdx.x / a.Hkv, g = blockIdx.x % a.Hkv;
  if (a.xcd_rows) {  // row tile t (8 rows x Hkv heads) on XCD t % 8
    int t, j;
    xcd_row_split(blockIdx.x, a.B * a.W / 8, t, j);
    r = 8 * t + j / a.Hkv;
    g = j % a.Hkv;
  }
  // GQA launches have G times fewer workgroups, and small launches (PF = 1)
  // too few to cover the load latency: keep two tiles per wave in flight
  attn_mfma_task<G, NP, YBF16, (G > 1 ? 1 : PF), NAT, OP>(a, r, g, sm, vst, ys);
}

// Windows (W > 1) on the bf16 cache: 16*NG query rows of one (segment, head)
// per workgroup; grid = B x H x ceil(W / (16*NG)).  At most 256 VGPRs, so at
// least two waves share a SIMD (NG <= 2 takes 152: three).
template <int NG, int NP, int YBF16>
__global__ __launch_bounds__(ATT_THREADS, 2) void attn_window_kernel(AttnP a) {
  __shared__ WinLds sm;
  const int nqb = (a.W + 16 * NG - 1) / (16 * NG);
  // Workgroups are dealt to the 8 XCDs round-robin by linear id.  Every query
  // block of a (segment, head) reads the same K/V tiles, so the blocks of one
  // (segment, head) go to one XCD, consecutively, and its tiles stay in that
  // XCD's L2 (a bijection of the ids when the grid is a multiple of 8).
  int L = blockIdx.x;
  if (gridDim.x % 8 == 0) L = (blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8;
  const int qb = L % nqb, bh = L / nqb;
  attn_window_task<NG, NP, YBF16>(a, bh / a.H, bh % a.H, qb * 16 * NG, sm);
}

// ---------------------------------------------------------------------------
// fp32 cache: VALU kernel on the natural [key][64] layout.
// ---------------------------------------------------------------------------

// Lanes: LPK = 16 lanes share a key (4 dims each); KPI = 4 keys per load.
constexpr int V_EPL = 4, V_LPK = HD / V_EPL, V_KPI = WAVE / V_LPK, V_NI = TILE / V_KPI;

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

// Four consecutive dims of cache row `row` (natural layout).
__device__ __forceinline__ f32x4 load4(const float* base, int64_t row, int d) {
  return __builtin_nontemporal_load((const f32x4*)(base + row * HD + d));
}
__device__ __forceinline__ float load1(const float* base, int64_t row, int d) { return base[row * HD + d]; }

// The fp32 cache (natural order; the bf16 natural order runs the MFMA kernel).
template <int G, int YBF16>
__global__ __launch_bounds__(ATT_THREADS) void attn_valu_kernel(AttnP a) {
  using KVT = float;
  __shared__ MergeLds<G> sm;
  {
    const int pairs = a.B * a.W * a.Hkv;
    if (a.helpers > 0 && (int)blockIdx.x >= pairs) {
      const int id = blockIdx.x - pairs;
      attn_prefetch_task<(int)sizeof(KVT)>(a, id % pairs, id / pairs);
      return;
    }
  }
  int r = blockIdx.x / a.Hkv, g = blockIdx.x % a.Hkv;
  if (a.xcd_rows) {  // row tile (8 rows x Hkv heads) tt on XCD tt % 8
    int tt, j;
    xcd_row_split(blockIdx.x, a.B * a.W / 8, tt, j);
    r = 8 * tt + j / a.Hkv;
    g = j % a.Hkv;
  }
  const int b = r / a.W, t = r % a.W;
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  int pb = a.pos[b];
  if (a.kv_tail >= 0 && pb > a.kv_tail) {  // the prefix would run into the window rows
    if (threadIdx.x == 0) flag_err(a.err, ALTXS_EDEV_POS);
    pb = a.kv_tail;
  }
  const int p = clamp_pos(a, b, t, pb);
  const int nkeys = p + 1;
  const int ntiles = (nkeys + TILE - 1) / TILE;
  const KVT* kb = (const KVT*)a.k + (int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD;
  const KVT* vb = (const KVT*)a.v + (int64_t)b * a.seg_stride + (int64_t)g * a.max_len * HD;
  const int dslice = V_EPL * (lane % V_LPK);
  const int ksub = lane / V_LPK;
  float qv[G][V_EPL];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const float* qh = a.q + ((int64_t)r * a.H + g * G + j) * HD + dslice;
#pragma unroll
    for (int e = 0; e < V_EPL; ++e) qv[j][e] = qh[e] * 0.125f;
  }
  float m_run[G], l_run[G], acc[G][V_EPL];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    m_run[j] = -INFINITY;
    l_run[j] = 0.f;
#pragma unroll
    for (int e = 0; e < V_EPL; ++e) acc[j][e] = 0.f;
  }
  for (int T = wave; T < ntiles; T += ATT_WAVES) {
    const int k0 = T * TILE;
    f32x4 kr[V_NI], vr[V_NI];
#pragma unroll
    for (int i = 0; i < V_NI; ++i) kr[i] = load4(kb, key_row(a, k0 + V_KPI * i + ksub, pb, p), dslice);
#pragma unroll
    for (int i = 0; i < V_NI; ++i) vr[i] = load4(vb, key_row(a, k0 + V_KPI * i + ksub, pb, p), dslice);
    const int my_key = k0 + V_KPI * (lane % V_LPK) + ksub;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      float s[V_NI];
#pragma unroll
      for (int i = 0; i < V_NI; ++i) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < V_EPL; ++e) d += qv[j][e] * kr[i][e];
        s[i] = d;
      }
      float sc = transpose_reduce<V_NI, V_LPK>(s, lane);
      if (my_key >= nkeys) sc = -INFINITY;
      const float m_new = fmaxf(m_run[j], wave_max(sc));
      const float alpha = __expf(m_run[j] - m_new);
      const float pl = __expf(sc - m_new);
      l_run[j] = l_run[j] * alpha + pl;
#pragma unroll
      for (int e = 0; e < V_EPL; ++e) acc[j][e] *= alpha;
#pragma unroll
      for (int i = 0; i < V_NI; ++i) {
        const float pk = __shfl(pl, (lane & ~(V_LPK - 1)) | i, WAVE);
#pragma unroll
        for (int e = 0; e < V_EPL; ++e) acc[j][e] += pk * vr[i][e];
      }
      m_run[j] = m_new;
    }
  }
#pragma unroll
  for (int j = 0; j < G; ++j) {
#pragma unroll
    for (int e = 0; e < V_EPL; ++e) {
#pragma unroll
      for (int msk = V_LPK; msk < WAVE; msk <<= 1) acc[j][e] += __shfl_xor(acc[j][e], msk, WAVE);
    }
    const float lsum = wave_sum(l_run[j]);
    if (lane < V_LPK) {
#pragma unroll
      for (int e = 0; e < V_EPL; ++e) sm.acc[wave][j][dslice + e] = acc[j][e];
    }
    if (lane == 0) {
      sm.m[wave][j] = m_run[j];
      sm.l[wave][j] = lsum;
    }
  }
  __syncthreads();
  merge_and_store<G, YBF16>(a, sm, r, g, p, wave, lane,
                            [&](int pp, int d) { return load1(vb, key_row(a, pp, pb, p), d); });
}

template <int YBF16>
hipError_t launch_y(const AttnP& p, int group, int kv_layout, bool ops_bf16, bool rows_only,
                    hipStream_t s) {
  const bool kv_bf16 = kv_layout == ALTXS_KV_BF16;  // the MFMA kernels read the tiled layout
  dim3 grid((unsigned)(p.B * p.W * p.Hkv)), block(ATT_THREADS);
#define ATT_GO(K) \
  do { hipLaunchKernelGGL(K, grid, block, 0, s, p); return hipGetLastError(); } while (0)
  if (kv_bf16 && p.W > 1 && !rows_only) {
    // 32 query rows per workgroup for longer windows: the 64-row variant needs
    // 253 VGPRs (two waves per SIMD) and measured slower (cfg4: 1.17 vs
    // 0.93 ms per slot); the bits are the same either way
    const int ng = p.W <= 16 ? 1 : 2;
    const int nqb = (p.W + 16 * ng - 1) / (16 * ng);
    dim3 wgrid((unsigned)((int64_t)p.B * p.H * nqb));
#define WIN_GO(K) \
  do { hipLaunchKernelGGL(K, wgrid, block, 0, s, p); return hipGetLastError(); } while (0)
    if (ops_bf16) {
      if (ng == 1) WIN_GO((attn_window_kernel<1, 1, YBF16>));
      WIN_GO((attn_window_kernel<2, 1, YBF16>));
    } else {
      if (ng == 1) WIN_GO((attn_window_kernel<1, 3, YBF16>));
      WIN_GO((attn_window_kernel<2, 3, YBF16>));
    }
#undef WIN_GO
  }
  if (kv_bf16) {
    // Fewer workgroups than CUs (small batches, B = 1 above all): each wave's
    // tiles are a dependent chain of HBM round trips that nothing else hides,
    // so the MHA kernel keeps its next tile's loads in flight as well (the
    // same arithmetic in the same order: the same bits).
    if (group == 1 && grid.x < kAttnSmallGrid && !p.xcd_rows) {
      AttnP ph = p;
      ph.helpers = attn_helpers(grid.x);
      const dim3 hgrid(grid.x * (1 + ph.helpers));
      if (ops_bf16) hipLaunchKernelGGL((attn_mfma_kernel<1, 1, YBF16, 1>), hgrid, block, 0, s, ph);
      else hipLaunchKernelGGL((attn_mfma_kernel<1, 3, YBF16, 1>), hgrid, block, 0, s, ph);
      return hipGetLastError();
    }
    if (ops_bf16) {
      if (group == 1) ATT_GO((attn_mfma_kernel<1, 1, YBF16, ALTXS_ATT_PF>));
      if (group == 2) ATT_GO((attn_mfma_kernel<2, 1, YBF16, 1>));
      if (group == 4) ATT_GO((attn_mfma_kernel<4, 1, YBF16, 1>));
    } else {
      if (group == 1) ATT_GO((attn_mfma_kernel<1, 3, YBF16, ALTXS_ATT_PF>));
      if (group == 2) ATT_GO((attn_mfma_kernel<2, 3, YBF16, 1>));
      if (group == 4) ATT_GO((attn_mfma_kernel<4, 3, YBF16, 1>));
    }
    return hipErrorInvalidValue;
  }
  // natural layouts: prefetch workgroups beside small launches as above
  AttnP ph = p;
  const unsigned pairs = grid.x;
  ph.helpers = p.xcd_rows ? 0 : attn_helpers(pairs);
  grid.x *= 1 + ph.helpers;
#undef ATT_GO
#define ATT_GO(K) \
  do { hipLaunchKernelGGL(K, grid, block, 0, s, ph); return hipGetLastError(); } while (0)
  if (kv_layout == ALTXS_KV_BF16_NATURAL) {
    // the MFMA kernel on the natural order (V staged through LDS): the bits
    // of the tiled layout; one query row per workgroup at every window width
    const bool pf = pairs < kAttnSmallGrid;  // (GQA launches keep two tiles in flight anyway)
    if (ops_bf16) {
      if (group == 1) { if (pf) ATT_GO((attn_mfma_kernel<1, 1, YBF16, 1, 1>)); ATT_GO((attn_mfma_kernel<1, 1, YBF16, 0, 1>)); }
      if (group == 2) ATT_GO((attn_mfma_kernel<2, 1, YBF16, 1, 1>));
      if (group == 4) ATT_GO((attn_mfma_kernel<4, 1, YBF16, 1, 1>));
    } else {
      if (group == 1) { if (pf) ATT_GO((attn_mfma_kernel<1, 3, YBF16, 1, 1>)); ATT_GO((attn_mfma_kernel<1, 3, YBF16, 0, 1>)); }
      if (group == 2) ATT_GO((attn_mfma_kernel<2, 3, YBF16, 1, 1>));
      if (group == 4) ATT_GO((attn_mfma_kernel<4, 3, YBF16, 1, 1>));
    }
  } else {
    if (group == 1) ATT_GO((attn_valu_kernel<1, YBF16>));
    if (group == 2) ATT_GO((attn_valu_kernel<2, YBF16>));
    if (group == 4) ATT_GO((attn_valu_kernel<4, YBF16>));
  }
#undef ATT_GO
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t altxs_launch_attn(const AltxsAttnArgs& a, hipStream_t s) {
  AttnP p;
  p.B = a.B; p.W = a.W; p.H = a.H; p.Hkv = a.Hkv; p.max_len = a.max_len;
  p.q = a.q; p.k = a.k; p.v = a.v; p.seg_stride = a.kv_seg_stride;
  p.pos = a.pos; p.gate = a.gate; p.use_xsa = a.use_xsa; p.y = a.y; p.err = a.err;
  const int group = a.H / a.Hkv;
  const bool ops_bf16 = (a.flags & ALTXS_ATTN_OPS_BF16) != 0;
  const bool rows_only = (a.flags & ALTXS_ATTN_ROWS) != 0;
  p.xcd_rows = ((a.flags & ALTXS_ATTN_XCD_ROWS) != 0 && (int64_t)a.B * a.W % 64 == 0) ? 1 : 0;
  p.kv_tail = a.kv_tail_end > 0 ? a.kv_tail_end - a.W : -1;
  return a.y_bf16 ? launch_y<1>(p, group, a.kv_bf16, ops_bf16, rows_only, s)
                  : launch_y<0>(p, group, a.kv_bf16, ops_bf16, rows_only, s);
}

// The decode launch with the out-projection terms (attn_mfma_task, OP = 1):
// W = 1 rows, MHA, the tiled bf16 cache, bf16 operands and output; o_bits in
// {2, 3, 4, 6}, o_n a multiple of 16 up to 512, H a multiple of 4.  The
// kernel variant and placement are those altxs_launch_attn picks.
hipError_t altxs_launch_attn_o(const AltxsAttnArgs& a, const uint8_t* o_codes, int o_bits, int o_n,
                               float* o_part, hipStream_t s) {
  if (a.W != 1 || a.H != a.Hkv || a.kv_bf16 != ALTXS_KV_BF16 || !a.y_bf16 ||
      (a.flags & ALTXS_ATTN_OPS_BF16) == 0 || a.kv_tail_end != 0 || a.H % 4 != 0 ||
      !(o_bits == 2 || o_bits == 3 || o_bits == 4 || o_bits == 6) || o_n < 16 || o_n > 512 ||
      o_n % 16 != 0 || !o_codes || !o_part)
    return hipErrorInvalidValue;
  AttnP p;
  p.B = a.B; p.W = a.W; p.H = a.H; p.Hkv = a.Hkv; p.max_len = a.max_len;
  p.q = a.q; p.k = a.k; p.v = a.v; p.seg_stride = a.kv_seg_stride;
  p.pos = a.pos; p.gate = a.gate; p.use_xsa = a.use_xsa; p.y = a.y; p.err = a.err;
  p.xcd_rows = ((a.flags & ALTXS_ATTN_XCD_ROWS) != 0 && (int64_t)a.B % 64 == 0) ? 1 : 0;
  p.o_codes = o_codes; p.o_bits = o_bits; p.o_n = o_n; p.o_part = o_part;
  const dim3 grid((unsigned)(p.B * p.Hkv)), block(ATT_THREADS);
  const bool small = grid.x < kAttnSmallGrid && !p.xcd_rows;  // as launch_y: prefetch workgroups beside
  if (small) p.helpers = attn_helpers(grid.x);
  const dim3 g2(small ? grid.x * (1 + p.helpers) : grid.x);
#define OP_GO(B)                                                                                \
  do {                                                                                          \
    if (small) hipLaunchKernelGGL((attn_mfma_kernel<1, 1, 1, 1, 0, B>), g2, block, 0, s, p);      \
    else hipLaunchKernelGGL((attn_mfma_kernel<1, 1, 1, ALTXS_ATT_PF, 0, B>), g2, block, 0, s, p); \
    return hipGetLastError();                                                                   \
  } while (0)
  switch (o_bits) {
    case 2: OP_GO(2);
    case 3: OP_GO(3);
    case 4: OP_GO(4);
    default: OP_GO(6);
  }
#undef OP_GO
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
  ALTXS_REQUIRE(a->max_len >= TILE && a->max_len % TILE == 0,
                "altxs_decode_attn: max_len=%d must be a positive multiple of %d", a->max_len, TILE);
  ALTXS_REQUIRE(a->kv_seg_stride == 0 || a->kv_seg_stride >= (int64_t)a->Hkv * a->max_len * HD,
                "altxs_decode_attn: kv_seg_stride too small");
  ALTXS_REQUIRE((a->flags & ~(ALTXS_ATTN_OPS_BF16 | ALTXS_ATTN_ROWS | ALTXS_ATTN_XCD_ROWS)) == 0,
                "altxs_decode_attn: unknown flags 0x%x", a->flags);
  ALTXS_REQUIRE(a->kv_bf16 == ALTXS_KV_F32 || a->kv_bf16 == ALTXS_KV_BF16 ||
                    a->kv_bf16 == ALTXS_KV_BF16_NATURAL,
                "altxs_decode_attn: kv_bf16=%d is not a KV layout", a->kv_bf16);
  ALTXS_REQUIRE(a->kv_tail_end == 0 || (a->kv_bf16 != ALTXS_KV_BF16 && a->kv_tail_end >= a->W &&
                                        a->kv_tail_end <= a->max_len),
                "altxs_decode_attn: kv_tail_end=%d needs a natural layout and W <= kv_tail_end <= "
                "max_len", a->kv_tail_end);
  ALTXS_REQUIRE(((uintptr_t)a->k & 15) == 0 && ((uintptr_t)a->v & 15) == 0 && ((uintptr_t)a->q & 15) == 0,
                "altxs_decode_attn: q, k and v must be 16-byte aligned");
  ALTXS_CHECK_HIP(altxs_launch_attn(*a, (hipStream_t)stream));
  return ALTXS_OK;
}
