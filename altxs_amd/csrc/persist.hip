// Persistent layer kernel: every slot of the step for every 16-row tile of a
// segment group in one launch.
//
// Work items ("tasks"): for each slot s and 16-row tile m, the QKV column
// tiles, the attention (row, kv head) pairs, then the O, UP and DOWN column
// tiles.  One workgroup per CU; the first `ng` workgroups to start are GEMM
// workers and take QKV/O/UP/DOWN tasks from one queue, the others stream
// attention tasks from a second queue.  A task waits (bounded spin) until the
// stage it reads is complete for its row tile, runs the same device code as the
// per-stage kernels, publishes its stores (one agent-scope release per
// workgroup) and bumps the completion counter of (s, m, stage).  Row tiles
// progress independently, so one tile's projections and MLP run while other
// tiles' attention streams the KV cache.
//
// Results are bit-identical to the per-stage kernels: each task is the same
// tile computation, and every reduction order depends only on the tile shape.
#include "attn.h"
#include "common.h"
#include "persist.h"
#include "step_ops.h"

using namespace altxs;
using namespace altxs_sk;

namespace {

constexpr int kThreads = 256;

// Tuning switches (compile time).  MINW: waves per SIMD the register budget
// is sized for (1: the full register file, one workgroup per CU, no spills).
// ATT_PF: attention tasks keep the next tile's loads in flight.
#ifndef ALTXS_PERSIST_MINW
#define ALTXS_PERSIST_MINW 1
#endif
#ifndef ALTXS_PERSIST_ATT_PF
#define ALTXS_PERSIST_ATT_PF 1
#endif
// A wait gives up after ~1 s of the 100 MHz wall clock (a step takes about a
// millisecond) and flags ALTXS_EDEV_SPIN; every other wait then sees the flag
// and returns at once, so the grid drains quickly with invalid results.
constexpr uint64_t kSpinTicks = 100000000ull;

#ifdef ALTXS_PERSIST_PROF
// Experiment hook (not part of the library build): per ticket the wall clock at
// task start, at the end of its dependency wait, at its end, and the stage.
__device__ uint64_t g_prof[1 << 17];
__shared__ uint64_t s_prof_wait;
#endif

// Wait until *ctr >= target (thread 0 polls), then make the producers' stores
// visible to every thread of the workgroup.
__device__ __forceinline__ void wait_ctr(const int* ctr, int target, int32_t* err) {
  if (threadIdx.x == 0) {
    const uint64_t t0 = (uint64_t)wall_clock64();
    int n = 0;
    while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      __builtin_amdgcn_s_sleep(1);
      if ((++n & 63) == 0) {
        if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & ALTXS_EDEV_SPIN) break;
        if ((uint64_t)wall_clock64() - t0 > kSpinTicks) {
          flag_err(err, ALTXS_EDEV_SPIN);
          break;
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // the barrier extends it to every wave
#ifdef ALTXS_PERSIST_PROF
    s_prof_wait = (uint64_t)wall_clock64();
#endif
  }
  __syncthreads();
}

struct CtrWait {
  const int* ctr;
  int target;
  int32_t* err;
  __device__ void operator()() const {
    if (ctr) wait_ctr(ctr, target, err);
  }
};

// Uniform (scalar) copies of values read from the plan.  The plan is reached
// through a pointer loaded from memory, so the compiler treats its fields as
// per-lane values; loops and branches that contain barriers (the GEMM
// column-tile loop, the dependency waits) must see scalars, or the compiler
// may build lane-split loops around the barriers.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float uni(float v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
template <class T>
__device__ __forceinline__ T* uni(T* p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
  return (T*)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ QT uni(const QT& q) {
  QT r;
  r.codes = uni(q.codes);
  r.scales = uni(q.scales);
  r.N = uni(q.N);
  r.K = uni(q.K);
  r.bits = uni(q.bits);
  return r;
}

template <int AM, int G>
struct Tasks {
  const PersistArgs& a;
  unsigned char* smem;

  __device__ int64_t rp() const { return (int64_t)a.nrt * 16; }
  __device__ const int* ctr(int s, int m, int st) const {
    return a.done + ((int64_t)s * a.nrt + m) * a.ctr_stride + st;
  }

  __device__ __forceinline__ void qkv(int s, int m, int nt) const {
    const SlotPlan& P = a.plan[s];
    const QT wq = uni(P.qkv);
    const int64_t Rp = rp(), D = a.D;
    const WS& w = a.w;
    const float* attn_in = uni(P.par) ? w.QIN + (s & 1) * Rp * D : w.XIN + (s & 1) * Rp * D;
    ProNorm pro{attn_in, nullptr, 0, uni(P.ln_scale), a.eps, a.D};
    pro.gate_w = (a.flags & ALTXS_F_SPARSE_GATE) ? uni(P.gate_w) : nullptr;
    pro.gate_out = w.GATE; pro.gate_scale = a.gate_scale; pro.H = a.H; pro.gw = a.gw;
    EpiQKV epi;
    epi.q = w.Q; epi.kv = a.kv + s * a.slot_kv_bytes; epi.kv_bf16 = 1; epi.H = a.H;
    epi.Hkv = a.Hkv; epi.W = a.W; epi.max_len = a.max_len; epi.rd = a.rd; epi.pos = a.pos;
    epi.cosb = a.rope_cos; epi.sinb = a.rope_sin; epi.q_gain = uni(P.q_gain); epi.eps = a.eps;
    epi.err = a.err;
    epi.rank = uni(P.lora_rank);
    if (epi.rank > 0) {
      epi.lqa = uni(P.lqa); epi.lqb = uni(P.lqb); epi.lva = uni(P.lva); epi.lvb = uni(P.lvb);
      epi.lora_s = uni(P.lora_s);
    }
    epi.D = a.D; epi.a_f32 = AM == A_F32 ? 1 : 0;
    const CtrWait wt{s > 0 ? ctr(s - 1, m, ST_DOWN) : nullptr, a.n_task[ST_DOWN], a.err};
    gemm_task<0, AM, 4, 1>(wq, a.R, 16 * m, nt, 1 << 30, ADirect{nullptr, 0}, pro, epi, smem, 0,
                           wt);
  }

  __device__ __forceinline__ void attn_g(int s, int r, int g) const {
    using altxs_attn::AttnP;
    using altxs_attn::MergeLds;
    const SlotPlan& P = a.plan[s];
    char* kv = a.kv + s * a.slot_kv_bytes;
    AttnP p;
    p.B = a.R / a.W; p.W = a.W; p.H = a.H; p.Hkv = a.Hkv; p.max_len = a.max_len;
    p.q = a.w.Q; p.k = kv; p.v = kv + (int64_t)a.Hkv * a.max_len * 64 * 2;
    p.seg_stride = 2ll * a.Hkv * a.max_len * 64; p.pos = a.pos;
    p.gate = (a.flags & ALTXS_F_SPARSE_GATE) ? a.w.GATE : nullptr;
    p.use_xsa = uni(P.use_xsa); p.y = a.w.Y; p.err = a.err; p.xcd_rows = 0;
    constexpr int NP = AM == A_BF16 ? 1 : 3;
    altxs_attn::attn_mfma_task<G, NP, AM == A_BF16 ? 1 : 0, ALTXS_PERSIST_ATT_PF>(
        p, r, g, *(MergeLds<G>*)smem);
  }

  __device__ __forceinline__ void attn(int s, int m, int k) const {
    wait_ctr(ctr(s, m, ST_QKV), a.n_task[ST_QKV], a.err);
    const int r = 16 * m + k / a.Hkv, g = k % a.Hkv;
    if (r >= a.R) return;
    attn_g(s, r, g);
  }

  template <int KS>
  __device__ __forceinline__ void o(int s, int m, int nt) const {
    const SlotPlan& P = a.plan[s];
    const WS& w = a.w;
    const int64_t Rp = rp(), D = a.D;
    EpiO epi{w.XIN + (s & 1) * Rp * D, uni(P.attn_scale), w.XOUT, a.D, uni(P.par)};
    const CtrWait wt{ctr(s, m, ST_ATT), a.n_task[ST_ATT], a.err};
    gemm_task<0, AM, 4 / KS, KS>(uni(P.o), a.R, 16 * m, nt, 1 << 30, ADirect{w.Y, 0}, ProNone{}, epi,
                                 smem, 0, wt);
  }

  template <int KS>
  __device__ __forceinline__ void up(int s, int m, int nt) const {
    const SlotPlan& P = a.plan[s];
    const WS& w = a.w;
    const int64_t Rp = rp(), D = a.D;
    const int par = uni(P.par);
    const float* lane1_in = par ? (uni(P.first_parallel) ? w.X0 + s * Rp * D : w.X1 + s * Rp * D)
                                : nullptr;
    ProNorm pro{par ? lane1_in : w.XOUT, nullptr, 0, uni(P.ln_scale), a.eps, a.D};
    EpiUp epi{w.HB, a.F, AM == A_BF16 ? 1 : 0};
    const CtrWait wt{ctr(s, m, ST_O), a.n_task[ST_O], a.err};
    gemm_task<0, AM, 4 / KS, KS>(uni(P.up), a.R, 16 * m, nt, 1 << 30, ADirect{nullptr, 0}, pro, epi,
                                 smem, 0, wt);
  }

  template <int KS>
  __device__ __forceinline__ void down(int s, int m, int nt) const {
    const SlotPlan& P = a.plan[s];
    const WS& w = a.w;
    const int64_t Rp = rp(), D = a.D;
    const int par = uni(P.par);
    const float* lane1_in = par ? (uni(P.first_parallel) ? w.X0 + s * Rp * D : w.X1 + s * Rp * D)
                                : nullptr;
    float* base_s = w.XIN + (s & 1) * Rp * D;
    EpiDown epi;
    epi.xout = w.XOUT; epi.mlp_scale = uni(P.mlp_scale);
    epi.out0 = w.X0 + (s + 1) * Rp * D; epi.out1 = w.X1 + (s + 1) * Rp * D;
    epi.lane0 = base_s; epi.lane1 = lane1_in; epi.pr = uni(P.par_resid); epi.pp = uni(P.par_post);
    epi.D = a.D; epi.parallel = par;
    if (uni(P.has_next)) {
      NextIn& nx = epi.next;
      const int src = uni(P.next_skip_src), npar = uni(P.next_par);
      nx.x0 = w.X0;
      nx.skip = src >= 0 ? w.X0 + (src + 1) * Rp * D : nullptr;
      nx.skip_w = uni(P.next_skip_w);
      nx.skip_g = uni(P.next_skip_g);
      nx.mix = uni(P.next_mix);
      nx.base = w.XIN + ((s + 1) & 1) * Rp * D;
      nx.attn = npar ? w.QIN + ((s + 1) & 1) * Rp * D : nx.base;
      nx.parallel = npar;
      nx.skip_self = uni(P.next_skip_self);
    }
    const CtrWait wt{ctr(s, m, ST_UP), a.n_task[ST_UP], a.err};
    gemm_task<0, AM, 4 / KS, KS>(uni(P.down), a.R, 16 * m, nt, 1 << 30, ADirect{w.HB, 0}, ProNone{},
                                 epi, smem, 0, wt);
  }
};

// Role-split schedule: GEMM workers and attention streamers (see PersistArgs).
// Each queue is consumed in an order consistent with one topological order of
// all tasks, so the smallest unfinished task always has a running worker of
// its role or is next in its queue: no deadlock while both roles have a
// resident workgroup (grid <= resident capacity; waits are bounded anyway).
template <int AM, int G, int KSO, int KSD>
__global__ __launch_bounds__(kThreads, ALTXS_PERSIST_MINW) void roles_kernel(const PersistArgs* __restrict__ pa) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ int s_task;
  const PersistArgs& a = *pa;
  const Tasks<AM, G> T{a, smem};
  if (threadIdx.x == 0) s_task = atomicAdd(a.role_ctr, 1);
  __syncthreads();
  const bool gemm = __builtin_amdgcn_readfirstlane(s_task) < a.ng;
  __syncthreads();
  int* const q = gemm ? a.gticket : a.aticket;
  const int nq = gemm ? a.n_gtask : a.n_atask;
  if (threadIdx.x == 0) s_task = atomicAdd(q, 1);
  __syncthreads();
  int t = __builtin_amdgcn_readfirstlane(s_task);
  const int nO = a.n_task[ST_O], nU = a.n_task[ST_UP], nD = a.n_task[ST_DOWN];
  while (t < nq) {
    int s, m, st, k;
    bool valid = true;
    if (gemm) {
      const int b = t / a.gblock;
      k = t - b * a.gblock;
      const int sp = b / a.nrt;
      m = b - sp * a.nrt;
      if (k < nO) { st = ST_O; s = sp - 1; }
      else if (k < nO + nU) { st = ST_UP; s = sp - 1; k -= nO; }
      else if (k < nO + nU + nD) { st = ST_DOWN; s = sp - 1; k -= nO + nU; }
      else { st = ST_QKV; s = sp; k -= nO + nU + nD; }
      valid = st == ST_QKV ? s < a.n_slots : s >= 0;
    } else {
      const int u = t / a.n_task[ST_ATT];
      k = t - u * a.n_task[ST_ATT];
      s = u / a.nrt;
      m = u - s * a.nrt;
      st = ST_ATT;
    }
#ifdef ALTXS_PERSIST_PROF
    uint64_t prof_t0 = 0;
    if (threadIdx.x == 0) prof_t0 = s_prof_wait = (uint64_t)wall_clock64();
#endif
    if (valid) {
      switch (st) {
        case ST_QKV: T.qkv(s, m, k); break;
        case ST_ATT: T.attn(s, m, k); break;
        case ST_O: T.template o<KSO>(s, m, k); break;
        case ST_UP: T.template up<KSO>(s, m, k); break;
        default: T.template down<KSD>(s, m, k); break;
      }
    }
    __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0): this wave's stores reached L2
    __syncthreads();
    if (threadIdx.x == 0) {
#ifdef ALTXS_PERSIST_PROF
      const int slot = gemm ? t : a.n_gtask + t;
      if (valid && slot < (1 << 15)) {
        g_prof[4 * slot] = prof_t0;
        g_prof[4 * slot + 1] = s_prof_wait;
        g_prof[4 * slot + 2] = (uint64_t)wall_clock64();
        g_prof[4 * slot + 3] = (uint64_t)st | ((uint64_t)s << 8) | ((uint64_t)m << 16) |
                               ((uint64_t)blockIdx.x << 24);
      }
#endif
      if (valid) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        // The release writes the XCD's L2 back (buffer_wbl2 sc1); the counter
        // may only move once that write-back has completed, or a consumer on
        // another XCD can read stale data from memory.  The compiled fence
        // was followed by no vmcnt wait before the atomic (the assembly of
        // this kernel showed buffer_wbl2 directly followed by the
        // flat_atomic_add), so the wait is spelled out here.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        atomicAdd(a.done + ((int64_t)s * a.nrt + m) * a.ctr_stride + st, 1);
      }
      s_task = atomicAdd(q, 1);
    }
    __syncthreads();
    t = __builtin_amdgcn_readfirstlane(s_task);
  }
}

template <int AM, int G, int KSO, int KSD>
size_t lds_bytes(const PersistArgs& a) {
  size_t b = task_lds_bytes<AM, 4, 1, ProNorm>(a.D);                 // QKV
  b = b > task_lds_bytes<AM, 4 / KSO, KSO, ProNorm>(a.D) ? b : task_lds_bytes<AM, 4 / KSO, KSO, ProNorm>(a.D);
  b = b > task_lds_bytes<AM, 4 / KSO, KSO, ProNone>(a.D) ? b : task_lds_bytes<AM, 4 / KSO, KSO, ProNone>(a.D);
  b = b > task_lds_bytes<AM, 4 / KSD, KSD, ProNone>(a.F) ? b : task_lds_bytes<AM, 4 / KSD, KSD, ProNone>(a.F);
  const size_t at = sizeof(altxs_attn::MergeLds<G>);
  return b > at ? b : at;
}

template <int AM, int G, int KSO, int KSD>
hipError_t launch_t(const PersistArgs& a, const PersistArgs* dev_args, int grid, hipStream_t s) {
  auto kfn = roles_kernel<AM, G, KSO, KSD>;
  const size_t lds = lds_bytes<AM, G, KSO, KSD>(a);
  static int resident = 0;  // workgroups that fit on the device at once (per instantiation)
  static size_t configured = 0;
  if (lds > 65536 && lds > configured) {
    hipError_t e = hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
    configured = lds;
  }
  if (resident == 0) {
    int dev = 0, per_cu = 0, cus = 0;
    hipError_t e;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
    if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess)
      return e;
    if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)kfn, kThreads, lds)) !=
        hipSuccess)
      return e;
    resident = (per_cu > 0 ? per_cu : 1) * cus;
  }
  // every workgroup resident at once, and at least one of each role
  int g = grid > 0 ? grid : resident;
  if (g > resident) g = resident;
  if (g <= a.ng || a.ng < 1) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(kfn, dim3(g), dim3(kThreads), lds, s, dev_args);
  return hipGetLastError();
}

}  // namespace

namespace altxs_sk {

hipError_t launch_persist(const PersistArgs& a, const PersistArgs* dev_args, int act_bf16, int ks_o,
                          int ks_d, int grid, hipStream_t s) {
  // one instantiation per (A mode, GQA group, K-splits): variant selection stays
  // outside the kernel so each compiles to the registers of its own code path
#define PERSIST_G(AMV, KO, KD)                                                        \
  if (ks_o == KO && ks_d == KD) {                                                     \
    if (a.G == 1) return launch_t<AMV, 1, KO, KD>(a, dev_args, grid, s);              \
    if (a.G == 2) return launch_t<AMV, 2, KO, KD>(a, dev_args, grid, s);              \
    if (a.G == 4) return launch_t<AMV, 4, KO, KD>(a, dev_args, grid, s);              \
  }
  if (act_bf16) {
    PERSIST_G(A_BF16, 1, 1) PERSIST_G(A_BF16, 1, 2) PERSIST_G(A_BF16, 1, 4)
    PERSIST_G(A_BF16, 2, 1) PERSIST_G(A_BF16, 2, 2) PERSIST_G(A_BF16, 2, 4)
  } else {
    PERSIST_G(A_F32, 1, 1) PERSIST_G(A_F32, 1, 2) PERSIST_G(A_F32, 1, 4)
    PERSIST_G(A_F32, 2, 1) PERSIST_G(A_F32, 2, 2) PERSIST_G(A_F32, 2, 4)
  }
#undef PERSIST_G
  return hipErrorInvalidValue;
}

}  // namespace altxs_sk

#ifdef ALTXS_PERSIST_PROF
extern "C" int altxs_prof_read(void* dst, int64_t n_u64) {
  return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_prof), (size_t)n_u64 * 8, 0, hipMemcpyDeviceToHost);
}
#endif
