// Types shared between the step's host orchestration (step.hip) and the
// persistent layer kernel (persist.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm.h"

namespace altxs_sk {

// Workspace pointers of one segment group.
struct WS {
  float *X0, *X1, *XIN, *QIN, *XOUT, *Q, *GATE;  // XIN, QIN: [2][Rp][D] (slot parity)
  void *Y, *HB;
  float2* STATS;
  int* SYNC;  // step counters (zeroed by the embedding kernel)
  int nsync;
  float* OPART;  // decode: the out-projection's per-head terms [Rp][H][D]
};

// One slot of the layer plan: everything a slot's tasks read besides the
// state.  Built once per model on the host (altxs_step_plan_build), like the
// reference's stacked persistent-step workspace (persistent_step.py:452-588).
struct SlotPlan {
  altxs::QT qkv, o, up, down;  // QT.bits: the run-time width of each tensor
  const float *resid_mix, *attn_scale, *mlp_scale, *q_gain, *gate_w, *par_resid, *par_post;
  float ln_scale;
  int use_xsa, par, first_parallel;
  // the following slot (inputs formed by this slot's DOWN); has_next == 0: last slot
  int has_next, next_par, next_skip_src, next_skip_self;
  const float *next_mix, *next_skip_w, *next_skip_g;
  // unmerged q/v LoRA of the slot (lora_rank 0: none)
  const uint16_t *lqa, *lqb, *lva, *lvb;
  float lora_s;
  int lora_rank;
};

enum : int { ST_QKV = 0, ST_ATT = 1, ST_O = 2, ST_UP = 3, ST_DOWN = 4, N_ST = 5 };

// Arguments of the persistent layer kernel (one segment group).
struct PersistArgs {
  const SlotPlan* plan;
  int n_slots, R, W, D, H, Hkv, F, max_len, rd, gw, flags, G;
  float eps, gate_scale;
  int nrt;               // 16-row tiles
  int n_task[N_ST];      // tasks of each stage per (slot, row tile)
  const int32_t* pos;
  char* kv;              // slot 0 of the group's first segment
  int64_t slot_kv_bytes;
  const float *rope_cos, *rope_sin;
  WS w;
  int* done;             // completed tasks of (slot s, row tile m, stage st) at
                         // done[(s * nrt + m) * ctr_stride + st]
  int ctr_stride;
  int32_t* err;
  // Roles: the first ng workgroups to start take GEMM tasks from one queue,
  // the others attention tasks from a second queue.
  // GEMM queue: blocks b = s' * nrt + m of gblock tickets holding O, UP, DOWN
  // of (s' - 1, m) then QKV of (s', m), for s' = 0 .. n_slots (entries of
  // slots outside [0, n_slots) are skipped).  Attention queue: (slot, row
  // tile)-major, 16 * Hkv tasks each.
  int ng, gblock, n_gtask, n_atask;
  int *role_ctr, *gticket, *aticket;
};

// Launch the persistent layer kernel on the arguments at dev_args (a device
// copy of `a`, which the host side reads for the launch shape): act_bf16
// selects the A operand mode, ks_o the K-split of the out-projection and
// MLP-up GEMMs (K = D), ks_d that of MLP-down (K = F).  grid <= 0: as many
// workgroups as can be resident (all of them must be; more than ng).
hipError_t launch_persist(const PersistArgs& a, const PersistArgs* dev_args, int act_bf16, int ks_o,
                          int ks_d, int grid, hipStream_t s);

}  // namespace altxs_sk
