// Shared host/device description of one MoE layer call.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace exl3m {

// Device-resident per-expert tensor table (the G5MoePrep equivalent, glm5.h:65-73):
// entries 0..E-1 are the routed experts, entry E the shared expert when it is a
// trellis. Index 0/1/2 = gate/up/down.
struct ExpertTab {
  const uint32_t *tr[3];
  const uint16_t *suh[3];
  const uint16_t *svh[3];
};

// Everything a kernel of one layer call needs, passed by value.
struct MoeArgs {
  // shape / config
  int N;       // token rows (B * L)
  int H;       // hidden
  int I;       // routed expert intermediate
  int SI;      // shared expert intermediate (0 = none)
  int Imax;    // max(I, SI): row stride of the per-slot intermediate buffers
  int E, topk, P, R;  // experts, top-k, pairs N*topk, run-table capacity min(E, P)
  int n_group, topk_group, norm_topk_prob;
  float routed_scaling_factor, swiglu_limit;
  int has_shared;
  int Sgu, Sdn;       // k-split counts of the gate/up and down partial planes (strides)
  int cnt_stride;     // counters per run
  // inputs
  const uint16_t *h;          // (N, H) f16
  const uint16_t *router_w;   // (E, H) f16
  const float *router_bias;   // (E) f32
  const ExpertTab *tab;       // E (+1) entries
  // workspace
  float *logits;       // (N, E)
  float *weights;      // (N, topk)
  int32_t *ids;        // (N, topk)
  int32_t *sorted_row;   // (P + N): slot -> token row; slots P.. are the shared rows
  int32_t *sorted_rank;  // (P + N): slot -> rank
  int32_t *slot;         // (P): pair b*topk + k -> slot
  int32_t *run_expert, *run_off, *run_len;  // (R)
  int32_t *n_runs;       // (1)
  float *gu_part;      // (P + N, 2, Sgu, Imax)
  uint16_t *act_hat;   // (P + N, Imax): rotated SwiGLU output = the down input xhat
  float *dn_part;      // (P + N, Sdn, H)
  uint16_t *yw;        // (P, H): f16(y * w) per slot
  uint16_t *sh_out;    // (N, H): shared expert output
  uint32_t *gu_cnt;    // (R + 1, cnt_stride)
  uint32_t *dn_cnt;    // (R + 1, cnt_stride)
  uint32_t *comb_cnt;  // (N, H / 128)
  int n_counters;      // total counter words (zeroed by the logits kernel)
  float *dsh_part;     // dense shared expert partials
  uint16_t *dsh_act;   // (N, SI) dense shared SwiGLU output
  uint16_t *out;       // (N, H)
};

}  // namespace exl3m
