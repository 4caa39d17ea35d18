// Shared host/device description of one MoE layer call.
//
// A decode call is six stream-ordered launches; every cross-workgroup dependency is
// a launch boundary (no device-scope fences or completion counters):
//   L1 k_moe_pre       router logits on the matrix cores (k-split partials)
//   L2 k_moe_route     split sums, top-k routing, expert-order dispatch, run table
//   L3 k_moe_gate_up   routed gate/up, one workgroup per (run, projection, 128-column
//                      block, k-slice); raw f32 slice partials per slot
//                      (+ the f16 shared expert's gate/up partials, extra workgroups)
//   L4 k_moe_act       per (slot, 128-block): slice sums, output Hadamards, SwiGLU with
//                      the clamp, the down input Hadamard (+ the f16 shared SwiGLU)
//   L5 k_moe_down      routed down, one workgroup per (run, 128-column block, k-slice);
//                      raw f32 slice partials per slot (+ the f16 shared down partials)
//   L6 k_moe_combine   per (token row, 128-column block): per rank, the slot's down
//                      slices summed in order, the output Hadamard (svh) and the routing
//                      weight; the ranks summed in order; + the shared expert
// A trellis shared expert runs the gate/up, act and down kernels on one extra "run"
// that holds every token row (three more launches; in long-run calls on the layer's
// second stream, forked after the dispatch and joined before L6).
// Calls of 32 rows or more add k_moe_rotate before L3 (each slot's gate/up input
// rotated once); calls of 65 rows or more take the long-run gate/up and down kernels
// over the pass table, and calls of 256 rows or more the tiled router logits kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "exl3_device.hpp"

namespace exl3m {

// Device-resident per-expert tensor table (the G5MoePrep equivalent, glm5.h:65-73):
// entries 0..E-1 are the routed experts, entry E the shared expert when it is a
// trellis. Index 0/1/2 = gate/up/down.
struct ExpertTab {
  const uint32_t *tr[3];
  const uint16_t *suh[3];
  const uint16_t *svh[3];
};

// One run of the dispatch as the short-run expert kernels read it, in one round of
// loads: the expert, its slots and first token row, and its tensors' pointers
// (p[2j] = trellis of projection j, p[2j + 1] = its suh, j = 0, 1; p[4] = the down
// trellis). Written by the dispatch from the expert table.
struct alignas(16) RunRec {
  int32_t e, off, len, row0;
  const void *p[6];
};

enum SharedKind { kSharedNone = 0, kSharedTrellis = 1, kSharedDense = 2 };

// Everything a kernel of one layer call needs, passed by value.
// Long-run mode (calls of at least EXL3_MOE_LONG_ROWS token rows, 65 by default): the
// expert kernels take passes of up to kLongBlocks 16-row MFMA blocks per decode.
constexpr int kLongBlocks = 4;
constexpr int kLongRows = 16 * kLongBlocks;

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
  int shared_kind;    // SharedKind
  int n_logit_blocks; // L1 workgroups computing router logits
  int logit_splits;   // k-split partials per logit (0: plain logits given by the caller)
  int fold;           // 1: expert kernels fold their k slices (one partial per output)
  int pass_rows;      // token rows per MFMA pass of the expert kernels (<= 16)
  int xrot_rows;      // 1: the short-run gate/up kernel copies the rows k_moe_rotate rotated
  int gu_items;       // 128-column blocks per short-run gate/up workgroup (one k slice)
  int dn_items;       // 128-column blocks per short-run down workgroup
  int weight_form;    // host side: the call's exl3_weight_form (the kernel codebooks)
  // inputs
  const uint16_t *h;          // (N, H) f16
  const uint16_t *router_w;   // (E, H) f16
  const float *router_bias;   // (E) f32
  const ExpertTab *tab;       // E (+1) entries
  const uint16_t *sh_dense[3];  // f16 shared expert weights, transposed (out, in), when dense
  // suh/svh of every expert stacked by expert (entry E: a trellis shared expert):
  // suh_s[0..1] (E + 1, H), svh_s[0..1] (E + 1, Imax), suh_s[2] (E + 1, Imax),
  // svh_s[2] (E + 1, H); an expert's scale is one load away from its id
  const uint16_t *suh_s[3];
  const uint16_t *svh_s[3];
  // workspace
  float *logits;       // (N, E, 8): router logit k-split partials, or (N, E) plain logits
  float *weights;      // (N, topk)
  int32_t *ids;        // (N, topk)
  int32_t *sorted_row;   // (P + N): slot -> token row; slots P.. are the shared rows
  int32_t *sorted_rank;  // (P + N): slot -> rank
  int32_t *slot_e;       // (P): slot -> expert
  int32_t *slot;         // (P): pair b*topk + k -> slot
  int32_t *run_expert, *run_off, *run_len;  // (R)
  int32_t *n_runs;
  RunRec *run_rec;       // (R) the runs with their pointers (short-run kernels)
  int32_t *pass_expert;  // (R + ceil(P / kLongRows)) runs cut into passes of <= kLongRows rows
  int32_t *pass_off;
  int32_t *pass_len;
  int32_t *n_passes;       // (1)
  int32_t *hist;           // (G, E): per-chunk expert counts of a many-workgroup dispatch
  float *yhat_gu;      // (P + N, 2, S, Imax): gate/up k-slice partials (S slices of H)
                       // before the output Hadamard
  uint16_t *act;       // (P + N, Imax): rotated SwiGLU output per slot, MFMA k order
  uint16_t *xrot;      // long-run mode or xrot_rows: (P + N, 2, H) f16 rotated gate/up
                       // inputs, staged order
  int S_dn;            // slot stride of yhat_dn in slices: max(slices(I), slices(SI))
  float *yhat_dn;      // (P + N, S_dn, H): down k-slice partials per slot, before the
                       // output Hadamard (slots P.. = a trellis shared expert)
  float *dsh_gu;       // (2, N, SI, 8): f16 shared gate/up k-split partials
  uint16_t *dsh_act;   // (N, SI): f16 shared expert SwiGLU output
  float *dsh_dn;       // (N, H, 8): f16 shared down k-split partials
  uint16_t *out;       // (N, H)
  // Optional hyper-connection mix behind the combine (g5_hc_mix): with hc_out set, the
  // combine also writes hc_out[row][n] = post[n] * out[row] + (comb^T @ residual)[n]
  int hc_n;                 // streams N
  const float *hc_post;     // (N_rows, hc_n) f32
  const float *hc_comb;     // (N_rows, hc_n, hc_n) f32
  const uint16_t *hc_res;   // (N_rows, hc_n, H) f16: the residual streams
  uint16_t *hc_out;         // (N_rows, hc_n, H) f16: the new streams, or NULL
};

// The hyper-connection mix (glm5_hc.cpp:342-355) of two adjacent elements d, d + 1 of one
// position, in the reference's f16 arithmetic (it runs in block_out's dtype): for every
// stream n, f16(f16(f16(post[n]) * b) + f16(sum_m f16(comb[m][n]) * residual[m])), the
// f16 products exact in f32 and the sum over m accumulated in f32 (a matmul's).
// res / out point at element d of stream 0; streams are D elements apart.
// The residual pairs are loaded once, up front (hc_mix_res), so that a caller can issue
// them long before the mix: rv[m] = stream m's pair, m < N <= kHcMixMax.
constexpr int kHcMixMax = 8;
__device__ __forceinline__ void hc_mix_res(const uint16_t *res, int D, int N, uint32_t (&rv)[kHcMixMax]) {
#pragma unroll
  for (int m = 0; m < kHcMixMax; ++m) rv[m] = *reinterpret_cast<const uint32_t *>(res + (int64_t)min(m, N - 1) * D);
}
__device__ __forceinline__ void hc_mix_pair(const float *post, const float *comb, const uint32_t (&rv)[kHcMixMax],
                                            int D, int N, float b0, float b1, uint16_t *out) {
  using exl3d::to_f16;
  auto h2f = [](uint32_t v) { return exl3d::f16_to_f32((uint16_t)v); };
  for (int n = 0; n < N; ++n) {
    const float pn = (float)to_f16(post[n]);
    const float a0 = (float)to_f16(pn * b0), a1 = (float)to_f16(pn * b1);
    float r0 = 0.0f, r1 = 0.0f;
#pragma unroll
    for (int m = 0; m < kHcMixMax; ++m)
      if (m < N) {
        const float cm = (float)to_f16(comb[m * N + n]);
        r0 = fmaf(cm, h2f(rv[m] & 0xffffu), r0);
        r1 = fmaf(cm, h2f(rv[m] >> 16), r1);
      }
    const float o0 = a0 + (float)to_f16(r0), o1 = a1 + (float)to_f16(r1);
    *reinterpret_cast<uint32_t *>(out + (int64_t)n * D) =
        (uint32_t)exl3d::bitcast<uint16_t>(to_f16(o0)) | ((uint32_t)exl3d::bitcast<uint16_t>(to_f16(o1)) << 16);
  }
}


// Column pair (c, c + 1) summed over n partial planes in plane order, p[0] + p[1] + ...
// (plane stride `stride` floats). MAXN planes are loaded at a time, unconditionally
// (plane indices clamped to n - 1, the extra values unused), before their adds: with
// no branch between them the loads are all in flight together. p: 8-byte aligned.
template <int MAXN>
__device__ __forceinline__ float2 ordered_sum2(const float *p, int64_t stride, int n) {
  float2 acc = make_float2(0.0f, 0.0f);
  for (int s0 = 0; s0 < n; s0 += MAXN) {
    float2 v[MAXN];
#pragma unroll
    for (int s = 0; s < MAXN; ++s)
      v[s] = *reinterpret_cast<const float2 *>(p + (int64_t)min(s0 + s, n - 1) * stride);
#pragma unroll
    for (int s = 0; s < MAXN; ++s) {
      if (s0 + s == 0) {
        acc = v[0];
      } else if (s0 + s < n) {
        acc.x += v[s].x;
        acc.y += v[s].y;
      }
    }
  }
  return acc;
}

}  // namespace exl3m
