// Expert launches of the MoE layer (grid set-up, steps in flight) and the input rotation
// and SwiGLU kernels between the expert kernels, gfx950. The expert kernels themselves
// are templates in moe_experts.hpp, instantiated in moe_experts_k*.hip.
#include "moe_experts.hpp"

using namespace exl3d;
using exl3m::MoeArgs;

namespace {

// Long-run mode: the input Hadamard of every (slot, projection) once, x_rot[slot][proj]
// = had_pre(h[row], suh of the slot's expert and projection) in the staged k order, so
// the gate/up workgroups of a pass (one per 256 output columns) copy it instead of each
// rotating it again. One wave per (slot, projection), kRotBatch 128-blocks at a time;
// slots [slot0, slot0 + n_slots): routed slots (below P, from the dispatch) or the N
// shared slots of a trellis shared expert (slot P + i is token row i, whatever the
// routing: so they can be rotated before the dispatch has run).
constexpr int kRotBatch = 8;

__global__ __launch_bounds__(256) void k_moe_rotate(MoeArgs a, int slot0, int n_slots) {
  const int lane = threadIdx.x & 63;
  const int nblk = a.H / 128;
  const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (gw >= (int64_t)n_slots * 2) return;
  const int proj = (int)(gw & 1);
  const int64_t slot = slot0 + (gw >> 1);
  const int e = slot < a.P ? a.slot_e[slot] : a.E;
  const int64_t row = slot < a.P ? a.sorted_row[slot] : slot - a.P;
  const uint16_t *hrow = a.h + row * a.H + 2 * lane;
  const uint16_t *suh = a.suh_s[proj] + (int64_t)e * a.H + 2 * lane;
  uint32_t *out = reinterpret_cast<uint32_t *>(a.xrot + (slot * 2 + proj) * a.H);
  for (int b0 = 0; b0 < nblk; b0 += kRotBatch) {
    uint32_t hx[kRotBatch], sx[kRotBatch];
#pragma unroll
    for (int q = 0; q < kRotBatch; ++q) {
      const int blk = min(b0 + q, nblk - 1);
      hx[q] = *reinterpret_cast<const uint32_t *>(hrow + blk * 128);
      sx[q] = *reinterpret_cast<const uint32_t *>(suh + blk * 128);
    }
    float v0[kRotBatch], v1[kRotBatch], s0[kRotBatch], s1[kRotBatch];
#pragma unroll
    for (int q = 0; q < kRotBatch; ++q) {
      v0[q] = lo16(hx[q]);
      v1[q] = hi16(hx[q]);
      s0[q] = lo16(sx[q]);
      s1[q] = hi16(sx[q]);
    }
    wave_had_pre_n<kRotBatch>(v0, v1, s0, s1);
#pragma unroll
    for (int q = 0; q < kRotBatch; ++q)
      if (b0 + q < nblk) stage_pair<false>(out, b0 + q, lane, pack16(v0[q], v1[q]));
  }
}

// One wave per (slot, 128-block of the intermediate): the gate/up slice partials
// summed in slice order, their output Hadamards (svh), SwiGLU with the swiglu_limit
// clamp (f16 op by op), and the down projection's input Hadamard (suh) -> act (f16, in
// the MFMA k order the down kernel stages). Routed slots come from the dispatch; in
// shared mode the slots P..P+N-1 of the trellis shared expert.
constexpr int kActThreads = 256;
constexpr int kActBatch = 4;  // (slot, block) items per wave of a long-run call

// Long-run calls (the gate/up slices already folded at slice position 0): a wave takes
// kActBatch consecutive (slot, block) items, issues all their loads before the first
// Hadamard and runs their rotations together; per item the arithmetic is k_moe_act's.
__device__ __forceinline__ void act_folded(const MoeArgs &a, int shared_mode, int64_t g0,
                                           int64_t n_items, int nblk) {
  const int lane = threadIdx.x & 63;
  const int gu_stride = n_slices(a.H / 16);
  int64_t slot[kActBatch];
  int blk[kActBatch], e[kActBatch];
  float2 vg[kActBatch], vu[kActBatch];
#pragma unroll
  for (int j = 0; j < kActBatch; ++j) {
    const int64_t item = min(g0 + j, n_items - 1);
    blk[j] = (int)(item % nblk);
    slot[j] = (shared_mode ? a.P : 0) + item / nblk;
    const int c = blk[j] * 128 + 2 * lane;
    vg[j] = *reinterpret_cast<const float2 *>(a.yhat_gu + (slot[j] * 2 + 0) * gu_stride * a.Imax + c);
    vu[j] = *reinterpret_cast<const float2 *>(a.yhat_gu + (slot[j] * 2 + 1) * gu_stride * a.Imax + c);
    e[j] = shared_mode ? a.E : a.slot_e[slot[j]];
  }
  uint32_t svg[kActBatch], svu[kActBatch], sud[kActBatch];
#pragma unroll
  for (int j = 0; j < kActBatch; ++j) {
    const int64_t so = (int64_t)e[j] * a.Imax + blk[j] * 128 + 2 * lane;
    svg[j] = *reinterpret_cast<const uint32_t *>(a.svh_s[0] + so);
    svu[j] = *reinterpret_cast<const uint32_t *>(a.svh_s[1] + so);
    sud[j] = *reinterpret_cast<const uint32_t *>(a.suh_s[2] + so);
  }
  float y0[2 * kActBatch], y1[2 * kActBatch], s0[2 * kActBatch], s1[2 * kActBatch];
#pragma unroll
  for (int j = 0; j < kActBatch; ++j) {
    y0[2 * j] = vg[j].x;
    y1[2 * j] = vg[j].y;
    y0[2 * j + 1] = vu[j].x;
    y1[2 * j + 1] = vu[j].y;
    s0[2 * j] = lo16(svg[j]);
    s1[2 * j] = hi16(svg[j]);
    s0[2 * j + 1] = lo16(svu[j]);
    s1[2 * j + 1] = hi16(svu[j]);
  }
  wave_had_post_n<2 * kActBatch>(y0, y1, s0, s1);
  const float L = rf16(a.swiglu_limit);
  float a0[kActBatch], a1[kActBatch], d0[kActBatch], d1[kActBatch];
#pragma unroll
  for (int j = 0; j < kActBatch; ++j) {
    a0[j] = swiglu1(rf16(y0[2 * j]), rf16(y0[2 * j + 1]), L);
    a1[j] = swiglu1(rf16(y1[2 * j]), rf16(y1[2 * j + 1]), L);
    d0[j] = lo16(sud[j]);
    d1[j] = hi16(sud[j]);
  }
  wave_had_pre_n<kActBatch>(a0, a1, d0, d1);
#pragma unroll
  for (int j = 0; j < kActBatch; ++j)
    if (g0 + j < n_items)
      stage_pair<false>(reinterpret_cast<uint32_t *>(a.act + slot[j] * a.Imax), blk[j], lane, pack16(a0[j], a1[j]));
}

__global__ __launch_bounds__(kActThreads) void k_moe_act(MoeArgs a, int shared_mode, int dense_blocks) {
  if ((int)blockIdx.x < dense_blocks) {
    shared_swiglu_block(a.dsh_gu, a.N, a.H, a.SI, a.swiglu_limit, a.dsh_act, blockIdx.x);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int in = shared_mode ? a.SI : a.I;
  const int nblk = in / 128;
  const int64_t gw = (int64_t)(blockIdx.x - dense_blocks) * (kActThreads / 64) + (threadIdx.x >> 6);
  const int n_slots = shared_mode ? a.N : a.P;
  if (a.fold) {
    const int64_t n_items = (int64_t)n_slots * nblk;
    if (gw * kActBatch < n_items) act_folded(a, shared_mode, gw * kActBatch, n_items, nblk);
    return;
  }
  if (gw >= (int64_t)n_slots * nblk) return;
  const int blk = (int)(gw % nblk);
  const int64_t slot = (shared_mode ? a.P : 0) + gw / nblk;
  const int gu_stride = n_slices(a.H / 16);       // slice positions per (slot, projection)
  const int gu_sl = a.fold ? 1 : gu_stride;        // partials to sum
  const float L = rf16(a.swiglu_limit);  // clipped always (glm5_moe.cpp:70-71)
  const int c = blk * 128 + 2 * lane;
  // the slice partials are loaded while the expert's scale pointers are fetched
  constexpr int kMaxSl = 8;
  const float *pg = a.yhat_gu + (slot * 2 + 0) * gu_stride * a.Imax + c;
  const float *pu = a.yhat_gu + (slot * 2 + 1) * gu_stride * a.Imax + c;
  float2 vg[kMaxSl], vu[kMaxSl];
  if (gu_sl == 1) {
    // long-run calls: the slices are already folded into slice position 0
    vg[0] = *reinterpret_cast<const float2 *>(pg);
    vu[0] = *reinterpret_cast<const float2 *>(pu);
  } else {
#pragma unroll
    for (int q = 0; q < kMaxSl; ++q) {
      const int64_t o = (int64_t)min(q, gu_sl - 1) * a.Imax;
      vg[q] = *reinterpret_cast<const float2 *>(pg + o);
      vu[q] = *reinterpret_cast<const float2 *>(pu + o);
    }
  }
  const int e = shared_mode ? a.E : a.slot_e[slot];
  const int64_t so = (int64_t)e * a.Imax;
  const uint16_t *svg_p = a.svh_s[0] + so, *svu_p = a.svh_s[1] + so, *sud_p = a.suh_s[2] + so;
  const uint32_t svg = *reinterpret_cast<const uint32_t *>(svg_p + c);
  const uint32_t svu = *reinterpret_cast<const uint32_t *>(svu_p + c);
  const uint32_t sud = *reinterpret_cast<const uint32_t *>(sud_p + c);
  float2 gs = vg[0], us = vu[0];
#pragma unroll
  for (int q = 1; q < kMaxSl; ++q)
    if (q < gu_sl) {
      gs.x += vg[q].x;
      gs.y += vg[q].y;
      us.x += vu[q].x;
      us.y += vu[q].y;
    }
  if (gu_sl > kMaxSl) {
    gs = exl3m::ordered_sum2<8>(pg, a.Imax, gu_sl);
    us = exl3m::ordered_sum2<8>(pu, a.Imax, gu_sl);
  }
  float g0 = gs.x, g1 = gs.y, u0 = us.x, u1 = us.y;
  float y0[2] = {g0, u0}, y1[2] = {g1, u1};
  const float s0[2] = {lo16(svg), lo16(svu)}, s1[2] = {hi16(svg), hi16(svu)};
  wave_had_post_n<2>(y0, y1, s0, s1);
  float a0 = swiglu1(rf16(y0[0]), rf16(y0[1]), L);
  float a1 = swiglu1(rf16(y1[0]), rf16(y1[1]), L);
  wave_had_pre(a0, a1, lo16(sud), hi16(sud));
  stage_pair<false>(reinterpret_cast<uint32_t *>(a.act + slot * a.Imax), blk, lane, pack16(a0, a1));
}

}  // namespace

namespace exl3h {

int moe_slices(int in) { return n_slices(in / 16); }

// Wave steps in flight: prefetch_steps(), or EXL3_MOE_PREFETCH (1, 2 or 4; capped by
// the slice length and, for K > 4, at 2), read once.
static int moe_prefetch(int k_tiles, int K) {
  static const int env = [] {
    const char *v = std::getenv("EXL3_MOE_PREFETCH");
    return v ? std::atoi(v) : 0;
  }();
  int pd = prefetch_steps(k_tiles, K);
  if (env == 1 || env == 2 || env == 4) pd = std::min(env, slice_steps(k_tiles));
  if (K > 4 && pd > 2) pd = 2;
  return pd;
}

// which: 0 = gate/up, 1 = down, over `runs` runs (routed: the dispatch's run table,
// bounded by R; shared_mode 1: the one trellis-shared run). cb is the kernel codebook
// (kernel_cb: the tensor codebook under the handle's weight form). dense: prepend the f16
// shared expert's workgroups for this projection (short-run kernels: whole z planes of
// the 3-D grid, the workgroups past the shared expert's tasks return at once).
exl3_status launch_moe_expert(int which, int K, int cb, int64_t runs, const MoeArgs &a,
                              int shared_mode, bool dense, hipStream_t st) {
  const int in = which == 0 ? a.H : (shared_mode ? a.SI : a.I);
  const int out = which == 0 ? (shared_mode ? a.SI : a.I) : a.H;
  const int n_sl = n_slices(in / 16);
  const int waves = a.fold ? kLongThreads / 64 : kGuThreads / 64;
  if ((a.fold ? long_lds(in, K, cb) : expert_lds(in, a.pass_rows, waves, K, cb)) > 128 * 1024)
    return fail(EXL3_ERR_UNSUPPORTED, "expert kernel LDS above 128 KB");
  const int items = which == 0 ? a.gu_items : a.dn_items;
  if (!a.fold && items < 1) return fail(EXL3_ERR_INVALID, "column blocks per expert workgroup below 1");
  const int groups = (out / 128 + items - 1) / items;  // short-run: column-block groups
  int64_t blocks;
  if (a.fold)
    blocks = runs * (which == 0 ? 2 : 1) * ((out / 32 + waves - 1) / waves);
  else
    blocks = runs * (which == 0 ? 2 : 1) * groups * n_sl;
  const int dense_blocks =
      !dense ? 0
             : (which == 0 ? shared_gate_up_blocks(a.N, a.H, a.SI, waves)
                           : shared_down_blocks(a.N, a.H, a.SI, waves));
  dim3 ub;
  int dense_arg = dense_blocks;
  if (a.fold) {
    blocks += dense_blocks;
    if (blocks == 0) return EXL3_OK;
    if (blocks > 0x7fffffff) return fail(EXL3_ERR_UNSUPPORTED, "expert launch too large");
    ub = dim3((unsigned)blocks);
  } else {
    // x = k-slice, y = column-block group, z = dense planes, then (run, projection)
    const int plane = n_sl * groups;
    const int dense_z = (dense_blocks + plane - 1) / plane;
    const int64_t z = runs * (which == 0 ? 2 : 1) + dense_z;
    if (z == 0) return EXL3_OK;
    if (z > 65535) return fail(EXL3_ERR_UNSUPPORTED, "expert launch too large");
    ub = dim3((unsigned)n_sl, (unsigned)groups, (unsigned)z);
    dense_arg = dense_z;
  }
  const int pd = a.fold ? std::min(moe_prefetch(in / 16, K), 2) : moe_prefetch(in / 16, K);
  exl3_status rc;
  if (K >= 1 && K <= 2) rc = launch_expert_k12(K, cb, pd, which, ub, st, a, shared_mode, dense_arg);
  else if (K <= 4) rc = launch_expert_k34(K, cb, pd, which, ub, st, a, shared_mode, dense_arg);
  else if (K <= 6) rc = launch_expert_k56(K, cb, pd, which, ub, st, a, shared_mode, dense_arg);
  else if (K <= 8) rc = launch_expert_k78(K, cb, pd, which, ub, st, a, shared_mode, dense_arg);
  else return fail(EXL3_ERR_INVALID, "K out of range");
  if (rc) return rc;
  EXL3_LAUNCHED(which == 0 ? "k_moe_gate_up" : "k_moe_down");
  return EXL3_OK;
}

// x_rot of slots [slot0, slot0 + n_slots): the P routed slots (after the dispatch) and,
// with a trellis shared expert, the N shared slots from P on (any time).
exl3_status launch_moe_rotate(const MoeArgs &a, int64_t slot0, int64_t n_slots, hipStream_t st) {
  const int64_t waves = n_slots * 2;
  if (waves == 0) return EXL3_OK;
  k_moe_rotate<<<(unsigned)((waves + 3) / 4), 256, 0, st>>>(a, (int)slot0, (int)n_slots);
  EXL3_LAUNCHED("k_moe_rotate");
  return EXL3_OK;
}

// Routed (shared_mode 0: P slots) or trellis-shared (shared_mode 1: N slots) SwiGLU
// activations, after `dense_blocks` workgroups of the f16 shared expert's SwiGLU.
exl3_status launch_moe_act(const MoeArgs &a, int shared_mode, int dense_blocks, hipStream_t st) {
  const int in = shared_mode ? a.SI : a.I;
  int64_t waves = (int64_t)(shared_mode ? a.N : a.P) * (in / 128);
  if (a.fold) waves = (waves + kActBatch - 1) / kActBatch;  // kActBatch items per wave
  const unsigned blocks = (unsigned)((waves + 3) / 4) + (unsigned)dense_blocks;
  if (blocks == 0) return EXL3_OK;
  k_moe_act<<<blocks, kActThreads, 0, st>>>(a, shared_mode, dense_blocks);
  EXL3_LAUNCHED("k_moe_act");
  return EXL3_OK;
}

}  // namespace exl3h
