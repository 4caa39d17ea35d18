// Routed (and trellis shared) expert kernels of the MoE layer, gfx950: the kernel
// templates and their launch helpers, included by moe_experts.hip (the grid set-up and
// the rotation and SwiGLU kernels) and by moe_experts_k*.hip, which instantiate the
// kernels of a few codebook widths K each (so that the instantiations compile in
// parallel).
//
// They replace the reference's per-bucket grouped launches (glm5_moe.cpp:329-405:
// hadamard-pre, grouped QMV, mx::sum over splits, hadamard-post, clip/sigmoid/
// multiply, take/concatenate). The device-side run table drives the grid: no host
// round trip, no member cap, and no cross-workgroup synchronisation inside a launch.
//
//  k_moe_gate_up  workgroup = (run, gate|up, 128-column block, k-slice of H), 4 waves:
//                 per pass of up to 16 token rows of the run, the input Hadamard of the
//                 slice's part of those rows into LDS, then one n-pair (32 columns) per
//                 wave over the slice on the MFMA core -> raw f32 slice partials in
//                 yhat_gu. Extra leading workgroups compute the f16 shared expert's
//                 gate/up partials.
//  k_moe_act      per (slot, 128-block): gate/up slice sums in order, output Hadamards
//                 (svh), SwiGLU with the swiglu_limit clamp (f16 op by op) and the down
//                 projection's input Hadamard (suh) -> act, in the MFMA k order.
//  k_moe_down     workgroup = (run, 128-column block of H, k-slice of the intermediate),
//                 4 waves, over act -> raw f32 slice partials in yhat_dn (the output
//                 Hadamard and the routing weight are applied by k_moe_combine). Extra
//                 leading workgroups compute the f16 shared expert's down partials.
//  *_long         calls of many rows: 64-row passes, every k slice in one workgroup,
//                 one accumulator chain per output over the whole k range;
//                 k_moe_rotate stages the rotated gate/up inputs once per (slot,
//                 projection).
//
// In the short-run kernels the arithmetic per token row and expert is
// exl3_trellis_linear's (same input Hadamard, k slices and slice order, output
// Hadamard), and the MFMA rows of a pass never mix, so a run of r rows gives the same
// bytes as r single-row calls, and a layer call the same bytes as its experts evaluated
// one linear at a time. The long-run kernels (the counterpart of the reference's staged
// path) accumulate over k in another association: within f32 round-off of it.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <type_traits>

#include "exl3_device.hpp"
#include "exl3_internal.hpp"
#include "moe_common.hpp"
#include "moe_dense.hpp"
#include "qmv_core.hpp"

using namespace exl3d;
using exl3m::MoeArgs;

namespace {

__device__ __forceinline__ float lo16(uint32_t v) { return (float)bitcast<f16>((uint16_t)(v & 0xffffu)); }
__device__ __forceinline__ float hi16(uint32_t v) { return (float)bitcast<f16>((uint16_t)(v >> 16)); }
__device__ __forceinline__ uint32_t pack16(float a, float b) { return pack_f16x2(a, b); }
__device__ __forceinline__ float rf16(float v) { return (float)to_f16(v); }

// A value every lane of the wave holds (a workgroup's run record, a staged row index),
// moved to a scalar register so that address arithmetic on it stays scalar.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
  return (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v) |
         ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32)) << 32);
}


constexpr int kGuThreads = 256;
constexpr int kDnThreads = 256;
// Waves per SIMD the short-run expert kernels are compiled for: 7 (<= 72 VGPRs) where
// that fits without spills (gate/up to K = 4, down to K = 5, whose LDS staging holds
// fewer registers), else 6 (<= 80).
template <int K>
constexpr int kGuWaves = K <= 4 ? 7 : 6;
template <int K>
constexpr int kDnWaves = K <= 5 ? 7 : 6;

struct RunInfo {
  int e, off, len;
};

// Workgroup = (run, projection, group of gu_items 128-column blocks, k-slice of H); 4
// waves, wave w owns n-pair 4*cb + w of each block cb of the group. Per pass of up to
// 16 token rows of the run: the input Hadamard of the slice's 128-blocks into LDS, then
// the slice of every block of the group in one ring-word stream per wave
// (qmv_slice_items), raw f32 partials to yhat_gu (summed in slice order by k_moe_act).
// Grid: x = k-slice, y = block group, z = dense_z planes of f16 shared-expert
// workgroups, then 2 * run + projection (a 3-D grid, so that no wave spends VALU on
// dividing its block index).
template <int K, int CB, int PD>
__global__ __launch_bounds__(kGuThreads) __attribute__((amdgpu_waves_per_eu(kGuWaves<K>, 8))) void k_moe_gate_up(MoeArgs a, int shared_mode, int dense_z) {
  extern __shared__ uint32_t smem[];
  if ((int)blockIdx.z < dense_z) {
    shared_gate_up_block(a.h, a.N, a.H, a.SI, a.sh_dense[0], a.sh_dense[1], a.dsh_gu,
                         (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x, kGuThreads / 64);
    return;
  }
  const int out = shared_mode ? a.SI : a.I;
  const int k_tiles = a.H / 16, ss = slice_steps(k_tiles), n_sl = gridDim.x;
  const int sl = blockIdx.x, cb0 = blockIdx.y * a.gu_items;
  const int items = min(a.gu_items, out / 128 - cb0);
  const int zz = blockIdx.z - dense_z;
  const int proj = zz & 1, u = zz >> 1;
  RunInfo ri;
  int row0;
  const uint32_t *base;
  const uint16_t *suh;
  if (shared_mode) {
    if (u > 0) return;
    ri = RunInfo{a.E, a.P, a.N};
    row0 = 0;
    base = a.tab[a.E].tr[proj];
    suh = a.tab[a.E].suh[proj];
  } else {
    // the run count and the run's record in one round of loads (the exit test reads
    // every loaded word, so none of the loads waits for it)
    const int nruns = *a.n_runs;
    const exl3m::RunRec *rr = a.run_rec + min(u, a.R - 1);
    const int4 hd = *reinterpret_cast<const int4 *>(rr);
    const ulonglong2 pp = *reinterpret_cast<const ulonglong2 *>(&rr->p[2 * proj]);
    if (u >= nruns || hd.z <= 0 || pp.x == 0 || pp.y == 0) return;
    // the record is the workgroup's: in scalar registers
    ri = RunInfo{uniform(hd.x), uniform(hd.y), uniform(hd.z)};
    row0 = uniform(hd.w);
    base = reinterpret_cast<const uint32_t *>(uniform64(pp.x));
    suh = reinterpret_cast<const uint16_t *>(uniform64(pp.y));
  }
  constexpr bool kDup = dup_cb(CB);
  // the wave index is uniform: in a scalar register, address arithmetic built on it
  // stays scalar
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int slice_k = kStepTiles * ss * 16;  // k values per slice
  const int nblk = slice_k / 128;           // a power of two (slice_steps)
  const int nblk_lg = __builtin_ctz(nblk);
  const int xs_stride = staged_row_words(k_tiles, kDup);  // words per staged row
  const int k_base = sl * slice_k;
  uint32_t *xs = smem;
  u32x4 *slot = reinterpret_cast<u32x4 *>(smem + a.pass_rows * xs_stride) + wave * slot_chunks(K);

  SliceStream<K, PD> S;
  for (int p0 = 0; p0 < ri.len; p0 += a.pass_rows) {
    const int nr = min(a.pass_rows, ri.len - p0);
    // the slice's first ring words are in flight while the rows are staged
    S.start(base, k_tiles, out / 16, sl * kStepTiles * ss, cb0 * 4 + wave);
    if (a.xrot_rows) {
      // rows already rotated by k_moe_rotate (x_rot of this projection, staged k
      // order): 16-byte copies of the slice
      const int q_row = slice_k / 8, q_lg = __builtin_ctz(q_row);  // 16-byte chunks per row
      for (int i = threadIdx.x; i < nr * q_row; i += kGuThreads) {
        const int r = i >> q_lg, q = i & (q_row - 1);
        stage_chunk<kDup>(xs + r * xs_stride, q, reinterpret_cast<const uint4 *>(
            a.xrot + ((int64_t)(ri.off + p0 + r) * 2 + proj) * a.H + k_base)[q]);
      }
    } else {
      for (int bi = wave; bi < nr * nblk; bi += kGuThreads / 64) {
        const int r = bi >> nblk_lg, blk = bi & (nblk - 1);
        // shared slots hold the rows in order; a run's first row is in its record
        const int row = shared_mode ? p0 + r : (p0 + r == 0 ? row0 : uniform(a.sorted_row[ri.off + p0 + r]));
        const int kc = k_base + blk * 128 + 2 * lane;
        const uint32_t hx = *reinterpret_cast<const uint32_t *>(a.h + (int64_t)row * a.H + kc);
        const uint32_t sx = *reinterpret_cast<const uint32_t *>(suh + kc);
        float v0 = lo16(hx), v1 = hi16(hx);
        wave_had_pre(v0, v1, lo16(sx), hi16(sx));
        stage_pair<kDup>(xs + r * xs_stride, blk, lane, pack16(v0, v1));
      }
    }
    __syncthreads();
    float *yp = a.yhat_gu + ((int64_t)((ri.off + p0) * 2 + proj) * n_sl + sl) * a.Imax + cb0 * 128 + wave * 32;
    const int row_stride = 2 * n_sl * a.Imax;  // a slot's partials: well below 2^31 floats
    qmv_slice_items<K, CB, PD>(S, ss, items, xs + min(lane & 15, nr - 1) * xs_stride, slot,
                               [=](int it, const f32x4 &D0, const f32x4 &D1) {
#pragma unroll
                                 for (int i = 0; i < 4; ++i) {
                                   const int r = d_row(i);
                                   if (r < nr) {
                                     const int o = r * row_stride + it * 128;
                                     yp[o + d_col(0)] = D0[i];
                                     yp[o + d_col(1)] = D1[i];
                                   }
                                 }
                               });
    __syncthreads();
  }
}

// Workgroup = (run, group of dn_items 128-column blocks of H, k-slice of the
// intermediate), 4 waves, wave w owns n-pair 4*cb + w of each block cb of the group. Per
// pass of up to 16 token rows: the rows' rotated SwiGLU outputs (k_moe_act, already in
// the MFMA k order) for the slice into LDS, then the slice of every block of the group
// in one stream per wave, raw f32 partials to yhat_dn (the output Hadamard and the
// routing weight are applied by k_moe_combine). Grid: x = k-slice, y = block group,
// z = dense_z planes of f16 shared-expert workgroups, then the run.
template <int K, int CB, int PD>
__global__ __launch_bounds__(kDnThreads) __attribute__((amdgpu_waves_per_eu(kDnWaves<K>, 8))) void k_moe_down(MoeArgs a, int shared_mode, int dense_z) {
  extern __shared__ uint32_t smem[];
  if ((int)blockIdx.z < dense_z) {
    shared_down_block(a.dsh_act, a.N, a.H, a.SI, a.sh_dense[2], a.dsh_dn,
                      (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x, kDnThreads / 64);
    return;
  }
  const int in = shared_mode ? a.SI : a.I;
  const int k_tiles = in / 16, ss = slice_steps(k_tiles);
  const int sl = blockIdx.x, cb0 = blockIdx.y * a.dn_items, u = blockIdx.z - dense_z;
  const int items = min(a.dn_items, a.H / 128 - cb0);
  RunInfo ri;
  const uint32_t *base;
  if (shared_mode) {
    if (u > 0) return;
    ri = RunInfo{a.E, a.P, a.N};
    base = a.tab[a.E].tr[2];
  } else {
    const int nruns = *a.n_runs;
    const exl3m::RunRec *rr = a.run_rec + min(u, a.R - 1);
    const int4 hd = *reinterpret_cast<const int4 *>(rr);
    const uint64_t p4 = *reinterpret_cast<const uint64_t *>(&rr->p[4]);
    if (u >= nruns || hd.z <= 0 || p4 == 0) return;
    ri = RunInfo{uniform(hd.x), uniform(hd.y), uniform(hd.z)};
    base = reinterpret_cast<const uint32_t *>(uniform64(p4));
  }
  constexpr bool kDup = dup_cb(CB);
  // the wave index is uniform: in a scalar register, address arithmetic built on it
  // stays scalar
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int slice_k = kStepTiles * ss * 16;
  const int xs_stride = staged_row_words(k_tiles, kDup);  // words per staged row
  uint32_t *xs = smem;
  u32x4 *slot = reinterpret_cast<u32x4 *>(smem + a.pass_rows * xs_stride) + wave * slot_chunks(K);

  SliceStream<K, PD> S;
  for (int p0 = 0; p0 < ri.len; p0 += a.pass_rows) {
    const int nr = min(a.pass_rows, ri.len - p0);
    S.start(base, k_tiles, a.H / 16, sl * kStepTiles * ss, cb0 * 4 + wave);
    const int q_row = slice_k / 8;  // 16-byte chunks of act per row (a power of two)
    const int q_lg = __builtin_ctz(q_row);
    for (int i = threadIdx.x; i < nr * q_row; i += kDnThreads) {
      const int r = i >> q_lg, q = i & (q_row - 1);
      stage_chunk<kDup>(xs + r * xs_stride, q, reinterpret_cast<const uint4 *>(
          a.act + (int64_t)(ri.off + p0 + r) * a.Imax + sl * slice_k)[q]);
    }
    __syncthreads();
    float *yp = a.yhat_dn + ((int64_t)(ri.off + p0) * a.S_dn + sl) * a.H + cb0 * 128 + wave * 32;
    const int row_stride = a.S_dn * a.H;
    qmv_slice_items<K, CB, PD>(S, ss, items, xs + min(lane & 15, nr - 1) * xs_stride, slot,
                               [=](int it, const f32x4 &D0, const f32x4 &D1) {
#pragma unroll
                                 for (int i = 0; i < 4; ++i) {
                                   const int r = d_row(i);
                                   if (r < nr) {
                                     const int o = r * row_stride + it * 128;
                                     yp[o + d_col(0)] = D0[i];
                                     yp[o + d_col(1)] = D1[i];
                                   }
                                 }
                               });
    __syncthreads();
  }
}

// Long runs (calls of 65 token rows or more): 8-wave workgroups, wave w owns n-pair
// 8*cb + w, passes of up to kLongRows rows with up to kLongBlocks 16-row MFMA blocks
// per decode (qmv_slice_rb over the pass's occupied blocks only), and every k slice of
// the tensor in one workgroup: each block's accumulators run on from the first k step
// to the last (the reference's staged path likewise sums in its own association, within
// 1% of max |value| of its QMV by its test, glm5_gemv_nt_test.cpp:221-247). One partial
// per output goes to slice position 0.
using exl3m::kLongBlocks;
using exl3m::kLongRows;
constexpr int kLongThreads = 512;
// Staging loads in flight per lane: a slice of 64 plain rows is 64 x 64 chunks, 8 per
// thread (two rounds of 4); a 4-step part of duplicated rows (the halves form) 64 x 32,
// 4 per thread (one round).
constexpr int kStageBatchGu = 4;
constexpr int kStageBatchDn = 4;

// Stages one part of a pass's rows into LDS: rows [0, nr) of the source, row r at byte
// r * row_bytes of `src` (a buffer resource that covers exactly those nr rows), their
// 16-byte chunks [kbyte0 / 16, kbyte0 / 16 + q_row) into staged rows xs + r * xs_stride.
// Thread t takes chunk t % q_row of rows t / q_row + j * (kLongThreads / q_row) (q_row a
// power of two that divides kLongThreads), so that its source offset and LDS row only
// step by whole rows; kBatch loads are issued before the first LDS store. A load of a row
// at or past nr falls outside the resource and reads zero (no address clamps).
template <bool kDup, int kBatch>
__device__ __forceinline__ void stage_part(__amdgpu_buffer_rsrc_t src, uint32_t row_bytes, uint32_t kbyte0,
                                           int q_row, int q_lg, int nr, uint32_t *xs, int xs_stride) {
  // the thread's offsets are derived afresh at each call (the empty volatile asm keeps the
  // compiler from hoisting them out of the slice loop, where they would hold VGPRs across
  // the MFMA loop)
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int cq = tid & (q_row - 1);
  const int r0 = tid >> q_lg;
  const int rstep = kLongThreads >> q_lg;
  const uint32_t vstep = (uint32_t)rstep * row_bytes;
  uint32_t vo = (uint32_t)r0 * row_bytes + (uint32_t)cq * 16 + kbyte0;
  uint32_t *dst = xs + r0 * xs_stride;
  const int dstep = rstep * xs_stride;
  for (int r = r0; r < nr; r += kBatch * rstep) {
    uint4 c[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q)
      c[q] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src, vo + q * vstep, 0, 0));
#pragma unroll
    for (int q = 0; q < kBatch; ++q)
      if (r + q * rstep < nr) stage_chunk<kDup>(dst + q * dstep, cq, c[q]);
    vo += kBatch * vstep;
    dst += kBatch * dstep;
  }
}

// Runs pass(std::integral_constant<int, NRB>) with NRB = the pass's occupied 16-row
// blocks, (nr + 15) / 16 of the kLongBlocks: a short pass computes no MFMAs and reads no
// A operands for its empty blocks (whose rows are never stored). Each block count is its
// own copy of the pass, so the accumulators of the blocks it has are all it holds.
template <typename F>
__device__ __forceinline__ void with_blocks(int nr, F &&pass) {
  static_assert(kLongBlocks == 4, "one case per block count");
  switch ((nr + 15) >> 4) {
    case 1: pass(std::integral_constant<int, 1>{}); break;
    case 2: pass(std::integral_constant<int, 2>{}); break;
    case 3: pass(std::integral_constant<int, 3>{}); break;
    default: pass(std::integral_constant<int, 4>{});
  }
}

// Double-buffered staging for the reference form (plain rows, one f16 per k-element):
// passes run in parts of up to kDbSteps wave steps, and part t + 1's rows are copied into
// the other of two LDS buffers by the 16-byte direct-to-LDS buffer load (lane i's 16
// bytes land at the row's LDS address + 16 i, no register holds them) while part t is
// decoded: one barrier per part, and the ring-word stream runs over the whole k range
// with no break at the part boundaries. The buffers are two objects, so that the
// compiler, which tracks the copies, does not hold reads of one buffer back for the copy
// into the other. Every step meets the same A operands and accumulators as in the
// single-buffered form, in the same order.
constexpr int kDbSteps = 4;
constexpr int kDbRowWords = kStepTiles * kDbSteps * 8 + 4;  // a part row + 4 words (bank offset)
constexpr int kDbBufWords = kLongRows * kDbRowWords;
static_assert(kLongThreads == 512, "eight waves copy a part's rows, wave + 8i");
typedef __attribute__((address_space(3))) void lds_void_t;
// The two part buffers: LDS of the plain-form long-run kernels only, the kernels that
// reference them.
__shared__ __align__(16) uint32_t g_db_a[kDbBufWords];
__shared__ __align__(16) uint32_t g_db_b[kDbBufWords];

// This wave's rows of a part (rows wave + 8i below nr): 16-byte chunks [0, q_row) of each
// row from byte kbyte0 of the row, into buf.
__device__ __forceinline__ void db_issue(__amdgpu_buffer_rsrc_t src, uint32_t row_bytes, uint32_t kbyte0,
                                         int q_row, int nr, uint32_t *buf) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < kLongRows / 8; ++i) {
    const int r = wave + 8 * i;
    if (r < nr && lane < q_row)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(src, (lds_void_t *)(buf + r * kDbRowWords), 16,
                                               (uint32_t)r * row_bytes + kbyte0 + 16u * (uint32_t)lane, 0, 0, 0);
  }
}

// One pass of up to 16 * NRB rows (nr >= 1) of a plain-form tensor over its whole k range
// into D (from zero): rows from src (row r at byte r * row_bytes, in the staged k order),
// ring words of n-pair np from base; active = this wave has an n-pair (idle waves copy
// rows and meet the barriers). Ends with a barrier, so the buffers are free afterwards.
template <int K, int CB, int PD, int NRB, int kPart>
__device__ __forceinline__ void long_pass_db_parts(const uint32_t *base, int k_tiles, int tiles_n, int np,
                                                   bool active, __amdgpu_buffer_rsrc_t src, uint32_t row_bytes,
                                                   int nr, u32x4 *slot, f32x4 (&D)[NRB][2], uint32_t *dbA,
                                                   uint32_t *dbB) {
  static_assert(!dup_cb(CB), "plain rows only");
  static_assert(kPart <= kDbSteps && kPart % PD == 0, "part steps");
  constexpr int kTw = tile_words(false);
  const int total = k_tiles / kStepTiles;                   // wave steps over the k range
  const int n_parts = total / kPart;
  constexpr int q_row = kPart * kStepTiles * kTw / 4;       // 16-byte chunks of a part row
  constexpr uint32_t part_bytes = 16u * q_row;
  // part 0's copies before the stream's first loads: the copies of a part are always
  // older than the ring loads in flight when the part's wait comes (below)
  db_issue(src, row_bytes, 0, q_row, nr, dbA);
  SliceStream<K, PD> S;
  if (active) S.start(base, k_tiles, tiles_n, 0, np);
  const StepLane sl = step_lane();
  const int lane = threadIdx.x & 63;
  const int wbase = (sl.kt * 2 + sl.nt) * 8 * K;
  // block r's A operands: staged row 16r + l % 16 (rows past nr hold stale values: their
  // MFMA rows are never stored, and an MFMA row depends on its own A row only), so the
  // blocks' offsets differ by constants that fold into the LDS reads
  const int xo0 = (lane & 15) * kDbRowWords + sl.kt * kTw;
  int xo[NRB];
#pragma unroll
  for (int r = 0; r < NRB; ++r) {
    xo[r] = xo0 + 16 * r * kDbRowWords;
    D[r][0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    D[r][1] = D[r][0];
  }
  // Loads complete in issue order. When part t's wait comes, a wave that decodes has
  // exactly PD steps of ring loads in flight (PD * (K > 4 ? 2 : 1) loads), all issued
  // after its copies of part t (at the start of part t - 1, or before the stream began):
  // waiting until no more than those are outstanding completes the copies; an idle wave
  // waits for everything. After the barrier every wave's copies of part t are in LDS, and
  // no wave reads the other buffer (part t - 1) any more.
  constexpr int kInFlight = PD * (K > 4 ? 2 : 1);
  static_assert(kInFlight < 16, "vmcnt field");
  auto run_part = [&](int t, uint32_t *cur, uint32_t *nxt) {
    if (active)
      __builtin_amdgcn_s_waitcnt(0x0F70 | kInFlight);  // vmcnt(kInFlight), expcnt/lgkmcnt unchecked
    else
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    // The workgroup barrier without __syncthreads' fences, which count the copies as LDS
    // writes and wait for every load in flight (vmcnt(0)), the ring words of the next
    // steps included. The copies are complete by the wait above; this wave's LDS reads of
    // the previous part have all been consumed by its MFMAs; the empty asm statements
    // keep the compiler from moving memory operations across the barrier.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (t + 1 < n_parts) db_issue(src, row_bytes, (uint32_t)(t + 1) * part_bytes, q_row, nr, nxt);
    if (active) {
#pragma unroll
      for (int sb = 0; sb < kPart; sb += PD) {
#pragma unroll
        for (int b = 0; b < PD; ++b) {
          uint32_t W[K + 1];
          step_words<K>(slot, wbase, sl.m, S.L[b], W);
          // past the last step: lane offsets beyond the tensor (zeros, no memory access),
          // so that every step issues the same loads
          const int nx = t * kPart + sb + b + PD;
          const bool past = nx >= total;
          step_load<K>(S.rsrc, past ? S.vo0 + kPastEnd : S.vo0, past ? S.vo1 + kPastEnd : S.vo1,
                       past ? 0u : S.so0 + (uint32_t)nx * S.step_bytes, S.L[b]);
          mfma_step_rb<K, CB, NRB>(W, cur + (sb + b) * (kStepTiles * kTw), xo, D);
        }
      }
    }
  };
  for (int t = 0; t < n_parts; t += 2) {
    run_part(t, dbA, dbB);
    if (t + 1 < n_parts) run_part(t + 1, dbB, dbA);
  }
  __syncthreads();
}

// Parts of 4 wave steps where they divide the k range, else of 2 (a tensor's k range is
// a multiple of 128, 2 wave steps): a part's steps unrolled, so that the loads in flight
// at each part's wait are known to the compiler as they are to the wait.
template <int K, int CB, int PD, int NRB>
__device__ __forceinline__ void long_pass_db(const uint32_t *base, int k_tiles, int tiles_n, int np, bool active,
                                             __amdgpu_buffer_rsrc_t src, uint32_t row_bytes, int nr,
                                             u32x4 *slot, f32x4 (&D)[NRB][2], uint32_t *dbA, uint32_t *dbB) {
  if ((k_tiles / kStepTiles) % kDbSteps == 0)
    long_pass_db_parts<K, CB, PD, NRB, kDbSteps>(base, k_tiles, tiles_n, np, active, src, row_bytes, nr, slot, D,
                                                 dbA, dbB);
  else
    long_pass_db_parts<K, CB, PD, NRB, 2>(base, k_tiles, tiles_n, np, active, src, row_bytes, nr, slot, D, dbA,
                                          dbB);
}

// Work unit u of the long-run kernels: pass u of the dispatch's pass table, or (shared
// mode) rows [u * kLongRows, u * kLongRows + kLongRows) of the trellis shared expert.
__device__ __forceinline__ bool pass_info(const MoeArgs &a, int u, int shared_mode, RunInfo &ri) {
  if (shared_mode) {
    if (u * kLongRows >= a.N) return false;
    ri.e = a.E;
    ri.off = a.P + u * kLongRows;
    ri.len = min(kLongRows, a.N - u * kLongRows);
    return true;
  }
  if (u >= *a.n_passes) return false;
  ri.e = a.pass_expert[u];
  ri.off = a.pass_off[u];
  ri.len = a.pass_len[u];
  return true;
}

// Workgroup b of the long-run grid -> its work item: the workgroups of one pass (and the
// passes of one expert, which follow each other) on one XCD, which then reads the pass's
// rows and the expert's weights through its own L2. Workgroups go to the 8 XCDs in turn
// (b % 8), each XCD taking its workgroups in b order; of the T live items [0, T), XCD
// class x takes a contiguous range, item x * (T / 8) + min(x, T % 8) + b / 8. Returns -1
// for b >= T (no work: the grid is sized for the most passes a call can have).
__device__ __forceinline__ int long_item(int b, int per_unit, int shared_mode, const MoeArgs &a) {
  const int units = shared_mode ? (a.N + kLongRows - 1) / kLongRows : *a.n_passes;
  const int T = units * per_unit;
  if (b >= T) return -1;
  const int x = b & 7, q = T >> 3, r = T & 7;
  return x * q + min(x, r) + (b >> 3);
}

template <int K, int CB, int PD>
__global__ __launch_bounds__(kLongThreads) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_moe_gate_up_long(MoeArgs a, int shared_mode, int dense_blocks) {
  extern __shared__ uint32_t smem[];
  constexpr int kWaves = kLongThreads / 64;
  if ((int)blockIdx.x < dense_blocks) {
    shared_gate_up_block(a.h, a.N, a.H, a.SI, a.sh_dense[0], a.sh_dense[1], a.dsh_gu, blockIdx.x,
                         kWaves);
    return;
  }
  const int out = shared_mode ? a.SI : a.I;
  const int n_np = out / 32, n_cb = (n_np + kWaves - 1) / kWaves;
  const int k_tiles = a.H / 16, ss = slice_steps(k_tiles), n_sl = n_slices(k_tiles);
  int b = long_item(blockIdx.x - dense_blocks, 2 * n_cb, shared_mode, a);
  if (b < 0) return;
  const int cb = b % n_cb;
  b /= n_cb;
  const int proj = b & 1, u = b >> 1;
  RunInfo ri;
  if (!pass_info(a, u, shared_mode, ri)) return;
  const exl3m::ExpertTab &tb = a.tab[ri.e];
  const uint32_t *base = tb.tr[proj];
  // uniform across the wave: in a scalar register, so that branches on it are scalar
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int np = cb * kWaves + wave;
  const bool active = np < n_np;  // idle waves still stage rows and meet the barriers
  constexpr bool kDup = dup_cb(CB);
  const int part = long_part_steps(k_tiles, kDup), n_parts = ss / part;
  const int part_k = kStepTiles * part * 16;
  const int xs_stride = long_row_words(k_tiles, kDup);
  // plain rows: the double buffers are static, the dynamic LDS holds the slots only
  uint32_t *xs = smem;
  u32x4 *slot = reinterpret_cast<u32x4 *>(smem + (kDup ? kLongRows * xs_stride : 0)) + wave * slot_chunks(K);

  const int q_row = part_k / 8;  // 16-byte chunks of xrot per row and part (a power of two)
  const int q_lg = __builtin_ctz(q_row);
  const uint32_t row_bytes = 4u * a.H;  // x_rot rows of a slot: gate's, then up's
  for (int p0 = 0; p0 < ri.len; p0 += kLongRows) {
    const int nr = min(kLongRows, ri.len - p0);
    // this projection's x_rot rows of the pass's slots (already rotated by k_moe_rotate,
    // in the staged k order)
    const __amdgpu_buffer_rsrc_t src = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.xrot + ((int64_t)(ri.off + p0) * 2 + proj) * a.H), (short)0, (int)(nr * row_bytes), 0x00020000);
    with_blocks(nr, [&](auto nrb) {
      constexpr int NRB = decltype(nrb)::value;
      f32x4 D[NRB][2];
      if constexpr (!kDup) {
        long_pass_db<K, CB, PD, NRB>(base, k_tiles, out / 16, np, active, src, row_bytes, nr, slot, D, g_db_a,
                                     g_db_b);
      } else
      for (int sl = 0; sl < n_sl; ++sl) {
        for (int pt = 0; pt < n_parts; ++pt) {
          const int k0 = (sl * n_parts + pt) * part_k;
          stage_part<kDup, kStageBatchGu>(src, row_bytes, 2u * k0, q_row, q_lg, nr, xs, xs_stride);
          __syncthreads();
          if (active)
            qmv_slice_rb<K, CB, PD, NRB>(base, k_tiles, out / 16, k0 / 16, np, part, xs, xs_stride, nr, slot,
                                         D, sl == 0 && pt == 0);
          __syncthreads();
        }
      }
      if (active) {
        const int col = np * 32;
        // the lane's first row, read here (not hoisted out of the pass loop, where the
        // rows of every block would each hold a VGPR through the decode)
        int lr = threadIdx.x;
        asm volatile("" : "+v"(lr));
        lr = 4 * ((lr & 63) >> 4);
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 16 * rb + lr + i;
            if (r < nr) {
              float *y = a.yhat_gu + (int64_t)((ri.off + p0 + r) * 2 + proj) * n_sl * a.Imax + col;
              y[d_col(0)] = D[rb][0][i];
              y[d_col(1)] = D[rb][1][i];
            }
          }
      }
    });
  }
}

template <int K, int CB, int PD>
__global__ __launch_bounds__(kLongThreads) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_moe_down_long(MoeArgs a, int shared_mode, int dense_blocks) {
  extern __shared__ uint32_t smem[];
  constexpr int kWaves = kLongThreads / 64;
  if ((int)blockIdx.x < dense_blocks) {
    shared_down_block(a.dsh_act, a.N, a.H, a.SI, a.sh_dense[2], a.dsh_dn, blockIdx.x, kWaves);
    return;
  }
  const int in = shared_mode ? a.SI : a.I;
  const int n_np = a.H / 32, n_cb = (n_np + kWaves - 1) / kWaves;
  const int k_tiles = in / 16, ss = slice_steps(k_tiles), n_sl = n_slices(k_tiles);
  const int b = long_item(blockIdx.x - dense_blocks, n_cb, shared_mode, a);
  if (b < 0) return;
  const int cb = b % n_cb, u = b / n_cb;
  RunInfo ri;
  if (!pass_info(a, u, shared_mode, ri)) return;
  const exl3m::ExpertTab &tb = a.tab[ri.e];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar branches
  const int np = cb * kWaves + wave;
  const bool active = np < n_np;
  constexpr bool kDup = dup_cb(CB);
  const int part = long_part_steps(k_tiles, kDup), n_parts = ss / part;
  const int part_k = kStepTiles * part * 16;
  const int xs_stride = long_row_words(k_tiles, kDup);
  const int q_row = part_k / 8;  // 16-byte chunks of act per row and part (a power of two)
  const int q_lg = __builtin_ctz(q_row);
  // plain rows: the double buffers are static, the dynamic LDS holds the slots only
  uint32_t *xs = smem;
  u32x4 *slot = reinterpret_cast<u32x4 *>(smem + (kDup ? kLongRows * xs_stride : 0)) + wave * slot_chunks(K);

  const uint32_t row_bytes = 2u * a.Imax;
  for (int p0 = 0; p0 < ri.len; p0 += kLongRows) {
    const int nr = min(kLongRows, ri.len - p0);
    const __amdgpu_buffer_rsrc_t src = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.act + (int64_t)(ri.off + p0) * a.Imax), (short)0, (int)(nr * row_bytes), 0x00020000);
    with_blocks(nr, [&](auto nrb) {
      constexpr int NRB = decltype(nrb)::value;
      f32x4 D[NRB][2];
      if constexpr (!kDup) {
        long_pass_db<K, CB, PD, NRB>(tb.tr[2], k_tiles, a.H / 16, np, active, src, row_bytes, nr, slot, D,
                                     g_db_a, g_db_b);
      } else
      for (int sl = 0; sl < n_sl; ++sl) {
        for (int pt = 0; pt < n_parts; ++pt) {
          const int k0 = (sl * n_parts + pt) * part_k;
          stage_part<kDup, kStageBatchDn>(src, row_bytes, 2u * k0, q_row, q_lg, nr, xs, xs_stride);
          __syncthreads();
          if (active)
            qmv_slice_rb<K, CB, PD, NRB>(tb.tr[2], k_tiles, a.H / 16, k0 / 16, np, part, xs, xs_stride, nr,
                                         slot, D, sl == 0 && pt == 0);
          __syncthreads();
        }
      }
      if (active) {
        const int col = np * 32;
        // the lane's first row, read here (not hoisted out of the pass loop, where the
        // rows of every block would each hold a VGPR through the decode)
        int lr = threadIdx.x;
        asm volatile("" : "+v"(lr));
        lr = 4 * ((lr & 63) >> 4);
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 16 * rb + lr + i;
            if (r < nr) {
              float *y = a.yhat_dn + (int64_t)(ri.off + p0 + r) * a.S_dn * a.H + col;
              y[d_col(0)] = D[rb][0][i];
              y[d_col(1)] = D[rb][1][i];
            }
          }
      }
    });
  }
}

}  // namespace

namespace exl3h {

// Staged activation rows of one k-slice (in the codebook's staging form), then one
// ring-word slot per wave.
static size_t expert_lds(int in, int pass_rows, int waves, int K, int cb) {
  return (size_t)pass_rows * staged_row_words(in / 16, dup_cb(cb)) * 4 + (size_t)waves * slot_chunks(K) * 16;
}
// Long-run kernels: the staged rows (halves form; the plain form's double buffers are
// static LDS), then one ring-word slot per wave.
static size_t long_lds(int in, int K, int cb) {
  return (dup_cb(cb) ? (size_t)kLongRows * long_row_words(in / 16, true) * 4 : 0) +
         (size_t)(kLongThreads / 64) * slot_chunks(K) * 16;
}

// Per kernel instantiation: the one-time LDS attribute, set under std::call_once so that
// threads making their first calls at once neither race on it nor launch before it is set.
struct KernelAttr {
  std::once_flag once;
  hipError_t rc = hipSuccess;
  size_t max_dynamic = 0;
};

template <typename Kern>
static exl3_status launch_kernel(Kern k, dim3 blocks, unsigned threads, size_t lds, hipStream_t st,
                                 const MoeArgs &a, int shared_mode, int dense_blocks, KernelAttr &attr) {
  // dynamic LDS above the 64 KB default, up to what the kernel's static LDS leaves of a
  // workgroup's 160 KB (at most 128 KB)
  std::call_once(attr.once, [&] {
    hipFuncAttributes fa{};
    attr.rc = hipFuncGetAttributes(&fa, (const void *)k);
    if (attr.rc != hipSuccess) return;
    attr.max_dynamic = std::min<size_t>(128 * 1024, 160 * 1024 - std::min<size_t>(fa.sharedSizeBytes, 160 * 1024));
    attr.rc = hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)attr.max_dynamic);
  });
  if (attr.rc != hipSuccess) return hip_check(attr.rc, "hipFuncSetAttribute");
  if (lds > attr.max_dynamic) return fail(EXL3_ERR_UNSUPPORTED, "expert kernel LDS above the workgroup's share");
  k<<<blocks, threads, lds, st>>>(a, shared_mode, dense_blocks);
  return EXL3_OK;
}

// which: 0 = gate/up, 1 = down.
template <int K, int CB, int PD>
static exl3_status moe_go(int which, dim3 blocks, hipStream_t st, const MoeArgs &a,
                          int shared_mode, int dense_blocks) {
  const int in = which == 0 ? a.H : (shared_mode ? a.SI : a.I);
  if (a.fold) {
    if constexpr (PD <= 2) {  // long-run kernels keep at most 2 steps in flight (VGPRs)
      const size_t lds = long_lds(in, K, CB);
      static KernelAttr set_gu, set_dn;
      return which == 0 ? launch_kernel(k_moe_gate_up_long<K, CB, PD>, blocks, kLongThreads, lds, st,
                                        a, shared_mode, dense_blocks, set_gu)
                        : launch_kernel(k_moe_down_long<K, CB, PD>, blocks, kLongThreads, lds, st, a,
                                        shared_mode, dense_blocks, set_dn);
    } else {
      return fail(EXL3_ERR_INVALID, "long-run expert kernels take at most 2 steps in flight");
    }
  }
  static KernelAttr set_gu, set_dn;
  return which == 0
             ? launch_kernel(k_moe_gate_up<K, CB, PD>, blocks, kGuThreads,
                             expert_lds(in, a.pass_rows, kGuThreads / 64, K, CB), st, a, shared_mode,
                             dense_blocks, set_gu)
             : launch_kernel(k_moe_down<K, CB, PD>, blocks, kDnThreads,
                             expert_lds(in, a.pass_rows, kDnThreads / 64, K, CB), st, a, shared_mode,
                             dense_blocks, set_dn);
}

template <int K, int CB>
static exl3_status moe_pd(int pd, int which, dim3 blocks, hipStream_t st, const MoeArgs &a,
                          int shared_mode, int dense_blocks) {
  if (pd == 1) return moe_go<K, CB, 1>(which, blocks, st, a, shared_mode, dense_blocks);
  if constexpr (K <= 4) {
    if (pd >= 4) return moe_go<K, CB, 4>(which, blocks, st, a, shared_mode, dense_blocks);
  }
  return moe_go<K, CB, 2>(which, blocks, st, a, shared_mode, dense_blocks);
}

// One codebook width's expert launch: the kernel codebook (kernel_cb) and the steps in
// flight select the instantiation.
template <int K>
static exl3_status launch_expert_k(int cb, int pd, int which, dim3 ub, hipStream_t st, const MoeArgs &a,
                                   int shared_mode, int dense_arg) {
  switch (cb) {
    case 0: return moe_pd<K, 0>(pd, which, ub, st, a, shared_mode, dense_arg);
    case 1: return moe_pd<K, 1>(pd, which, ub, st, a, shared_mode, dense_arg);
    case 2: return moe_pd<K, 2>(pd, which, ub, st, a, shared_mode, dense_arg);
    case 3: return moe_pd<K, 3>(pd, which, ub, st, a, shared_mode, dense_arg);
    case 4: return moe_pd<K, 4>(pd, which, ub, st, a, shared_mode, dense_arg);
    default: return fail(EXL3_ERR_INVALID, "kernel codebook out of range");
  }
}

// Defined in moe_experts_k12.hip, _k34, _k56 and _k78: the launches for K in 1..2, 3..4,
// 5..6 and 7..8.
exl3_status launch_expert_k12(int K, int cb, int pd, int which, dim3 ub, hipStream_t st, const MoeArgs &a,
                              int shared_mode, int dense_arg);
exl3_status launch_expert_k34(int K, int cb, int pd, int which, dim3 ub, hipStream_t st, const MoeArgs &a,
                              int shared_mode, int dense_arg);
exl3_status launch_expert_k56(int K, int cb, int pd, int which, dim3 ub, hipStream_t st, const MoeArgs &a,
                              int shared_mode, int dense_arg);
exl3_status launch_expert_k78(int K, int cb, int pd, int which, dim3 ub, hipStream_t st, const MoeArgs &a,
                              int shared_mode, int dense_arg);

}  // namespace exl3h
