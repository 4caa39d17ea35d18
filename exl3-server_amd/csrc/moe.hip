// MoE layer: router logits, top-k routing + expert-order dispatch (one workgroup, no
// host round trip), the dense f16 shared expert, and the C ABI of the layer.
// Reference: src/glm5_moe.{h,cpp} (muyouming/exl3-server).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "exl3_device.hpp"
#include "exl3_internal.hpp"
#include "exl3_moe.h"
#include "moe_common.hpp"
#include "moe_dense.hpp"
#include "qmv_core.hpp"

using namespace exl3d;
using exl3m::ExpertTab;
using exl3m::MoeArgs;
using exl3m::kLongRows;

namespace exl3h {
exl3_status launch_moe_expert(int which, int K, int cb, int64_t runs, const MoeArgs &a,
                              int shared_mode, bool dense, hipStream_t st);
int moe_slices(int in);
exl3_status launch_moe_act(const MoeArgs &a, int shared_mode, int dense_blocks, hipStream_t st);
exl3_status launch_moe_rotate(const MoeArgs &a, int64_t slot0, int64_t n_slots, hipStream_t st);
}

namespace {

__device__ __forceinline__ float lo16(uint32_t v) { return (float)bitcast<f16>((uint16_t)(v & 0xffffu)); }
__device__ __forceinline__ float hi16(uint32_t v) { return (float)bitcast<f16>((uint16_t)(v >> 16)); }
__device__ __forceinline__ float rf16(float v) { return (float)to_f16(v); }


// ---------------------------------------------------------------------------------
// L1. Router logits: logits[t][e] = sum_k f32(h[t][k]) * f32(router_w[e][k])
// (glm5_moe.cpp:127-128) on the matrix cores, one workgroup per (16 rows, 16 experts,
// k split), its 4 waves on quarters of the split; f16*f16 products are exact in f32.
// The router sums the split partials in order.
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_moe_pre(MoeArgs a) {
  __shared__ float red[4 * 64 * 4];
  dense_mfma_wg4(a.h, a.N, a.H, a.router_w, a.E, a.logits, blockIdx.x, red);
}

// The same logits for calls of many rows, tiled: a workgroup computes a 64-row x
// 64-expert tile of one k split, staging both operands through LDS 128 k at a time, so
// each h row and router row is read once per tile instead of once per 16 x 16 task.
// Per output the arithmetic is k_moe_pre's: the split's four quarters each accumulated
// from zero by 16x16x32 MFMAs in step order, then ((q0 + q1) + q2) + q3, so the logits
// (and the routing) are bit-identical whichever kernel ran. Grid: x = split, y =
// expert block, z = row block; wave w owns rows 32(w & 1) .. +32 and experts
// 32(w >> 1) .. +32 of the tile (2 x 2 MFMA tiles).
constexpr int kPreTile = 64;
constexpr int kPreChunk = 128;  // k per staging round
constexpr int kPreStride = kPreChunk + 8;  // halves per staged row (16-byte pad)
constexpr int kPreTiledMinRows = 256;
constexpr int kPreLoads = kPreTile * (kPreChunk / 8) / 256;  // 16-byte chunks per thread per operand
static_assert(kPreLoads == 4, "the staging registers below are four per operand");

// One staging round's global loads into registers, all issued before any is used:
// chunk c of the round is row c / cpr, k offset 8 (c % cpr); rows and experts past the
// end load the last valid one (never stored). The loads take no branch (chunks past
// the round's last one load that one again, unused): a load under a branch is waited
// for before the branch ends, which would serialise them. Named native vectors, not an
// array of HIP's uint4: carried across the rounds' loop, those are kept in scratch memory.
struct PreRegs {
  u32x4 a0, a1, a2, a3, b0, b1, b2, b3;
};

__device__ __forceinline__ void pre_tiled_chunk(const MoeArgs &a, int64_t r0, int e0, int kk, int cpr,
                                                int i, u32x4 &ra, u32x4 &rb) {
  const int c = min((int)threadIdx.x + 256 * i, kPreTile * cpr - 1);
  const int r = c / cpr, kc = (c % cpr) * 8;
  const int64_t row = min<int64_t>(r0 + r, a.N - 1);
  const int e = min(e0 + r, a.E - 1);
  ra = *reinterpret_cast<const u32x4 *>(a.h + row * a.H + kk + kc);
  rb = *reinterpret_cast<const u32x4 *>(a.router_w + (int64_t)e * a.H + kk + kc);
}

__device__ __forceinline__ void pre_tiled_load(const MoeArgs &a, int64_t r0, int e0, int kk, int cpr,
                                               PreRegs &g) {
  pre_tiled_chunk(a, r0, e0, kk, cpr, 0, g.a0, g.b0);
  pre_tiled_chunk(a, r0, e0, kk, cpr, 1, g.a1, g.b1);
  pre_tiled_chunk(a, r0, e0, kk, cpr, 2, g.a2, g.b2);
  pre_tiled_chunk(a, r0, e0, kk, cpr, 3, g.a3, g.b3);
}

__device__ __forceinline__ void pre_tiled_put(uint16_t *sA, uint16_t *sB, int cpr, int i,
                                              const u32x4 &ra, const u32x4 &rb) {
  const int c = (int)threadIdx.x + 256 * i;
  if (c < kPreTile * cpr) {
    const int r = c / cpr, kc = (c % cpr) * 8;
    *reinterpret_cast<u32x4 *>(sA + r * kPreStride + kc) = ra;
    *reinterpret_cast<u32x4 *>(sB + r * kPreStride + kc) = rb;
  }
}

__device__ __forceinline__ void pre_tiled_store(uint16_t *sA, uint16_t *sB, int cpr, const PreRegs &g) {
  pre_tiled_put(sA, sB, cpr, 0, g.a0, g.b0);
  pre_tiled_put(sA, sB, cpr, 1, g.a1, g.b1);
  pre_tiled_put(sA, sB, cpr, 2, g.a2, g.b2);
  pre_tiled_put(sA, sB, cpr, 3, g.a3, g.b3);
}

// Staging rounds: quarter q of the split in chunks of kPreChunk k. Round s + 1's loads
// are issued before round s's MFMAs, so a workgroup waits on one memory round trip per
// round.
__global__ __launch_bounds__(256) void k_moe_pre_tiled(MoeArgs a) {
  __shared__ __align__(16) uint16_t sA[kPreTile * kPreStride];
  __shared__ __align__(16) uint16_t sB[kPreTile * kPreStride];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4;
  const int H = a.H;
  const int S = dense_mfma_splits(H), sk = H / S, qk = sk / 4;  // k per quarter
  const int sp = blockIdx.x;
  const int e0 = blockIdx.y * kPreTile;
  const int64_t r0 = (int64_t)blockIdx.z * kPreTile;
  const int wr = (wave & 1) * 32, we = (wave >> 1) * 32;
  const int n_ch = (qk + kPreChunk - 1) / kPreChunk, n_st = 4 * n_ch;
  f32x4_ acc[2][2], D[2][2];
  PreRegs regs;
  // round s: quarter s / n_ch, chunk (s % n_ch); ck a multiple of 32
  auto round_k = [&](int s, int &ck) {
    const int q = s / n_ch, c0 = (s % n_ch) * kPreChunk;
    ck = min(kPreChunk, qk - c0);
    return sp * sk + q * qk + c0;
  };
  int ck;
  int kk = round_k(0, ck);
  pre_tiled_load(a, r0, e0, kk, ck / 8, regs);
  for (int s = 0; s < n_st; ++s) {
    const int q = s / n_ch, chunk = s % n_ch;
    const int cur_ck = ck;
    if (chunk == 0) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) D[i][j] = f32x4_{0.0f, 0.0f, 0.0f, 0.0f};
    }
    if (s > 0) __syncthreads();  // every wave is done reading the previous round
    pre_tiled_store(sA, sB, cur_ck / 8, regs);
    __syncthreads();
    if (s + 1 < n_st) {
      kk = round_k(s + 1, ck);
      pre_tiled_load(a, r0, e0, kk, ck / 8, regs);
    }
    for (int st = 0; st < cur_ck / 32; ++st) {
      const int ko = st * 32 + 8 * g;
      f16x8_ A[2], B[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        A[i] = *reinterpret_cast<const f16x8_ *>(sA + (wr + 16 * i + (lane & 15)) * kPreStride + ko);
        B[i] = *reinterpret_cast<const f16x8_ *>(sB + (we + 16 * i + (lane & 15)) * kPreStride + ko);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) D[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[i], B[j], D[i][j], 0, 0, 0);
    }
    if (chunk == n_ch - 1) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int t = 0; t < 4; ++t) acc[i][j][t] = q == 0 ? D[i][j][t] : acc[i][j][t] + D[i][j][t];
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int e = e0 + we + 16 * j + (lane & 15);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int64_t row = r0 + wr + 16 * i + 4 * g + t;
        if (row < a.N && e < a.E) a.logits[(row * a.E + e) * kDenseSlots + sp] = acc[i][j][t];
      }
    }
}

// ---------------------------------------------------------------------------------
// Routing + dispatch, one workgroup of 16 waves (glm5_moe.cpp:16-60, 158-255).
// ---------------------------------------------------------------------------------
constexpr int kMaxE = 1024;
constexpr int kIdBatch = 16;  // pair experts per lane loaded at once by the counting sort
// Chunks of the dispatch's counting sort, one workgroup each: 1024 pairs (a round of 64
// per wave) up to kDispatchMaxWg chunks, above that kDispatchMaxWg chunks of a multiple of
// 1024 pairs; one workgroup up to 1024 pairs.
constexpr int kDispatchMaxWg = 64;
__host__ __device__ constexpr int64_t dispatch_chunk_pairs(int64_t P) {
  return 1024 * (((P + 1023) / 1024 + kDispatchMaxWg - 1) / kDispatchMaxWg);
}
__host__ __device__ constexpr int dispatch_wgs(int64_t P) {
  return P > 0 ? (int)((P + dispatch_chunk_pairs(P) - 1) / dispatch_chunk_pairs(P)) : 1;
}
// Route kernels are instantiated for E <= 64 * JN experts (JN 64-expert chunks per lane).
template <typename F>
static void with_route_chunks(int E, F &&f) {
  if (E <= 128) f(std::integral_constant<int, 2>{});
  else if (E <= 256) f(std::integral_constant<int, 4>{});
  else if (E <= 320) f(std::integral_constant<int, 5>{});
  else if (E <= 512) f(std::integral_constant<int, 8>{});
  else f(std::integral_constant<int, 16>{});
}

__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

__device__ __forceinline__ uint64_t match_mask(int e, bool valid) {
  uint64_t m = __ballot(valid);
#pragma unroll
  for (int b = 0; b < 10; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t bb = __ballot(bit);
    m &= bit ? bb : ~bb;
  }
  return m;
}

__device__ __forceinline__ uint64_t lanes_below() {
  const int lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}


// Monotone map of an f32 (not NaN) to u32: a > b  <=>  key(a) > key(b); -0 is taken as +0.
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Wave-wide max / min of a u32: DPP within rows of 16 lanes, then the 4 row values.
__device__ __forceinline__ uint32_t row_reduce_max(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false));   // lane ^ 1
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false));   // lane ^ 2
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false));  // half-row mirror
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false));  // row mirror
  return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = row_reduce_max(v);
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) { return ~wave_max_u32(~v); }

// The run record of run `run_i`: expert e's pointers from the expert table.
__device__ __forceinline__ void write_run_rec(const MoeArgs &a, int run_i, int e, int off, int len,
                                              int row0, const ExpertTab &t) {
  exl3m::RunRec r;
  r.e = e;
  r.off = off;
  r.len = len;
  r.row0 = row0;
  r.p[0] = t.tr[0];
  r.p[1] = t.suh[0];
  r.p[2] = t.tr[1];
  r.p[3] = t.suh[1];
  r.p[4] = t.tr[2];
  r.p[5] = nullptr;
  a.run_rec[run_i] = r;
}

// The dispatch of P <= 64 pairs by one wave (lane i = pair i, its expert in ids[i]):
// the same stable sort by expert, run table and pass table as the workgroup-wide
// counting sort. The 64 keys (expert, pair index) are sorted across the lanes by a
// bitonic network (21 compare-exchange stages over lane exchanges), after which lane
// p holds the pair at sorted position p; runs start where the expert changes.
static_assert(64 < 2 * (kLongRows + 1), "at most one run of 64 pairs exceeds a pass");

template <int J>
__device__ __forceinline__ uint32_t bitonic_step(uint32_t key, int k) {
  const int lane = threadIdx.x & 63;
  const uint32_t other = __builtin_bit_cast(uint32_t, xor_lanes<J>(__builtin_bit_cast(float, key)));
  const bool keep_min = ((lane & J) == 0) == ((lane & k) == 0);
  return keep_min ? min(key, other) : max(key, other);
}

__device__ __forceinline__ void dispatch_small(const MoeArgs &a, const int *ids) {
  const int lane = threadIdx.x & 63;
  const int P = a.P, K = a.topk;
  // pair `lane`'s expert table entry, loaded while the keys are sorted
  const ExpertTab tab_l = a.tab[lane < P ? ids[lane] : 0];
  uint32_t key = lane < P ? (((uint32_t)ids[lane] << 6) | (uint32_t)lane) : 0xFFFFFFFFu;
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1) {
    if (k >= 64) key = bitonic_step<32>(key, k);
    if (k >= 32) key = bitonic_step<16>(key, k);
    if (k >= 16) key = bitonic_step<8>(key, k);
    if (k >= 8) key = bitonic_step<4>(key, k);
    if (k >= 4) key = bitonic_step<2>(key, k);
    key = bitonic_step<1>(key, k);
  }
  // lane p: sorted position p
  const bool valid = lane < P;
  const int se = (int)(key >> 6), pair = (int)(key & 63u);
  if (valid) {
    a.sorted_row[lane] = pair / K;
    a.sorted_rank[lane] = pair % K;
    a.slot_e[lane] = se;
    a.slot[pair] = lane;
  }
  const int prev = __shfl(se, lane > 0 ? lane - 1 : 0, 64);
  const bool start = valid && (lane == 0 || prev != se);
  const uint64_t starts = __ballot(start);
  const uint64_t upto = lanes_below() | (1ull << lane);
  const int run_i = __builtin_popcountll(starts & upto) - 1;
  const uint64_t later = starts & ~upto;
  const int run_end = later ? __builtin_ctzll(later) : P;
  const int len = run_end - lane;
  // passes of <= kLongRows rows: with P <= 64 only one run can need two
  const uint64_t big = __ballot(start && len > kLongRows);
  const int pass_i = run_i + (big && __builtin_ctzll(big) < lane ? 1 : 0);
  // the expert table entry of this position's pair (loaded by lane `pair`)
  ExpertTab tp;
  for (int j = 0; j < 3; ++j) {
    tp.tr[j] = (const uint32_t *)__shfl((long long)(uintptr_t)tab_l.tr[j], pair, 64);
    tp.suh[j] = (const uint16_t *)__shfl((long long)(uintptr_t)tab_l.suh[j], pair, 64);
    tp.svh[j] = nullptr;
  }
  if (start) {
    a.run_expert[run_i] = se;
    a.run_off[run_i] = lane;
    a.run_len[run_i] = len;
    write_run_rec(a, run_i, se, lane, len, pair / K, tp);
    for (int q = 0; q * kLongRows < len; ++q) {
      a.pass_expert[pass_i + q] = se;
      a.pass_off[pass_i + q] = lane + q * kLongRows;
      a.pass_len[pass_i + q] = min(kLongRows, len - q * kLongRows);
    }
  }
  if (lane == 0) {
    *a.n_runs = __builtin_popcountll(starts);
    *a.n_passes = __builtin_popcountll(starts) + (big ? 1 : 0);
  }
  for (int i = lane; i < a.N; i += 64) {
    a.sorted_row[P + i] = i;
    a.sorted_rank[P + i] = 0;
  }
}

// Stable counting sort of the P = N*K pairs by expert (pair order b*K + k), the order of
// the reference's stable_sort (glm5_moe.cpp:191-200), over G workgroups of 16 waves:
// workgroup g takes chunk g of the pairs, [g * cs, (g + 1) * cs), each of its waves a
// segment of the chunk in pair order, 64 pairs at a time. Slot of a pair = the expert's
// first slot + the pairs of that expert in earlier chunks (a.hist, G > 1), in earlier
// segments of the chunk, and in earlier lanes of the round.
struct DispatchChunk {
  int c0, c1, seg;
};
__device__ __forceinline__ DispatchChunk dispatch_chunk(int P, int g) {
  const int cs = (int)dispatch_chunk_pairs(P);
  DispatchChunk ch;
  ch.c0 = min(P, g * cs);
  ch.c1 = min(P, ch.c0 + cs);
  ch.seg = ((ch.c1 - ch.c0 + 15) / 16 + 63) / 64 * 64;
  return ch;
}

// Per-wave counts of the chunk's pairs by expert into cnt[wave * kMaxE + e].
__device__ __forceinline__ void chunk_counts(const MoeArgs &a, const int32_t *id_out, const DispatchChunk &ch,
                                             int *cnt) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < 16 * kMaxE; i += 1024)
    if ((i & (kMaxE - 1)) < a.E) cnt[i] = 0;
  __syncthreads();
  const int pbeg = ch.c0 + wave * ch.seg, pend = min(ch.c1, pbeg + ch.seg);
  // A wave's pairs go 64 at a time; their experts are loaded kIdBatch rounds at once (the
  // addresses clamped, so that no branch separates the loads): one memory round trip
  // per batch instead of one per round.
  for (int c0 = pbeg; c0 < pend; c0 += 64 * kIdBatch) {
    int ev[kIdBatch];
#pragma unroll
    for (int q = 0; q < kIdBatch; ++q) ev[q] = id_out[min(c0 + 64 * q + lane, a.P - 1)];
#pragma unroll
    for (int q = 0; q < kIdBatch; ++q) {
      if (c0 + 64 * q >= pend) break;
      const int p = c0 + 64 * q + lane;
      const bool valid = p < pend;
      const int e = valid ? ev[q] : 0;
      const uint64_t m = match_mask(e, valid);
      if (valid && (__builtin_ctzll(m) == lane)) cnt[wave * kMaxE + e] += __builtin_popcountll(m);
      __builtin_amdgcn_wave_barrier();
    }
  }
  __syncthreads();
}

// Workgroup g of the dispatch: its chunk's per-wave counts; per expert the total and the
// pairs of earlier chunks (from a.hist when G > 1); the expert bases and run / pass /
// record indices by block scans (every workgroup computes the same ones); then the
// scatter of its chunk. Workgroup 0 writes the run and pass tables; a run's record is
// written by the workgroup that holds the run's first pair (it knows the run's first row).
__device__ void dispatch_wg(const MoeArgs &a, const int32_t *id_out, int g, int G, int *cnt) {
  __shared__ int s_run_of[kMaxE], s_base[kMaxE];  // per expert: its run record, its first slot
  __shared__ int s_wv[16], s_wf[16], s_wg[16], s_wq[16];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int E = a.E, K = a.topk, P = a.P;
  const ExpertTab tab_t = a.tab[threadIdx.x < E ? threadIdx.x : 0];  // loaded during the count
  const DispatchChunk ch = dispatch_chunk(P, g);
  chunk_counts(a, id_out, ch, cnt);
  // Per expert: total, pairs in earlier chunks, base offset (exclusive scan over experts),
  // per-wave offsets.
  const int t = threadIdx.x;
  int tot = 0, pre = 0;
  if (t < E) {
    if (G == 1) {
      for (int w = 0; w < 16; ++w) tot += cnt[w * kMaxE + t];
    } else {
      // the chunks' counts 8 at a time, all loads of a batch in flight together
      for (int q0 = 0; q0 < G; q0 += 8) {
        int h[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = a.hist[(int64_t)min(q0 + j, G - 1) * E + t];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int hj = q0 + j < G ? h[j] : 0;
          tot += hj;
          pre += q0 + j < g ? hj : 0;
        }
      }
    }
  }
  // block exclusive scans of tot, of (tot > 0) and of the run's pass count (passes of
  // at most kLongRows rows, the work units of the long-run expert kernels)
  const int npass = (tot + kLongRows - 1) / kLongRows;
  // runs that need several row passes of the short-run kernels go first in the run
  // records, so that their longer workgroups start early instead of ending the launch
  const int big = tot > a.pass_rows ? 1 : 0;
  int v = tot, f = tot > 0 ? 1 : 0, gp = npass, q = big;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int ov = __shfl_up(v, d, 64), of = __shfl_up(f, d, 64), og = __shfl_up(gp, d, 64);
    const int oq = __shfl_up(q, d, 64);
    if (lane >= d) {
      v += ov;
      f += of;
      gp += og;
      q += oq;
    }
  }
  if (lane == 63) {
    s_wv[wave] = v;
    s_wf[wave] = f;
    s_wg[wave] = gp;
    s_wq[wave] = q;
  }
  __syncthreads();
  int pv = 0, pf = 0, pg = 0, pq = 0, nbig = 0;
  for (int w = 0; w < 16; ++w) {
    if (w < wave) {
      pv += s_wv[w];
      pf += s_wf[w];
      pg += s_wg[w];
      pq += s_wq[w];
    }
    nbig += s_wq[w];
  }
  const int base_e = pv + v - tot;           // exclusive
  const int run_i = pf + f - (tot > 0 ? 1 : 0);
  const int pass_i = pg + gp - npass;
  const int big_i = pq + q - big;            // among the big runs
  const int rec_i = big ? big_i : nbig + (run_i - big_i);  // big runs first, order kept
  if (t < E) {
    int run = base_e + pre;
    for (int w = 0; w < 16; ++w) {
      const int x = cnt[w * kMaxE + t];
      cnt[w * kMaxE + t] = run;
      run += x;
    }
    // the chunk that holds the expert's first pair writes its run record (row0 set by
    // the scatter below)
    if (pre == 0 && run > base_e) write_run_rec(a, rec_i, t, base_e, tot, 0, tab_t);
    if (g == 0) {
      if (tot > 0) {
        a.run_expert[run_i] = t;
        a.run_off[run_i] = base_e;
        a.run_len[run_i] = tot;
      }
      for (int j = 0; j < npass; ++j) {
        a.pass_expert[pass_i + j] = t;
        a.pass_off[pass_i + j] = base_e + j * kLongRows;
        a.pass_len[pass_i + j] = min(kLongRows, tot - j * kLongRows);
      }
    }
    s_run_of[t] = rec_i;
    s_base[t] = base_e;
  }
  if (g == 0 && t == 1023) {
    int nrun = 0, npas = 0;
    for (int w = 0; w < 16; ++w) {
      nrun += s_wf[w];
      npas += s_wg[w];
    }
    *a.n_runs = nrun;
    *a.n_passes = npas;
  }
  __syncthreads();
  const int pbeg = ch.c0 + wave * ch.seg, pend = min(ch.c1, pbeg + ch.seg);
  for (int c0 = pbeg; c0 < pend; c0 += 64 * kIdBatch) {
    int ev[kIdBatch];
#pragma unroll
    for (int qq = 0; qq < kIdBatch; ++qq) ev[qq] = id_out[min(c0 + 64 * qq + lane, P - 1)];
#pragma unroll
    for (int qq = 0; qq < kIdBatch; ++qq) {
      if (c0 + 64 * qq >= pend) break;
      const int p = c0 + 64 * qq + lane;
      const bool valid = p < pend;
      const int e = valid ? ev[qq] : 0;
      const uint64_t m = match_mask(e, valid);
      if (valid) {
        const int pos = cnt[wave * kMaxE + e] + __builtin_popcountll(m & lanes_below());
        a.sorted_row[pos] = p / K;
        a.sorted_rank[pos] = p % K;
        a.slot_e[pos] = e;
        a.slot[p] = pos;
        if (pos == s_base[e]) a.run_rec[s_run_of[e]].row0 = p / K;
      }
      __builtin_amdgcn_wave_barrier();
      if (valid && (__builtin_ctzll(m) == lane)) cnt[wave * kMaxE + e] += __builtin_popcountll(m);
      __builtin_amdgcn_wave_barrier();
    }
  }
  if (g == 0)
    for (int i = threadIdx.x; i < a.N; i += 1024) {
      a.sorted_row[P + i] = i;
      a.sorted_rank[P + i] = 0;
    }
}

// L2. Routing + dispatch. mode bit 0: top-k routing of rows blockIdx.x*16 + wave,
// strided by the grid; bit 1: the dispatch (one workgroup, after the routing of every
// row: the same workgroup's or an earlier launch's).
template <int kJ>
__global__ __launch_bounds__(1024) void k_moe_route(MoeArgs a, float *w_out, int32_t *id_out,
                                                    int mode) {
  // group path: scores_for_choice per wave; top-k: a wave's candidates (8-byte keys);
  // dispatch: counts
  __shared__ __align__(16) float s_buf[16][kMaxE];
  __shared__ int s_keep[16][64];
  __shared__ int s_small[64];         // the pairs' experts when P <= 64 (one-wave dispatch)
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int E = a.E, K = a.topk;
  const int ng = a.n_group > 1 ? a.n_group : 1;
  const int tg = a.topk_group > 0 ? min(a.topk_group, ng) : 1;
  const int gsize = E / ng;

  const int jn = (E + 63) / 64;
  const int S = a.logit_splits;  // 0: plain logits (N, E); else S partials in (N, E, 8)
  for (int b = (mode & 1) ? blockIdx.x * 16 + wave : a.N; b < a.N; b += 16 * gridDim.x) {
    // the logit partial and bias loads of kLoadJ chunks at once (clamped addresses, so
    // no branches split them; every chunk at once up to 320 experts, 4 at a time above,
    // which keeps the partials in registers), then the split sums in split order, the
    // sigmoid and the biased score
    constexpr int kLoadJ = kJ <= 5 ? kJ : 4;
    static_assert(kJ % kLoadJ == 0, "route chunks");
    float sc[kJ], sfc[kJ];
#pragma unroll
    for (int j0 = 0; j0 < kJ; j0 += kLoadJ) {
      float4 lp[kLoadJ][2];
      float bias[kLoadJ];
#pragma unroll
      for (int jj = 0; jj < kLoadJ; ++jj) {
        const int e = min(lane + 64 * (j0 + jj), E - 1);
        if (S == 0) {
          lp[jj][0].x = a.logits[(int64_t)b * E + e];
        } else {
          const float4 *q = reinterpret_cast<const float4 *>(a.logits + ((int64_t)b * E + e) * kDenseSlots);
          lp[jj][0] = q[0];
          lp[jj][1] = q[1];
        }
        bias[jj] = a.router_bias[e];
      }
#pragma unroll
      for (int jj = 0; jj < kLoadJ; ++jj) {
        const int j = j0 + jj;
        const float v[8] = {lp[jj][0].x, lp[jj][0].y, lp[jj][0].z, lp[jj][0].w,
                            lp[jj][1].x, lp[jj][1].y, lp[jj][1].z, lp[jj][1].w};
        float lg = v[0];
#pragma unroll
        for (int s = 1; s < 8; ++s)
          if (s < S) lg += v[s];
        const int e = lane + 64 * j;
        sc[j] = 0.0f;
        sfc[j] = -INFINITY;
        if (e < E) {
          sc[j] = 1.0f / (1.0f + expf(-lg));
          sfc[j] = sc[j] + bias[jj];
        }
      }
    }
    if (ng > 1) {
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const int e = lane + 64 * j;
        if (e < E) s_buf[wave][e] = sfc[j];
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      float gs = -INFINITY;
      if (lane < ng) {
        float m1 = -INFINITY, m2 = -INFINITY;
        for (int j = 0; j < gsize; ++j) {
          const float v = s_buf[wave][lane * gsize + j];
          if (v > m1) {
            m2 = m1;
            m1 = v;
          } else if (v > m2) {
            m2 = v;
          }
        }
        gs = gsize >= 2 ? m1 + m2 : m1;
      }
      bool kept = false;
      for (int i = 0; i < tg; ++i) {
        float bv = (lane < ng && !kept) ? gs : -INFINITY;
        int bi = (lane < ng && !kept) ? lane : 1 << 30;
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
          const float ov = __shfl_xor(bv, d, 64);
          const int oi = __shfl_xor(bi, d, 64);
          if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
          }
        }
        if (lane == bi) kept = true;
      }
      s_keep[wave][lane] = kept ? 1 : 0;
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const int e = lane + 64 * j;
        if (e < E && !s_keep[wave][e / gsize]) sfc[j] = -INFINITY;
      }
    }
    // top_k: largest sfc, ties to the lower expert id. T = the K-th largest of the 64
    // lanes' largest order keys: every lane counts the lane maxima above its own (64
    // broadcast LDS reads, independent of each other), and T is the smallest lane maximum
    // with fewer than K above it. K lanes hold a key >= T, each a different expert, so
    // the top K keys are all >= T. Those candidates (about K) go to LDS and each one ranks
    // itself against all of them by the key above the complemented expert id: its rank
    // is its pick index. More than 64 candidates (scores tied across many experts) take
    // the repeated wave argmax below, which picks the same experts in the same order.
    float denom = 0.0f;
    float my_w = 0.0f;
    int my_id = 0;
    uint32_t okey[kJ];
    uint32_t lmax = 0;
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
      const int e = lane + 64 * j;
      okey[j] = (j < jn && e < E) ? order_key(sfc[j]) : 0u;
      lmax = max(lmax, okey[j]);
    }
    uint32_t *lm = reinterpret_cast<uint32_t *>(&s_buf[wave][320]);
    lm[lane] = lmax;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    int gt0 = 0, gt1 = 0, gt2 = 0, gt3 = 0;
#pragma unroll
    for (int i = 0; i < 64; i += 4) {
      gt0 += lm[i] > lmax ? 1 : 0;
      gt1 += lm[i + 1] > lmax ? 1 : 0;
      gt2 += lm[i + 2] > lmax ? 1 : 0;
      gt3 += lm[i + 3] > lmax ? 1 : 0;
    }
    const uint32_t thr = wave_min_u32((gt0 + gt1) + (gt2 + gt3) < K ? lmax : 0xFFFFFFFFu);
    uint64_t *cand = reinterpret_cast<uint64_t *>(&s_buf[wave][0]);  // 64 keys
    float *cand_sc = &s_buf[wave][128];
    int *pick_id = reinterpret_cast<int *>(&s_buf[wave][192]);
    float *pick_sc = &s_buf[wave][256];
    int n_c = 0;
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
      const bool cj = okey[j] >= thr && okey[j] != 0u;
      const uint64_t m = __ballot(cj);
      const int pos = n_c + __builtin_popcountll(m & lanes_below());
      if (cj && pos < 64) {
        cand[pos] = ((uint64_t)okey[j] << 32) | (uint64_t)(~(uint32_t)(lane + 64 * j));
        cand_sc[pos] = sc[j];
      }
      n_c += __builtin_popcountll(m);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (n_c <= 64) {
      const uint64_t mine = lane < n_c ? cand[lane] : 0;
      const float msc = lane < n_c ? cand_sc[lane] : 0.0f;
      // every candidate's key by a broadcast LDS read (independent reads, issued ahead)
      int rank = 0;
      for (int i = 0; i < n_c; ++i) rank += cand[i] > mine ? 1 : 0;
      if (lane < n_c && rank < K) {
        pick_id[rank] = (int)~(uint32_t)mine;
        pick_sc[rank] = msc;
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      if (lane < K) {
        my_id = pick_id[lane];
        my_w = pick_sc[lane];
      }
      // the weights' sum in pick order, as the argmax loop adds them
      for (int k = 0; k < K; ++k) denom += pick_sc[k];
    }
    uint32_t taken = 0;
    for (int k = 0; k < (n_c <= 64 ? 0 : K); ++k) {
      uint32_t bkey = 0;
      int bj = 0;
      float bsc = 0.0f;
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        if (!((taken >> j) & 1u)) {
          const uint32_t key = okey[j];
          if (key > bkey) {
            bkey = key;
            bj = j;
            bsc = sc[j];
          }
        }
      }
      const uint32_t mkey = wave_max_u32(bkey);
      // the lane holding the maximum; on a tie between lanes, the lowest expert id
      const uint64_t hold = __ballot(bkey == mkey && bkey != 0);
      uint32_t ewin;
      if (__builtin_popcountll(hold) == 1) {
        const int hl = __builtin_ctzll(hold);
        ewin = (uint32_t)(hl + 64 * __builtin_amdgcn_readlane(bj, hl));
      } else {
        ewin = wave_min_u32(bkey == mkey && bkey != 0 ? (uint32_t)(lane + 64 * bj) : 0xFFFFFFFFu);
      }
      const int wl = (int)(ewin & 63u);
      const float bs = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bsc), wl));
      if (lane == wl) taken |= 1u << (ewin >> 6);
      denom += bs;
      if (lane == k) {
        my_w = bs;
        my_id = (int)ewin;
      }
    }
    if (lane < K) {
      float w = my_w;
      if (a.norm_topk_prob) w = w / (denom + 1e-20f);
      w = w * a.routed_scaling_factor;
      w_out[(int64_t)b * K + lane] = w;
      id_out[(int64_t)b * K + lane] = my_id;
      if ((mode & 2) && b * K + lane < 64) s_small[b * K + lane] = my_id;
    }
  }
  if (!(mode & 2)) return;
  __syncthreads();
  if (a.P <= 64) {
    if (wave == 0) {
      // a dispatch-only launch (mode 2) did not route here: its pairs' experts come from
      // the routing launch's id_out, not from this workgroup's LDS
      if (!(mode & 1)) {
        if (lane < a.P) s_small[lane] = id_out[lane];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      }
      dispatch_small(a, s_small);
    }
    return;
  }

  // the one-workgroup form of the counting sort (the pairs as one chunk)
  dispatch_wg(a, id_out, 0, 1, reinterpret_cast<int *>(&s_buf[0][0]));
}

// Dispatch of many pairs over G workgroups: k_moe_count writes each chunk's per-expert
// counts to a.hist, then k_moe_dispatch (G workgroups again) scatters each chunk.
__global__ __launch_bounds__(1024) void k_moe_count(MoeArgs a, const int32_t *id_out) {
  __shared__ int cnt[16 * kMaxE];
  const DispatchChunk ch = dispatch_chunk(a.P, blockIdx.x);
  chunk_counts(a, id_out, ch, cnt);
  for (int e = threadIdx.x; e < a.E; e += 1024) {
    int t = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) t += cnt[w * kMaxE + e];
    a.hist[(int64_t)blockIdx.x * a.E + e] = t;
  }
}

__global__ __launch_bounds__(1024) void k_moe_dispatch(MoeArgs a, const int32_t *id_out, int G) {
  __shared__ int cnt[16 * kMaxE];
  dispatch_wg(a, id_out, blockIdx.x, G, cnt);
}

// ---------------------------------------------------------------------------------
// L6. Combine (glm5_moe.cpp:369-416): one wave per (token row, 128-column block). Per
// rank k (in rank order): the slot's down slice partials summed in slice order, the
// output Hadamard with the expert's svh, y = f16 (the linear's output), then
// f16(f32(y) * w_k); routed = f16(sum of those f16 terms in rank order), then
// out = f16(routed + shared).
// ---------------------------------------------------------------------------------
// Ranks are taken 8 at a time: their slot/expert/weight, their down slice partials and
// svh words are all loaded before the first output Hadamard, so a row costs a few
// memory round trips instead of a few per rank.
constexpr int kCombineBatch = 8;
constexpr int kCombineSlices = 2;  // down slices loaded at once (intermediate <= 1024)

__device__ __forceinline__ void down_out(float2 y, uint32_t sv, float &y0, float &y1) {
  y0 = y.x;
  y1 = y.y;
  wave_had_post(y0, y1, lo16(sv), hi16(sv));
  y0 = rf16(y0);
  y1 = rf16(y1);
}

// kFold: a long-run call (one folded down partial per slot, a.fold). Its variant holds
// few enough VGPRs for 7 waves per SIMD (the general one: 4), so that many more rows'
// loads are in flight over a long call's many rows; the f16 shared expert's partials are
// then loaded after the ranks.
template <bool kFold>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kFold ? 7 : 1))) void k_moe_combine(MoeArgs a) {
  const int lane = threadIdx.x & 63;
  const int n_cb = a.H / 128;
  const int64_t gw = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (gw >= (int64_t)a.N * n_cb) return;
  const int row = (int)(gw / n_cb), cb = (int)(gw % n_cb);
  const int c = cb * 128 + 2 * lane;
  const int n_sl = kFold ? 1 : n_slices(a.I / 16);  // down partials per output
  const int64_t plane = a.H;  // floats between slice planes of one slot
  // the f16 shared expert's down partials (addresses known at entry): in flight with the
  // first round of the ranks' loads
  static_assert(kDenseSlots == 8, "two outputs' partials are four float4");
  float4 dsh[4];
  auto load_dsh = [&] {
    const float4 *pd = reinterpret_cast<const float4 *>(a.dsh_dn + ((int64_t)row * a.H + c) * kDenseSlots);
#pragma unroll
    for (int q = 0; q < 4; ++q) dsh[q] = pd[q];
  };
  if (!kFold && a.shared_kind == exl3m::kSharedDense) load_dsh();
  // the mix's residual pairs (its only per-lane inputs), in flight with the rest (the
  // folded form, held to 72 VGPRs, loads them at the mix)
  uint32_t rv[exl3m::kHcMixMax];
  if (!kFold && a.hc_out) exl3m::hc_mix_res(a.hc_res + (int64_t)row * a.hc_n * a.H + c, a.H, a.hc_n, rv);
  float r0 = 0.0f, r1 = 0.0f;
  for (int k0 = 0; k0 < a.topk; k0 += kCombineBatch) {
    const int nk = min(kCombineBatch, a.topk - k0);
    // three rounds of loads, each for all ranks of the batch at once (rank indices
    // clamped, so no branch separates them): pair -> slot/expert/weight -> the expert's
    // svh pointer -> svh words and the slot's down slice partials
    int slot[kCombineBatch], e[kCombineBatch];
    float w[kCombineBatch];
#pragma unroll
    for (int j = 0; j < kCombineBatch; ++j) {
      const int64_t pk = (int64_t)row * a.topk + min(k0 + j, a.topk - 1);
      slot[j] = a.slot[pk];
      e[j] = a.ids[pk];
      w[j] = a.weights[pk];
    }
    const uint16_t *svb = a.svh_s[2] + c;
    uint32_t sv[kCombineBatch];
    float2 y[kCombineBatch];
    if (kFold || n_sl == 1) {
      // long-run calls: one folded partial per slot
#pragma unroll
      for (int j = 0; j < kCombineBatch; ++j) {
        sv[j] = *reinterpret_cast<const uint32_t *>(svb + (int64_t)e[j] * a.H);
        y[j] = *reinterpret_cast<const float2 *>(a.yhat_dn + (int64_t)slot[j] * a.S_dn * plane + c);
      }
    } else if (n_sl <= kCombineSlices) {
      float2 part[kCombineBatch][kCombineSlices];
#pragma unroll
      for (int j = 0; j < kCombineBatch; ++j) {
        sv[j] = *reinterpret_cast<const uint32_t *>(svb + (int64_t)e[j] * a.H);
#pragma unroll
        for (int q = 0; q < kCombineSlices; ++q)
          part[j][q] = *reinterpret_cast<const float2 *>(
              a.yhat_dn + ((int64_t)slot[j] * a.S_dn + min(q, n_sl - 1)) * plane + c);
      }
#pragma unroll
      for (int j = 0; j < kCombineBatch; ++j) {
        y[j] = part[j][0];
#pragma unroll
        for (int q = 1; q < kCombineSlices; ++q)
          if (q < n_sl) {
            y[j].x += part[j][q].x;
            y[j].y += part[j][q].y;
          }
      }
    } else {
#pragma unroll
      for (int j = 0; j < kCombineBatch; ++j) {
        sv[j] = *reinterpret_cast<const uint32_t *>(svb + (int64_t)e[j] * a.H);
        y[j] = exl3m::ordered_sum2<4>(a.yhat_dn + (int64_t)slot[j] * a.S_dn * plane + c, plane, n_sl);
      }
    }
    // the output Hadamards kHadGroup ranks at a time (their stages interleaved), in rank
    // order into the sums
    constexpr int kHadGroup = kFold ? 4 : kCombineBatch;
#pragma unroll
    for (int g0 = 0; g0 < kCombineBatch; g0 += kHadGroup) {
      float v0[kHadGroup], v1[kHadGroup], s0[kHadGroup], s1[kHadGroup];
#pragma unroll
      for (int j = 0; j < kHadGroup; ++j) {
        v0[j] = y[g0 + j].x;
        v1[j] = y[g0 + j].y;
        s0[j] = lo16(sv[g0 + j]);
        s1[j] = hi16(sv[g0 + j]);
      }
      wave_had_post_n<kHadGroup>(v0, v1, s0, s1);
#pragma unroll
      for (int j = 0; j < kHadGroup; ++j) {
        if (g0 + j < nk) {
          r0 += rf16(rf16(v0[j]) * w[g0 + j]);
          r1 += rf16(rf16(v1[j]) * w[g0 + j]);
        }
      }
    }
  }
  r0 = rf16(r0);
  r1 = rf16(r1);
  if (a.shared_kind == exl3m::kSharedTrellis) {
    const int64_t slot = (int64_t)a.P + row;
    const float2 ys = kFold ? *reinterpret_cast<const float2 *>(a.yhat_dn + slot * a.S_dn * plane + c)
                            : exl3m::ordered_sum2<4>(a.yhat_dn + slot * a.S_dn * plane + c, plane,
                                                     n_slices(a.SI / 16));
    float y0, y1;
    down_out(ys, *reinterpret_cast<const uint32_t *>(a.svh_s[2] + (int64_t)a.E * a.H + c), y0, y1);
    r0 += y0;
    r1 += y1;
  } else if (a.shared_kind == exl3m::kSharedDense) {
    if (kFold) load_dsh();
    // dense_slots_sum's order over the two outputs' kDenseSlots partials
    const int S = dense_mfma_splits(a.SI);
    const float v0[8] = {dsh[0].x, dsh[0].y, dsh[0].z, dsh[0].w, dsh[1].x, dsh[1].y, dsh[1].z, dsh[1].w};
    const float v1[8] = {dsh[2].x, dsh[2].y, dsh[2].z, dsh[2].w, dsh[3].x, dsh[3].y, dsh[3].z, dsh[3].w};
    float d0 = v0[0], d1 = v1[0];
#pragma unroll
    for (int q = 1; q < 8; ++q)
      if (q < S) {
        d0 += v0[q];
        d1 += v1[q];
      }
    r0 += rf16(d0);
    r1 += rf16(d1);
  }
  const uint32_t o = pack_f16x2(r0, r1);
  *reinterpret_cast<uint32_t *>(a.out + (int64_t)row * a.H + c) = o;
  if (a.hc_out) {
    // the hyper-connection mix behind the layer (g5_hc_mix), on the f16 output
    const int64_t so = (int64_t)row * a.hc_n * a.H + c;
    if (kFold) exl3m::hc_mix_res(a.hc_res + so, a.H, a.hc_n, rv);
    exl3m::hc_mix_pair(a.hc_post + (int64_t)row * a.hc_n, a.hc_comb + (int64_t)row * a.hc_n * a.hc_n, rv,
                       a.H, a.hc_n, lo16(o), hi16(o), a.hc_out + so);
  }
}

// Stacks every expert's suh/svh (entry e of tab) into the layer's scale arrays: block
// (e, j) copies suh[j] (length in_j) and svh[j] (out_j) of entry e, rows of stride
// stride_in[j] / stride_out[j]. Entries without a tensor (no shared expert) are skipped.
struct ScaleGather {
  uint16_t *suh[3], *svh[3];
  int len_in[2][3], len_out[2][3];  // [routed, shared][j]
  int stride_in[3], stride_out[3];
};

__global__ __launch_bounds__(256) void k_gather_scales(const ExpertTab *tab, int E, ScaleGather g) {
  const int e = blockIdx.x / 3, j = blockIdx.x % 3;
  const ExpertTab &t = tab[e];
  const int sh = e == E ? 1 : 0;
  if (t.suh[j])
    for (int i = threadIdx.x; i < g.len_in[sh][j]; i += 256) g.suh[j][(int64_t)e * g.stride_in[j] + i] = t.suh[j][i];
  if (t.svh[j])
    for (int i = threadIdx.x; i < g.len_out[sh][j]; i += 256) g.svh[j][(int64_t)e * g.stride_out[j] + i] = t.svh[j][i];
}

// (in, out) f16 -> (out, in) f16 through a 64x64 LDS tile per workgroup (256 threads);
// used once per f16 shared expert projection when the layer is created.
__global__ __launch_bounds__(256) void k_transpose_f16(const uint16_t *__restrict__ src, int in,
                                                       int out, uint16_t *__restrict__ dst) {
  __shared__ uint16_t t[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4)
    if (r0 + r < in && c0 + tx < out) t[r][tx] = src[(int64_t)(r0 + r) * out + c0 + tx];
  __syncthreads();
  for (int c = ty; c < 64; c += 4)
    if (c0 + c < out && r0 + tx < in) dst[(int64_t)(c0 + c) * in + r0 + tx] = t[tx][c];
}

}  // namespace

using namespace exl3h;

// ---------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------
struct exl3_moe_layer_s {
  exl3_moe_config cfg;
  int H, I, E, topk;
  int gu_K, gu_cb, dn_K, dn_cb;
  int shared;        // exl3m::SharedKind
  int SI, sh_K, sh_cb, sh_dn_K, sh_dn_cb;
  const uint16_t *sh_dense[3];  // the caller's (in, out) f16 weights
  uint16_t *sh_dense_t[3];      // layer-owned (out, in) copies read by the kernels
  const uint16_t *router_w;
  const float *router_bias;
  ExpertTab *tab_dev;  // E + 1 entries
  uint16_t *scales;    // stacked suh/svh (MoeArgs::suh_s/svh_s), E + 1 entries each
  size_t scale_off[6]; // suh 0..2, svh 0..2 (f16 elements)
  std::vector<int64_t> expert_bytes;  // trellis bytes of gate + up + down per routed expert
  std::vector<int64_t> gu_bytes, dn_bytes;  // trellis bytes of gate+up / down per expert
  exl3_tuning tuning;  // the handle's knobs: staged-path window (diag), weight form
  std::vector<void *> owned;           // device buffers of a loaded layer (exl3_moe_layer_load)
  int64_t loaded_in_place = 0, loaded_repacked = 0;
  int diag_on;
  exl3_moe_diag diag;
  int timing_on;
  exl3_moe_timing timing;
  hipEvent_t ev[5];
  bool ev_made;
  // calls of the long-run kernels with a trellis shared expert: the shared expert's
  // launches go on a second stream, beside the routed ones, joined before the combine
  hipStream_t side;
  hipEvent_t fork, join;
  bool side_made;
  std::mutex mu;
};

namespace exl3h {
void layer_adopt(exl3_moe_layer_t layer, const std::vector<void *> &bufs, int64_t in_place, int64_t repacked) {
  layer->owned.insert(layer->owned.end(), bufs.begin(), bufs.end());
  layer->loaded_in_place += in_place;
  layer->loaded_repacked += repacked;
}
int layer_hidden(exl3_moe_layer_t layer) { return layer->H; }
}  // namespace exl3h

namespace {

struct MoeLayout {
  size_t total;
  size_t logits, weights, ids, sorted_row, sorted_rank, slot_e, slot, run_expert, run_off, run_len,
      n_runs, run_rec, pass_expert, pass_off, pass_len, n_passes, hist;
  size_t yhat_gu, act, yhat_dn, dsh_gu, dsh_act, dsh_dn, xrot;
  int P, R, Imax, S_dn, max_passes;
};

// Calls of at least this many token rows take the long-run expert kernels (one
// accumulator chain over the whole k range: within the reference's staged-path bound of
// the short-run path, not bit-identical to it): EXL3_MOE_LONG_ROWS, read once, default 65
// (at 64 rows the slice-parallel short-run kernels are still faster).
int64_t long_min_rows() {
  static const int64_t v = [] {
    const char *e = std::getenv("EXL3_MOE_LONG_ROWS");
    const long long x = e ? std::atoll(e) : 0;
    return x > 0 ? (int64_t)x : (int64_t)65;
  }();
  return v;
}

// Short-run calls of at least this many token rows rotate each (slot, projection)'s
// input once (k_moe_rotate) and the gate/up workgroups copy it, instead of every
// column block rotating its rows again: EXL3_MOE_XROT_ROWS, read once, default 32 (at
// 64 rows 0.290 -> 0.275 ms; at 8 rows the extra launch costs more than it saves).
int64_t xrot_min_rows() {
  static const int64_t v = [] {
    const char *e = std::getenv("EXL3_MOE_XROT_ROWS");
    const long long x = e ? std::atoll(e) : 0;
    return x > 0 ? (int64_t)x : (int64_t)32;
  }();
  return v;
}

// Token rows staged per pass of the short-run expert kernels (at most 16, one MFMA row
// block): EXL3_MOE_PASS_ROWS, read once. Runs longer than a pass take several passes.
int pass_rows_cap() {
  static const int v = [] {
    const char *e = std::getenv("EXL3_MOE_PASS_ROWS");
    const int x = e ? std::atoi(e) : 0;
    return x >= 1 && x <= 16 ? x : 16;
  }();
  return v;
}

// 128-column blocks per short-run expert workgroup (one ring-word stream per wave over
// the group): EXL3_MOE_ITEMS_GU / EXL3_MOE_ITEMS_DN, read once. No output bit depends on
// them.
int env_items(const char *name, int dflt) {
  const char *e = std::getenv(name);
  const int x = e ? std::atoi(e) : 0;
  return x > 0 ? x : dflt;
}
int gu_items_default() {
  static const int v = env_items("EXL3_MOE_ITEMS_GU", 2);
  return v;
}
// Down: one 128-column block per workgroup (GLM-5 layer: at B=1, 43.7 -> 41.9 us per
// call, where 256 workgroups of two blocks leave most SIMDs one wave; at B=8 the down
// launch 1.0-1.6 us shorter than with two blocks in three A/B runs, three blocks slower).
// EXL3_MOE_ITEMS_DN (read once) overrides it.
int dn_items_default(int64_t N) {
  (void)N;
  static const int v = env_items("EXL3_MOE_ITEMS_DN", 1);
  return v;
}

MoeLayout moe_layout(const exl3_moe_layer_s *L, int64_t N) {
  MoeLayout m{};
  const int H = L->H, I = L->I, E = L->E, K = L->topk, SI = L->shared ? L->SI : 0;
  m.P = (int)(N * K);
  m.R = std::min<int64_t>(E, m.P);
  m.Imax = std::max(I, SI);
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align_up(o + bytes, 256);
    return at;
  };
  const int64_t slots = m.P + N;
  const bool dense = L->shared == exl3m::kSharedDense;
  m.logits = take(4 * N * E * kDenseSlots);
  m.weights = take(4 * (size_t)m.P);
  m.ids = take(4 * (size_t)m.P);
  m.sorted_row = take(4 * (size_t)slots);
  m.sorted_rank = take(4 * (size_t)slots);
  m.slot_e = take(4 * (size_t)slots);
  m.slot = take(4 * (size_t)m.P);
  m.run_expert = take(4 * (size_t)m.R);
  m.run_off = take(4 * (size_t)m.R);
  m.run_len = take(4 * (size_t)m.R);
  m.n_runs = take(4);
  m.run_rec = take(sizeof(exl3m::RunRec) * (size_t)m.R);
  m.max_passes = m.R + (m.P + kLongRows - 1) / kLongRows;
  m.pass_expert = take(4 * (size_t)m.max_passes);
  m.pass_off = take(4 * (size_t)m.max_passes);
  m.pass_len = take(4 * (size_t)m.max_passes);
  m.n_passes = take(4);
  m.hist = take(4 * (size_t)dispatch_wgs(m.P) * E);
  m.yhat_gu = take(4 * (size_t)slots * 2 * moe_slices(H) * m.Imax);
  m.act = take(2 * (size_t)slots * m.Imax);
  m.S_dn = std::max(moe_slices(I), SI > 0 ? moe_slices(SI) : 1);
  m.yhat_dn = take(4 * (size_t)slots * m.S_dn * H);
  m.dsh_gu = take(dense ? 4 * (size_t)2 * N * SI * kDenseSlots : 0);
  m.dsh_act = take(dense ? 2 * (size_t)N * SI : 0);
  m.dsh_dn = take(dense ? 4 * (size_t)N * H * kDenseSlots : 0);
  m.xrot = take(N >= long_min_rows() || N >= xrot_min_rows() ? 2 * (size_t)slots * 2 * H : 0);
  m.total = o;
  return m;
}

MoeArgs make_args(const exl3_moe_layer_s *L, const MoeLayout &m, int64_t N, const uint16_t *h,
                  uint16_t *out, char *ws) {
  MoeArgs a{};
  a.N = (int)N;
  a.H = L->H;
  a.I = L->I;
  a.SI = L->shared ? L->SI : 0;
  a.Imax = m.Imax;
  a.E = L->E;
  a.topk = L->topk;
  a.P = m.P;
  a.R = m.R;
  a.n_group = L->cfg.n_group;
  a.topk_group = L->cfg.topk_group;
  a.norm_topk_prob = L->cfg.norm_topk_prob;
  a.routed_scaling_factor = L->cfg.routed_scaling_factor;
  a.swiglu_limit = L->cfg.swiglu_limit;
  a.shared_kind = L->shared;
  a.logit_splits = dense_mfma_splits(a.H);
  a.n_logit_blocks = (int)dense_mfma_tasks(N, a.H, a.E);  // one task per workgroup
  a.fold = N >= long_min_rows();  // long runs: kLongRows-row passes, slices folded
  a.pass_rows = (int)std::min<int64_t>(N, pass_rows_cap());
  a.xrot_rows = !a.fold && N >= xrot_min_rows();
  a.gu_items = gu_items_default();
  a.dn_items = dn_items_default(N);
  a.h = h;
  a.router_w = L->router_w;
  a.router_bias = L->router_bias;
  a.tab = L->tab_dev;
  for (int j = 0; j < 3; ++j) {
    a.suh_s[j] = L->scales + L->scale_off[j];
    a.svh_s[j] = L->scales + L->scale_off[3 + j];
  }
  for (int j = 0; j < 3; ++j) a.sh_dense[j] = L->sh_dense_t[j];
  a.logits = (float *)(ws + m.logits);
  a.weights = (float *)(ws + m.weights);
  a.ids = (int32_t *)(ws + m.ids);
  a.sorted_row = (int32_t *)(ws + m.sorted_row);
  a.sorted_rank = (int32_t *)(ws + m.sorted_rank);
  a.slot_e = (int32_t *)(ws + m.slot_e);
  a.slot = (int32_t *)(ws + m.slot);
  a.run_expert = (int32_t *)(ws + m.run_expert);
  a.run_off = (int32_t *)(ws + m.run_off);
  a.run_len = (int32_t *)(ws + m.run_len);
  a.n_runs = (int32_t *)(ws + m.n_runs);
  a.run_rec = (exl3m::RunRec *)(ws + m.run_rec);
  a.pass_expert = (int32_t *)(ws + m.pass_expert);
  a.pass_off = (int32_t *)(ws + m.pass_off);
  a.pass_len = (int32_t *)(ws + m.pass_len);
  a.n_passes = (int32_t *)(ws + m.n_passes);
  a.hist = (int32_t *)(ws + m.hist);
  a.yhat_gu = (float *)(ws + m.yhat_gu);
  a.act = (uint16_t *)(ws + m.act);
  a.yhat_dn = (float *)(ws + m.yhat_dn);
  a.S_dn = m.S_dn;
  a.dsh_gu = (float *)(ws + m.dsh_gu);
  a.dsh_act = (uint16_t *)(ws + m.dsh_act);
  a.dsh_dn = (float *)(ws + m.dsh_dn);
  a.xrot = (uint16_t *)(ws + m.xrot);
  a.out = out;
  return a;
}

exl3_status check_linear(const exl3_linear_desc &d, int in, int out, const char *what) {
  if (d.in_features != in || d.out_features != out)
    return fail(EXL3_ERR_INVALID, std::string(what) + ": shape mismatch");
  if (d.dense) return EXL3_OK;
  exl3_status rc = check_desc(&d.tw, true);
  if (rc) return fail(rc, std::string(what) + ": " + exl3_last_error());
  if (d.tw.in_features != in || d.tw.out_features != out)
    return fail(EXL3_ERR_INVALID, std::string(what) + ": trellis shape mismatch");
  return EXL3_OK;
}

// Routing (+ dispatch): one workgroup for up to kRouteOneWg rows (routing and dispatch
// in one launch); above that the rows' routing spreads over workgroups of 16 rows and
// the dispatch follows in a one-workgroup launch.
constexpr int kRouteOneWg = 16;

void launch_route(const MoeArgs &a, float *w_out, int32_t *id_out, int do_dispatch, hipStream_t st) {
  with_route_chunks(a.E, [&](auto jn) {
    constexpr int J = decltype(jn)::value;
    if (a.N <= kRouteOneWg) {
      k_moe_route<J><<<1, 1024, 0, st>>>(a, w_out, id_out, do_dispatch ? 3 : 1);
    } else {
      const unsigned g = (unsigned)std::min<int64_t>((a.N + 15) / 16, 4096);
      k_moe_route<J><<<g, 1024, 0, st>>>(a, w_out, id_out, 1);
      if (do_dispatch) {
        const int G = dispatch_wgs(a.P);
        if (G == 1) {
          k_moe_route<J><<<1, 1024, 0, st>>>(a, w_out, id_out, 2);
        } else {
          k_moe_count<<<G, 1024, 0, st>>>(a, id_out);
          k_moe_dispatch<<<G, 1024, 0, st>>>(a, id_out, G);
        }
      }
    }
  });
}

// L1 + L2: logits, then routing/dispatch. w_out / id_out receive the routing.
exl3_status launch_logits_route(exl3_moe_layer_s *L, const MoeArgs &a, float *w_out, int32_t *id_out,
                                int do_dispatch, hipStream_t st) {
  (void)L;
  if (a.N >= kPreTiledMinRows && (a.N + kPreTile - 1) / kPreTile <= 65535) {
    const dim3 grid((unsigned)dense_mfma_splits(a.H), (unsigned)((a.E + kPreTile - 1) / kPreTile),
                    (unsigned)((a.N + kPreTile - 1) / kPreTile));
    k_moe_pre_tiled<<<grid, 256, 0, st>>>(a);
    EXL3_LAUNCHED("k_moe_pre_tiled");
  } else {
    k_moe_pre<<<a.n_logit_blocks, 256, 0, st>>>(a);
    EXL3_LAUNCHED("k_moe_pre");
  }
  launch_route(a, w_out, id_out, do_dispatch, st);
  EXL3_LAUNCHED("k_moe_route");
  return EXL3_OK;
}

exl3_status check_ws(void *ws, size_t bytes, size_t need) {
  if (!ws || bytes < need)
    return fail(EXL3_ERR_WORKSPACE, "workspace too small: need " + std::to_string(need) +
                                        " bytes, got " + std::to_string(bytes));
  if (reinterpret_cast<uintptr_t>(ws) % 256)
    return fail(EXL3_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return EXL3_OK;
}

}  // namespace

extern "C" {

exl3_status exl3_moe_layer_create(const exl3_moe_layer_desc *desc, const exl3_moe_config *cfg,
                                  exl3_moe_layer_t *out) {
  if (!desc || !cfg || !out) return fail(EXL3_ERR_INVALID, "null argument");
  *out = nullptr;
  const int H = cfg->hidden_size, I = cfg->moe_intermediate_size, E = cfg->n_routed_experts;
  const int K = cfg->num_experts_per_tok;
  if (H <= 0 || H % 128 || I <= 0 || I % 128)
    return fail(EXL3_ERR_INVALID, "hidden and intermediate sizes must be positive multiples of 128");
  if (H > 8192 || I > 8192)
    return fail(EXL3_ERR_UNSUPPORTED, "hidden and intermediate sizes must be <= 8192");
  if (E <= 0 || E > 1024) return fail(EXL3_ERR_UNSUPPORTED, "n_routed_experts must be in 1..1024");
  if (K <= 0 || K > E || K > 64) return fail(EXL3_ERR_INVALID, "num_experts_per_tok must be in 1..min(E, 64)");
  const int ng = cfg->n_group > 1 ? cfg->n_group : 1;
  if (ng > 64 || E % ng) return fail(EXL3_ERR_INVALID, "n_group must divide E and be <= 64");
  if (!desc->experts || !desc->router_w || !desc->router_bias)
    return fail(EXL3_ERR_INVALID, "missing experts or router tensors");
  const exl3_linear_desc *ex = desc->experts;
  for (int e = 0; e < E; ++e) {
    for (int j = 0; j < 3; ++j) {
      const exl3_linear_desc &d = ex[3 * e + j];
      exl3_status rc = check_linear(d, j == 2 ? I : H, j == 2 ? H : I, "expert");
      if (rc) return rc;
      if (d.dense) return fail(EXL3_ERR_UNSUPPORTED, "routed experts must be EXL3 trellis tensors");
      const exl3_linear_desc &r0 = ex[j == 2 ? 2 : 0];
      if (d.tw.K != r0.tw.K || d.tw.codebook != r0.tw.codebook)
        return fail(EXL3_ERR_INVALID,
                    "every routed gate/up (and every down) projection must share K and codebook");
    }
  }
  auto *L = new exl3_moe_layer_s();
  L->cfg = *cfg;
  L->H = H;
  L->I = I;
  L->E = E;
  L->topk = K;
  L->gu_K = ex[0].tw.K;
  L->gu_cb = ex[0].tw.codebook;
  L->dn_K = ex[2].tw.K;
  L->dn_cb = ex[2].tw.codebook;
  L->router_w = desc->router_w;
  L->router_bias = desc->router_bias;
  L->shared = 0;
  L->SI = 0;
  if (desc->shared) {
    const exl3_linear_desc *sh = desc->shared;
    const int SI = sh[0].out_features;
    if (SI <= 0 || SI % 128) {
      delete L;
      return fail(EXL3_ERR_INVALID, "shared intermediate must be a positive multiple of 128");
    }
    if (SI > 8192) {
      delete L;
      return fail(EXL3_ERR_UNSUPPORTED, "shared intermediate size must be <= 8192");
    }
    for (int j = 0; j < 3; ++j) {
      exl3_status rc = check_linear(sh[j], j == 2 ? SI : H, j == 2 ? H : SI, "shared expert");
      if (rc) {
        delete L;
        return rc;
      }
    }
    const bool dense = sh[0].dense && sh[1].dense && sh[2].dense;
    const bool quant = !sh[0].dense && !sh[1].dense && !sh[2].dense;
    if (!dense && !quant) {
      delete L;
      return fail(EXL3_ERR_UNSUPPORTED, "shared expert must be all-trellis or all-f16");
    }
    if (quant && (sh[0].tw.K != sh[1].tw.K || sh[0].tw.codebook != sh[1].tw.codebook)) {
      delete L;
      return fail(EXL3_ERR_INVALID, "shared gate/up must share K and codebook");
    }
    L->SI = SI;
    L->shared = dense ? 2 : 1;
    L->sh_K = quant ? sh[0].tw.K : 0;
    L->sh_cb = quant ? sh[0].tw.codebook : 0;
    L->sh_dn_K = quant ? sh[2].tw.K : 0;
    L->sh_dn_cb = quant ? sh[2].tw.codebook : 0;
    for (int j = 0; j < 3; ++j) L->sh_dense[j] = sh[j].dense;
    if (dense) {
      const size_t n = (size_t)H * SI;
      hipError_t e0 = hipMalloc(&L->sh_dense_t[0], 3 * n * sizeof(uint16_t));
      if (e0 != hipSuccess) {
        delete L;
        return hip_check(e0, "hipMalloc(shared expert copy)");
      }
      L->sh_dense_t[1] = L->sh_dense_t[0] + n;
      L->sh_dense_t[2] = L->sh_dense_t[0] + 2 * n;
      for (int j = 0; j < 3 && e0 == hipSuccess; ++j) {
        const int in = j == 2 ? SI : H, out_f = j == 2 ? H : SI;
        k_transpose_f16<<<dim3((out_f + 63) / 64, (in + 63) / 64), 256, 0, 0>>>(
            sh[j].dense, in, out_f, L->sh_dense_t[j]);
        e0 = hipGetLastError();
      }
      if (e0 == hipSuccess) e0 = hipStreamSynchronize(0);
      if (e0 != hipSuccess) {
        (void)hipFree(L->sh_dense_t[0]);
        delete L;
        return hip_check(e0, "transpose(shared expert)");
      }
    }
  }
  std::vector<ExpertTab> tab((size_t)E + 1);
  L->expert_bytes.resize(E);
  L->gu_bytes.resize(E);
  L->dn_bytes.resize(E);
  for (int e = 0; e < E; ++e) {
    int64_t bytes[3];
    for (int j = 0; j < 3; ++j) {
      const exl3_trellis_desc &t = ex[3 * e + j].tw;
      tab[e].tr[j] = (const uint32_t *)t.trellis;
      tab[e].suh[j] = t.suh;
      tab[e].svh[j] = t.svh;
      bytes[j] = (int64_t)t.in_features * t.out_features / 256 * 32 * t.K;
    }
    L->gu_bytes[e] = bytes[0] + bytes[1];
    L->dn_bytes[e] = bytes[2];
    L->expert_bytes[e] = bytes[0] + bytes[1] + bytes[2];
  }
  if (L->shared == 1) {
    for (int j = 0; j < 3; ++j) {
      const exl3_trellis_desc &t = desc->shared[j].tw;
      tab[E].tr[j] = (const uint32_t *)t.trellis;
      tab[E].suh[j] = t.suh;
      tab[E].svh[j] = t.svh;
    }
  }
  hipError_t e1 = hipMalloc(&L->tab_dev, sizeof(ExpertTab) * tab.size());
  if (e1 != hipSuccess) {
    if (L->sh_dense_t[0]) (void)hipFree(L->sh_dense_t[0]);
    delete L;
    return hip_check(e1, "hipMalloc(expert table)");
  }
  e1 = hipMemcpy(L->tab_dev, tab.data(), sizeof(ExpertTab) * tab.size(), hipMemcpyHostToDevice);
  if (e1 != hipSuccess) {
    (void)hipFree(L->tab_dev);
    if (L->sh_dense_t[0]) (void)hipFree(L->sh_dense_t[0]);
    delete L;
    return hip_check(e1, "hipMemcpy(expert table)");
  }
  {
    // stacked scales: suh 0,1 (E+1, H), suh 2 (E+1, Imax), svh 0,1 (E+1, Imax), svh 2 (E+1, H)
    const int Imax = std::max(I, L->SI);
    const size_t rows = (size_t)E + 1;
    const size_t sz[6] = {rows * H, rows * H, rows * Imax, rows * Imax, rows * Imax, rows * H};
    size_t total = 0;
    for (int j = 0; j < 6; ++j) {
      L->scale_off[j] = total;
      total += align_up(sz[j], 128);
    }
    hipError_t e2 = hipMalloc(&L->scales, total * sizeof(uint16_t));
    if (e2 == hipSuccess) e2 = hipMemset(L->scales, 0, total * sizeof(uint16_t));
    if (e2 == hipSuccess) {
      ScaleGather g{};
      for (int j = 0; j < 3; ++j) {
        g.suh[j] = L->scales + L->scale_off[j];
        g.svh[j] = L->scales + L->scale_off[3 + j];
      }
      const int SI = L->SI;
      const int in_r[3] = {H, H, I}, out_r[3] = {I, I, H};
      const int in_s[3] = {H, H, SI}, out_s[3] = {SI, SI, H};
      for (int j = 0; j < 3; ++j) {
        g.len_in[0][j] = in_r[j];
        g.len_out[0][j] = out_r[j];
        g.len_in[1][j] = L->shared == 1 ? in_s[j] : 0;
        g.len_out[1][j] = L->shared == 1 ? out_s[j] : 0;
      }
      g.stride_in[0] = H;
      g.stride_in[1] = H;
      g.stride_in[2] = Imax;
      g.stride_out[0] = Imax;
      g.stride_out[1] = Imax;
      g.stride_out[2] = H;
      k_gather_scales<<<(unsigned)(rows * 3), 256, 0, 0>>>(L->tab_dev, E, g);
      e2 = hipGetLastError();
      if (e2 == hipSuccess) e2 = hipStreamSynchronize(0);
    }
    if (e2 != hipSuccess) {
      if (L->scales) (void)hipFree(L->scales);
      (void)hipFree(L->tab_dev);
      if (L->sh_dense_t[0]) (void)hipFree(L->sh_dense_t[0]);
      delete L;
      return hip_check(e2, "stacked scales");
    }
  }
  L->tuning = tuning();
  L->diag_on = 0;
  std::memset(&L->diag, 0, sizeof(L->diag));
  L->timing_on = 0;
  std::memset(&L->timing, 0, sizeof(L->timing));
  L->ev_made = false;
  L->side_made = false;
  if (L->shared == exl3m::kSharedTrellis) {
    // the second stream of long-run calls, made here so that no call creates it (a
    // call may be under graph capture)
    hipError_t e3 = hipStreamCreateWithFlags(&L->side, hipStreamNonBlocking);
    if (e3 == hipSuccess) {
      e3 = hipEventCreateWithFlags(&L->fork, hipEventDisableTiming);
      if (e3 == hipSuccess) {
        e3 = hipEventCreateWithFlags(&L->join, hipEventDisableTiming);
        if (e3 == hipSuccess) L->side_made = true;
        else (void)hipEventDestroy(L->fork);
      }
      if (!L->side_made) (void)hipStreamDestroy(L->side);
    }
    if (!L->side_made) {
      (void)exl3_moe_layer_destroy(L);
      return hip_check(e3, "layer stream");
    }
  }
  *out = L;
  return EXL3_OK;
}

exl3_status exl3_moe_layer_destroy(exl3_moe_layer_t layer) {
  if (!layer) return EXL3_OK;
  for (void *p : layer->owned) (void)hipFree(p);
  layer->owned.clear();
  if (layer->ev_made)
    for (int i = 0; i < 5; ++i) (void)hipEventDestroy(layer->ev[i]);
  if (layer->side_made) {
    (void)hipEventDestroy(layer->fork);
    (void)hipEventDestroy(layer->join);
    (void)hipStreamDestroy(layer->side);
  }

  if (layer->scales) (void)hipFree(layer->scales);
  if (layer->sh_dense_t[0]) {
    hipError_t e = hipFree(layer->sh_dense_t[0]);
    if (e != hipSuccess) {
      (void)hipFree(layer->tab_dev);
      delete layer;
      return hip_check(e, "hipFree(shared expert copy)");
    }
  }
  if (layer->tab_dev) {
    hipError_t e = hipFree(layer->tab_dev);
    if (e != hipSuccess) {
      delete layer;
      return hip_check(e, "hipFree(expert table)");
    }
  }
  delete layer;
  return EXL3_OK;
}

size_t exl3_moe_workspace_size(exl3_moe_layer_t layer, int64_t rows) {
  if (!layer || rows <= 0 || rows > (1 << 24) / layer->topk) return 0;  // as exl3_moe_layer's limit
  return moe_layout(layer, rows).total;
}

exl3_status exl3_moe_route(exl3_moe_layer_t layer, const uint16_t *h, int64_t rows, float *weights,
                           int32_t *ids, void *workspace, size_t workspace_bytes,
                           exl3_stream_t stream) {
  if (!layer || !h || !weights || !ids || rows < 0) return fail(EXL3_ERR_INVALID, "bad route arguments");
  if (rows == 0) return EXL3_OK;
  const MoeLayout m = moe_layout(layer, rows);
  exl3_status rc = check_ws(workspace, workspace_bytes, m.total);
  if (rc) return rc;
  const MoeArgs a = make_args(layer, m, rows, h, nullptr, (char *)workspace);
  return launch_logits_route(layer, a, weights, ids, 0, stream_of(stream));
}

exl3_status exl3_moe_topk_route(const float *logits, const float *bias, int64_t rows,
                                const exl3_moe_config *cfg, float *weights, int32_t *ids,
                                exl3_stream_t stream) {
  if (!logits || !bias || !cfg || !weights || !ids || rows < 0)
    return fail(EXL3_ERR_INVALID, "bad topk_route arguments");
  const int E = cfg->n_routed_experts, K = cfg->num_experts_per_tok;
  const int ng = cfg->n_group > 1 ? cfg->n_group : 1;
  if (E <= 0 || E > 1024) return fail(EXL3_ERR_UNSUPPORTED, "n_routed_experts must be in 1..1024");
  if (K <= 0 || K > E || K > 64) return fail(EXL3_ERR_INVALID, "num_experts_per_tok must be in 1..min(E, 64)");
  if (ng > 64 || E % ng) return fail(EXL3_ERR_INVALID, "n_group must divide E and be <= 64");
  if (rows == 0) return EXL3_OK;
  if (rows > (1 << 24)) return fail(EXL3_ERR_UNSUPPORTED, "too many rows");
  MoeArgs a{};
  a.N = (int)rows;
  a.E = E;
  a.topk = K;
  a.P = (int)(rows * K);
  a.n_group = cfg->n_group;
  a.topk_group = cfg->topk_group;
  a.norm_topk_prob = cfg->norm_topk_prob;
  a.routed_scaling_factor = cfg->routed_scaling_factor;
  a.router_bias = bias;
  a.logits = const_cast<float *>(logits);
  a.logit_splits = 0;  // plain (N, E) logits
  launch_route(a, weights, ids, 0, stream_of(stream));
  EXL3_LAUNCHED("k_moe_route");
  return EXL3_OK;
}

namespace {
// EXL3_MOE_SIDE_STREAM=0 keeps the trellis shared expert on the caller's stream.
bool side_stream_on() {
  static const bool v = [] {
    const char *e = std::getenv("EXL3_MOE_SIDE_STREAM");
    return !(e && std::atoi(e) == 0);
  }();
  return v;
}

// The trellis shared expert: every token row through the expert kernels (one run of
// the short-run kernels, or kLongRows-row passes of the long-run kernels).
exl3_status launch_shared_trellis(const exl3_moe_layer_s *layer, const MoeArgs &a, int64_t N,
                                  hipStream_t st) {
  const int64_t sh_units = a.fold ? (N + kLongRows - 1) / kLongRows : 1;
  exl3_status rc = launch_moe_expert(0, layer->sh_K, kernel_cb(layer->sh_cb, a.weight_form), sh_units, a, 1,
                                     false, st);
  if (rc) return rc;
  rc = launch_moe_act(a, 1, 0, st);
  if (rc) return rc;
  return launch_moe_expert(1, layer->sh_dn_K, kernel_cb(layer->sh_dn_cb, a.weight_form), sh_units, a, 1,
                           false, st);
}
}  // namespace

}  // extern "C"

namespace {

// Rows of one layer call (checked), or a status.
exl3_status call_rows(exl3_moe_layer_t layer, const uint16_t *h, const uint16_t *out, int64_t B,
                      int64_t Lq, int64_t &N) {
  if (!layer || !h || !out || B < 0 || Lq < 0) return fail(EXL3_ERR_INVALID, "bad layer arguments");
  if (B > 0 && Lq > ((int64_t)1 << 24) / B) return fail(EXL3_ERR_UNSUPPORTED, "too many rows in one call");
  N = B * Lq;  // no overflow: checked above
  if (N > (1 << 24) / layer->topk) return fail(EXL3_ERR_UNSUPPORTED, "too many rows in one call");
  return EXL3_OK;
}

// The hyper-connection mix fused behind the combine (exl3_moe_block).
struct HcEpilogue {
  int n;
  const float *post, *comb;
  const uint16_t *residual;
  uint16_t *streams_out;
};

exl3_status moe_layer_run(exl3_moe_layer_t layer, const uint16_t *h, int64_t N, uint16_t *out,
                          void *workspace, const MoeLayout &m, exl3_stream_t stream, bool instrumented,
                          const HcEpilogue *epi = nullptr);

}  // namespace

// ---------------------------------------------------------------------------------
// Allocation-free calls: the workspace is this file-scope device array (one copy per
// GPU, held until the process ends), not caller memory. Its device address is looked
// up once per device with that device current; host code uses only that address (the
// array's name is a host-side stand-in).
// ---------------------------------------------------------------------------------
constexpr size_t kScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
struct ScratchSlot {
  std::once_flag once;
  hipError_t rc = hipSuccess;
  void *ptr = nullptr;
};
ScratchSlot g_scratch[kMaxDevices];

exl3_status scratch_of_current_device(void **ptr) {
  int dev = 0;
  EXL3_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(EXL3_ERR_UNSUPPORTED, "device index beyond the scratch table");
  ScratchSlot &sl = g_scratch[dev];
  std::call_once(sl.once, [&] {
    void *p = nullptr;
    sl.rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (sl.rc == hipSuccess) sl.ptr = p;
  });
  if (sl.rc != hipSuccess || !sl.ptr) return hip_check(sl.rc == hipSuccess ? hipErrorInvalidSymbol : sl.rc,
                                                      "hipGetSymbolAddress(scratch)");
  *ptr = sl.ptr;
  return EXL3_OK;
}

}  // namespace

extern "C" {

size_t exl3_moe_scratch_capacity(void) { return kScratchBytes; }

exl3_status exl3_moe_layer_noalloc(exl3_moe_layer_t layer, const uint16_t *h, int64_t B, int64_t L,
                                   uint16_t *out, exl3_stream_t stream) {
  int64_t N = 0;
  exl3_status rc = call_rows(layer, h, out, B, L, N);
  if (rc) return rc;
  if (N == 0) return EXL3_OK;
  const MoeLayout m = moe_layout(layer, N);
  if (m.total > kScratchBytes)
    return fail(EXL3_ERR_UNSUPPORTED, "exl3_moe_layer_noalloc: this call needs " + std::to_string(m.total) +
                                          " bytes of workspace, above the " + std::to_string(kScratchBytes) +
                                          "-byte scratch array (use exl3_moe_layer with a caller workspace)");
  void *ws = nullptr;
  rc = scratch_of_current_device(&ws);
  if (rc) return rc;
  return moe_layer_run(layer, h, N, out, ws, m, stream, false);
}

namespace {
// exl3_moe_block's workspace: the hyper-connection partials, the normalised rows h, post,
// comb, the MoE output rows, then the layer call's own workspace.
struct BlockLayout {
  size_t part, h, post, comb, out, moe, total;
};
BlockLayout block_layout(exl3_moe_layer_t layer, int n, int64_t P, const MoeLayout &m) {
  BlockLayout b{};
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align_up(o + bytes, 256);
    return at;
  };
  b.part = take(hc_part_bytes(n, layer->H, P));
  b.h = take(2 * (size_t)P * layer->H);
  b.post = take(4 * (size_t)P * n);
  b.comb = take(4 * (size_t)P * n * n);
  b.out = take(2 * (size_t)P * layer->H);
  b.moe = take(m.total);
  b.total = o;
  return b;
}
}  // namespace

size_t exl3_moe_block_workspace_size(exl3_moe_layer_t layer, int32_t hc_mult, int64_t P) {
  if (!layer || P < 0 || hc_mult < 1 || hc_mult > 8 || check_hc_shape(hc_mult, layer->H)) return 0;
  if (P == 0) return 0;
  if (P > (1 << 24) / layer->topk) return 0;
  return block_layout(layer, hc_mult, P, moe_layout(layer, P)).total;
}

exl3_status exl3_moe_block(exl3_moe_layer_t layer, const exl3_hc_site *hc, const uint16_t *norm_w, float norm_eps,
                           const uint16_t *streams, int64_t P, uint16_t *streams_out, void *workspace,
                           size_t workspace_bytes, exl3_stream_t stream) {
  if (!layer || P < 0) return fail(EXL3_ERR_INVALID, "bad block arguments");
  exl3_status rc = check_hc(hc, layer->H);
  if (rc) return rc;
  if (P == 0) return EXL3_OK;
  if (!norm_w || !streams || !streams_out) return fail(EXL3_ERR_INVALID, "null block argument");
  if (P > (1 << 24) / layer->topk) return fail(EXL3_ERR_UNSUPPORTED, "too many rows in one call");
  if (reinterpret_cast<uintptr_t>(streams) % 8 || reinterpret_cast<uintptr_t>(streams_out) % 4 ||
      reinterpret_cast<uintptr_t>(norm_w) % 4 || reinterpret_cast<uintptr_t>(hc->fn) % 16)
    return fail(EXL3_ERR_INVALID, "streams must be 8-byte, streams_out and norm_w 4-byte, fn 16-byte aligned");
  if (overlaps(streams, streams_out, (size_t)P * hc->mult * layer->H * 2))
    return fail(EXL3_ERR_INVALID, "streams_out must not overlap streams");
  const MoeLayout m = moe_layout(layer, P);
  const BlockLayout b = block_layout(layer, hc->mult, P, m);
  rc = check_ws(workspace, workspace_bytes, b.total);
  if (rc) return rc;
  char *ws = (char *)workspace;
  uint16_t *h = (uint16_t *)(ws + b.h);
  float *post = (float *)(ws + b.post), *comb = (float *)(ws + b.comb);
  hipStream_t st = stream_of(stream);
  // hc_prepare + rms_norm (glm5_forward.cpp:435-436)
  rc = launch_hc_prepare(hc, streams, P, layer->H, norm_w, norm_eps, h, post, comb, (float *)(ws + b.part), st);
  if (rc) return rc;
  // moe_layer_rows (:437) with g5_hc_mix (:438) behind its combine
  const HcEpilogue epi{hc->mult, post, comb, streams, streams_out};
  return moe_layer_run(layer, h, P, (uint16_t *)(ws + b.out), ws + b.moe, m, stream, true, &epi);
}

exl3_status exl3_moe_layer(exl3_moe_layer_t layer, const uint16_t *h, int64_t B, int64_t Lq,
                           uint16_t *out, void *workspace, size_t workspace_bytes,
                           exl3_stream_t stream) {
  int64_t N = 0;
  exl3_status rc = call_rows(layer, h, out, B, Lq, N);
  if (rc) return rc;
  if (N == 0) return EXL3_OK;
  const MoeLayout m = moe_layout(layer, N);
  rc = check_ws(workspace, workspace_bytes, m.total);
  if (rc) return rc;
  return moe_layer_run(layer, h, N, out, workspace, m, stream, true);
}

}  // extern "C"

namespace {

// MoeRowsDiag of one finished call (synchronises the stream).
exl3_status collect_diag(exl3_moe_layer_t layer, const MoeArgs &a, const MoeLayout &m, hipStream_t st) {
  std::lock_guard<std::mutex> lk(layer->mu);
  EXL3_HIP(hipStreamSynchronize(st));
  int32_t nr = 0;
  EXL3_HIP(hipMemcpy(&nr, a.n_runs, 4, hipMemcpyDeviceToHost));
  std::vector<int32_t> rl(nr), re(nr);
  if (nr > 0) {
    EXL3_HIP(hipMemcpy(rl.data(), a.run_len, 4 * (size_t)nr, hipMemcpyDeviceToHost));
    EXL3_HIP(hipMemcpy(re.data(), a.run_expert, 4 * (size_t)nr, hipMemcpyDeviceToHost));
  }
  exl3_moe_diag &d = layer->diag;
  d.calls += 1;
  d.pairs += m.P;
  d.runs += nr;
  d.distinct_experts += nr;
  // a run's weights are streamed once per pass: passes of pass_rows rows on the
  // short-run kernels, of kLongRows rows on the long-run ones (glm5_moe.cpp:280-287
  // counts trellis_path_info(tw, r).passes the same way); a run counts as staged by
  // the handle's mat_min_rows/mat_max_rows window
  const int prow = a.fold ? kLongRows : a.pass_rows;
  const exl3_tuning &tn = layer->tuning;
  for (int i = 0; i < nr; ++i) {
    const int r = rl[i];
    d.run_hist[r >= 64 ? 64 : r] += 1;
    d.shared_bytes += layer->expert_bytes[re[i]];
    d.streamed_bytes += layer->expert_bytes[re[i]] * ((r + prow - 1) / prow);
    if (tn.mat_min_rows > 0 && r >= tn.mat_min_rows && (tn.mat_max_rows <= 0 || r <= tn.mat_max_rows))
      d.staged_runs += 1;
  }
  return EXL3_OK;
}

// One layer call over N token rows with its workspace. instrumented: honour the
// handle's timing and diagnostics (both synchronise the stream; the allocation-free
// entry point skips them).
exl3_status moe_layer_run(exl3_moe_layer_t layer, const uint16_t *h, int64_t N, uint16_t *out,
                          void *workspace, const MoeLayout &m, exl3_stream_t stream, bool instrumented,
                          const HcEpilogue *epi) {
  exl3_status rc = EXL3_OK;
  hipStream_t st = stream_of(stream);
  MoeArgs a = make_args(layer, m, N, h, out, (char *)workspace);
  {
    // the handle's weight form, read once per call
    std::lock_guard<std::mutex> lk(layer->mu);
    a.weight_form = layer->tuning.weight_form;
  }
  if (epi) {
    a.hc_n = epi->n;
    a.hc_post = epi->post;
    a.hc_comb = epi->comb;
    a.hc_res = epi->residual;
    a.hc_out = epi->streams_out;
  }
  const bool timed = instrumented && layer->timing_on != 0;
  if (timed && !layer->ev_made) {
    for (int i = 0; i < 5; ++i) EXL3_HIP(hipEventCreate(&layer->ev[i]));
    layer->ev_made = true;
  }
  const int H = layer->H;
  const bool dense_sh = layer->shared == exl3m::kSharedDense;
  const bool trellis_sh = layer->shared == exl3m::kSharedTrellis;
  const int64_t units = a.fold ? m.max_passes : m.R;  // work units: runs or long-run passes
  // Long-run calls: a trellis shared expert (under one wave of the machine on its own)
  // does not depend on the routing, so it runs on the layer's second stream from the
  // start of the call: beside the router and the dispatch (latency-bound launches that
  // leave most of the machine idle), then beside the routed experts.
  const bool side = a.fold && layer->side_made && side_stream_on();
  // Every return after the fork joins the side stream back into the caller's (an
  // unjoined fork would leave a graph capture of this call unable to end).
  bool forked = false;
  auto join_side = [&](bool locked) {
    if (!forked) return;
    forked = false;
    std::unique_lock<std::mutex> lk(layer->mu, std::defer_lock);
    if (!locked) lk.lock();
    (void)hipEventRecord(layer->join, layer->side);
    (void)hipStreamWaitEvent(st, layer->join, 0);
  };
  auto fail_joined = [&](exl3_status r) {
    join_side(false);
    return r;
  };
  if (timed) EXL3_HIP(hipEventRecord(layer->ev[0], st));
  if (side) {
    // one caller at a time records the fork and join (calls on other threads and
    // streams would otherwise interleave them)
    std::lock_guard<std::mutex> lk(layer->mu);
    EXL3_HIP(hipEventRecord(layer->fork, st));
    EXL3_HIP(hipStreamWaitEvent(layer->side, layer->fork, 0));
    forked = true;
    rc = launch_moe_rotate(a, a.P, N, layer->side);  // the shared slots: row i at slot P + i
    if (!rc) rc = launch_shared_trellis(layer, a, N, layer->side);
    if (rc) {
      join_side(true);
      return rc;
    }
    const hipError_t e = hipEventRecord(layer->join, layer->side);
    if (e != hipSuccess) {
      join_side(true);
      return hip_check(e, "hipEventRecord(join)");
    }
  }
  rc = launch_logits_route(layer, a, a.weights, a.ids, 1, st);
  if (rc) return fail_joined(rc);
  if (timed) {
    const hipError_t e = hipEventRecord(layer->ev[1], st);
    if (e != hipSuccess) return fail_joined(hip_check(e, "hipEventRecord"));
  }
  // L3: routed gate/up (+ the f16 shared expert's gate/up partials), after the input
  // rotation of the routed slots (and of a trellis shared expert's slots when it runs on
  // this stream)
  if (a.fold || a.xrot_rows) {
    rc = launch_moe_rotate(a, 0, (int64_t)a.P + (trellis_sh && !side ? N : 0), st);
    if (rc) return fail_joined(rc);
  }
  rc = launch_moe_expert(0, layer->gu_K, kernel_cb(layer->gu_cb, a.weight_form), units, a, 0, dense_sh, st);
  if (rc) return fail_joined(rc);
  if (timed) {
    const hipError_t e = hipEventRecord(layer->ev[2], st);
    if (e != hipSuccess) return fail_joined(hip_check(e, "hipEventRecord"));
  }
  // L4: routed SwiGLU activations (+ the f16 shared expert's SwiGLU), L5: routed down
  // (+ the f16 shared expert's down partials)
  rc = launch_moe_act(a, 0, dense_sh ? shared_swiglu_blocks(N, layer->SI) : 0, st);
  if (rc) return fail_joined(rc);
  rc = launch_moe_expert(1, layer->dn_K, kernel_cb(layer->dn_cb, a.weight_form), units, a, 0, dense_sh, st);
  if (rc) return fail_joined(rc);
  if (timed) {
    const hipError_t e = hipEventRecord(layer->ev[3], st);
    if (e != hipSuccess) return fail_joined(hip_check(e, "hipEventRecord"));
  }
  // a trellis shared expert: one run of every token row through the same kernels
  if (side) {
    const hipError_t e = hipStreamWaitEvent(st, layer->join, 0);
    if (e != hipSuccess) return fail_joined(hip_check(e, "hipStreamWaitEvent(join)"));
    forked = false;
  } else if (layer->shared == exl3m::kSharedTrellis) {
    rc = launch_shared_trellis(layer, a, N, st);
    if (rc) return rc;
  }
  // L6: combine
  if (a.fold)
    k_moe_combine<true><<<(unsigned)((N * (H / 128) + 3) / 4), 256, 0, st>>>(a);
  else
    // one wave per workgroup: the waves' loads spread over every CU (5.48 -> 5.11 us at
    // B=8 against four-wave workgroups)
    k_moe_combine<false><<<(unsigned)(N * (H / 128)), 64, 0, st>>>(a);
  EXL3_LAUNCHED("k_moe_combine");
  if (timed) {
    EXL3_HIP(hipEventRecord(layer->ev[4], st));
    EXL3_HIP(hipEventSynchronize(layer->ev[4]));
    float ms[4];
    for (int i = 0; i < 4; ++i) EXL3_HIP(hipEventElapsedTime(&ms[i], layer->ev[i], layer->ev[i + 1]));
    int32_t nr = 0;
    EXL3_HIP(hipMemcpy(&nr, a.n_runs, 4, hipMemcpyDeviceToHost));
    std::vector<int32_t> re(nr);
    if (nr > 0) EXL3_HIP(hipMemcpy(re.data(), a.run_expert, 4 * (size_t)nr, hipMemcpyDeviceToHost));
    std::lock_guard<std::mutex> lk(layer->mu);
    exl3_moe_timing &t = layer->timing;
    t.calls += 1;
    t.router_ms += ms[0];
    t.gate_up_ms += ms[1];
    t.down_ms += ms[2];
    t.combine_ms += ms[3];
    t.total_ms += ms[0] + ms[1] + ms[2] + ms[3];
    for (int i = 0; i < nr; ++i) {
      t.gate_up_trellis_bytes += layer->gu_bytes[re[i]];
      t.down_trellis_bytes += layer->dn_bytes[re[i]];
    }
  }

  if (instrumented && layer->diag_on) return collect_diag(layer, a, m, st);
  return EXL3_OK;
}

}  // namespace

extern "C" {

exl3_status exl3_moe_timing_enable(exl3_moe_layer_t layer, int32_t enabled) {
  if (!layer) return fail(EXL3_ERR_INVALID, "null layer");
  layer->timing_on = enabled ? 1 : 0;
  return EXL3_OK;
}

exl3_status exl3_moe_timing_get(exl3_moe_layer_t layer, exl3_moe_timing *out) {
  if (!layer || !out) return fail(EXL3_ERR_INVALID, "null argument");
  std::lock_guard<std::mutex> lk(layer->mu);
  *out = layer->timing;
  return EXL3_OK;
}

exl3_status exl3_moe_timing_reset(exl3_moe_layer_t layer) {
  if (!layer) return fail(EXL3_ERR_INVALID, "null layer");
  std::lock_guard<std::mutex> lk(layer->mu);
  std::memset(&layer->timing, 0, sizeof(layer->timing));
  return EXL3_OK;
}

exl3_status exl3_moe_diag_enable(exl3_moe_layer_t layer, int32_t enabled) {
  if (!layer) return fail(EXL3_ERR_INVALID, "null layer");
  layer->diag_on = enabled ? 1 : 0;
  return EXL3_OK;
}

exl3_status exl3_moe_diag_get(exl3_moe_layer_t layer, exl3_moe_diag *out) {
  if (!layer || !out) return fail(EXL3_ERR_INVALID, "null argument");
  std::lock_guard<std::mutex> lk(layer->mu);
  *out = layer->diag;
  return EXL3_OK;
}

exl3_status exl3_moe_layer_load_info(exl3_moe_layer_t layer, int64_t *in_place, int64_t *repacked) {
  if (!layer || !in_place || !repacked) return fail(EXL3_ERR_INVALID, "null argument");
  *in_place = layer->loaded_in_place;
  *repacked = layer->loaded_repacked;
  return EXL3_OK;
}

exl3_status exl3_moe_set_tuning(exl3_moe_layer_t layer, const exl3_tuning *t) {
  if (!layer) return fail(EXL3_ERR_INVALID, "null argument");
  exl3_status rc = check_tuning(t);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(layer->mu);
  layer->tuning = *t;
  return EXL3_OK;
}

exl3_status exl3_moe_get_tuning(exl3_moe_layer_t layer, exl3_tuning *t) {
  if (!layer || !t) return fail(EXL3_ERR_INVALID, "null argument");
  std::lock_guard<std::mutex> lk(layer->mu);
  *t = layer->tuning;
  return EXL3_OK;
}

exl3_status exl3_moe_diag_reset(exl3_moe_layer_t layer) {
  if (!layer) return fail(EXL3_ERR_INVALID, "null layer");
  std::lock_guard<std::mutex> lk(layer->mu);
  std::memset(&layer->diag, 0, sizeof(layer->diag));
  return EXL3_OK;
}

}  // extern "C"
