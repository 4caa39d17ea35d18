// The dequant-GEMV core shared by the standalone linear and the MoE expert kernels:
// trellis decode in VALU registers, products on the matrix cores.
//
// Wave step. One wave step covers 4 k-tiles x 2 n-tiles (64 k x 32 output columns).
// Lane l = 16*kt + 8*nt + m loads ring words [m*K - 1, m*K + K) of tile (k0 + kt,
// n0 + nt): the bit range of reference lanes 4m..4m+3 (exl3.cpp:84-99), i.e. all 16
// k-rows of columns m and m + 8 of that tile (exl3_device.hpp). It decodes them as 8
// "quads" of 4 weights, quad (j, h) = stream positions 8j + 4h + 0..3 = k-rows
// {2j, 2j+1, 2j+8, 2j+9} of column m + 8h. That is already the operand layout of
// v_mfma_f32_16x16x32_f16: lane l supplies B[k-group l/16][column l%16], so k-group =
// kt and column = (nt, m). MFMA (h, jp) takes quads (2jp, h), (2jp+1, h) as its 8
// k-values; the activations are staged in LDS in the matching k order, so the wave
// feeds the matrix cores straight from its decode registers with no shuffle. The A
// operand's 16 rows are 16 token rows: one decode serves up to 16 rows.
//
// Activation order in LDS. Per token row and k-tile, the 16 values are stored as
// k-rows [0,1,8,9, 2,3,10,11, 4,5,12,13, 6,7,14,15] (32 bytes): the 16 bytes at
// offset 16*jp are MFMA jp's A operand. f16 pair u (k-rows 2u, 2u+1) of a k-tile sits
// at word xpos(u).
//
// Exact weights. Each weight is the reference's f16 value: mcg/3inst add the two f16
// halves of the masked hash with one RNE (trellis_gemm.cpp:348-356), written with
// v_add_f16 SDWA straight into the half of the operand register it occupies.
//
// k partition (a function of the tensor's k-tile count only): the k range is cut
// into slices of slice_steps(k_tiles) wave steps. A slice is accumulated from zero by
// one wave, in step order, in the MFMA accumulator; an output is the in-order f32 sum
// of its slice partials. Every entry point (standalone, grouped, MoE) follows this
// order, so they agree bit for bit on a shape whatever workgroup ran a slice.
#pragma once

#include "exl3_device.hpp"

namespace exl3d {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kStepTiles = 4;     // k-tiles per wave step
constexpr int kPassRows = 16;     // token rows per MFMA pass (the A operand's rows)
constexpr int kMaxPrefetch = 4;   // wave steps of ring words in flight per wave

constexpr int kMaxSliceSteps = 8;

__host__ __device__ constexpr int slice_steps(int k_tiles) {
  return (k_tiles / kStepTiles) % 8 == 0   ? 8
         : (k_tiles / kStepTiles) % 4 == 0 ? 4
         : (k_tiles / kStepTiles) % 2 == 0 ? 2
                                            : 1;
}
__host__ __device__ constexpr int n_slices(int k_tiles) {
  return k_tiles / (kStepTiles * slice_steps(k_tiles));
}
// Wave steps kept in flight: 4 (2 for K > 4, whose steps take two chunk registers per
// lane), at most one slice.
__host__ __device__ constexpr int prefetch_steps(int k_tiles, int K) {
  return slice_steps(k_tiles) < (K <= 4 ? kMaxPrefetch : 2) ? slice_steps(k_tiles)
                                                            : (K <= 4 ? kMaxPrefetch : 2);
}

// Word position of f16 pair u (k-rows 2u, 2u+1) inside a staged k-tile.
__host__ __device__ constexpr int xpos(int u) { return ((u & 3) << 1) | (u >> 2); }

// ---------------------------------------------------------------------------------
// Decode
// ---------------------------------------------------------------------------------
template <int CB>
__device__ __forceinline__ uint32_t cb_bits(uint32_t s) {
  return (cb_hash<CB>(s) & 0x8FFF8FFFu) ^ 0x3B603B60u;
}

// Eight masked hash words -> the 4-register B operand of one MFMA: operand half i =
// f16(m_i.lo + m_i.hi), one RNE (v_add_f16 SDWA writes each sum straight into its half).
// The compiler's hazard tracking does not see into inline assembly, so the block ends
// with the wait states a VALU-written VGPR needs before an MFMA reads it.
__device__ __forceinline__ f16x8 hadd_operand(const uint32_t (&m)[8]) {
  typedef uint32_t u32x4_ __attribute__((ext_vector_type(4)));
  uint32_t b0, b1, b2, b3;
  asm("v_add_f16_sdwa %0, %4, %4 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
      "v_add_f16_sdwa %1, %6, %6 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
      "v_add_f16_sdwa %2, %8, %8 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
      "v_add_f16_sdwa %3, %10, %10 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
      "v_add_f16_sdwa %0, %5, %5 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1\n\t"
      "v_add_f16_sdwa %1, %7, %7 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1\n\t"
      "v_add_f16_sdwa %2, %9, %9 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1\n\t"
      "v_add_f16_sdwa %3, %11, %11 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1\n\t"
      "s_nop 1"
      : "=&v"(b0), "=&v"(b1), "=&v"(b2), "=&v"(b3)
      : "v"(m[0]), "v"(m[1]), "v"(m[2]), "v"(m[3]), "v"(m[4]), "v"(m[5]), "v"(m[6]), "v"(m[7]));
  const u32x4_ v = {b0, b1, b2, b3};
  return __builtin_bit_cast(f16x8, v);
}

// mul1: one f16 fma per state on packed pairs (trellis_gemm.cpp:336-345).
__device__ __forceinline__ uint32_t mul1_pair(uint32_t s0, uint32_t s1) {
  const uint32_t a0 = __builtin_amdgcn_sad_u8(s0 * 0x83DCD12Du, 0u, 0x6400u);
  const uint32_t a1 = __builtin_amdgcn_sad_u8(s1 * 0x83DCD12Du, 0u, 0x6400u);
  const f16x2 v = bitcast<f16x2>(a0 | (a1 << 16));
  const f16x2 inv = {bitcast<f16>((uint16_t)0x1EEE), bitcast<f16>((uint16_t)0x1EEE)};
  const f16x2 bias = {bitcast<f16>((uint16_t)0xC931), bitcast<f16>((uint16_t)0xC931)};
  return bitcast<uint32_t>(__builtin_elementwise_fma(v, inv, bias));
}

// The B operand of MFMA (h, jp): quads (2jp, h) and (2jp+1, h), i.e. stream positions
// 16jp + 4h + {0..3} and 16jp + 8 + 4h + {0..3} of this lane's bit string.
template <int K, int CB, int T0>
__device__ __forceinline__ f16x8 b_operand(const uint32_t (&W)[K + 1], const uint32_t (&F)[K + 1]) {
  if constexpr (CB == 2) {
    typedef uint32_t u32x4_ __attribute__((ext_vector_type(4)));
    const u32x4_ v = {mul1_pair(lane_state<K, T0 + 0>(W, F), lane_state<K, T0 + 1>(W, F)),
                      mul1_pair(lane_state<K, T0 + 2>(W, F), lane_state<K, T0 + 3>(W, F)),
                      mul1_pair(lane_state<K, T0 + 8>(W, F), lane_state<K, T0 + 9>(W, F)),
                      mul1_pair(lane_state<K, T0 + 10>(W, F), lane_state<K, T0 + 11>(W, F))};
    return __builtin_bit_cast(f16x8, v);
  } else {
    const uint32_t m[8] = {cb_bits<CB>(lane_state<K, T0 + 0>(W, F)),
                           cb_bits<CB>(lane_state<K, T0 + 1>(W, F)),
                           cb_bits<CB>(lane_state<K, T0 + 2>(W, F)),
                           cb_bits<CB>(lane_state<K, T0 + 3>(W, F)),
                           cb_bits<CB>(lane_state<K, T0 + 8>(W, F)),
                           cb_bits<CB>(lane_state<K, T0 + 9>(W, F)),
                           cb_bits<CB>(lane_state<K, T0 + 10>(W, F)),
                           cb_bits<CB>(lane_state<K, T0 + 11>(W, F))};
    return hadd_operand(m);
  }
}

// One wave step: this lane's 32 weights into 4 MFMAs. A0/A1: the A operands of the
// two k-row halves (jp = 0, 1); D0/D1 accumulate columns m and m + 8.
template <int K, int CB>
__device__ __forceinline__ void mfma_step(const uint32_t (&W)[K + 1], const f16x8 &A0,
                                          const f16x8 &A1, f32x4 &D0, f32x4 &D1) {
  uint32_t F[K + 1];
  lane_funnels<K>(W, F);
  D0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, b_operand<K, CB, 0>(W, F), D0, 0, 0, 0);
  D1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, b_operand<K, CB, 4>(W, F), D1, 0, 0, 0);
  D0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, b_operand<K, CB, 16>(W, F), D0, 0, 0, 0);
  D1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, b_operand<K, CB, 20>(W, F), D1, 0, 0, 0);
}

// Ring words of a wave step. The step's 4 k-rows x 2 tiles are 16K chunks of 16 bytes
// (each k-row's two tiles are contiguous). Lane l loads chunk l and, for K > 4, chunk
// 64 + l with aligned 16-byte buffer loads, so every load instruction of the wave reads
// whole, fully used cache lines. A wave-private LDS slot then transposes the chunks
// into each lane's ring words: W[1..K] = words [m*K, m*K + K) of its tile, W[0] = the
// word before them (the ring wraps: word 8K - 1 for m = 0).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kBufNT = 2;           // non-temporal: the ring words are streamed once
constexpr int kSlotChunks = 128;    // 16-byte chunks of one wave's LDS slot (K <= 8)
constexpr uint32_t kNoChunk = 0x80000000u;  // offset past any tensor: the load returns 0

template <int K>
struct StepLoads {
  u32x4 c0, c1;
};

template <int K>
__device__ __forceinline__ void step_load(__amdgpu_buffer_rsrc_t r, uint32_t vo0, uint32_t vo1,
                                          uint32_t so, StepLoads<K> &L) {
  L.c0 = __builtin_amdgcn_raw_buffer_load_b128(r, vo0, so, kBufNT);
  if constexpr (K > 4) L.c1 = __builtin_amdgcn_raw_buffer_load_b128(r, vo1, so, kBufNT);
}

// Chunks into the wave's slot, then this lane's K + 1 ring words out of it. LDS
// operations of one wave complete in issue order, so the reads see the writes of
// every lane; the wave barriers keep the compiler from reordering them.
template <int K>
__device__ __forceinline__ void step_words(u32x4 *slot, int wbase, int m, const StepLoads<K> &L,
                                           uint32_t (&W)[K + 1]) {
  const int lane = threadIdx.x & 63;
  slot[lane] = L.c0;
  if constexpr (K > 4) slot[64 + lane] = L.c1;
  __builtin_amdgcn_wave_barrier();
  const uint32_t *sw = reinterpret_cast<const uint32_t *>(slot) + wbase;
#pragma unroll
  for (int w = 0; w < K; ++w) W[w + 1] = sw[m * K + w];
  W[0] = sw[(m * K + 8 * K - 1) % (8 * K)];
  __builtin_amdgcn_wave_barrier();
}

// Lane geometry of a wave step.
struct StepLane {
  int kt, nt, m;
};
__device__ __forceinline__ StepLane step_lane() {
  const int l = threadIdx.x & 63;
  return StepLane{l >> 4, (l >> 3) & 1, l & 7};
}

// One k-slice of one n-pair (32 output columns): D0/D1 = the slice's partial sums from
// zero over `nsteps` wave steps starting at k-tile kt0. `base` = the tensor's first ring
// word, (k_tiles, tiles_n) its tile grid; n-pair np covers n-tiles 2np, 2np+1. xrow =
// this lane's staged activation row (A-operand row l % 16), positioned at the slice's
// first k-tile; slot = this wave's kSlotChunks-chunk LDS slot. PD = steps in flight
// (divides nsteps). Split in two so that callers can issue the first PD steps' ring
// loads (SliceStream::start) before staging their activations, and run the slice
// (qmv_slice_run) once the staged rows are visible.
template <int K, int PD>
struct SliceStream {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t vo0, vo1, so0, step_bytes;
  StepLoads<K> L[PD];

  __device__ __forceinline__ void start(const uint32_t *base, int k_tiles, int tiles_n, int kt0, int np) {
    constexpr uint32_t kTileBytes = 32 * K;
    constexpr int kChunks = 16 * K, kRowChunks = 4 * K;
    const int lane = threadIdx.x & 63;
    rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0,
                                             (int)((uint32_t)k_tiles * tiles_n * kTileBytes), 0x00020000);
    step_bytes = (uint32_t)kStepTiles * tiles_n * kTileBytes;
    auto chunk_off = [&](int c) -> uint32_t {
      return c < kChunks ? ((uint32_t)(c / kRowChunks) * tiles_n + 2 * np) * kTileBytes +
                               (uint32_t)(c % kRowChunks) * 16
                         : kNoChunk;
    };
    vo0 = chunk_off(lane);
    vo1 = chunk_off(64 + lane);
    so0 = (uint32_t)kt0 * tiles_n * kTileBytes;
#pragma unroll
    for (int b = 0; b < PD; ++b) step_load<K>(rsrc, vo0, vo1, so0 + b * step_bytes, L[b]);
  }
};

template <int K, int CB, int PD>
__device__ __forceinline__ void qmv_slice_run(SliceStream<K, PD> &S, int nsteps, const uint32_t *xrow,
                                              u32x4 *slot, f32x4 &D0, f32x4 &D1) {
  static_assert(16 * K <= kSlotChunks, "slot size");
  const StepLane sl = step_lane();
  const int wbase = (sl.kt * 2 + sl.nt) * 8 * K;  // this lane's tile in the slot, in words
  D0 = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  D1 = D0;
  // A operand of step s: 32 bytes at k-tile 4s + kt of the row (8 words per k-tile).
  const uint32_t *xa = xrow + sl.kt * 8;
  int s0 = 0;
  for (; s0 < nsteps - PD; s0 += PD) {
#pragma unroll
    for (int b = 0; b < PD; ++b) {
      uint32_t W[K + 1];
      step_words<K>(slot, wbase, sl.m, S.L[b], W);
      step_load<K>(S.rsrc, S.vo0, S.vo1, S.so0 + (s0 + b + PD) * S.step_bytes, S.L[b]);
      const uint32_t *xs = xa + (s0 + b) * (kStepTiles * 8);
      const f16x8 A0 = *reinterpret_cast<const f16x8 *>(xs);
      const f16x8 A1 = *reinterpret_cast<const f16x8 *>(xs + 4);
      mfma_step<K, CB>(W, A0, A1, D0, D1);
    }
  }
#pragma unroll
  for (int b = 0; b < PD; ++b) {
    uint32_t W[K + 1];
    step_words<K>(slot, wbase, sl.m, S.L[b], W);
    const uint32_t *xs = xa + (s0 + b) * (kStepTiles * 8);
    const f16x8 A0 = *reinterpret_cast<const f16x8 *>(xs);
    const f16x8 A1 = *reinterpret_cast<const f16x8 *>(xs + 4);
    mfma_step<K, CB>(W, A0, A1, D0, D1);
  }
}

template <int K, int CB, int PD>
__device__ __forceinline__ void qmv_slice(const uint32_t *base, int k_tiles, int tiles_n, int kt0,
                                          int np, int nsteps, const uint32_t *xrow, u32x4 *slot,
                                          f32x4 &D0, f32x4 &D1) {
  SliceStream<K, PD> S;
  S.start(base, k_tiles, tiles_n, kt0, np);
  qmv_slice_run<K, CB, PD>(S, nsteps, xrow, slot, D0, D1);
}

// Long runs: RB blocks of 16 token rows share one decode. The four B operands of a
// wave step are decoded once and each block b runs its 4 MFMAs with its own A
// operands (staged row 16b + l%16 at word offset xo[b] of xs) and accumulators; per
// block the accumulation is exactly mfma_step's, so every row's result is
// bit-identical to a 16-row pass.
template <int K, int CB, int RB>
__device__ __forceinline__ void mfma_step_rb(const uint32_t (&W)[K + 1], const uint32_t *xs,
                                             const int (&xo)[RB], f32x4 (&D)[RB][2]) {
  uint32_t F[K + 1];
  lane_funnels<K>(W, F);
  // k-rows 0..7 of the step (A0) before 8..15 (A1), as in mfma_step; two B operands
  // live at a time
  const f16x8 B0 = b_operand<K, CB, 0>(W, F), B1 = b_operand<K, CB, 4>(W, F);
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const f16x8 A0 = *reinterpret_cast<const f16x8 *>(xs + xo[r]);
    D[r][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, B0, D[r][0], 0, 0, 0);
    D[r][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, B1, D[r][1], 0, 0, 0);
  }
  const f16x8 B2 = b_operand<K, CB, 16>(W, F), B3 = b_operand<K, CB, 20>(W, F);
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const f16x8 A1 = *reinterpret_cast<const f16x8 *>(xs + xo[r] + 4);
    D[r][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, B2, D[r][0], 0, 0, 0);
    D[r][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, B3, D[r][1], 0, 0, 0);
  }
}

// qmv_slice over up to 16 * RB staged token rows: xs = the first staged row (row
// stride xs_stride words), nrows = rows staged (>= 1); rows past nrows read the last
// row and are never stored. D[b] = the slice partials of rows 16b .. 16b + 15.
template <int K, int CB, int PD, int RB>
__device__ __forceinline__ void qmv_slice_rb(const uint32_t *base, int k_tiles, int tiles_n, int kt0,
                                             int np, int nsteps, const uint32_t *xs, int xs_stride,
                                             int nrows, u32x4 *slot, f32x4 (&D)[RB][2]) {
  static_assert(16 * K <= kSlotChunks, "slot size");
  const StepLane sl = step_lane();
  const int lane = threadIdx.x & 63;
  constexpr uint32_t kTileBytes = 32 * K;
  constexpr int kChunks = 16 * K, kRowChunks = 4 * K;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void *)base, (short)0, (int)((uint32_t)k_tiles * tiles_n * kTileBytes), 0x00020000);
  const uint32_t step_bytes = (uint32_t)kStepTiles * tiles_n * kTileBytes;
  auto chunk_off = [&](int c) -> uint32_t {
    return c < kChunks ? ((uint32_t)(c / kRowChunks) * tiles_n + 2 * np) * kTileBytes +
                             (uint32_t)(c % kRowChunks) * 16
                       : kNoChunk;
  };
  const uint32_t vo0 = chunk_off(lane), vo1 = chunk_off(64 + lane);
  const int wbase = (sl.kt * 2 + sl.nt) * 8 * K;
  const uint32_t so0 = (uint32_t)kt0 * tiles_n * kTileBytes;
  int xo[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) xo[r] = min(16 * r + (lane & 15), nrows - 1) * xs_stride + sl.kt * 8;
  StepLoads<K> L[PD];
#pragma unroll
  for (int b = 0; b < PD; ++b) step_load<K>(rsrc, vo0, vo1, so0 + b * step_bytes, L[b]);
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    D[r][0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    D[r][1] = D[r][0];
  }
  int s0 = 0;
  for (; s0 < nsteps - PD; s0 += PD) {
#pragma unroll
    for (int b = 0; b < PD; ++b) {
      uint32_t W[K + 1];
      step_words<K>(slot, wbase, sl.m, L[b], W);
      step_load<K>(rsrc, vo0, vo1, so0 + (s0 + b + PD) * step_bytes, L[b]);
      mfma_step_rb<K, CB, RB>(W, xs + (s0 + b) * (kStepTiles * 8), xo, D);
    }
  }
#pragma unroll
  for (int b = 0; b < PD; ++b) {
    uint32_t W[K + 1];
    step_words<K>(slot, wbase, sl.m, L[b], W);
    mfma_step_rb<K, CB, RB>(W, xs + (s0 + b) * (kStepTiles * 8), xo, D);
  }
}

// Output position of accumulator element D_h[i] of this lane inside its n-pair's 32
// columns: token row 4*(l/16) + i, column 16*nt + m + 8h.
__device__ __forceinline__ int d_row(int i) { return 4 * ((threadIdx.x & 63) >> 4) + i; }
__device__ __forceinline__ int d_col(int h) {
  const int l = threadIdx.x & 63;
  return 16 * ((l >> 3) & 1) + (l & 7) + 8 * h;
}

// Stages one Hadamard-rotated activation pair: lane's pair covers k = 128*blk + 2*lane,
// 2*lane + 1 of a row whose staged copy starts at `row` (k-tile 0 of the staged range).
__device__ __forceinline__ void stage_pair(uint32_t *row, int blk, int lane, uint32_t packed) {
  row[(blk * 8 + (lane >> 3)) * 8 + xpos(lane & 7)] = packed;
}

}  // namespace exl3d
