// The dequant-GEMV core shared by the standalone linear and the MoE expert kernels:
// trellis decode in VALU registers, products on the matrix cores.
//
// Wave step. One wave step covers 4 k-tiles x 2 n-tiles (64 k x 32 output columns).
// Lane l = 16*kt + 8*nt + m loads ring words [m*K - 1, m*K + K) of tile (k0 + kt,
// n0 + nt): the bit range of reference lanes 4m..4m+3 (exl3.cpp:84-99), i.e. all 16
// k-rows of columns m and m + 8 of that tile (exl3_device.hpp). It decodes them as 8
// "quads" of 4 weights, quad (j, h) = stream positions 8j + 4h + 0..3 = k-rows
// {2j, 2j+1, 2j+8, 2j+9} of column m + 8h. In the operand layout of
// v_mfma_f32_16x16x32_f16 lane l supplies B[k-group l/16][column l%16], so k-group = kt
// and column = (nt, m): the wave feeds the matrix cores straight from its decode
// registers with no shuffle. The A operand's 16 rows are 16 token rows staged in LDS
// in the matching k order: one decode serves up to 16 rows.
//
// B forms. The CB template parameter of the GEMV kernels is a kernel codebook: the
// tensor's codebook in the reference-weight form (0 = 3inst, 1 = mcg, 2 = mul1), or
// 3 = 3inst, 4 = mcg in the exact-halves form (exl3_tuning.weight_form).
//  - reference (packed): every weight is the reference's f16 value, two per register;
//    MFMA (h, jp) takes quads (2jp, h), (2jp+1, h). mcg/3inst: the f16 sum of the two
//    halves of the masked hash word with one RNE (trellis_gemm.cpp:348-356), written by
//    v_add_f16 SDWA straight into its half of the operand register; mul1: one f16 fma
//    (trellis_gemm.cpp:336-345), exact for two weights per packed register.
//  - halves (mcg, 3inst): the masked word itself is the B register: its halves are two
//    k-elements, multiplied by the same activation, so the MFMA forms x*lo + x*hi in
//    f32 and no VALU add is spent per weight. MFMA (h, j) takes quad (j, h): 4 words = 8
//    k-elements. The activations are staged duplicated, each f16 value in both halves
//    of a word. The product is x*(lo + hi) without the f16 rounding of lo + hi, so it
//    differs from the reference's by up to 2^-11 of each weight.
//
// Staged activation order in LDS, per token row and k-tile (xpos: f16 pair u = k-rows
// 2u, 2u+1):
//  - plain (reference forms): 8 words [p0, p4, p1, p5, p2, p6, p3, p7]; words 4jp..4jp+3
//    are MFMA jp's A operand. Pair u sits at word xpos(u). This is also the layout of
//    the rotated activations the MoE kernels keep in HBM (act, xrot).
//  - duplicated (halves forms): 16 words, word 2w = (lo, lo) and 2w + 1 = (hi, hi) of
//    plain word w; words 4j..4j+3 are MFMA j's A operand.
//
// k partition (a function of the tensor's k-tile count only): the k range is cut
// into slices of slice_steps(k_tiles) wave steps. A slice is accumulated from zero by
// one wave, in step order, in the MFMA accumulator; an output is the in-order f32 sum
// of its slice partials. Every entry point (standalone, grouped, MoE) follows this
// order, so they agree bit for bit on a shape whatever workgroup ran a slice.
#pragma once

#include "exl3_device.hpp"
#include "exl3_moe.h"

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

// Word position of f16 pair u (k-rows 2u, 2u+1) inside a plain staged k-tile.
__host__ __device__ constexpr int xpos(int u) { return ((u & 3) << 1) | (u >> 2); }

// Kernel codebooks (see the B forms above).
constexpr int kHalvesCb = 3;
// The tensor codebook of kernel codebook kcb.
__host__ __device__ constexpr int cb_base(int kcb) { return kcb >= kHalvesCb ? kcb - kHalvesCb : kcb; }
// The kernel codebook of a tensor codebook under a weight form (mul1 has one form).
__host__ __device__ constexpr int kernel_cb(int cb, int form) {
  return form == EXL3_FORM_HALVES && cb != 2 ? cb + kHalvesCb : cb;
}
// Staging form of a kernel codebook: duplicated activations for the halves B form.
__host__ __device__ constexpr bool dup_cb(int kcb) { return kcb >= kHalvesCb; }
// Staged words per token row and k-tile.
__host__ __device__ constexpr int tile_words(bool dup) { return dup ? 16 : 8; }
// Staged words per token row of one k slice of a tensor with k_tiles k-tiles.
__host__ __device__ constexpr int slice_words(int k_tiles, bool dup) {
  return kStepTiles * slice_steps(k_tiles) * tile_words(dup);
}
// Row stride of the staged rows in LDS: the slice plus 16 bytes, so that the 16-byte A
// reads of consecutive rows (one row per lane) fall on different banks.
__host__ __device__ constexpr int staged_row_words(int k_tiles, bool dup) {
  return slice_words(k_tiles, dup) + 4;
}
// The long-run kernels stage a slice of duplicated rows in parts of at most 4 wave
// steps (a part of 64 rows is ~66 KB of LDS, so that two 8-wave workgroups share a CU;
// a whole slice of plain rows is that size already).
__host__ __device__ constexpr int long_part_steps(int k_tiles, bool dup) {
  return !dup || slice_steps(k_tiles) < 4 ? slice_steps(k_tiles) : 4;
}
__host__ __device__ constexpr int long_row_words(int k_tiles, bool dup) {
  return kStepTiles * long_part_steps(k_tiles, dup) * tile_words(dup) + 4;
}
// 16-byte ring-word chunks of one wave's LDS slot: one wave step's 16K chunks, and at
// least one per lane (every lane stores its first chunk register, K < 4 included).
__host__ __device__ constexpr int slot_chunks(int K) { return 16 * K > 64 ? 16 * K : 64; }

// ---------------------------------------------------------------------------------
// Decode
// ---------------------------------------------------------------------------------
// The masked hash word of a state (mcg/3inst): two f16 halves whose sum is the weight.
template <int CB>
__device__ __forceinline__ uint32_t cb_bits(uint32_t s) {
  return (cb_hash<cb_base(CB)>(s) & 0x8FFF8FFFu) ^ 0x3B603B60u;
}

// Eight masked hash words -> the 4-register B operand of one MFMA in the reference
// form: half i of the operand = f16(m_i.lo + m_i.hi), one RNE, the reference's weight
// (trellis_gemm.cpp:348-356). Both halves are f16 values of magnitude in [2^-3, 2), so
// their exact sum is a multiple of 2^-13 and never subnormal. v_add_f16 SDWA writes
// each sum straight into its half of the operand register (the compiler spells a pair
// as two funnel shifts, two packed adds and a pack). The compiler's hazard tracking does not
// see into inline assembly, so the block ends with the wait states a VALU-written VGPR
// needs before an MFMA reads it.
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

// mul1: two states -> their f16 weights packed in one register, each one f16 fma
// (trellis_gemm.cpp:336-345). v_sad_u8 adds state 0's byte sum to 0x64006400 and
// v_sad_hi_u8 adds state 1's, shifted into the high half, so the pair arrives packed;
// byte sums are at most 1020, so no carry crosses the halves.
__device__ __forceinline__ uint32_t mul1_pair(uint32_t s0, uint32_t s1) {
  const uint32_t a = __builtin_amdgcn_sad_u8(s0 * 0x83DCD12Du, 0u, 0x64006400u);
  const uint32_t v2 = __builtin_amdgcn_sad_hi_u8(s1 * 0x83DCD12Du, 0u, a);
  const f16x2 v = bitcast<f16x2>(v2);
  const f16x2 inv = {bitcast<f16>((uint16_t)0x1EEE), bitcast<f16>((uint16_t)0x1EEE)};
  const f16x2 bias = {bitcast<f16>((uint16_t)0xC931), bitcast<f16>((uint16_t)0xC931)};
  return bitcast<uint32_t>(__builtin_elementwise_fma(v, inv, bias));
}

// Reference-form B operand of MFMA (h, jp): quads (2jp, h) and (2jp+1, h), i.e. stream
// positions 16jp + 4h + {0..3} and 16jp + 8 + 4h + {0..3} of this lane's bit string
// (T0 = 16jp + 4h), two f16 weights per register.
template <int K, int CB, int T0>
__device__ __forceinline__ f16x8 b_packed(const uint32_t (&W)[K + 1], const uint32_t (&F)[K + 1]) {
  if constexpr (CB == 2) {
    typedef uint32_t u32x4_ __attribute__((ext_vector_type(4)));
    const u32x4_ v = {mul1_pair(lane_state<K, T0 + 0>(W, F), lane_state<K, T0 + 1>(W, F)),
                      mul1_pair(lane_state<K, T0 + 2>(W, F), lane_state<K, T0 + 3>(W, F)),
                      mul1_pair(lane_state<K, T0 + 8>(W, F), lane_state<K, T0 + 9>(W, F)),
                      mul1_pair(lane_state<K, T0 + 10>(W, F), lane_state<K, T0 + 11>(W, F))};
    return __builtin_bit_cast(f16x8, v);
  } else {
    const uint32_t m[8] = {cb_bits<CB>(lane_state<K, T0 + 0>(W, F)),  cb_bits<CB>(lane_state<K, T0 + 1>(W, F)),
                           cb_bits<CB>(lane_state<K, T0 + 2>(W, F)),  cb_bits<CB>(lane_state<K, T0 + 3>(W, F)),
                           cb_bits<CB>(lane_state<K, T0 + 8>(W, F)),  cb_bits<CB>(lane_state<K, T0 + 9>(W, F)),
                           cb_bits<CB>(lane_state<K, T0 + 10>(W, F)), cb_bits<CB>(lane_state<K, T0 + 11>(W, F))};
    return hadd_operand(m);
  }
}

// Halves B operand of MFMA (h, j): the masked hash words of quad (j, h), stream positions
// T0 = 8j + 4h .. T0 + 3; word i's halves are k-elements 2i and 2i + 1.
template <int K, int CB, int T0>
__device__ __forceinline__ f16x8 b_halves(const uint32_t (&W)[K + 1], const uint32_t (&F)[K + 1]) {
  typedef uint32_t u32x4_ __attribute__((ext_vector_type(4)));
  const u32x4_ v = {cb_bits<CB>(lane_state<K, T0 + 0>(W, F)), cb_bits<CB>(lane_state<K, T0 + 1>(W, F)),
                    cb_bits<CB>(lane_state<K, T0 + 2>(W, F)), cb_bits<CB>(lane_state<K, T0 + 3>(W, F))};
  return __builtin_bit_cast(f16x8, v);
}

__device__ __forceinline__ f16x8 lds_a(const uint32_t *p) { return *reinterpret_cast<const f16x8 *>(p); }

__device__ __forceinline__ f32x4 mfma16(const f16x8 &a, const f16x8 &b, const f32x4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// One wave step: this lane's 32 weights into the MFMAs. xa = this lane's staged row at
// its k-tile of the step; D0/D1 accumulate columns m and m + 8. Reference forms: 4
// MFMAs, jp major; halves: 8 MFMAs, j major.
template <int K, int CB>
__device__ __forceinline__ void mfma_step(const uint32_t (&W)[K + 1], const uint32_t *xa, f32x4 &D0,
                                          f32x4 &D1) {
  uint32_t F[K + 1];
  lane_funnels<K>(W, F);
  if constexpr (!dup_cb(CB)) {
    const f16x8 A0 = lds_a(xa), A1 = lds_a(xa + 4);
    D0 = mfma16(A0, b_packed<K, CB, 0>(W, F), D0);
    D1 = mfma16(A0, b_packed<K, CB, 4>(W, F), D1);
    D0 = mfma16(A1, b_packed<K, CB, 16>(W, F), D0);
    D1 = mfma16(A1, b_packed<K, CB, 20>(W, F), D1);
  } else {
    const f16x8 A0 = lds_a(xa), A1 = lds_a(xa + 4);
    D0 = mfma16(A0, b_halves<K, CB, 0>(W, F), D0);
    D1 = mfma16(A0, b_halves<K, CB, 4>(W, F), D1);
    D0 = mfma16(A1, b_halves<K, CB, 8>(W, F), D0);
    D1 = mfma16(A1, b_halves<K, CB, 12>(W, F), D1);
    const f16x8 A2 = lds_a(xa + 8), A3 = lds_a(xa + 12);
    D0 = mfma16(A2, b_halves<K, CB, 16>(W, F), D0);
    D1 = mfma16(A2, b_halves<K, CB, 20>(W, F), D1);
    D0 = mfma16(A3, b_halves<K, CB, 24>(W, F), D0);
    D1 = mfma16(A3, b_halves<K, CB, 28>(W, F), D1);
  }
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
constexpr uint32_t kNoChunk = 0x80000000u;  // offset past any tensor: the load returns 0
// Lane offset past any tensor (tensors are below 1 GiB, buffer sizes are 31-bit), added
// to a lane's chunk offset (voffset, which the raw buffer's range check covers; the
// scalar soffset is left at 0): with any chunk offset, kNoChunk included, the sum stays
// at or above 1 GiB and below 2^32, so the load returns 0 and touches no memory.
constexpr uint32_t kPastEnd = 0x40000000u;

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

// Chunks into the wave's slot (slot_chunks(K) >= 64 chunks), then this lane's K + 1 ring words
// out of it. LDS operations of one wave complete in issue order, so the reads see the
// writes of every lane; the wave barriers keep the compiler from reordering them.
template <int K>
__device__ __forceinline__ void step_words(u32x4 *slot, int wbase, int m, const StepLoads<K> &L,
                                           uint32_t (&W)[K + 1]) {
  const int lane = threadIdx.x & 63;
  slot[lane] = L.c0;
  if constexpr (K > 4) {
    if (lane < 16 * K - 64) slot[64 + lane] = L.c1;
  }
  __builtin_amdgcn_wave_barrier();
  const uint32_t *sw = reinterpret_cast<const uint32_t *>(slot) + wbase;
  // the lane's K words in as few reads as their alignment allows (a tile is 32K bytes,
  // so word m*K sits at 16 bytes * m for K = 4, 8 and at 8 bytes * m*K/2 for K = 2, 6):
  // each wide read covers whole 128-byte rows of 8 lanes, free of bank conflicts, where
  // one dword at a time puts the 4 tiles of a half-wave on the same 8 banks
  if constexpr (K % 4 == 0) {
#pragma unroll
    for (int q = 0; q < K / 4; ++q) {
      const u32x4 v = *reinterpret_cast<const u32x4 *>(sw + m * K + 4 * q);
      W[4 * q + 1] = v.x;
      W[4 * q + 2] = v.y;
      W[4 * q + 3] = v.z;
      W[4 * q + 4] = v.w;
    }
  } else if constexpr (K % 2 == 0) {
#pragma unroll
    for (int q = 0; q < K / 2; ++q) {
      const u32x2 v = *reinterpret_cast<const u32x2 *>(sw + m * K + 2 * q);
      W[2 * q + 1] = v.x;
      W[2 * q + 2] = v.y;
    }
  } else {
#pragma unroll
    for (int w = 0; w < K; ++w) W[w + 1] = sw[m * K + w];
  }
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
// first k-tile, in the codebook's staging form; slot = this wave's slot_chunks(K)-chunk
// LDS slot. PD = steps in flight (divides nsteps). Split in two so that callers can
// issue the first PD steps' ring loads (SliceStream::start) before staging their
// activations, and run the slice (qmv_slice_run) once the staged rows are visible.
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
  constexpr int kTw = tile_words(dup_cb(CB));
  const StepLane sl = step_lane();
  const int wbase = (sl.kt * 2 + sl.nt) * 8 * K;  // this lane's tile in the slot, in words
  D0 = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  D1 = D0;
  // A operands of step s: the staged k-tile 4s + kt of the row
  const uint32_t *xa = xrow + sl.kt * kTw;
  int s0 = 0;
  for (; s0 < nsteps - PD; s0 += PD) {
#pragma unroll
    for (int b = 0; b < PD; ++b) {
      uint32_t W[K + 1];
      step_words<K>(slot, wbase, sl.m, S.L[b], W);
      step_load<K>(S.rsrc, S.vo0, S.vo1, S.so0 + (s0 + b + PD) * S.step_bytes, S.L[b]);
      mfma_step<K, CB>(W, xa + (s0 + b) * (kStepTiles * kTw), D0, D1);
    }
  }
#pragma unroll
  for (int b = 0; b < PD; ++b) {
    uint32_t W[K + 1];
    step_words<K>(slot, wbase, sl.m, S.L[b], W);
    mfma_step<K, CB>(W, xa + (s0 + b) * (kStepTiles * kTw), D0, D1);
  }
}

// The same k slice of `items` column blocks in one stream: item i is n-pair np0 + 4i
// (the next 128-column block of the wave's workgroup), 8 tiles further into each k-row.
// The ring loads run PD steps ahead across the item boundary (PD divides nsteps, so a
// group of PD steps never straddles two items), and the wave's pipeline does not drain
// between blocks. After each item's last step store(i, D0, D1) receives that item's
// slice partials (the same f32 operations, in the same order, as a separate
// qmv_slice_run of that item). nsteps is a power of two.
template <int K, int CB, int PD, typename Store>
__device__ __forceinline__ void qmv_slice_items(SliceStream<K, PD> &S, int nsteps, int items,
                                                const uint32_t *xrow, u32x4 *slot, Store &&store) {
  constexpr int kTw = tile_words(dup_cb(CB));
  constexpr uint32_t kItemBytes = 8u * 32u * K;  // 4 n-pairs = 8 tiles of a k-row
  const StepLane sl = step_lane();
  const int wbase = (sl.kt * 2 + sl.nt) * 8 * K;
  const uint32_t *xa = xrow + sl.kt * kTw;
  const int smask = nsteps - 1, slg = __builtin_ctz(nsteps);
  // lane offsets past the tensor for the loads after the last step
  const uint32_t vd0 = S.vo0 + kPastEnd, vd1 = S.vo1 + kPastEnd;
  for (int it = 0; it < items; ++it) {
    f32x4 D0 = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, D1 = D0;
    for (int s0 = 0; s0 < nsteps; s0 += PD) {
      // the steps PD ahead: this item's, then the next item's first ones; past the last
      // step the loads take lane offsets beyond the tensor, which return zeros without a
      // memory access (so every group issues the same instructions)
      const int tn = it * nsteps + s0 + PD;
      const bool past = tn >= items * nsteps;
      const uint32_t next =
          past ? 0u : S.so0 + (uint32_t)(tn & smask) * S.step_bytes + (uint32_t)(tn >> slg) * kItemBytes;
      const uint32_t v0 = past ? vd0 : S.vo0, v1 = past ? vd1 : S.vo1;
#pragma unroll
      for (int b = 0; b < PD; ++b) {
        uint32_t W[K + 1];
        step_words<K>(slot, wbase, sl.m, S.L[b], W);
        step_load<K>(S.rsrc, v0, v1, past ? 0u : next + b * S.step_bytes, S.L[b]);
        mfma_step<K, CB>(W, xa + (s0 + b) * (kStepTiles * kTw), D0, D1);
      }
    }
    store(it, D0, D1);
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

// Halves form of one quad index j of a long-run wave step: both B operands of quad j
// (h = 0, 1) decoded once, then every block's two MFMAs.
template <int K, int CB, int RB, int J>
__device__ __forceinline__ void mfma_quad_rb(const uint32_t (&W)[K + 1], const uint32_t (&F)[K + 1],
                                             const uint32_t *xs, const int (&xo)[RB], f32x4 (&D)[RB][2]) {
  const f16x8 B0 = b_halves<K, CB, 8 * J>(W, F), B1 = b_halves<K, CB, 8 * J + 4>(W, F);
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const f16x8 A = lds_a(xs + xo[r] + 4 * J);
    D[r][0] = mfma16(A, B0, D[r][0]);
    D[r][1] = mfma16(A, B1, D[r][1]);
  }
}

// Long runs: RB blocks of 16 token rows share one decode. The B operands of a wave step
// are decoded once and each block b runs the step's MFMAs with its own A operands
// (staged row 16b + l%16 at word offset xo[b] of xs) and accumulators; per block a
// step's MFMAs are exactly mfma_step's (the same operands in the same order).
template <int K, int CB, int RB>
__device__ __forceinline__ void mfma_step_rb(const uint32_t (&W)[K + 1], const uint32_t *xs,
                                             const int (&xo)[RB], f32x4 (&D)[RB][2]) {
  uint32_t F[K + 1];
  lane_funnels<K>(W, F);
  if constexpr (!dup_cb(CB)) {
    // k-rows 0..7 of the step (A0) before 8..15 (A1), as in mfma_step; two B operands
    // live at a time
    const f16x8 B0 = b_packed<K, CB, 0>(W, F), B1 = b_packed<K, CB, 4>(W, F);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const f16x8 A0 = lds_a(xs + xo[r]);
      D[r][0] = mfma16(A0, B0, D[r][0]);
      D[r][1] = mfma16(A0, B1, D[r][1]);
    }
    const f16x8 B2 = b_packed<K, CB, 16>(W, F), B3 = b_packed<K, CB, 20>(W, F);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const f16x8 A1 = lds_a(xs + xo[r] + 4);
      D[r][0] = mfma16(A1, B2, D[r][0]);
      D[r][1] = mfma16(A1, B3, D[r][1]);
    }
  } else {
    mfma_quad_rb<K, CB, RB, 0>(W, F, xs, xo, D);
    mfma_quad_rb<K, CB, RB, 1>(W, F, xs, xo, D);
    mfma_quad_rb<K, CB, RB, 2>(W, F, xs, xo, D);
    mfma_quad_rb<K, CB, RB, 3>(W, F, xs, xo, D);
  }
}

// qmv_slice over up to 16 * RB staged token rows: xs = the first staged row (row
// stride xs_stride words), nrows = rows staged (>= 1); rows past nrows read the last
// row and are never stored. D[b] = the slice partials of rows 16b .. 16b + 15, from
// zero, or (zero = false) continuing the accumulation already in D: a slice run as
// consecutive parts adds every step into its accumulator in the same order as one call.
template <int K, int CB, int PD, int RB>
__device__ __forceinline__ void qmv_slice_rb(const uint32_t *base, int k_tiles, int tiles_n, int kt0,
                                             int np, int nsteps, const uint32_t *xs, int xs_stride,
                                             int nrows, u32x4 *slot, f32x4 (&D)[RB][2], bool zero = true) {
  constexpr int kTw = tile_words(dup_cb(CB));
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
  for (int r = 0; r < RB; ++r) xo[r] = min(16 * r + (lane & 15), nrows - 1) * xs_stride + sl.kt * kTw;
  StepLoads<K> L[PD];
#pragma unroll
  for (int b = 0; b < PD; ++b) step_load<K>(rsrc, vo0, vo1, so0 + b * step_bytes, L[b]);
  if (zero) {
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      D[r][0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      D[r][1] = D[r][0];
    }
  }
  int s0 = 0;
  for (; s0 < nsteps - PD; s0 += PD) {
#pragma unroll
    for (int b = 0; b < PD; ++b) {
      uint32_t W[K + 1];
      step_words<K>(slot, wbase, sl.m, L[b], W);
      step_load<K>(rsrc, vo0, vo1, so0 + (s0 + b + PD) * step_bytes, L[b]);
      mfma_step_rb<K, CB, RB>(W, xs + (s0 + b) * (kStepTiles * kTw), xo, D);
    }
  }
#pragma unroll
  for (int b = 0; b < PD; ++b) {
    uint32_t W[K + 1];
    step_words<K>(slot, wbase, sl.m, L[b], W);
    mfma_step_rb<K, CB, RB>(W, xs + (s0 + b) * (kStepTiles * kTw), xo, D);
  }
}

// Output position of accumulator element D_h[i] of this lane inside its n-pair's 32
// columns: token row 4*(l/16) + i, column 16*nt + m + 8h.
__device__ __forceinline__ int d_row(int i) { return 4 * ((threadIdx.x & 63) >> 4) + i; }
__device__ __forceinline__ int d_col(int h) {
  const int l = threadIdx.x & 63;
  return 16 * ((l >> 3) & 1) + (l & 7) + 8 * h;
}

// ---------------------------------------------------------------------------------
// Staging of activations
// ---------------------------------------------------------------------------------
// (lo, lo) and (hi, hi) of a packed f16 pair.
__device__ __forceinline__ uint32_t dup_lo(uint32_t v) { return __builtin_amdgcn_perm(v, v, 0x01000100u); }
__device__ __forceinline__ uint32_t dup_hi(uint32_t v) { return __builtin_amdgcn_perm(v, v, 0x03020302u); }

// Stages one Hadamard-rotated activation pair: the lane's pair covers k = 128*blk +
// 2*lane, 2*lane + 1 of a row whose staged copy starts at `row` (k-tile 0 of the staged
// range). DUP: the duplicated form (two words).
template <bool DUP>
__device__ __forceinline__ void stage_pair(uint32_t *row, int blk, int lane, uint32_t packed) {
  const int w = (blk * 8 + (lane >> 3)) * 8 + xpos(lane & 7);  // plain word
  if constexpr (DUP) {
    *reinterpret_cast<u32x2 *>(row + 2 * w) = u32x2{dup_lo(packed), dup_hi(packed)};
  } else {
    row[w] = packed;
  }
}

// Stages plain 16-byte chunk q of a row (4 plain words, already in the plain staged
// order) at `row`: the chunk itself, or (DUP) its 32-byte duplicated form.
template <bool DUP>
__device__ __forceinline__ void stage_chunk(uint32_t *row, int q, const uint4 &c) {
  if constexpr (DUP) {
    uint4 *d = reinterpret_cast<uint4 *>(row) + 2 * q;
    d[0] = uint4{dup_lo(c.x), dup_hi(c.x), dup_lo(c.y), dup_hi(c.y)};
    d[1] = uint4{dup_lo(c.z), dup_hi(c.z), dup_lo(c.w), dup_hi(c.w)};
  } else {
    reinterpret_cast<uint4 *>(row)[q] = c;
  }
}

}  // namespace exl3d
