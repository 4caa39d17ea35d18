// The dequant-GEMV core shared by the standalone linear and the MoE expert kernels.
//
// k partition (a function of the tensor's k-tile count only): the k range is cut into
// chunks of chunk_tiles(k_tiles) consecutive k-tiles. One wave computes one chunk's
// partial sums from zero, visiting its k-tiles in order; an output is the in-order
// sum of its chunk partials (c = 0, 1, 2, ...). Every entry point -- standalone,
// grouped, MoE -- follows this order, so they agree bit for bit on a shape, whatever
// workgroup or launch a chunk ran in.
//
// A wave covers 8 n-tiles (128 output columns, one Hadamard block) of one member; lane
// l holds columns (l/8)*16 + l%8 and that + 8 (see exl3_device.hpp).
#pragma once

#include "exl3_device.hpp"

namespace exl3d {

constexpr int kMaxRowsPerPass = 4;

__host__ __device__ constexpr int chunk_tiles(int k_tiles) { return (k_tiles % 16 == 0) ? 16 : 8; }

typedef const __attribute__((address_space(1))) uint32_t *gu32p;

template <int K>
__device__ __forceinline__ void lane_load_g(gu32p tile, int m, uint32_t (&W)[K + 1]) {
  gu32p p = tile + m * K;
#pragma unroll
  for (int w = 0; w < K; ++w) W[w + 1] = __builtin_nontemporal_load(p + w);
  W[0] = __builtin_nontemporal_load(tile + ((m * K + 8 * K - 1) % (8 * K)));
}

// x values of k-tile kt for MB rows from LDS: xs row r holds 8 packed f16 pairs per
// k-tile starting at word kt * 8 (row stride `stride` words).
template <int MB>
__device__ __forceinline__ void load_x(const uint32_t *xs, int stride, int kt,
                                       uint32_t (&X)[MB][8]) {
#pragma unroll
  for (int r = 0; r < MB; ++r) {
    const uint4 a = *reinterpret_cast<const uint4 *>(xs + r * stride + kt * 8);
    const uint4 b = *reinterpret_cast<const uint4 *>(xs + r * stride + kt * 8 + 4);
    X[r][0] = a.x; X[r][1] = a.y; X[r][2] = a.z; X[r][3] = a.w;
    X[r][4] = b.x; X[r][5] = b.y; X[r][6] = b.z; X[r][7] = b.w;
  }
}

// One chunk: acc = sum over k-tiles [kt0, kt0 + nkt) of this lane's 32 weights times x,
// from zero. `base` = member's trellis words, tn = this lane's n-tile, m = lane slot in
// its tile; xs/xkt0: the LDS x row holding k-tile kt0 at word offset xkt0 * 8.
// Two k-tiles of ring words are kept in flight per lane (nkt is even).
template <int K, int CB, int MB>
__device__ __forceinline__ void qmv_chunk(const uint32_t *base, int tiles_n, int tn, int m,
                                          int kt0, int nkt, const uint32_t *xs, int stride,
                                          int xkt0, float (&acc)[MB][2]) {
#pragma unroll
  for (int r = 0; r < MB; ++r) acc[r][0] = acc[r][1] = 0.0f;
  gu32p g = (gu32p)base;
  const int64_t tstride = (int64_t)tiles_n * 8 * K;  // words between consecutive k-tiles
  gu32p t0 = g + ((int64_t)kt0 * tiles_n + tn) * 8 * K;
  uint32_t Wa[K + 1], Wb[K + 1];
  lane_load_g<K>(t0, m, Wa);
  lane_load_g<K>(t0 + tstride, m, Wb);
  for (int t = 0; t < nkt; t += 2) {
    uint32_t X[MB][8];
    load_x<MB>(xs, stride, xkt0 + t, X);
    lane_tile_fma<K, CB, MB>(Wa, X, acc);
    if (t + 2 < nkt) lane_load_g<K>(t0 + (t + 2) * tstride, m, Wa);
    load_x<MB>(xs, stride, xkt0 + t + 1, X);
    lane_tile_fma<K, CB, MB>(Wb, X, acc);
    if (t + 3 < nkt) lane_load_g<K>(t0 + (t + 3) * tstride, m, Wb);
  }
}

// Column of acc[r][h] inside the wave's 128-column block.
__device__ __forceinline__ int lane_col(int lane, int h) {
  return (lane >> 3) * 16 + (lane & 7) + 8 * h;
}

}  // namespace exl3d
