// The dequant-GEMV core shared by the standalone linear and the MoE expert kernels,
// so that every entry point that sees one tensor shape sums it in the same f32 order.
//
// Workgroup = 4 waves. A workgroup owns one 128-column block (8 n-tiles) of one
// member and a contiguous range of 4*T k-tiles; wave w streams the T k-tiles starting
// at k0 + w*T in order, double-buffering one k-tile of ring words in registers.
// Per output element the result is ((wave0 + wave1) + wave2) + wave3.
#pragma once

#include "exl3_device.hpp"

namespace exl3d {

constexpr int kQmvWaves = 4;
constexpr int kQmvMaxKtPerWg = 64;  // 4 waves x at most 16 k-tiles

// xs: LDS, MB rows of (4*T k-tiles x 16) f16 packed as u32 pairs; row stride
// kQmvMaxKtPerWg * 8 words. Rows past the valid count must hold zeros.
template <int K, int CB, int MB>
__device__ __forceinline__ void qmv_wave_loop(const uint32_t *__restrict__ base, int tiles_n,
                                              int tn, int m, int kw, int T, int wave,
                                              const uint32_t *xs, float (&acc)[MB][2]) {
#pragma unroll
  for (int r = 0; r < MB; ++r) acc[r][0] = acc[r][1] = 0.0f;
  uint32_t Wc[K + 1], Wn[K + 1];
  lane_load<K>(base + ((int64_t)kw * tiles_n + tn) * 8 * K, m, Wc);
  for (int t = 0; t < T; ++t) {
    if (t + 1 < T) lane_load<K>(base + ((int64_t)(kw + t + 1) * tiles_n + tn) * 8 * K, m, Wn);
    uint32_t X[MB][8];
#pragma unroll
    for (int r = 0; r < MB; ++r)
#pragma unroll
      for (int u = 0; u < 8; ++u) X[r][u] = xs[r * (kQmvMaxKtPerWg * 8) + (wave * T + t) * 8 + u];
    lane_tile_fma<K, CB, MB>(Wc, X, acc);
#pragma unroll
    for (int w = 0; w <= K; ++w) Wc[w] = Wn[w];
  }
}

// Lane l of a wave holds columns (l/8)*16 + l%8 (acc[r][0]) and that + 8 (acc[r][1]).
template <int MB>
__device__ __forceinline__ void qmv_stash(float *red /* [4][MB][128] */, int wave, int lane,
                                          const float (&acc)[MB][2]) {
  const int c = (lane >> 3) * 16 + (lane & 7);
#pragma unroll
  for (int r = 0; r < MB; ++r) {
    red[(wave * MB + r) * 128 + c] = acc[r][0];
    red[(wave * MB + r) * 128 + c + 8] = acc[r][1];
  }
}

template <int MB>
__device__ __forceinline__ float qmv_wave_sum(const float *red, int r, int c) {
  float v = red[(0 * MB + r) * 128 + c];
  v += red[(1 * MB + r) * 128 + c];
  v += red[(2 * MB + r) * 128 + c];
  v += red[(3 * MB + r) * 128 + c];
  return v;
}

// The k partition (mirrors exl3h::kpart on the host).
__device__ __forceinline__ int qmv_T(int k_tiles) {
  if (k_tiles >= 256 && k_tiles % 64 == 0) return 16;
  if (k_tiles % 32 == 0) return 8;
  if (k_tiles % 16 == 0) return 4;
  return 2;
}

}  // namespace exl3d
