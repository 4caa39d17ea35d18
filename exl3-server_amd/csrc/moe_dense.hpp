// The f16 shared expert (g5_linear's mx::matmul branch, glm5_kda.cpp:120) and the
// router logits (glm5_moe.cpp:127-128): skinny f16 GEMVs with f32 accumulation.
#pragma once

#include "exl3_device.hpp"

namespace exl3d {

__device__ __forceinline__ float lo16f(uint32_t v) { return (float)bitcast<f16>((uint16_t)(v & 0xffffu)); }
__device__ __forceinline__ float hi16f(uint32_t v) { return (float)bitcast<f16>((uint16_t)(v >> 16)); }

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kDenseKR = 256;   // k rows per dense workgroup (one k split)

// k splits of a dense_skinny GEMV over `in` rows.
__host__ __device__ constexpr int dense_splits(int in) { return (in + kDenseKR - 1) / kDenseKR; }
constexpr int kDenseRows = 8;   // token rows per pass

// LDS words a dense_skinny workgroup needs.
constexpr int kDenseLdsWords = kDenseRows * kDenseKR / 2 + 4 * kDenseRows * 128;

// One workgroup of 4 waves: part[s][row][n] = sum over k in [s*KR, s*KR + KR) of
// x[row][k] * W[k][n] for the 128 columns of block cb of an (in, out) row-major f16 W.
// Lane l of wave w reads 8 bytes (4 columns) of k-row s*KR + w*64 + 2*i + l/32 for
// i = 0..31, so one wave load covers 2 k-rows x 128 columns (512 B). Per output the sum
// is: per lane, its 32 k-rows in order; then the 2 lanes of a column (xor-shuffle); then
// the 4 waves in order.
__device__ __forceinline__ void dense_skinny(const uint16_t *__restrict__ x, int64_t rows, int in,
                                             int out, const uint16_t *__restrict__ W,
                                             float *__restrict__ part, int cb, int s,
                                             uint32_t *lds) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int q = lane >> 5, g = lane & 31;
  const int k0 = s * kDenseKR;
  const int col = cb * 128 + g * 4;
  uint32_t *xs = lds;                                           // [8 rows][KR/2 words]
  float *red = reinterpret_cast<float *>(lds + kDenseRows * kDenseKR / 2);  // [4][8][128]
  for (int64_t r0 = 0; r0 < rows; r0 += kDenseRows) {
    const int nr = (int)min<int64_t>(kDenseRows, rows - r0);
    static_assert(kDenseRows * kDenseKR / 8 == 256, "one 16-byte x chunk per thread");
    {
      const int r = threadIdx.x / (kDenseKR / 8), c8 = threadIdx.x % (kDenseKR / 8);
      reinterpret_cast<uint4 *>(xs)[threadIdx.x] =
          (r < nr && k0 + 8 * c8 < in)
              ? *reinterpret_cast<const uint4 *>(x + (r0 + r) * in + k0 + 8 * c8)
              : make_uint4(0u, 0u, 0u, 0u);
    }
    __syncthreads();
    float acc[kDenseRows][4];
#pragma unroll
    for (int r = 0; r < kDenseRows; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[r][c] = 0.0f;
#pragma unroll 1
    for (int i0 = 0; i0 < 32; i0 += 8) {
      u32x2 wv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int k = k0 + wave * 64 + 2 * (i0 + i) + q;
        wv[i] = k < in ? __builtin_nontemporal_load(
                             reinterpret_cast<const u32x2 *>(W + (int64_t)k * out + col))
                       : u32x2{0u, 0u};
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int kk = wave * 64 + 2 * (i0 + i) + q;  // k row inside this split
#pragma unroll
        for (int r = 0; r < kDenseRows; ++r) {
          const uint32_t xw = xs[r * (kDenseKR / 2) + (kk >> 1)];
          const float xv = q ? hi16f(xw) : lo16f(xw);
          acc[r][0] = fmaf(xv, lo16f(wv[i].x), acc[r][0]);
          acc[r][1] = fmaf(xv, hi16f(wv[i].x), acc[r][1]);
          acc[r][2] = fmaf(xv, lo16f(wv[i].y), acc[r][2]);
          acc[r][3] = fmaf(xv, hi16f(wv[i].y), acc[r][3]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kDenseRows; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[r][c] += __shfl_xor(acc[r][c], 32, 64);
    if (q == 0) {
#pragma unroll
      for (int r = 0; r < kDenseRows; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) red[(wave * kDenseRows + r) * 128 + g * 4 + c] = acc[r][c];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nr * 128; i += 256) {
      const int r = i >> 7, cc = i & 127;
      float v = red[(0 * kDenseRows + r) * 128 + cc];
      v += red[(1 * kDenseRows + r) * 128 + cc];
      v += red[(2 * kDenseRows + r) * 128 + cc];
      v += red[(3 * kDenseRows + r) * 128 + cc];
      part[((int64_t)s * rows + r0 + r) * out + cb * 128 + cc] = v;
    }
    __syncthreads();
  }
}

// Router logits for 4 experts per wave-group: one wave per expert e, logits[t][e] =
// sum_k f32(h[t][k]) * f32(router_w[e][k]) for token rows [r0, r0 + 8). Lane l holds
// the 16-byte chunks k = 8l + 512j of the expert's row (all loads issued at once); the
// lane partials are reduced with an xor-shuffle tree. xs: LDS, 8 rows x H/2 words.
__device__ __forceinline__ void router_logits(const uint16_t *__restrict__ h, int64_t rows,
                                              int H, const uint16_t *__restrict__ rw, int E,
                                              float *__restrict__ logits, int e0, int64_t r0,
                                              uint32_t *xs) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nr = (int)min<int64_t>(8, rows - r0);
  for (int i0 = threadIdx.x; i0 < H; i0 += 4 * 256) {  // 8 rows x H/8 16-byte chunks
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + 256 * u, r = i / (H / 8), c8 = i % (H / 8);
      v[u] = (i < H && r < nr) ? *reinterpret_cast<const uint4 *>(h + (r0 + r) * H + 8 * c8)
                               : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (i0 + 256 * u < H) reinterpret_cast<uint4 *>(xs)[i0 + 256 * u] = v[u];
  }
  __syncthreads();
  const int e = e0 + wave;
  if (e >= E) return;
  constexpr int kMaxChunks = 16;  // H <= 8192
  const int nch = (H + 511) / 512;
  uint4 wv[kMaxChunks];
#pragma unroll
  for (int j = 0; j < kMaxChunks; ++j) {
    wv[j] = make_uint4(0u, 0u, 0u, 0u);  // lanes past H contribute zero
    if (j < nch && 512 * j + 8 * lane < H)
      wv[j] = *reinterpret_cast<const uint4 *>(rw + (int64_t)e * H + 512 * j + 8 * lane);
  }
  float acc[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int j = 0; j < kMaxChunks; ++j) {
    const uint32_t w4[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
    if (j >= nch || 512 * j + 8 * lane >= H) continue;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const uint4 x4 = *reinterpret_cast<const uint4 *>(xs + r * (H / 2) + 256 * j + 4 * lane);
      const uint32_t xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        acc[r] = fmaf(lo16f(xv[c]), lo16f(w4[c]), acc[r]);
        acc[r] = fmaf(hi16f(xv[c]), hi16f(w4[c]), acc[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    float v = acc[r];
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
    if (lane == 0 && r < nr) logits[(r0 + r) * E + e] = v;
  }
}

}  // namespace exl3d
