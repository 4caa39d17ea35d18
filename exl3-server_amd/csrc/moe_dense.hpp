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
    // all 32 of this lane's weight loads are issued before the first product
    u32x2 wv[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      // rows past `in` load row in - 1: their staged x is zero, so they add nothing
      const int k = min(k0 + wave * 64 + 2 * i + q, in - 1);
      wv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(W + (int64_t)k * out + col));
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int kk = wave * 64 + 2 * i + q;  // k row inside this split
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

// Router logits on the matrix cores (glm5_moe.cpp:127-128): logits = f32(h) f32(W)^T
// with W = router_w (E, H) f16 as on disk. Products of f16 values are exact in f32,
// so only the summation order differs from a scalar f32 dot product. H is cut into
// logit_splits(H) <= 8 equal k splits; a wave task is (16 experts, one split): lane l
// loads 8 consecutive k of expert 16nb + l%16 (the B operand, k-group l/16) for 16
// 32-k steps at a time, the matching h values of 16 token rows (the A operand), and
// accumulates the 16x16x32 MFMAs in step order. The split partials go to
// part[(row * E + e) * kLogitSlots + s], summed in split order by the router.
typedef _Float16 f16x8_ __attribute__((ext_vector_type(8)));
typedef float f32x4_ __attribute__((ext_vector_type(4)));

constexpr int kLogitSlots = 8;      // partial slots per logit (splits <= 8)
constexpr int kLogitChunk = 16;     // 32-k MFMA steps whose operands are loaded at once

__host__ __device__ constexpr int logit_splits(int H) {
  return (H / 128) % 8 == 0 ? 8 : ((H / 128) % 4 == 0 ? 4 : ((H / 128) % 2 == 0 ? 2 : 1));
}

__device__ __forceinline__ void router_logits_mfma(const uint16_t *__restrict__ h, int64_t rows,
                                                   int H, const uint16_t *__restrict__ rw, int E,
                                                   float *__restrict__ part, int task) {
  const int lane = threadIdx.x & 63;
  const int S = logit_splits(H), sk = H / S, nsteps = sk / 32;
  const int nb = task / S, sp = task % S;
  const int e = nb * 16 + (lane & 15), g = lane >> 4;
  const int ec = e < E ? e : E - 1;  // out-of-range columns load a valid row, never stored
  const int k0 = sp * sk + 8 * g;
  for (int64_t r0 = 0; r0 < rows; r0 += 16) {
    const int64_t row = r0 + (lane & 15);
    const int64_t rc = row < rows ? row : rows - 1;
    f32x4_ D = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int q0 = 0; q0 < nsteps; q0 += kLogitChunk) {
      f16x8_ A[kLogitChunk], B[kLogitChunk];
#pragma unroll
      for (int q = 0; q < kLogitChunk; ++q) {
        const int k = k0 + 32 * min(q0 + q, nsteps - 1);
        B[q] = *reinterpret_cast<const f16x8_ *>(rw + (int64_t)ec * H + k);
        A[q] = *reinterpret_cast<const f16x8_ *>(h + rc * H + k);
      }
#pragma unroll
      for (int q = 0; q < kLogitChunk; ++q)
        if (q0 + q < nsteps) D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[q], B[q], D, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t rr = r0 + 4 * g + i;
      if (rr < rows && e < E) part[(rr * E + e) * kLogitSlots + sp] = D[i];
    }
  }
}

}  // namespace exl3d
