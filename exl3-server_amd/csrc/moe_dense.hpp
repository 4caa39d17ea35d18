// The f16 shared expert (g5_linear's mx::matmul branch, glm5_kda.cpp:120) and the
// router logits (glm5_moe.cpp:127-128): skinny f16 GEMVs with f32 accumulation.
#pragma once

#include "exl3_device.hpp"
#include "moe_common.hpp"

namespace exl3d {

__device__ __forceinline__ float lo16f(uint32_t v) { return (float)bitcast<f16>((uint16_t)(v & 0xffffu)); }
__device__ __forceinline__ float hi16f(uint32_t v) { return (float)bitcast<f16>((uint16_t)(v >> 16)); }

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float rf16d(float v) { return (float)to_f16(v); }

// silu(min(g, L)) * clamp(u, -L, L), every MLX f16 op rounded (glm5_moe.cpp:66-74,
// 369-371): sigmoid, the product with g, and the product with u each round to f16.
__device__ __forceinline__ float swiglu1(float g, float u, float L) {
  if (L > 0.0f) {
    g = fminf(g, L);
    u = fminf(fmaxf(u, -L), L);
  }
  const float sg = rf16d(1.0f / (1.0f + expf(-g)));
  const float act = rf16d(g * sg);
  return rf16d(act * u);
}

constexpr int kDenseKR = 256;   // k rows per dense workgroup (one k split)

// k splits of a dense_skinny GEMV over `in` rows.
__host__ __device__ constexpr int dense_splits(int in) { return (in + kDenseKR - 1) / kDenseKR; }
constexpr int kDenseRows = 8;   // token rows per pass

// LDS words a dense_skinny workgroup needs.
constexpr int kDenseLdsWords = kDenseRows * kDenseKR / 2 + 4 * kDenseRows * 128;

// One workgroup of 4 waves: part[s][row][n] = sum over k in [s*KR, s*KR + KR) of
// x[row][k] * W[k][n] for the 128 columns of block cb of an (in, out) row-major f16 W.
// Lane l reads the 4 bytes of columns 2l, 2l + 1 of one k-row per load, so one wave
// load covers a whole 256-byte k-row of the block; wave w takes k-rows s*KR + 64w + i,
// i = 0..63, 8 loads in flight at a time. Per output the sum is: per lane, its 64
// k-rows in order; then the 4 waves in order. Small enough (about 50 VGPRs) to run as
// extra workgroups of the routed expert kernels without lowering their occupancy.
__device__ __forceinline__ void dense_skinny(const uint16_t *__restrict__ x, int64_t rows, int in,
                                             int out, const uint16_t *__restrict__ W,
                                             float *__restrict__ part, int cb, int s,
                                             uint32_t *lds) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k0 = s * kDenseKR;
  const int col = cb * 128 + 2 * lane;
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
    float acc[kDenseRows][2];
#pragma unroll
    for (int r = 0; r < kDenseRows; ++r) acc[r][0] = acc[r][1] = 0.0f;
#pragma unroll 1
    for (int i0 = 0; i0 < 64; i0 += 8) {
      uint32_t wv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        // rows past `in` load row in - 1: their staged x is zero, so they add nothing
        const int k = min(k0 + wave * 64 + i0 + i, in - 1);
        wv[i] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(W + (int64_t)k * out + col));
      }
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        const int kk = wave * 64 + i0 + i;  // even k row inside this split
#pragma unroll
        for (int r = 0; r < kDenseRows; ++r) {
          const uint32_t xw = xs[r * (kDenseKR / 2) + (kk >> 1)];  // k rows kk, kk + 1
          acc[r][0] = fmaf(lo16f(xw), lo16f(wv[i]), acc[r][0]);
          acc[r][1] = fmaf(lo16f(xw), hi16f(wv[i]), acc[r][1]);
          acc[r][0] = fmaf(hi16f(xw), lo16f(wv[i + 1]), acc[r][0]);
          acc[r][1] = fmaf(hi16f(xw), hi16f(wv[i + 1]), acc[r][1]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kDenseRows; ++r) {
      red[(wave * kDenseRows + r) * 128 + 2 * lane] = acc[r][0];
      red[(wave * kDenseRows + r) * 128 + 2 * lane + 1] = acc[r][1];
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

// The f16 shared expert (g5_linear's mx::matmul branch, glm5_kda.cpp:120), as extra
// workgroups of the routed expert launches: gate/up k-split partials beside the routed
// gate/up, their SwiGLU beside the routed activations, the down k-split partials beside
// the routed down (the combine sums them in split order).
__host__ __device__ inline int shared_gate_up_blocks(int H, int SI) {
  return 2 * (SI / 128) * dense_splits(H);
}
__host__ __device__ inline int shared_down_blocks(int H, int SI) {
  return (H / 128) * dense_splits(SI);
}
__host__ __device__ inline int shared_swiglu_blocks(int64_t N, int SI) {
  return (int)((N * SI / 2 + 255) / 256);
}

__device__ __forceinline__ void shared_gate_up_block(const uint16_t *h, int64_t N, int H, int SI,
                                                     const uint16_t *wg, const uint16_t *wu,
                                                     float *dsh_gu, int b, uint32_t *lds) {
  const int n_cb = SI / 128, S = dense_splits(H);
  const int proj = b / (n_cb * S), rem = b % (n_cb * S);
  dense_skinny(h, N, H, SI, proj ? wu : wg, dsh_gu + (int64_t)proj * S * N * SI, rem % n_cb,
               rem / n_cb, lds);
}

// One element pair (i, i + 1) per thread of 256-thread workgroup b.
__device__ __forceinline__ void shared_swiglu_block(const float *dsh_gu, int64_t N, int H, int SI,
                                                    float limit, uint16_t *dsh_act, int b) {
  const int64_t i = 2 * ((int64_t)b * 256 + (threadIdx.x & 255));
  const int64_t n = N * SI;
  if (i >= n) return;
  const int S = dense_splits(H);
  const float2 g = exl3m::ordered_sum2<16>(dsh_gu + i, n, S);
  const float2 u = exl3m::ordered_sum2<16>(dsh_gu + (int64_t)S * n + i, n, S);
  const float L = limit > 0.0f ? rf16d(limit) : 0.0f;
  const uint32_t o = (uint32_t)bitcast<uint16_t>(to_f16(swiglu1(rf16d(g.x), rf16d(u.x), L))) |
                     ((uint32_t)bitcast<uint16_t>(to_f16(swiglu1(rf16d(g.y), rf16d(u.y), L))) << 16);
  *reinterpret_cast<uint32_t *>(dsh_act + i) = o;
}

__device__ __forceinline__ void shared_down_block(const uint16_t *dsh_act, int64_t N, int H, int SI,
                                                  const uint16_t *wd, float *dsh_dn, int b,
                                                  uint32_t *lds) {
  const int n_cb = H / 128;
  dense_skinny(dsh_act, N, SI, H, wd, dsh_dn, b % n_cb, b / n_cb, lds);
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
