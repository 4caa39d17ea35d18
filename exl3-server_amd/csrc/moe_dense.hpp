// The f16 shared expert (g5_linear's mx::matmul branch, glm5_kda.cpp:120) and the
// router logits (glm5_moe.cpp:127-128): f16 GEMVs on the matrix cores, f32 accumulation.
#pragma once

#include "exl3_device.hpp"
#include "moe_common.hpp"

namespace exl3d {

__device__ __forceinline__ float rf16d(float v) { return (float)to_f16(v); }

// silu(min(g, L)) * clamp(u, -L, L), every MLX f16 op rounded (glm5_moe.cpp:66-74,
// 369-371): sigmoid, the product with g, and the product with u each round to f16. The
// clips apply whatever L is, as mx::clip does there (L = 0 gives 0; the up clip is
// max then min, as mx::clip's bounds are applied).
__device__ __forceinline__ float swiglu1(float g, float u, float L) {
  g = fminf(g, L);
  u = fminf(fmaxf(u, -L), L);
  const float sg = rf16d(1.0f / (1.0f + expf(-g)));
  const float act = rf16d(g * sg);
  return rf16d(act * u);
}

// Dense f16 GEMV on the matrix cores: part = f32(x) f32(Wt)^T for x (rows, in) and Wt
// (out, in), both f16 row-major (the router weight as stored; the f16 shared expert's
// weights transposed once when the layer is created). Products of f16 values are exact
// in f32, so only the summation order differs from a scalar f32 dot product. `in` is
// cut into S = dense_mfma_splits(in) <= 8 equal k splits; a wave task is (16 token
// rows, 16 outputs, one split): lane l loads 8 consecutive k of output 16nb + l%16 (the
// B operand, k-group l/16) and of token row 16rb + l%16 (the A operand), CHUNK 32-k
// steps at a time, and accumulates the 16x16x32 MFMAs in step order. Split partials
// are written to part[(row * out + n) * kDenseSlots + split] and summed in split order
// by the consumer.
typedef _Float16 f16x8_ __attribute__((ext_vector_type(8)));
typedef float f32x4_ __attribute__((ext_vector_type(4)));

constexpr int kDenseSlots = 8;   // partial slots per output (splits <= 8)

__host__ __device__ constexpr int dense_mfma_splits(int in) {
  return (in / 128) % 8 == 0 ? 8 : ((in / 128) % 4 == 0 ? 4 : ((in / 128) % 2 == 0 ? 2 : 1));
}
// Wave tasks of an (rows x in) @ (in x out) dense GEMV.
__host__ __device__ inline int64_t dense_mfma_tasks(int64_t rows, int in, int out) {
  return ((rows + 15) / 16) * ((out + 15) / 16) * dense_mfma_splits(in);
}

template <int CHUNK>
__device__ __forceinline__ void dense_mfma(const uint16_t *__restrict__ x, int64_t rows, int in,
                                           const uint16_t *__restrict__ wt, int out,
                                           float *__restrict__ part, int64_t task) {
  const int lane = threadIdx.x & 63;
  const int S = dense_mfma_splits(in), sk = in / S, nsteps = sk / 32;
  const int n_nb = (out + 15) / 16;
  const int sp = (int)(task % S);
  const int nb = (int)((task / S) % n_nb);
  const int64_t r0 = 16 * (task / ((int64_t)S * n_nb));
  const int n = nb * 16 + (lane & 15), g = lane >> 4;
  const int nc = n < out ? n : out - 1;  // out-of-range outputs load a valid row, never stored
  const int k0 = sp * sk + 8 * g;
  const int64_t row = r0 + (lane & 15);
  const int64_t rc = row < rows ? row : rows - 1;
  f32x4_ D = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
  for (int q0 = 0; q0 < nsteps; q0 += CHUNK) {
    f16x8_ A[CHUNK], B[CHUNK];
#pragma unroll
    for (int q = 0; q < CHUNK; ++q) {
      const int k = k0 + 32 * min(q0 + q, nsteps - 1);
      B[q] = *reinterpret_cast<const f16x8_ *>(wt + (int64_t)nc * in + k);
      A[q] = *reinterpret_cast<const f16x8_ *>(x + rc * in + k);
    }
#pragma unroll
    for (int q = 0; q < CHUNK; ++q)
      if (q0 + q < nsteps) D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[q], B[q], D, 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t rr = r0 + 4 * g + i;
    if (rr < rows && n < out) part[(rr * out + n) * kDenseSlots + sp] = D[i];
  }
}

// The same task (and output layout) computed by the 4 waves of a workgroup: wave w
// takes the w-th quarter of the split's MFMA steps, and the split partial is
// ((q0 + q1) + q2) + q3 of the quarters' accumulators, summed by wave 0 through LDS
// (red: 4 * 64 * 4 floats). Four times the memory parallelism of dense_mfma for
// launches too small to fill the machine (the router logits at decode batch sizes).
__device__ __forceinline__ void dense_mfma_wg4(const uint16_t *__restrict__ x, int64_t rows, int in,
                                               const uint16_t *__restrict__ wt, int out,
                                               float *__restrict__ part, int64_t task, float *red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int S = dense_mfma_splits(in), sk = in / S, nsteps = sk / 32, nq = nsteps / 4;
  const int n_nb = (out + 15) / 16;
  const int sp = (int)(task % S);
  const int nb = (int)((task / S) % n_nb);
  const int64_t r0 = 16 * (task / ((int64_t)S * n_nb));
  const int n = nb * 16 + (lane & 15), g = lane >> 4;
  const int nc = n < out ? n : out - 1;
  const int k0 = sp * sk + wave * nq * 32 + 8 * g;
  const int64_t row = r0 + (lane & 15);
  const int64_t rc = row < rows ? row : rows - 1;
  constexpr int kQ = 4;  // steps per load round
  f32x4_ D = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
  for (int q0 = 0; q0 < nq; q0 += kQ) {
    f16x8_ A[kQ], B[kQ];
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      const int k = k0 + 32 * min(q0 + q, nq - 1);
      B[q] = *reinterpret_cast<const f16x8_ *>(wt + (int64_t)nc * in + k);
      A[q] = *reinterpret_cast<const f16x8_ *>(x + rc * in + k);
    }
#pragma unroll
    for (int q = 0; q < kQ; ++q)
      if (q0 + q < nq) D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[q], B[q], D, 0, 0, 0);
  }
  reinterpret_cast<f32x4_ *>(red)[wave * 64 + lane] = D;
  __syncthreads();
  if (wave == 0) {
    const f32x4_ *rq = reinterpret_cast<const f32x4_ *>(red);
    f32x4_ t = rq[lane];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const f32x4_ u = rq[w * 64 + lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) t[i] = t[i] + u[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t rr = r0 + 4 * g + i;
      if (rr < rows && n < out) part[(rr * out + n) * kDenseSlots + sp] = t[i];
    }
  }
}

// One output from its kDenseSlots contiguous split partials, summed in split order.
__device__ __forceinline__ float dense_slots_sum(const float *p, int S) {
  const float4 a = *reinterpret_cast<const float4 *>(p);
  const float4 b = *reinterpret_cast<const float4 *>(p + 4);
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float acc = v[0];
#pragma unroll
  for (int s = 1; s < 8; ++s)
    if (s < S) acc += v[s];
  return acc;
}

// The f16 shared expert (g5_linear's mx::matmul branch, glm5_kda.cpp:120; SwiGLU as in
// glm5_moe.cpp:66-74) as extra workgroups (one MFMA task per wave) of the
// routed expert launches: the gate/up partials beside the routed gate/up, their SwiGLU
// beside the routed activations, the down partials beside the routed down (the combine
// sums those in split order). Weights: the layer's transposed (out, in) copies.
constexpr int kSharedChunk = 4;  // MFMA steps per load round (keeps the expert kernels' VGPRs)

// Workgroups of `waves` waves, one task per wave.
__host__ __device__ inline int shared_gate_up_blocks(int64_t N, int H, int SI, int waves) {
  return (int)((2 * dense_mfma_tasks(N, H, SI) + waves - 1) / waves);
}
__host__ __device__ inline int shared_down_blocks(int64_t N, int H, int SI, int waves) {
  return (int)((dense_mfma_tasks(N, SI, H) + waves - 1) / waves);
}
__host__ __device__ inline int shared_swiglu_blocks(int64_t N, int SI) {
  return (int)((N * SI / 2 + 255) / 256);
}

__device__ __forceinline__ void shared_gate_up_block(const uint16_t *h, int64_t N, int H, int SI,
                                                     const uint16_t *wg_t, const uint16_t *wu_t,
                                                     float *dsh_gu, int b, int waves) {
  const int64_t per = dense_mfma_tasks(N, H, SI);
  const int64_t task = (int64_t)b * waves + (threadIdx.x >> 6);
  if (task >= 2 * per) return;
  const int proj = task >= per;
  dense_mfma<kSharedChunk>(h, N, H, proj ? wu_t : wg_t, SI,
                           dsh_gu + (int64_t)proj * N * SI * kDenseSlots, task - proj * per);
}

// One element pair (i, i + 1) per thread of 256-thread workgroup b.
__device__ __forceinline__ void shared_swiglu_block(const float *dsh_gu, int64_t N, int H, int SI,
                                                    float limit, uint16_t *dsh_act, int b) {
  const int64_t i = 2 * ((int64_t)b * 256 + (threadIdx.x & 255));
  const int64_t n = N * SI;
  if (i >= n) return;
  const int S = dense_mfma_splits(H);
  const float *pg = dsh_gu + i * kDenseSlots, *pu = dsh_gu + (n + i) * kDenseSlots;
  const float g0 = dense_slots_sum(pg, S), g1 = dense_slots_sum(pg + kDenseSlots, S);
  const float u0 = dense_slots_sum(pu, S), u1 = dense_slots_sum(pu + kDenseSlots, S);
  const float L = rf16d(limit);
  const uint32_t o = (uint32_t)bitcast<uint16_t>(to_f16(swiglu1(rf16d(g0), rf16d(u0), L))) |
                     ((uint32_t)bitcast<uint16_t>(to_f16(swiglu1(rf16d(g1), rf16d(u1), L))) << 16);
  *reinterpret_cast<uint32_t *>(dsh_act + i) = o;
}

__device__ __forceinline__ void shared_down_block(const uint16_t *dsh_act, int64_t N, int H, int SI,
                                                  const uint16_t *wd_t, float *dsh_dn, int b,
                                                  int waves) {
  const int64_t task = (int64_t)b * waves + (threadIdx.x >> 6);
  if (task >= dense_mfma_tasks(N, SI, H)) return;
  dense_mfma<kSharedChunk>(dsh_act, N, SI, wd_t, H, dsh_dn, task);
}

}  // namespace exl3d
