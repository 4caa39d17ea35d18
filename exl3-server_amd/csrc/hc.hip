// The steps either side of the MoE in the GLM-5 batch step (glm5_forward.cpp:434-438):
// the hyper-connection prepare (g5_hc_prepare, glm5_hc.cpp:242-340), the RMSNorm of its
// collapsed stream (rms_norm, glm5_attn.cpp:12-22) and the hyper-connection mix
// (g5_hc_mix, glm5_hc.cpp:342-355), gfx950.
//
//  k_hc_proj      grid (k chunk of the N*D axis, group of kHcRows positions): per position
//                 the chunk's sum of squares and its part of the W = (2+N)*N projections
//                 x . fn[j] (fn stored (W, N*D), as the reference's F.linear weight);
//                 f32 partials per chunk. Each wave keeps its projections' fn slice in
//                 registers and reuses it for every position of the group.
//  k_hc_finalize  one workgroup per position: the partials summed in chunk order, the RMS
//                 factor (w = rms * x.fn, the fused reference kernel's per-term product
//                 folded out of the sum), pre/post/comb with the softmax over the last
//                 axis, the Sinkhorn in the reference's loop order (glm5_hc.cpp:321-324),
//                 the collapsed stream sum_n pre[n] * streams[n] rounded to f16, and,
//                 given a norm weight, the RMSNorm of that row fused behind it.
//  k_rms_norm     the RMSNorm alone, one workgroup per row.
//  k_hc_mix       post[n] * out + comb^T @ residual in f16 (also fused into the MoE
//                 combine, which then writes the new streams directly).
#include <hip/hip_runtime.h>

#include <cmath>
#include <string>

#include "exl3_device.hpp"
#include "exl3_internal.hpp"
#include "exl3_moe.h"
#include "moe_common.hpp"

using namespace exl3d;

namespace {

constexpr int kHcMaxN = 4;                       // streams (W <= 24), as the reference's fused path
constexpr int kHcMaxW = (2 + kHcMaxN) * kHcMaxN;
constexpr int kHcChunk = 256;                    // elements of the N*D axis per workgroup
constexpr int kHcRows = 8;                       // positions per projection workgroup
constexpr int kHcVals = kHcMaxW + 1;             // per chunk: W projections, then the sum of squares

__device__ __forceinline__ float wave_sum(float v) {
  v += xor_lanes<1>(v);
  v += xor_lanes<2>(v);
  v += xor_lanes<4>(v);
  v += xor_lanes<8>(v);
  v += xor_lanes<16>(v);
  v += xor_lanes<32>(v);
  return v;
}

__device__ __forceinline__ float h2f(uint16_t v) { return (float)bitcast<f16>(v); }

__global__ __launch_bounds__(256) void k_hc_proj(const uint16_t *__restrict__ streams, int64_t P, int ND, int W,
                                                 const float *__restrict__ fn, float *__restrict__ part) {
  const int chunk = blockIdx.x, n_chunks = gridDim.x;
  const int64_t p0 = (int64_t)blockIdx.y * kHcRows;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int k0 = chunk * kHcChunk + 4 * lane;  // this lane's 4 elements
  // projections j = wave, wave + 4, ...: their fn slices, kept for every position
  constexpr int kPer = kHcMaxW / 4;
  float4 f[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int j = wave + 4 * q;
    f[q] = j < W ? *reinterpret_cast<const float4 *>(fn + (int64_t)j * ND + k0) : float4{0, 0, 0, 0};
  }
  for (int r = 0; r < kHcRows && p0 + r < P; ++r) {
    const int64_t p = p0 + r;
    const uint2 sv = *reinterpret_cast<const uint2 *>(streams + p * ND + k0);
    const float s0 = h2f(sv.x & 0xffff), s1 = h2f(sv.x >> 16), s2 = h2f(sv.y & 0xffff), s3 = h2f(sv.y >> 16);
    float *out = part + (p * n_chunks + chunk) * kHcVals;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int j = wave + 4 * q;
      float d = s0 * f[q].x;
      d = fmaf(s1, f[q].y, d);
      d = fmaf(s2, f[q].z, d);
      d = fmaf(s3, f[q].w, d);
      d = wave_sum(d);
      if (j < W && lane == 0) out[j] = d;
    }
    if (wave == 0) {
      float ss = s0 * s0;
      ss = fmaf(s1, s1, ss);
      ss = fmaf(s2, s2, ss);
      ss = fmaf(s3, s3, ss);
      ss = wave_sum(ss);
      if (lane == 0) out[kHcMaxW] = ss;
    }
  }
}

// Sum of one value over a workgroup of 4 waves, the waves' sums added in wave order.
__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  const float t = ((red[0] + red[1]) + red[2]) + red[3];
  __syncthreads();
  return t;
}

// y = f16(f16(x * r) * w) for this thread's elements (x already f16 values in f32).
template <int PER>
__device__ __forceinline__ void rms_apply(const float (&x)[PER], int D, float eps, const uint16_t *w, uint16_t *y,
                                          float *red) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = threadIdx.x + 256 * i;
    if (d < D) ss = fmaf(x[i], x[i], ss);
  }
  const float total = block_sum(ss, red);
  const float r = 1.0f / sqrtf(total / (float)D + eps);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = threadIdx.x + 256 * i;
    if (d < D) {
      const float n = (float)to_f16(x[i] * r);
      y[d] = f32_to_f16(n * h2f(w[d]));
    }
  }
}

constexpr int kHcMaxD = 8192;
constexpr int kHcPer = kHcMaxD / 256;

__global__ __launch_bounds__(256) void k_hc_finalize(const uint16_t *__restrict__ streams, int N, int D, int W,
                                                     int n_chunks, const float *__restrict__ part,
                                                     const float *__restrict__ base, const float *__restrict__ scale,
                                                     int iters, float eps, const uint16_t *__restrict__ norm_w,
                                                     float norm_eps, uint16_t *__restrict__ out,
                                                     float *__restrict__ post_out, float *__restrict__ comb_out) {
  __shared__ float vals[kHcVals];
  __shared__ float pre[kHcMaxN];
  __shared__ float red[4];
  const int64_t p = blockIdx.x;
  const int64_t ND = (int64_t)N * D;
  const int t = threadIdx.x;
  // the chunk partials in chunk order
  if (t < W || t == kHcMaxW) {
    const float *pp = part + p * n_chunks * kHcVals + t;
    float acc = pp[0];
    for (int c = 1; c < n_chunks; ++c) acc += pp[(int64_t)c * kHcVals];
    vals[t] = acc;
  }
  __syncthreads();
  if (t == 0) {
    const float rms = 1.0f / sqrtf(vals[kHcMaxW] / (float)ND + eps);
    float w[kHcMaxW];
    for (int j = 0; j < W; ++j) w[j] = vals[j] * rms;
    for (int n = 0; n < N; ++n) {
      pre[n] = 1.0f / (1.0f + expf(-(w[n] * scale[0] + base[n]))) + eps;
      post_out[p * N + n] = 2.0f * (1.0f / (1.0f + expf(-(w[N + n] * scale[1] + base[N + n]))));
    }
    float c[kHcMaxN * kHcMaxN];
    for (int i = 0; i < N; ++i) {
      float m = -INFINITY;
      for (int j = 0; j < N; ++j) {
        const float z = w[2 * N + i * N + j] * scale[2] + base[2 * N + i * N + j];
        c[i * N + j] = z;
        m = fmaxf(m, z);
      }
      float s = 0.0f;
      for (int j = 0; j < N; ++j) {
        c[i * N + j] = expf(c[i * N + j] - m);
        s += c[i * N + j];
      }
      for (int j = 0; j < N; ++j) c[i * N + j] = c[i * N + j] / s + eps;
    }
    for (int j = 0; j < N; ++j) {
      float cs = 0.0f;
      for (int i = 0; i < N; ++i) cs += c[i * N + j];
      for (int i = 0; i < N; ++i) c[i * N + j] = c[i * N + j] / (cs + eps);
    }
    for (int it = 0; it < iters - 1; ++it) {
      for (int i = 0; i < N; ++i) {
        float rs = 0.0f;
        for (int j = 0; j < N; ++j) rs += c[i * N + j];
        for (int j = 0; j < N; ++j) c[i * N + j] = c[i * N + j] / (rs + eps);
      }
      for (int j = 0; j < N; ++j) {
        float cs = 0.0f;
        for (int i = 0; i < N; ++i) cs += c[i * N + j];
        for (int i = 0; i < N; ++i) c[i * N + j] = c[i * N + j] / (cs + eps);
      }
    }
    for (int k = 0; k < N * N; ++k) comb_out[p * N * N + k] = c[k];
  }
  __syncthreads();
  // collapsed = sum_n pre[n] * streams[n], in f16
  const uint16_t *s = streams + p * ND;
  float x[kHcPer];
#pragma unroll
  for (int i = 0; i < kHcPer; ++i) {
    const int d = t + 256 * i;
    float a = 0.0f;
    if (d < D) {
      for (int n = 0; n < N; ++n) a = fmaf(pre[n], h2f(s[(int64_t)n * D + d]), a);
    }
    x[i] = (float)to_f16(a);
  }
  if (!norm_w) {
#pragma unroll
    for (int i = 0; i < kHcPer; ++i) {
      const int d = t + 256 * i;
      if (d < D) out[p * D + d] = f32_to_f16(x[i]);
    }
    return;
  }
  rms_apply<kHcPer>(x, D, norm_eps, norm_w, out + p * D, red);
}

__global__ __launch_bounds__(256) void k_rms_norm(const uint16_t *__restrict__ xin, int D, const uint16_t *__restrict__ w,
                                                  float eps, uint16_t *__restrict__ y) {
  __shared__ float red[4];
  const int64_t p = blockIdx.x;
  float x[kHcPer];
#pragma unroll
  for (int i = 0; i < kHcPer; ++i) {
    const int d = threadIdx.x + 256 * i;
    x[i] = d < D ? h2f(xin[p * D + d]) : 0.0f;
  }
  rms_apply<kHcPer>(x, D, eps, w, y + p * D, red);
}

// post[n] * out + comb^T @ residual, f16 as the reference (its g5_hc_mix runs in
// block_out's dtype): each thread two adjacent d of one position, every n.
__global__ __launch_bounds__(256) void k_hc_mix(const uint16_t *__restrict__ bout, const float *__restrict__ post,
                                                const float *__restrict__ comb, const uint16_t *__restrict__ res,
                                                int64_t P, int N, int D, uint16_t *__restrict__ out) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int half_d = D / 2;
  if (g >= P * half_d) return;
  const int64_t p = g / half_d;
  const int d = (int)(g % half_d) * 2;
  const uint32_t b = *reinterpret_cast<const uint32_t *>(bout + p * D + d);
  exl3m::hc_mix_pair(post + p * N, comb + p * N * N, res + p * N * D + d, D, N, h2f(b & 0xffff), h2f(b >> 16),
                     out + p * N * D + d);
}

}  // namespace

namespace exl3h {

exl3_status check_hc(const exl3_hc_site *hc, int D) {
  if (!hc || !hc->fn || !hc->base || !hc->scale) return fail(EXL3_ERR_INVALID, "null hyper-connection site");
  if (hc->mult < 1 || hc->mult > kHcMaxN)
    return fail(EXL3_ERR_UNSUPPORTED, "hc_mult must be 1..4 (the fused path's range)");
  if (hc->sinkhorn_iters < 1) return fail(EXL3_ERR_INVALID, "hc_sinkhorn_iters must be >= 1");
  if (D <= 0 || D > kHcMaxD || D % 2 || ((int64_t)hc->mult * D) % kHcChunk)
    return fail(EXL3_ERR_UNSUPPORTED, "hidden size must be even, at most 8192, and N*hidden a multiple of 256");
  return EXL3_OK;
}

size_t hc_part_bytes(int N, int D, int64_t P) {
  return align_up((size_t)P * ((size_t)N * D / kHcChunk) * kHcVals * 4, 256);
}

exl3_status launch_hc_prepare(const exl3_hc_site *hc, const uint16_t *streams, int64_t P, int D,
                              const uint16_t *norm_w, float norm_eps, uint16_t *out, float *post,
                              float *comb, float *part, hipStream_t st) {
  const int N = hc->mult, W = (2 + N) * N, ND = N * D, n_chunks = ND / kHcChunk;
  if (P == 0) return EXL3_OK;
  const int64_t groups = (P + kHcRows - 1) / kHcRows;
  if (groups > 65535) return fail(EXL3_ERR_UNSUPPORTED, "too many positions in one call");
  k_hc_proj<<<dim3((unsigned)n_chunks, (unsigned)groups), 256, 0, st>>>(streams, P, ND, W, hc->fn, part);
  EXL3_LAUNCHED("k_hc_proj");
  k_hc_finalize<<<(unsigned)P, 256, 0, st>>>(streams, N, D, W, n_chunks, part, hc->base, hc->scale,
                                              hc->sinkhorn_iters, hc->eps, norm_w, norm_eps, out, post, comb);
  EXL3_LAUNCHED("k_hc_finalize");
  return EXL3_OK;
}

}  // namespace exl3h

using namespace exl3h;

extern "C" {

size_t exl3_hc_workspace_size(int32_t mult, int32_t hidden, int64_t P) {
  if (mult < 1 || mult > kHcMaxN || hidden <= 0 || P < 0 || ((int64_t)mult * hidden) % kHcChunk) return 0;
  return hc_part_bytes(mult, hidden, P);
}

exl3_status exl3_hc_prepare(const exl3_hc_site *hc, const uint16_t *streams, int64_t P, int32_t hidden,
                            const uint16_t *norm_w, float norm_eps, uint16_t *out, float *post, float *comb,
                            void *workspace, size_t workspace_bytes, exl3_stream_t stream) {
  exl3_status rc = check_hc(hc, hidden);
  if (rc) return rc;
  if (P < 0 || P > ((int64_t)1 << 31)) return fail(EXL3_ERR_INVALID, "exl3_hc_prepare: bad row count");
  if (P == 0) return EXL3_OK;
  if (!streams || !out || !post || !comb) return fail(EXL3_ERR_INVALID, "exl3_hc_prepare: null argument");
  const size_t need = hc_part_bytes(hc->mult, hidden, P);
  if (!workspace || workspace_bytes < need)
    return fail(EXL3_ERR_WORKSPACE, "exl3_hc_prepare: workspace too small: need " + std::to_string(need) + " bytes");
  if (reinterpret_cast<uintptr_t>(workspace) % 256)
    return fail(EXL3_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  if (reinterpret_cast<uintptr_t>(streams) % 8 || reinterpret_cast<uintptr_t>(hc->fn) % 16)
    return fail(EXL3_ERR_INVALID, "streams must be 8-byte and fn 16-byte aligned");
  return launch_hc_prepare(hc, streams, P, hidden, norm_w, norm_eps, out, post, comb, (float *)workspace,
                           stream_of(stream));
}

exl3_status exl3_rms_norm(const uint16_t *x, int64_t P, int32_t hidden, const uint16_t *w, float eps, uint16_t *y,
                          exl3_stream_t stream) {
  if (P < 0 || P > ((int64_t)1 << 31) || hidden <= 0 || hidden > kHcMaxD)
    return fail(EXL3_ERR_INVALID, "exl3_rms_norm: bad shape (hidden at most 8192)");
  if (P == 0) return EXL3_OK;
  if (!x || !w || !y) return fail(EXL3_ERR_INVALID, "exl3_rms_norm: null argument");
  k_rms_norm<<<(unsigned)P, 256, 0, stream_of(stream)>>>(x, hidden, w, eps, y);
  EXL3_LAUNCHED("k_rms_norm");
  return EXL3_OK;
}

exl3_status exl3_hc_mix(const uint16_t *block_out, const float *post, const float *comb, const uint16_t *residual,
                        int64_t P, int32_t mult, int32_t hidden, uint16_t *out, exl3_stream_t stream) {
  if (P < 0 || mult < 1 || mult > kHcMaxN || hidden <= 0 || hidden % 2)
    return fail(EXL3_ERR_INVALID, "exl3_hc_mix: bad shape (hc_mult 1..4, even hidden)");
  if (P == 0) return EXL3_OK;
  if (!block_out || !post || !comb || !residual || !out) return fail(EXL3_ERR_INVALID, "exl3_hc_mix: null argument");
  if ((reinterpret_cast<uintptr_t>(block_out) | reinterpret_cast<uintptr_t>(residual) |
       reinterpret_cast<uintptr_t>(out)) % 4)
    return fail(EXL3_ERR_INVALID, "exl3_hc_mix: block_out, residual and out must be 4-byte aligned");
  if (P > ((int64_t)1 << 40) / hidden) return fail(EXL3_ERR_UNSUPPORTED, "exl3_hc_mix: too large");
  if (overlaps(residual, out, (size_t)P * mult * hidden * 2))
    return fail(EXL3_ERR_INVALID, "exl3_hc_mix: out must not overlap residual");
  const int64_t threads = P * (hidden / 2);
  if (threads == 0) return EXL3_OK;
  k_hc_mix<<<(unsigned)((threads + 255) / 256), 256, 0, stream_of(stream)>>>(block_out, post, comb, residual, P,
                                                                             mult, hidden, out);
  EXL3_LAUNCHED("k_hc_mix");
  return EXL3_OK;
}

}  // extern "C"
