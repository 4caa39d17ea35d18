// The steps either side of the MoE in the GLM-5 batch step (glm5_forward.cpp:434-438):
// the hyper-connection prepare (g5_hc_prepare, glm5_hc.cpp:242-340), the RMSNorm of its
// collapsed stream (rms_norm, glm5_attn.cpp:12-22) and the hyper-connection mix
// (g5_hc_mix, glm5_hc.cpp:342-355), gfx950.
//
//  k_hc_proj      grid (k chunk of the N*D axis, group of positions): per position
//                 the chunk's sum of squares and its part of the W = (2+N)*N projections
//                 x . fn[j] (fn stored (W, N*D), as the reference's F.linear weight);
//                 f32 partials per chunk. Each wave keeps its projections' fn slice in
//                 registers and reuses it for every position of the group.
//  k_hc_finalize  two workgroups per position, side by side: both sum the partials in
//                 chunk order and take the RMS factor (w = rms * x.fn, the fused
//                 reference kernel's per-term product folded out of the sum); one forms
//                 pre and the collapsed stream sum_n pre[n] * streams[n] rounded to f16
//                 (and, given a norm weight, the RMSNorm of that row fused behind it),
//                 the other post and comb, with the softmax over the last axis and the
//                 Sinkhorn in the reference's loop order (glm5_hc.cpp:321-324).
//  k_rms_norm     the RMSNorm alone, one workgroup per row.
//  k_hc_mix       post[n] * out + comb^T @ residual in f16 (also fused into the MoE
//                 combine, which then writes the new streams directly).
#include <hip/hip_runtime.h>

#include <cmath>
#include <string>
#include <type_traits>

#include "exl3_device.hpp"
#include "exl3_internal.hpp"
#include "exl3_moe.h"
#include "moe_common.hpp"

using namespace exl3d;

namespace {

constexpr int kHcMaxN = 8;                       // streams (W <= 80)
static_assert(kHcMaxN <= exl3m::kHcMixMax, "the mix's residual registers");
constexpr int kHcNarrowN = 4;                    // the narrow kernels' streams (W <= 24; GLM-5's 4)
constexpr int kHcChunk = 64;                     // elements of the N*D axis per workgroup

// Per kernel variant (kN = 4: 1..4 streams; kN = 8: 5..8): the W = (2+N)*N projections'
// bound, the values per (position, chunk) partial (the W projections, then the sum of
// squares, at index kMaxW), positions per projection workgroup, and the finalize's
// reduction of the chunk partials by kG groups of kJ threads.
template <int kN>
struct HcShape {
  static constexpr int kMaxW = (2 + kN) * kN;
  static constexpr int kVals = kMaxW + 1;
  static constexpr int kRows = kN <= kHcNarrowN ? 8 : 3;
  static constexpr int kProjThreads = kVals * kRows;  // 200, 243
  static constexpr int kJ = kN <= kHcNarrowN ? 32 : 128;
  static constexpr int kG = 256 / kJ;
  static_assert(kProjThreads <= 256 && kVals <= kJ, "hc shape");
};
// Values per (position, chunk) partial for N streams (the part buffer's layout).
constexpr int hc_vals(int N) { return N <= kHcNarrowN ? HcShape<kHcNarrowN>::kVals : HcShape<kHcMaxN>::kVals; }

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

// Thread (j, r): projection j < W of position p0 + r (r < kRows), the dot product of
// the workgroup's chunk of the N*D axis with fn row j, in k order; threads past the
// projections: the chunk's sum of squares of position p0 + r. All of a thread's loads are
// in flight at once; no cross-lane reduction.
template <int kN>
__global__ __launch_bounds__(256) void k_hc_proj(const uint16_t *__restrict__ streams, int64_t P, int ND, int W,
                                                 const float *__restrict__ fn, float *__restrict__ part) {
  using S = HcShape<kN>;
  const int chunk = blockIdx.x, n_chunks = gridDim.x;
  const int t = threadIdx.x;
  if (t >= S::kProjThreads) return;
  const bool sq = t >= S::kMaxW * S::kRows;
  const int j = sq ? S::kMaxW : t / S::kRows, r = t % S::kRows;
  const int64_t p = (int64_t)blockIdx.y * S::kRows + r;
  if (p >= P || (!sq && j >= W)) return;
  const int k0 = chunk * kHcChunk;
  const uint16_t *s = streams + p * ND + k0;
  const float *f = fn + (int64_t)(sq ? 0 : j) * ND + k0;
  // the chunk's 16 groups of 4 elements, every load in flight at once
  constexpr int kGroups = kHcChunk / 4;
  uint2 sv[kGroups];
  float4 fv[kGroups];
#pragma unroll
  for (int q = 0; q < kGroups; ++q) {
    sv[q] = *reinterpret_cast<const uint2 *>(s + 4 * q);
    if (!sq) fv[q] = *reinterpret_cast<const float4 *>(f + 4 * q);
  }
  float acc = 0.0f;
  {
#pragma unroll
    for (int q = 0; q < kGroups; ++q) {
      const float s0 = h2f(sv[q].x & 0xffff), s1 = h2f(sv[q].x >> 16), s2 = h2f(sv[q].y & 0xffff),
                  s3 = h2f(sv[q].y >> 16);
      if (sq) {
        acc = fmaf(s0, s0, acc);
        acc = fmaf(s1, s1, acc);
        acc = fmaf(s2, s2, acc);
        acc = fmaf(s3, s3, acc);
      } else {
        acc = fmaf(s0, fv[q].x, acc);
        acc = fmaf(s1, fv[q].y, acc);
        acc = fmaf(s2, fv[q].z, acc);
        acc = fmaf(s3, fv[q].w, acc);
      }
    }
  }
  part[(p * n_chunks + chunk) * S::kVals + j] = acc;
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

constexpr int kHcMaxD = 8192;
constexpr int kHcPairs = kHcMaxD / 512;  // element pairs per thread at the largest hidden size

// This thread's pairs of a row: d = 2 * (threadIdx.x + 256 * i).
__device__ __forceinline__ int pair_d(int i) { return 2 * ((int)threadIdx.x + 256 * i); }

// This thread's pairs of the norm weights (w: at least D values; callers issue these
// loads early, so that they are not a round trip of their own at the end).
__device__ __forceinline__ void load_pairs(const uint16_t *w, int D, uint32_t (&wv)[kHcPairs]) {
#pragma unroll
  for (int i = 0; i < kHcPairs; ++i) wv[i] = *reinterpret_cast<const uint32_t *>(w + min(pair_d(i), D - 2));
}

// y = f16(f16(x * r) * w) on this thread's pairs (x0/x1: the pairs' f16 values in f32;
// wv: the norm weights' pairs, from load_pairs), r = rsqrt(mean(x^2) + eps) of the row:
// the thread's squares summed in pair order, then the workgroup's sum.
__device__ __forceinline__ void rms_pairs(const float (&x0)[kHcPairs], const float (&x1)[kHcPairs], int D,
                                          float eps, const uint32_t (&wv)[kHcPairs], uint16_t *y, float *red) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kHcPairs; ++i)
    if (pair_d(i) < D) {
      ss = fmaf(x0[i], x0[i], ss);
      ss = fmaf(x1[i], x1[i], ss);
    }
  const float total = block_sum(ss, red);
  const float r = 1.0f / sqrtf(total / (float)D + eps);
#pragma unroll
  for (int i = 0; i < kHcPairs; ++i)
    if (pair_d(i) < D) {
      const float n0 = (float)to_f16(x0[i] * r), n1 = (float)to_f16(x1[i] * r);
      *reinterpret_cast<uint32_t *>(y + pair_d(i)) =
          pack_f16x2(n0 * h2f(wv[i] & 0xffff), n1 * h2f(wv[i] >> 16));
    }
}

template <int kN>
__global__ __launch_bounds__(256) void k_hc_finalize(const uint16_t *__restrict__ streams, int N, int D, int W,
                                                     int n_chunks, const float *__restrict__ part,
                                                     const float *__restrict__ base, const float *__restrict__ scale,
                                                     int iters, float eps, const uint16_t *__restrict__ norm_w,
                                                     float norm_eps, uint16_t *__restrict__ out,
                                                     float *__restrict__ post_out, float *__restrict__ comb_out) {
  using S = HcShape<kN>;
  constexpr bool kNarrow = kN <= kHcNarrowN;
  __shared__ float vals[S::kVals];
  __shared__ float grp[S::kG][S::kJ];
  __shared__ float pre[kN];
  __shared__ float red[4];
  // workgroup 2p: pre and the collapsed stream of position p; 2p + 1: post and comb (the
  // latency-bound Sinkhorn of one wave runs beside the collapse and its norm)
  const int64_t p = blockIdx.x >> 1;
  const bool collapse = (blockIdx.x & 1) == 0;
  const int64_t ND = (int64_t)N * D;
  const int t = threadIdx.x;
  // the row's stream pairs, in flight while the projections are finished (the narrow
  // variant; the wide one loads each stream at the collapse, to keep its registers)
  const uint16_t *srow = streams + p * ND;
  uint32_t sp[kNarrow ? kN : 1][kHcPairs];
  if (kNarrow && collapse) {
#pragma unroll
    for (int n = 0; n < kN; ++n)
#pragma unroll
      for (int i = 0; i < kHcPairs; ++i)
        sp[n][i] = n < N && pair_d(i) < D ? *reinterpret_cast<const uint32_t *>(srow + (int64_t)n * D + pair_d(i))
                                          : 0u;
  }
  // the norm weights too (the row's own streams stand in when there is no norm: same
  // length, never used)
  uint32_t wv[kHcPairs];
  if (collapse) load_pairs(norm_w ? norm_w : srow, D, wv);
  // the chunk partials: thread (g, j) sums value j over chunks g, g + kG, ... in order
  // (their loads in flight together), then value j is the sum of the kG group sums in
  // group order
  {
    const int j = t % S::kJ, g = t / S::kJ;
    float acc = 0.0f;
    if (j < W || j == S::kMaxW) {
      const float *pp = part + p * n_chunks * S::kVals + j;
      for (int c0 = g; c0 < n_chunks; c0 += S::kG * 32) {
        float v[32];
#pragma unroll
        for (int q = 0; q < 32; ++q) v[q] = pp[(int64_t)min(c0 + S::kG * q, n_chunks - 1) * S::kVals];
#pragma unroll
        for (int q = 0; q < 32; ++q)
          if (c0 + S::kG * q < n_chunks) acc += v[q];
      }
    }
    grp[g][j] = acc;
  }
  __syncthreads();
  if (t < W || t == S::kMaxW) {
    float acc = grp[0][t];
#pragma unroll
    for (int g = 1; g < S::kG; ++g) acc += grp[g][t];
    vals[t] = acc;
  }
  __syncthreads();
  if (t < 64 && !kNarrow) {
    // wave 0, the wide variant: lane l holds comb entry (l / 8, l % 8) of an 8 x 8
    // layout (entries outside N x N stay 0): a row is 8 consecutive lanes, a column the
    // lanes 8 apart; sums by lane exchanges at distances 1, 2, 4 (rows) and 8, 16, 32
    // (columns)
    const float rms = 1.0f / sqrtf(vals[S::kMaxW] / (float)ND + eps);
    const int lane = t;
    if (collapse) {
      if (lane < N) {
        const float wp = vals[lane] * rms;
        pre[lane] = 1.0f / (1.0f + expf(-(wp * scale[0] + base[lane]))) + eps;
      }
    } else {
      if (lane < N) {
        const float wq = vals[N + lane] * rms;
        post_out[p * N + lane] = 2.0f * (1.0f / (1.0f + expf(-(wq * scale[1] + base[N + lane]))));
      }
      const int ci = lane >> 3, cj = lane & 7;
      const bool live = ci < N && cj < N;
      auto row_sum = [&](float v) {
        const float s = v + xor_lanes<1>(v);
        const float s2 = s + xor_lanes<2>(s);
        return s2 + xor_lanes<4>(s2);
      };
      auto col_sum = [&](float v) {
        const float s = v + xor_lanes<8>(v);
        const float s2 = s + xor_lanes<16>(s);
        return s2 + xor_lanes<32>(s2);
      };
      const float z = live ? vals[2 * N + ci * N + cj] * rms * scale[2] + base[2 * N + ci * N + cj] : -INFINITY;
      float m = fmaxf(z, xor_lanes<1>(z));
      m = fmaxf(m, xor_lanes<2>(m));
      m = fmaxf(m, xor_lanes<4>(m));
      float c = live ? expf(z - m) : 0.0f;
      const float rs = row_sum(c);
      c = live ? c / rs + eps : 0.0f;
      auto norm = [&](float v, float sum) { return live ? v / (sum + eps) : 0.0f; };
      c = norm(c, col_sum(c));
      for (int it = 0; it < iters - 1; ++it) {
        c = norm(c, row_sum(c));
        c = norm(c, col_sum(c));
      }
      if (live) comb_out[p * N * N + ci * N + cj] = c;
    }
  }
  if (t < 64 && kNarrow) {
    // wave 0: lane l < 16 holds comb entry (l / 4, l % 4) of a 4 x 4 layout (entries
    // outside N x N stay 0), so a row is a quad and a column the lanes j, j + 4, j + 8,
    // j + 12 of the first 16: row sums by quad-permute DPP, column sums by row-rotate DPP,
    // no LDS round trip per reduction
    const float rms = 1.0f / sqrtf(vals[S::kMaxW] / (float)ND + eps);
    const int lane = t;
    if (collapse) {
      if (lane < N) {
        const float wp = vals[lane] * rms;
        pre[lane] = 1.0f / (1.0f + expf(-(wp * scale[0] + base[lane]))) + eps;
      }
    } else {
      if (lane < N) {
        const float wq = vals[N + lane] * rms;
        post_out[p * N + lane] = 2.0f * (1.0f / (1.0f + expf(-(wq * scale[1] + base[N + lane]))));
      }
      const int ci = (lane >> 2) & 3, cj = lane & 3;
      const bool live = lane < 16 && ci < N && cj < N;
      auto dpp = [](float v, auto ctrl) {
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), decltype(ctrl)::value,
                                                                   0xF, 0xF, false));
      };
      using X1 = std::integral_constant<int, 0xB1>;   // lane ^ 1
      using X2 = std::integral_constant<int, 0x4E>;   // lane ^ 2
      using R4 = std::integral_constant<int, 0x124>;  // rotate right by 4 within 16 lanes
      using R8 = std::integral_constant<int, 0x128>;  // rotate right by 8 within 16 lanes
      auto row_sum = [&](float v) {
        const float s = v + dpp(v, X1{});
        return s + dpp(s, X2{});
      };
      auto col_sum = [&](float v) {
        const float s = v + dpp(v, R4{});
        return s + dpp(s, R8{});
      };
      // softmax over the last axis (j), then + eps
      const float z = live ? vals[2 * N + ci * N + cj] * rms * scale[2] + base[2 * N + ci * N + cj] : -INFINITY;
      float m = fmaxf(z, dpp(z, X1{}));
      m = fmaxf(m, dpp(m, X2{}));
      float c = live ? expf(z - m) : 0.0f;
      const float rs = row_sum(c);
      c = live ? c / rs + eps : 0.0f;
      // Sinkhorn: columns, then (iters - 1) x (rows, columns); the entries outside N x N
      // are set to 0 at every step (a padded row or column sums to 0, so at eps = 0 its
      // own division would be 0 / 0; the sums themselves run on every lane for the DPP)
      auto norm = [&](float v, float sum) { return live ? v / (sum + eps) : 0.0f; };
      c = norm(c, col_sum(c));
      for (int it = 0; it < iters - 1; ++it) {
        c = norm(c, row_sum(c));
        c = norm(c, col_sum(c));
      }
      if (live) comb_out[p * N * N + ci * N + cj] = c;
    }
  }
  if (!collapse) return;
  __syncthreads();
  // collapsed = sum_n pre[n] * streams[n], in f16
  float x0[kHcPairs], x1[kHcPairs];
  if constexpr (kNarrow) {
#pragma unroll
    for (int i = 0; i < kHcPairs; ++i) {
      float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
      for (int n = 0; n < kN; ++n)
        if (n < N) {
          a0 = fmaf(pre[n], h2f(sp[n][i] & 0xffff), a0);
          a1 = fmaf(pre[n], h2f(sp[n][i] >> 16), a1);
        }
      x0[i] = (float)to_f16(a0);
      x1[i] = (float)to_f16(a1);
    }
  } else {
    // stream by stream (the same fma chain per element, n ascending)
#pragma unroll
    for (int i = 0; i < kHcPairs; ++i) x0[i] = x1[i] = 0.0f;
    for (int n = 0; n < N; ++n) {
      uint32_t v[kHcPairs];
#pragma unroll
      for (int i = 0; i < kHcPairs; ++i)
        v[i] = *reinterpret_cast<const uint32_t *>(srow + (int64_t)n * D + min(pair_d(i), D - 2));
#pragma unroll
      for (int i = 0; i < kHcPairs; ++i) {
        x0[i] = fmaf(pre[n], h2f(v[i] & 0xffff), x0[i]);
        x1[i] = fmaf(pre[n], h2f(v[i] >> 16), x1[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < kHcPairs; ++i) {
      x0[i] = (float)to_f16(x0[i]);
      x1[i] = (float)to_f16(x1[i]);
    }
  }
  if (!norm_w) {
#pragma unroll
    for (int i = 0; i < kHcPairs; ++i)
      if (pair_d(i) < D)
        *reinterpret_cast<uint32_t *>(out + p * D + pair_d(i)) =
            pack_f16x2(x0[i], x1[i]);
    return;
  }
  rms_pairs(x0, x1, D, norm_eps, wv, out + p * D, red);
}

__global__ __launch_bounds__(256) void k_rms_norm(const uint16_t *__restrict__ xin, int D, const uint16_t *__restrict__ w,
                                                  float eps, uint16_t *__restrict__ y) {
  __shared__ float red[4];
  const int64_t p = blockIdx.x;
  float x0[kHcPairs], x1[kHcPairs];
  uint32_t wv[kHcPairs];
  load_pairs(w, D, wv);
#pragma unroll
  for (int i = 0; i < kHcPairs; ++i) {
    const uint32_t v = pair_d(i) < D ? *reinterpret_cast<const uint32_t *>(xin + p * D + pair_d(i)) : 0u;
    x0[i] = h2f(v & 0xffff);
    x1[i] = h2f(v >> 16);
  }
  rms_pairs(x0, x1, D, eps, wv, y + p * D, red);
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
  uint32_t rv[exl3m::kHcMixMax];
  exl3m::hc_mix_res(res + p * N * D + d, D, N, rv);
  exl3m::hc_mix_pair(post + p * N, comb + p * N * N, rv, D, N, h2f(b & 0xffff), h2f(b >> 16),
                     out + p * N * D + d);
}

}  // namespace

namespace exl3h {

exl3_status check_hc(const exl3_hc_site *hc, int D) {
  if (!hc || !hc->fn || !hc->base || !hc->scale) return fail(EXL3_ERR_INVALID, "null hyper-connection site");
  if (hc->mult < 1 || hc->mult > kHcMaxN)
    return fail(EXL3_ERR_UNSUPPORTED, "hc_mult must be 1..8");
  if (hc->sinkhorn_iters < 1) return fail(EXL3_ERR_INVALID, "hc_sinkhorn_iters must be >= 1");
  if (D <= 0 || D > kHcMaxD || D % 2 || ((int64_t)hc->mult * D) % kHcChunk)
    return fail(EXL3_ERR_UNSUPPORTED, "hidden size must be even, at most 8192, and N*hidden a multiple of 64");
  return EXL3_OK;
}

size_t hc_part_bytes(int N, int D, int64_t P) {
  return align_up((size_t)P * ((size_t)N * D / kHcChunk) * hc_vals(N) * 4, 256);
}

template <int kN>
static void hc_prepare_go(const exl3_hc_site *hc, const uint16_t *streams, int64_t P, int D, int64_t groups,
                          const uint16_t *norm_w, float norm_eps, uint16_t *out, float *post, float *comb,
                          float *part, hipStream_t st) {
  const int N = hc->mult, W = (2 + N) * N, ND = N * D, n_chunks = ND / kHcChunk;
  k_hc_proj<kN><<<dim3((unsigned)n_chunks, (unsigned)groups), 256, 0, st>>>(streams, P, ND, W, hc->fn, part);
  k_hc_finalize<kN><<<(unsigned)(2 * P), 256, 0, st>>>(streams, N, D, W, n_chunks, part, hc->base, hc->scale,
                                                  hc->sinkhorn_iters, hc->eps, norm_w, norm_eps, out, post, comb);
}

exl3_status launch_hc_prepare(const exl3_hc_site *hc, const uint16_t *streams, int64_t P, int D,
                              const uint16_t *norm_w, float norm_eps, uint16_t *out, float *post,
                              float *comb, float *part, hipStream_t st) {
  if (P == 0) return EXL3_OK;
  const bool narrow = hc->mult <= kHcNarrowN;
  const int rows = narrow ? HcShape<kHcNarrowN>::kRows : HcShape<kHcMaxN>::kRows;
  const int64_t groups = (P + rows - 1) / rows;
  if (groups > 65535) return fail(EXL3_ERR_UNSUPPORTED, "too many positions in one call");
  if (narrow)
    hc_prepare_go<kHcNarrowN>(hc, streams, P, D, groups, norm_w, norm_eps, out, post, comb, part, st);
  else
    hc_prepare_go<kHcMaxN>(hc, streams, P, D, groups, norm_w, norm_eps, out, post, comb, part, st);
  EXL3_LAUNCHED("k_hc_proj / k_hc_finalize");
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
  if (reinterpret_cast<uintptr_t>(streams) % 8 || reinterpret_cast<uintptr_t>(hc->fn) % 16 ||
      (reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(norm_w)) % 4)
    return fail(EXL3_ERR_INVALID, "streams must be 8-byte, fn 16-byte, out and norm_w 4-byte aligned");
  return launch_hc_prepare(hc, streams, P, hidden, norm_w, norm_eps, out, post, comb, (float *)workspace,
                           stream_of(stream));
}

exl3_status exl3_rms_norm(const uint16_t *x, int64_t P, int32_t hidden, const uint16_t *w, float eps, uint16_t *y,
                          exl3_stream_t stream) {
  if (P < 0 || P > ((int64_t)1 << 31) || hidden <= 0 || hidden > kHcMaxD || hidden % 2)
    return fail(EXL3_ERR_INVALID, "exl3_rms_norm: bad shape (hidden even, at most 8192)");
  if (P == 0) return EXL3_OK;
  if (!x || !w || !y) return fail(EXL3_ERR_INVALID, "exl3_rms_norm: null argument");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(y)) % 4)
    return fail(EXL3_ERR_INVALID, "exl3_rms_norm: x, w and y must be 4-byte aligned");
  k_rms_norm<<<(unsigned)P, 256, 0, stream_of(stream)>>>(x, hidden, w, eps, y);
  EXL3_LAUNCHED("k_rms_norm");
  return EXL3_OK;
}

exl3_status exl3_hc_mix(const uint16_t *block_out, const float *post, const float *comb, const uint16_t *residual,
                        int64_t P, int32_t mult, int32_t hidden, uint16_t *out, exl3_stream_t stream) {
  if (P < 0 || mult < 1 || mult > kHcMaxN || hidden <= 0 || hidden % 2)
    return fail(EXL3_ERR_INVALID, "exl3_hc_mix: bad shape (hc_mult 1..8, even hidden)");
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
