// Routed (and trellis shared) expert kernels of the MoE layer, gfx950.
//
// One launch per projection class replaces the reference's per-bucket grouped
// launches (glm5_moe.cpp:329-405: hadamard-pre, grouped QMV, mx::sum over splits,
// hadamard-post, clip/sigmoid/multiply, take/concatenate). The run table built on the
// device by the router kernel drives the grid, so there is no host round trip and no
// member cap.
//
//  k_moe_gate_up  workgroup = (run, gate|up, 128-column block, k-split). Each pass of
//                 up to 4 rows of the run: input Hadamard of the token rows into LDS,
//                 the QMV wave loop, the wave sum into a split partial. The last of the
//                 2*S workgroups of a (run, block) to finish (completion counter) sums
//                 the splits in order, applies the output Hadamards with svh, SwiGLU
//                 with the swiglu_limit clamp (f16 op by op), and the down projection's
//                 input Hadamard for that 128-block, writing act_hat.
//  k_moe_down     workgroup = (run, 128-column block, k-split) over act_hat. The last
//                 workgroup of a (run, block) applies the output Hadamard, scales by the
//                 routing weight (f16(f32(y) * w)); the last contribution to a
//                 (token row, block) sums the top_k terms in rank order, adds the shared
//                 expert and writes the layer output.
//
// Per token row and expert the arithmetic is exactly exl3_trellis_linear's (same
// input Hadamard, k partition, wave and split order, output Hadamard), so a run of r
// rows gives the same bytes as r single-row calls.
#include <hip/hip_runtime.h>

#include "exl3_device.hpp"
#include "exl3_internal.hpp"
#include "moe_common.hpp"
#include "qmv_core.hpp"

using namespace exl3d;
using exl3m::MoeArgs;

namespace {

constexpr int kXsRow = kQmvMaxKtPerWg * 8;  // LDS words per staged row

__device__ __forceinline__ float lo16(uint32_t v) { return (float)bitcast<f16>((uint16_t)(v & 0xffffu)); }
__device__ __forceinline__ float hi16(uint32_t v) { return (float)bitcast<f16>((uint16_t)(v >> 16)); }
__device__ __forceinline__ uint32_t pack16(float a, float b) {
  return (uint32_t)bitcast<uint16_t>(to_f16(a)) | ((uint32_t)bitcast<uint16_t>(to_f16(b)) << 16);
}
__device__ __forceinline__ float rf16(float v) { return (float)to_f16(v); }

// silu(min(g, L)) * clamp(u, -L, L), every MLX f16 op rounded (glm5_moe.cpp:369-371).
__device__ __forceinline__ float swiglu1(float g, float u, float L) {
  if (L > 0.0f) {
    g = fminf(g, L);
    u = fminf(fmaxf(u, -L), L);
  }
  const float sg = rf16(1.0f / (1.0f + expf(-g)));
  const float act = rf16(g * sg);
  return rf16(act * u);
}

struct RunInfo {
  int e, off, len, cidx;
};

__device__ __forceinline__ bool run_info(const MoeArgs &a, int u, int shared_mode, RunInfo &ri) {
  if (shared_mode) {
    if (u > 0) return false;
    ri.e = a.E;
    ri.off = a.P;
    ri.len = a.N;
    ri.cidx = a.R;
    return true;
  }
  if (u >= *a.n_runs) return false;
  ri.e = a.run_expert[u];
  ri.off = a.run_off[u];
  ri.len = a.run_len[u];
  ri.cidx = u;
  return true;
}

// One pass of nr <= MB rows: wave loop on the staged xs, wave sum, partial write.
template <int K, int CB, int MB>
__device__ __forceinline__ void expert_pass(const uint32_t *base, int tiles_n, int cb, int k0,
                                            int T, const uint32_t *xs, float *red, int nr,
                                            float *dst, int64_t dst_row_stride) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float acc[MB][2];
  qmv_wave_loop<K, CB, MB>(base, tiles_n, cb * 8 + (lane >> 3), lane & 7, k0 + wave * T, T, wave,
                           xs, acc);
  qmv_stash<MB>(red, wave, lane, acc);
  __syncthreads();
  for (int i = threadIdx.x; i < nr * 128; i += 256) {
    const int r = i >> 7, c = i & 127;
    dst[r * dst_row_stride + cb * 128 + c] = qmv_wave_sum<MB>(red, r, c);
  }
}

template <int K, int CB>
__device__ __forceinline__ void expert_pass_rt(const uint32_t *base, int tiles_n, int cb, int k0,
                                               int T, const uint32_t *xs, float *red, int nr,
                                               float *dst, int64_t dst_row_stride) {
  if (nr == 1)
    expert_pass<K, CB, 1>(base, tiles_n, cb, k0, T, xs, red, nr, dst, dst_row_stride);
  else if (nr == 2)
    expert_pass<K, CB, 2>(base, tiles_n, cb, k0, T, xs, red, nr, dst, dst_row_stride);
  else
    expert_pass<K, CB, 4>(base, tiles_n, cb, k0, T, xs, red, nr, dst, dst_row_stride);
}

template <int K, int CB>
__global__ __launch_bounds__(256) void k_moe_gate_up(MoeArgs a, int shared_mode) {
  __shared__ uint32_t xs[4 * kXsRow];
  __shared__ float red[kQmvWaves * 4 * 128];
  __shared__ int s_last;
  const int out = shared_mode ? a.SI : a.I;
  const int n_cb = out / 128;
  const int k_tiles = a.H / 16;
  const int T = qmv_T(k_tiles), S = k_tiles / (kQmvWaves * T), kt_wg = kQmvWaves * T;
  const int per_run = 2 * n_cb * S;
  const int u = blockIdx.x / per_run;
  int rem = blockIdx.x % per_run;
  const int proj = rem / (n_cb * S);
  rem %= n_cb * S;
  const int cb = rem % n_cb, s = rem / n_cb;
  RunInfo ri;
  if (!run_info(a, u, shared_mode, ri)) return;
  const exl3m::ExpertTab &tb = a.tab[ri.e];
  const uint32_t *base = tb.tr[proj];
  const uint16_t *suh = tb.suh[proj];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k0 = s * kt_wg;
  const int nblk = kt_wg / 8;  // Hadamard blocks in this workgroup's k range
  const int64_t slot_stride = (int64_t)2 * a.Sgu * a.Imax;

  for (int p0 = 0; p0 < ri.len; p0 += 4) {
    const int nr = min(4, ri.len - p0);
    for (int bi = wave; bi < 4 * nblk; bi += kQmvWaves) {
      const int r = bi / nblk, blk = bi % nblk;
      uint32_t packed = 0;
      if (r < nr) {
        const int row = a.sorted_row[ri.off + p0 + r];
        const int kc = k0 * 16 + blk * 128 + 2 * lane;
        const uint32_t hx = *reinterpret_cast<const uint32_t *>(a.h + (int64_t)row * a.H + kc);
        const uint32_t sx = *reinterpret_cast<const uint32_t *>(suh + kc);
        float v0 = lo16(hx), v1 = hi16(hx);
        wave_had_pre(v0, v1, lo16(sx), hi16(sx));
        packed = pack16(v0, v1);
      }
      xs[r * kXsRow + blk * 64 + lane] = packed;
    }
    __syncthreads();
    float *dst = a.gu_part + (int64_t)(ri.off + p0) * slot_stride + (int64_t)(proj * a.Sgu + s) * a.Imax;
    expert_pass_rt<K, CB>(base, out / 16, cb, k0, T, xs, red, nr, dst, slot_stride);
    __syncthreads();
  }

  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = atomicAdd(&a.gu_cnt[ri.cidx * a.cnt_stride + cb], 1u) == (unsigned)(2 * S - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  const int c = cb * 128 + 2 * lane;
  const uint32_t svg = *reinterpret_cast<const uint32_t *>(tb.svh[0] + c);
  const uint32_t svu = *reinterpret_cast<const uint32_t *>(tb.svh[1] + c);
  const uint32_t sud = *reinterpret_cast<const uint32_t *>(tb.suh[2] + c);
  const float L = a.swiglu_limit > 0.0f ? rf16(a.swiglu_limit) : 0.0f;
  for (int i = wave; i < ri.len; i += kQmvWaves) {
    const int64_t slot = ri.off + i;
    const float *pg = a.gu_part + slot * slot_stride + c;
    const float *pu = pg + (int64_t)a.Sgu * a.Imax;
    float g0 = pg[0], g1 = pg[1], u0 = pu[0], u1 = pu[1];
    for (int k = 1; k < S; ++k) {
      g0 += pg[(int64_t)k * a.Imax];
      g1 += pg[(int64_t)k * a.Imax + 1];
      u0 += pu[(int64_t)k * a.Imax];
      u1 += pu[(int64_t)k * a.Imax + 1];
    }
    wave_had_post(g0, g1, lo16(svg), hi16(svg));
    wave_had_post(u0, u1, lo16(svu), hi16(svu));
    float a0 = swiglu1(rf16(g0), rf16(u0), L);
    float a1 = swiglu1(rf16(g1), rf16(u1), L);
    wave_had_pre(a0, a1, lo16(sud), hi16(sud));
    *reinterpret_cast<uint32_t *>(a.act_hat + slot * a.Imax + c) = pack16(a0, a1);
  }
  if (threadIdx.x == 0) a.gu_cnt[ri.cidx * a.cnt_stride + cb] = 0;
}

template <int K, int CB>
__global__ __launch_bounds__(256) void k_moe_down(MoeArgs a, int shared_mode) {
  __shared__ uint32_t xs[4 * kXsRow];
  __shared__ float red[kQmvWaves * 4 * 128];
  __shared__ int s_last;
  __shared__ int s_rows[256];
  const int in = shared_mode ? a.SI : a.I;
  const int n_cb = a.H / 128;
  const int k_tiles = in / 16;
  const int T = qmv_T(k_tiles), S = k_tiles / (kQmvWaves * T), kt_wg = kQmvWaves * T;
  const int per_run = n_cb * S;
  const int u = blockIdx.x / per_run;
  const int rem = blockIdx.x % per_run;
  const int cb = rem % n_cb, s = rem / n_cb;
  RunInfo ri;
  if (!run_info(a, u, shared_mode, ri)) return;
  const exl3m::ExpertTab &tb = a.tab[ri.e];
  const uint32_t *base = tb.tr[2];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k0 = s * kt_wg;
  const int64_t slot_stride = (int64_t)a.Sdn * a.H;

  for (int p0 = 0; p0 < ri.len; p0 += 4) {
    const int nr = min(4, ri.len - p0);
    for (int i = threadIdx.x; i < 4 * kt_wg * 8; i += 256) {
      const int r = i / (kt_wg * 8), wd = i % (kt_wg * 8);
      uint32_t v = 0;
      if (r < nr)
        v = reinterpret_cast<const uint32_t *>(a.act_hat + (int64_t)(ri.off + p0 + r) * a.Imax +
                                               k0 * 16)[wd];
      xs[r * kXsRow + wd] = v;
    }
    __syncthreads();
    float *dst = a.dn_part + (int64_t)(ri.off + p0) * slot_stride + (int64_t)s * a.H;
    expert_pass_rt<K, CB>(base, a.H / 16, cb, k0, T, xs, red, nr, dst, slot_stride);
    __syncthreads();
  }

  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = atomicAdd(&a.dn_cnt[ri.cidx * a.cnt_stride + cb], 1u) == (unsigned)(S - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  const int c = cb * 128 + 2 * lane;
  const uint32_t svd = *reinterpret_cast<const uint32_t *>(tb.svh[2] + c);
  for (int i = wave; i < ri.len; i += kQmvWaves) {
    const int64_t slot = ri.off + i;
    const float *pd = a.dn_part + slot * slot_stride + c;
    float y0 = pd[0], y1 = pd[1];
    for (int k = 1; k < S; ++k) {
      y0 += pd[(int64_t)k * a.H];
      y1 += pd[(int64_t)k * a.H + 1];
    }
    wave_had_post(y0, y1, lo16(svd), hi16(svd));
    if (shared_mode) {
      *reinterpret_cast<uint32_t *>(a.sh_out + (int64_t)i * a.H + c) = pack16(y0, y1);
    } else {
      const int row = a.sorted_row[slot], rank = a.sorted_rank[slot];
      const float w = a.weights[(int64_t)row * a.topk + rank];
      *reinterpret_cast<uint32_t *>(a.yw + slot * a.H + c) = pack16(rf16(y0) * w, rf16(y1) * w);
    }
  }
  if (threadIdx.x == 0) a.dn_cnt[ri.cidx * a.cnt_stride + cb] = 0;
  if (shared_mode) return;

  // Combine: the last of a token row's top_k contributions to this block writes it.
  __threadfence();
  __syncthreads();
  for (int c0 = 0; c0 < ri.len; c0 += 256) {
    const int nloc = min(256, ri.len - c0);
    if ((int)threadIdx.x < nloc) {
      const int row = a.sorted_row[ri.off + c0 + threadIdx.x];
      const unsigned old = atomicAdd(&a.comb_cnt[(int64_t)row * n_cb + cb], 1u);
      s_rows[threadIdx.x] = old == (unsigned)(a.topk - 1) ? row : -1;
    }
    __syncthreads();
    for (int i = wave; i < nloc; i += kQmvWaves) {
      const int row = s_rows[i];
      if (row < 0) continue;
      __threadfence();
      float r0 = 0.0f, r1 = 0.0f;
      for (int k = 0; k < a.topk; ++k) {
        const int sl = a.slot[(int64_t)row * a.topk + k];
        const uint32_t v = __builtin_nontemporal_load(
            reinterpret_cast<const uint32_t *>(a.yw + (int64_t)sl * a.H + c));
        r0 += lo16(v);
        r1 += hi16(v);
      }
      r0 = rf16(r0);
      r1 = rf16(r1);
      if (a.has_shared) {
        const uint32_t sv = *reinterpret_cast<const uint32_t *>(a.sh_out + (int64_t)row * a.H + c);
        r0 += lo16(sv);
        r1 += hi16(sv);
      }
      *reinterpret_cast<uint32_t *>(a.out + (int64_t)row * a.H + c) = pack16(r0, r1);
      if (lane == 0) a.comb_cnt[(int64_t)row * n_cb + cb] = 0;
    }
    __syncthreads();
  }
}

}  // namespace

namespace exl3h {

template <int K, int CB>
static void moe_go(int which, dim3 grid, hipStream_t st, const MoeArgs &a, int shared_mode) {
  if (which == 0)
    k_moe_gate_up<K, CB><<<grid, 256, 0, st>>>(a, shared_mode);
  else
    k_moe_down<K, CB><<<grid, 256, 0, st>>>(a, shared_mode);
}

// which: 0 = gate/up, 1 = down.
exl3_status launch_moe_expert(int which, int K, int cb, unsigned blocks, const MoeArgs &a,
                              int shared_mode, hipStream_t st) {
  if (blocks == 0) return EXL3_OK;
  dim3 grid(blocks);
#define EXL3_KC(KK)                                                      \
  case KK:                                                               \
    if (cb == 0) moe_go<KK, 0>(which, grid, st, a, shared_mode);         \
    else if (cb == 1) moe_go<KK, 1>(which, grid, st, a, shared_mode);    \
    else moe_go<KK, 2>(which, grid, st, a, shared_mode);                 \
    break;
  switch (K) {
    EXL3_KC(1) EXL3_KC(2) EXL3_KC(3) EXL3_KC(4) EXL3_KC(5) EXL3_KC(6) EXL3_KC(7) EXL3_KC(8)
    default: return fail(EXL3_ERR_INVALID, "K out of range");
  }
#undef EXL3_KC
  EXL3_LAUNCHED(which == 0 ? "k_moe_gate_up" : "k_moe_down");
  return EXL3_OK;
}

}  // namespace exl3h
