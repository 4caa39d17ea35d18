// Routed (and trellis shared) expert kernels of the MoE layer, gfx950.
//
// They replace the reference's per-bucket grouped launches (glm5_moe.cpp:329-405:
// hadamard-pre, grouped QMV, mx::sum over splits, hadamard-post, clip/sigmoid/
// multiply, take/concatenate). The device-side run table drives the grid: no host
// round trip, no member cap, and no cross-workgroup synchronisation inside a launch.
//
//  k_moe_gate_up  workgroup = (run, gate|up, 128-column block), 4 waves, the whole k
//                 range: per pass of up to 2 token rows of the run, the input
//                 Hadamard of those rows into LDS, one k chunk per wave at a time, the
//                 chunk partials summed in chunk order -> yhat_gu (f32, per slot).
//                 Extra workgroups compute the f16 shared expert's down partials.
//  k_moe_down     workgroup = (run, 128-column block), 4 waves: prologue = output
//                 Hadamards of gate/up (svh), SwiGLU with the swiglu_limit clamp (f16 op
//                 by op) and the down projection's input Hadamard (suh), for the whole
//                 intermediate of each row; then the QMV over it, the output Hadamard,
//                 and f16(f32(y) * w) per slot (or the shared expert's output).
//
// Per token row and expert the arithmetic is exl3_trellis_linear's (same input
// Hadamard, k chunks and chunk order, output Hadamard), so a run of r rows gives the
// same bytes as r single-row calls, and a layer call the same bytes as its experts
// evaluated one linear at a time.
#include <hip/hip_runtime.h>

#include "exl3_device.hpp"
#include "exl3_internal.hpp"
#include "moe_common.hpp"
#include "moe_dense.hpp"
#include "qmv_core.hpp"

using namespace exl3d;
using exl3m::MoeArgs;

namespace {

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

constexpr int kGuThreads = 256;
constexpr int kDnThreads = 256;
// Token rows per pass of an expert kernel. At decode batch sizes nearly every run has
// one or two rows; a longer run takes more passes over its (L2-resident) tile range.
constexpr int kRowsPerPass = 2;
static_assert(kRowsPerPass <= kMaxRowsPerPass, "row pass");

struct RunInfo {
  int e, off, len;
};

__device__ __forceinline__ bool run_info(const MoeArgs &a, int u, int shared_mode, RunInfo &ri) {
  if (shared_mode) {
    if (u > 0) return false;
    ri.e = a.E;
    ri.off = a.P;
    ri.len = a.N;
    return true;
  }
  if (u >= *a.n_runs) return false;
  ri.e = a.run_expert[u];
  ri.off = a.run_off[u];
  ri.len = a.run_len[u];
  return true;
}

// Waves [0, nwaves) take chunks wave, wave + nwaves, ...; each chunk partial goes to
// part[c][r][col] in LDS.
template <int K, int CB, int MB>
__device__ __forceinline__ void run_chunks(const uint32_t *base, int tiles_n, int cb,
                                           int n_chunks, int ct, int nwaves,
                                           const uint32_t *xs, int xs_stride, float *part) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int c = wave; c < n_chunks; c += nwaves) {
    float acc[MB][2];
    qmv_chunk<K, CB, MB>(base, tiles_n, cb * 8 + (lane >> 3), lane & 7, c * ct, ct, xs,
                         xs_stride, c * ct, acc);
#pragma unroll
    for (int r = 0; r < MB; ++r) {
      part[(c * kRowsPerPass + r) * 128 + lane_col(lane, 0)] = acc[r][0];
      part[(c * kRowsPerPass + r) * 128 + lane_col(lane, 1)] = acc[r][1];
    }
  }
}

template <int K, int CB>
__device__ __forceinline__ void run_chunks_rt(int nr, const uint32_t *base, int tiles_n, int cb,
                                              int n_chunks, int ct, int nwaves,
                                              const uint32_t *xs, int xs_stride, float *part) {
  if (nr == 1)
    run_chunks<K, CB, 1>(base, tiles_n, cb, n_chunks, ct, nwaves, xs, xs_stride, part);
  else
    run_chunks<K, CB, 2>(base, tiles_n, cb, n_chunks, ct, nwaves, xs, xs_stride, part);
}

__device__ __forceinline__ float chunk_sum(const float *part, int n_chunks, int r, int col) {
  float v = part[r * 128 + col];
  for (int c = 1; c < n_chunks; ++c) v += part[(c * kRowsPerPass + r) * 128 + col];
  return v;
}


template <int K, int CB>
__global__ __launch_bounds__(kGuThreads) void k_moe_gate_up(MoeArgs a, int shared_mode,
                                                            int routed_blocks) {
  extern __shared__ uint32_t smem[];
  if (!shared_mode && (int)blockIdx.x >= routed_blocks) {
    // f16 shared expert down partials: H/128 column blocks x 256-row k splits of SI
    static_assert(kGuThreads == 256, "dense_skinny runs on 4 waves");
    const int b = blockIdx.x - routed_blocks;
    const int n_cb = a.H / 128;
    dense_skinny(a.dsh_act, a.N, a.SI, a.H, a.sh_dense[2], a.dsh_dn, b % n_cb, b / n_cb, smem);
    return;
  }
  const int out = shared_mode ? a.SI : a.I;
  const int n_cb = out / 128;
  const int u = blockIdx.x / (2 * n_cb);
  const int proj = (blockIdx.x / n_cb) % 2;
  const int cb = blockIdx.x % n_cb;
  RunInfo ri;
  if (!run_info(a, u, shared_mode, ri)) return;
  const exl3m::ExpertTab &tb = a.tab[ri.e];
  const uint32_t *base = tb.tr[proj];
  const uint16_t *suh = tb.suh[proj];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k_tiles = a.H / 16, ct = chunk_tiles(k_tiles), n_chunks = k_tiles / ct;
  const int xs_stride = a.H / 2;  // words per staged row
  uint32_t *xs = smem;
  float *part = reinterpret_cast<float *>(smem + kRowsPerPass * xs_stride);
  const int nblk = a.H / 128;

  for (int p0 = 0; p0 < ri.len; p0 += kRowsPerPass) {
    const int nr = min(kRowsPerPass, ri.len - p0);
    for (int bi = wave; bi < kRowsPerPass * nblk; bi += kGuThreads / 64) {
      const int r = bi / nblk, blk = bi % nblk;
      uint32_t packed = 0;
      if (r < nr) {
        const int row = a.sorted_row[ri.off + p0 + r];
        const int kc = blk * 128 + 2 * lane;
        const uint32_t hx = *reinterpret_cast<const uint32_t *>(a.h + (int64_t)row * a.H + kc);
        const uint32_t sx = *reinterpret_cast<const uint32_t *>(suh + kc);
        float v0 = lo16(hx), v1 = hi16(hx);
        wave_had_pre(v0, v1, lo16(sx), hi16(sx));
        packed = pack16(v0, v1);
      }
      xs[r * xs_stride + blk * 64 + lane] = packed;
    }
    __syncthreads();
    run_chunks_rt<K, CB>(nr, base, out / 16, cb, n_chunks, ct, kGuThreads / 64, xs, xs_stride, part);
    __syncthreads();
    for (int i = threadIdx.x; i < nr * 128; i += kGuThreads) {
      const int r = i >> 7, col = i & 127;
      a.yhat_gu[((int64_t)(ri.off + p0 + r) * 2 + proj) * a.Imax + cb * 128 + col] =
          chunk_sum(part, n_chunks, r, col);
    }
    __syncthreads();
  }
}

template <int K, int CB>
__global__ __launch_bounds__(kDnThreads) void k_moe_down(MoeArgs a, int shared_mode) {
  extern __shared__ uint32_t smem[];
  const int in = shared_mode ? a.SI : a.I;
  const int n_cb = a.H / 128;
  const int u = blockIdx.x / n_cb, cb = blockIdx.x % n_cb;
  RunInfo ri;
  if (!run_info(a, u, shared_mode, ri)) return;
  const exl3m::ExpertTab &tb = a.tab[ri.e];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k_tiles = in / 16, ct = chunk_tiles(k_tiles), n_chunks = k_tiles / ct;
  const int xs_stride = in / 2;
  uint32_t *xs = smem;
  float *part = reinterpret_cast<float *>(smem + kRowsPerPass * xs_stride);
  const int nblk = in / 128;
  const float L = a.swiglu_limit > 0.0f ? rf16(a.swiglu_limit) : 0.0f;

  for (int p0 = 0; p0 < ri.len; p0 += kRowsPerPass) {
    const int nr = min(kRowsPerPass, ri.len - p0);
    // SwiGLU of the gate/up outputs and the down input Hadamard, per 128-block.
    for (int bi = wave; bi < kRowsPerPass * nblk; bi += kDnThreads / 64) {
      const int r = bi / nblk, blk = bi % nblk;
      uint32_t packed = 0;
      if (r < nr) {
        const int64_t slot = ri.off + p0 + r;
        const int c = blk * 128 + 2 * lane;
        const float *yg = a.yhat_gu + (slot * 2 + 0) * a.Imax + c;
        const float *yu = a.yhat_gu + (slot * 2 + 1) * a.Imax + c;
        float g0 = yg[0], g1 = yg[1], u0 = yu[0], u1 = yu[1];
        const uint32_t svg = *reinterpret_cast<const uint32_t *>(tb.svh[0] + c);
        const uint32_t svu = *reinterpret_cast<const uint32_t *>(tb.svh[1] + c);
        const uint32_t sud = *reinterpret_cast<const uint32_t *>(tb.suh[2] + c);
        wave_had_post(g0, g1, lo16(svg), hi16(svg));
        wave_had_post(u0, u1, lo16(svu), hi16(svu));
        float a0 = swiglu1(rf16(g0), rf16(u0), L);
        float a1 = swiglu1(rf16(g1), rf16(u1), L);
        wave_had_pre(a0, a1, lo16(sud), hi16(sud));
        packed = pack16(a0, a1);
      }
      xs[r * xs_stride + blk * 64 + lane] = packed;
    }
    __syncthreads();
    run_chunks_rt<K, CB>(nr, tb.tr[2], a.H / 16, cb, n_chunks, ct, kDnThreads / 64, xs, xs_stride,
                         part);
    __syncthreads();
    const int c = cb * 128 + 2 * lane;
    const uint32_t svd = *reinterpret_cast<const uint32_t *>(tb.svh[2] + c);
    for (int r = wave; r < nr; r += kDnThreads / 64) {
      float y0 = chunk_sum(part, n_chunks, r, 2 * lane);
      float y1 = chunk_sum(part, n_chunks, r, 2 * lane + 1);
      wave_had_post(y0, y1, lo16(svd), hi16(svd));
      const int64_t slot = ri.off + p0 + r;
      if (shared_mode) {
        *reinterpret_cast<uint32_t *>(a.sh_out + (slot - a.P) * a.H + c) = pack16(y0, y1);
      } else {
        const int row = a.sorted_row[slot], rank = a.sorted_rank[slot];
        const float w = a.weights[(int64_t)row * a.topk + rank];
        *reinterpret_cast<uint32_t *>(a.yw + slot * a.H + c) = pack16(rf16(y0) * w, rf16(y1) * w);
      }
    }
    __syncthreads();
  }
}

}  // namespace

namespace exl3h {

size_t moe_gate_up_lds(int H) {
  const int k_tiles = H / 16;
  return (size_t)kRowsPerPass * (H / 2) * 4 + (size_t)(k_tiles / chunk_tiles(k_tiles)) *
                                                      kRowsPerPass * 128 * 4;
}

size_t moe_down_lds(int in) {
  const int k_tiles = in / 16;
  return (size_t)kRowsPerPass * (in / 2) * 4 + (size_t)(k_tiles / chunk_tiles(k_tiles)) *
                                                       kRowsPerPass * 128 * 4;
}

template <int K, int CB>
static exl3_status moe_go(int which, unsigned blocks, hipStream_t st, const MoeArgs &a,
                          int shared_mode, int routed_blocks) {
  if (which == 0) {
    const size_t lds = std::max(moe_gate_up_lds(a.H), (size_t)4 * kDenseLdsWords);
    static bool attr_set = false;
    if (!attr_set) {
      EXL3_HIP(hipFuncSetAttribute((const void *)k_moe_gate_up<K, CB>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
      attr_set = true;
    }
    k_moe_gate_up<K, CB><<<blocks, kGuThreads, lds, st>>>(a, shared_mode, routed_blocks);
  } else {
    const size_t lds = moe_down_lds(shared_mode ? a.SI : a.I);
    static bool attr_set = false;
    if (!attr_set) {
      EXL3_HIP(hipFuncSetAttribute((const void *)k_moe_down<K, CB>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
      attr_set = true;
    }
    k_moe_down<K, CB><<<blocks, kDnThreads, lds, st>>>(a, shared_mode);
  }
  return EXL3_OK;
}

// which: 0 = gate/up (routed_blocks = workgroups of routed runs; the rest compute the
// f16 shared expert's down partials), 1 = down.
exl3_status launch_moe_expert(int which, int K, int cb, unsigned blocks, const MoeArgs &a,
                              int shared_mode, int routed_blocks, hipStream_t st) {
  if (blocks == 0) return EXL3_OK;
  exl3_status rc = EXL3_OK;
#define EXL3_KC(KK)                                                                          \
  case KK:                                                                                   \
    if (cb == 0) rc = moe_go<KK, 0>(which, blocks, st, a, shared_mode, routed_blocks);       \
    else if (cb == 1) rc = moe_go<KK, 1>(which, blocks, st, a, shared_mode, routed_blocks);  \
    else rc = moe_go<KK, 2>(which, blocks, st, a, shared_mode, routed_blocks);               \
    break;
  switch (K) {
    EXL3_KC(1) EXL3_KC(2) EXL3_KC(3) EXL3_KC(4) EXL3_KC(5) EXL3_KC(6) EXL3_KC(7) EXL3_KC(8)
    default: return fail(EXL3_ERR_INVALID, "K out of range");
  }
#undef EXL3_KC
  if (rc) return rc;
  EXL3_LAUNCHED(which == 0 ? "k_moe_gate_up" : "k_moe_down");
  return EXL3_OK;
}

}  // namespace exl3h
