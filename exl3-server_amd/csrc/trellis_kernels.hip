// Trellis tensor kernels for gfx950: decode (W_hat), reconstruct (W), the Hadamard
// steps, and the dequant-GEMV (QMV) with its split-sum / output-Hadamard epilogue.
//
// Reference counterparts (muyouming/exl3-server):
//   decode       exl3.cpp:101-125      (bit-exact)
//   reconstruct  exl3.cpp:152-209      (bit-exact: same f32 butterfly order, one RNE)
//   hadamard     trellis_gemm.cpp:367-400, 582-603 (same rounding points)
//   qmv          trellis_gemm.cpp:30-141 (Metal scalar QMV) + mx::sum over splits
//                (:980, :1185) + the output Hadamard (:1186)
#include <hip/hip_runtime.h>

#include <algorithm>

#include "exl3_device.hpp"
#include "exl3_internal.hpp"
#include "qmv_core.hpp"

using namespace exl3d;

namespace {

// ---------------------------------------------------------------------------------
// decode: one workgroup per tile, one thread per stream position.
// ---------------------------------------------------------------------------------
__device__ __forceinline__ int tile_element(int p) {
  const int L = p >> 3, i = p & 7, q = i & 3;
  const int row = 2 * (L & 3) + (q < 2 ? q : q + 6);
  const int col = (L >> 2) + 8 * (i >> 2);
  return row * 16 + col;
}

__device__ __forceinline__ uint32_t tile_state_rt(const uint32_t *__restrict__ tile, int K, int p) {
  const int nw = 8 * K;
  const int lb = (p + 1) * K - 1;  // ring bit of the state's LSB
  const int last = lb >> 5;
  const uint32_t lo = tile[last % nw];
  const uint32_t hi = tile[(last - 1 + nw) % nw];
  const uint64_t pair = ((uint64_t)hi << 32) | lo;
  return (uint32_t)(pair >> (31 - (lb & 31))) & 0xffffu;
}

template <int CB>
__global__ __launch_bounds__(256) void k_decode(const uint32_t *__restrict__ trellis, int K,
                                                int tiles_n, int out, uint16_t *__restrict__ w_hat) {
  const int tn = blockIdx.x, tk = blockIdx.y, p = threadIdx.x;
  const uint32_t *tile = trellis + ((int64_t)tk * tiles_n + tn) * 8 * K;
  const f16 v = decode_one<CB>(tile_state_rt(tile, K, p));
  const int e = tile_element(p);
  w_hat[(int64_t)(tk * 16 + (e >> 4)) * out + tn * 16 + (e & 15)] = bitcast<uint16_t>(v);
}

// ---------------------------------------------------------------------------------
// reconstruct: one workgroup per 128x128 block. The block is decoded into LDS as f32,
// then the left butterflies (across rows), the row scale, the right butterflies
// (across columns), the column scale and one RNE -- the operation order of
// exl3.cpp:156-197, element for element.
// ---------------------------------------------------------------------------------
template <int CB>
__global__ __launch_bounds__(256) void k_reconstruct(const uint32_t *__restrict__ trellis, int K,
                                                     int tiles_n, int out,
                                                     const uint16_t *__restrict__ suh,
                                                     const uint16_t *__restrict__ svh,
                                                     uint16_t *__restrict__ w) {
  __shared__ float buf[128][129];
  const int cbk = blockIdx.x, rbk = blockIdx.y, tid = threadIdx.x;
  for (int idx = tid; idx < 64 * 256; idx += 256) {
    const int t = idx >> 8, p = idx & 255;
    const int tr = t >> 3, tc = t & 7;
    const uint32_t *tile =
        trellis + ((int64_t)(rbk * 8 + tr) * tiles_n + (cbk * 8 + tc)) * 8 * K;
    const int e = tile_element(p);
    buf[tr * 16 + (e >> 4)][tc * 16 + (e & 15)] = (float)decode_one<CB>(tile_state_rt(tile, K, p));
  }
  __syncthreads();
  for (int len = 1; len < 128; len <<= 1) {
    for (int idx = tid; idx < 64 * 128; idx += 256) {
      const int q = idx >> 7, c = idx & 127;
      const int j = (q / len) * 2 * len + (q % len);
      const float a = buf[j][c], b = buf[j + len][c];
      buf[j][c] = a + b;
      buf[j + len][c] = a - b;
    }
    __syncthreads();
  }
  for (int idx = tid; idx < 128 * 128; idx += 256) {
    const int i = idx >> 7, c = idx & 127;
    const float s = f16_to_f32(suh[rbk * 128 + i]) * kHadScale;
    buf[i][c] = buf[i][c] * s;
  }
  __syncthreads();
  for (int len = 1; len < 128; len <<= 1) {
    for (int idx = tid; idx < 128 * 64; idx += 256) {
      const int i = idx >> 6, q = idx & 63;
      const int j = (q / len) * 2 * len + (q % len);
      const float a = buf[i][j], b = buf[i][j + len];
      buf[i][j] = a + b;
      buf[i][j + len] = a - b;
    }
    __syncthreads();
  }
  for (int idx = tid; idx < 128 * 128; idx += 256) {
    const int i = idx >> 7, c = idx & 127;
    const float s = f16_to_f32(svh[cbk * 128 + c]) * kHadScale;
    w[(int64_t)(rbk * 128 + i) * out + cbk * 128 + c] = f32_to_f16(buf[i][c] * s);
  }
}

// ---------------------------------------------------------------------------------
// Hadamard pre/post: one wave per (row, 128-block).
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_hadamard(const uint16_t *__restrict__ x16,
                                                  const float *__restrict__ x32, int64_t rows,
                                                  int n, exl3h::PtrTable s,
                                                  int64_t rows_per_member,
                                                  uint16_t *__restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nb = n / 128;
  if (gw >= rows * nb) return;
  const int blk = (int)(gw % nb);
  const int64_t row = gw / nb;
  const uint16_t *sv = (const uint16_t *)s.p[row / rows_per_member] + blk * 128 + 2 * lane;
  const int64_t o = row * n + blk * 128 + 2 * lane;
  float v0, v1;
  if (x16) {
    v0 = f16_to_f32(x16[o]);
    v1 = f16_to_f32(x16[o + 1]);
    wave_had_pre(v0, v1, f16_to_f32(sv[0]), f16_to_f32(sv[1]));
  } else {
    v0 = x32[o];
    v1 = x32[o + 1];
    wave_had_post(v0, v1, f16_to_f32(sv[0]), f16_to_f32(sv[1]));
  }
  y[o] = f32_to_f16(v0);
  y[o + 1] = f32_to_f16(v1);
}

// ---------------------------------------------------------------------------------
// QMV: grid (out/128 column blocks x k-slices, row passes, members); 4 waves per
// workgroup, wave w owns n-pair 4*cb + w of one k-slice. The workgroup stages its
// slice of up to 16 xhat rows into LDS in the MFMA k order and writes the slice
// partials part[member][slice][row][col].
// ---------------------------------------------------------------------------------
template <int K, int CB, int PD>
__global__ __launch_bounds__(256) void k_qmv(exl3h::PtrTable trellis, int tiles_n, int in,
                                             int out, const uint16_t *__restrict__ xhat,
                                             int64_t x_member_stride, int64_t rows,
                                             int pass_rows, float *__restrict__ part,
                                             exl3h::PtrTable suh, int rotate) {
  constexpr bool kDup = dup_cb(CB);
  // one ring-word slot per wave, then the slice's staged rows (pass_rows of them: the
  // launch sizes the LDS to the pass, so a one-row call is not held to the occupancy of
  // a 16-row one)
  extern __shared__ u32x4 qmv_smem[];
  u32x4 *slots = qmv_smem;
  uint32_t *xs = reinterpret_cast<uint32_t *>(qmv_smem + 4 * slot_chunks(K));
  const int k_tiles = in / 16, ss = slice_steps(k_tiles), n_sl = n_slices(k_tiles);
  const int slice_k = kStepTiles * ss * 16, xs_stride = staged_row_words(k_tiles, kDup);
  // grid: x = 128-column block, y = row block * n_sl + k-slice, z = member (one row
  // block, the decode case, needs no division)
  const int cb = blockIdx.x;
  const int sl = (int)gridDim.y == n_sl ? (int)blockIdx.y : (int)blockIdx.y % n_sl;
  const int64_t r0 = (int64_t)((int)gridDim.y == n_sl ? 0 : (int)blockIdx.y / n_sl) * pass_rows;
  const int nr = (int)min<int64_t>(pass_rows, rows - r0);
  const int member = blockIdx.z;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;

  if (rotate) {
    // x, not xhat: the input Hadamard of the slice's 128-blocks (member's suh), in the
    // workgroup, kBatch blocks per wave at a time with every load issued first
    constexpr int kBatch = 4;
    const uint16_t *xr = xhat + member * x_member_stride + r0 * in + sl * slice_k + 2 * lane;
    const uint16_t *su = (const uint16_t *)suh.p[member] + sl * slice_k + 2 * lane;
    // blocks per row: slice_k / 128 = ss / 2, a power of two
    const int nblk = slice_k / 128, nblk_lg = __builtin_ctz(nblk), items = nr * nblk;
    for (int b0 = wave; b0 < items; b0 += 4 * kBatch) {
      uint32_t hx[kBatch], sx[kBatch];
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        const int bi = min(b0 + 4 * q, items - 1);
        hx[q] = *reinterpret_cast<const uint32_t *>(xr + (int64_t)(bi >> nblk_lg) * in +
                                                    (bi & (nblk - 1)) * 128);
        sx[q] = *reinterpret_cast<const uint32_t *>(su + (bi & (nblk - 1)) * 128);
      }
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        const int bi = b0 + 4 * q;
        if (bi < items) {
          float v0 = f16_to_f32((uint16_t)(hx[q] & 0xffffu)), v1 = f16_to_f32((uint16_t)(hx[q] >> 16));
          wave_had_pre(v0, v1, f16_to_f32((uint16_t)(sx[q] & 0xffffu)), f16_to_f32((uint16_t)(sx[q] >> 16)));
          stage_pair<kDup>(xs + (bi >> nblk_lg) * xs_stride, bi & (nblk - 1), lane,
                           pack_f16x2(v0, v1));
        }
      }
    }
  } else {
    // xhat rows: pair w of a k-tile (k-rows 2w, 2w + 1) to its staged position
    const uint16_t *xm = xhat + member * x_member_stride + r0 * in + sl * slice_k;
    const int pr_row = slice_k / 2, pr_lg = __builtin_ctz(pr_row);  // pairs per row
    for (int i = threadIdx.x; i < nr * pr_row; i += 256) {
      const int r = i >> pr_lg, w = i & (pr_row - 1);
      const uint32_t v = reinterpret_cast<const uint32_t *>(xm + (int64_t)r * in)[w];
      const int pw = (w & ~7) + xpos(w & 7);  // plain staged word
      if constexpr (kDup) {
        *reinterpret_cast<u32x2 *>(xs + r * xs_stride + 2 * pw) = u32x2{dup_lo(v), dup_hi(v)};
      } else {
        xs[r * xs_stride + pw] = v;
      }
    }
  }
  __syncthreads();
  f32x4 D0, D1;
  qmv_slice<K, CB, PD>((const uint32_t *)trellis.p[member], k_tiles, tiles_n, sl * kStepTiles * ss,
                       cb * 4 + wave, ss, xs + min(lane & 15, nr - 1) * xs_stride,
                       slots + wave * slot_chunks(K), D0, D1);
  float *p = part + (((int64_t)member * n_sl + sl) * rows + r0) * out + cb * 128 + wave * 32;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = d_row(i);
    if (r < nr) {
      p[(int64_t)r * out + d_col(0)] = D0[i];
      p[(int64_t)r * out + d_col(1)] = D1[i];
    }
  }
}

// One wave per (member, row, 128-column block): slice partials summed in slice order,
// then the raw f32 result or the output Hadamard.
__global__ __launch_bounds__(256) void k_qmv_finalize(int n, int n_sl, int64_t rows, int out,
                                                      const float *__restrict__ part,
                                                      float *__restrict__ y32,
                                                      uint16_t *__restrict__ y16,
                                                      exl3h::PtrTable svh) {
  const int lane = threadIdx.x & 63;
  const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int n_cb = out / 128;
  if (gw >= (int64_t)n * rows * n_cb) return;
  const int cb = (int)(gw % n_cb);
  const int64_t rest = gw / n_cb;
  const int64_t row = rest % rows;
  const int member = (int)(rest / rows);
  const int c = cb * 128 + 2 * lane;
  const float *p = part + ((int64_t)member * n_sl * rows + row) * out + c;
  // slice partials summed in slice order; the loads of 8 slices are issued together
  float v0 = 0.0f, v1 = 0.0f;
  for (int s0 = 0; s0 < n_sl; s0 += 8) {
    float2 v[8];
#pragma unroll
    for (int s = 0; s < 8; ++s)
      v[s] = *reinterpret_cast<const float2 *>(p + (int64_t)min(s0 + s, n_sl - 1) * rows * out);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (s0 + s == 0) {
        v0 = v[0].x;
        v1 = v[0].y;
      } else if (s0 + s < n_sl) {
        v0 += v[s].x;
        v1 += v[s].y;
      }
    }
  }
  const int64_t o = ((int64_t)member * rows + row) * out + c;
  if (y32) {
    y32[o] = v0;
    y32[o + 1] = v1;
    return;
  }
  const uint16_t *sv = (const uint16_t *)svh.p[member] + c;
  wave_had_post(v0, v1, f16_to_f32(sv[0]), f16_to_f32(sv[1]));
  y16[o] = f32_to_f16(v0);
  y16[o + 1] = f32_to_f16(v1);
}

}  // namespace

namespace exl3h {

exl3_status launch_decode(const exl3_trellis_desc &w, uint16_t *w_hat, hipStream_t st) {
  const int tiles_n = w.out_features / 16, tiles_k = w.in_features / 16;
  dim3 grid(tiles_n, tiles_k);
  const uint32_t *t = (const uint32_t *)w.trellis;
  switch (w.codebook) {
    case 0: k_decode<0><<<grid, 256, 0, st>>>(t, w.K, tiles_n, w.out_features, w_hat); break;
    case 1: k_decode<1><<<grid, 256, 0, st>>>(t, w.K, tiles_n, w.out_features, w_hat); break;
    default: k_decode<2><<<grid, 256, 0, st>>>(t, w.K, tiles_n, w.out_features, w_hat); break;
  }
  EXL3_LAUNCHED("k_decode");
  return EXL3_OK;
}

exl3_status launch_reconstruct(const exl3_trellis_desc &w, uint16_t *w_out, hipStream_t st) {
  const int tiles_n = w.out_features / 16;
  dim3 grid(w.out_features / 128, w.in_features / 128);
  const uint32_t *t = (const uint32_t *)w.trellis;
  switch (w.codebook) {
    case 0:
      k_reconstruct<0><<<grid, 256, 0, st>>>(t, w.K, tiles_n, w.out_features, w.suh, w.svh, w_out);
      break;
    case 1:
      k_reconstruct<1><<<grid, 256, 0, st>>>(t, w.K, tiles_n, w.out_features, w.suh, w.svh, w_out);
      break;
    default:
      k_reconstruct<2><<<grid, 256, 0, st>>>(t, w.K, tiles_n, w.out_features, w.suh, w.svh, w_out);
      break;
  }
  EXL3_LAUNCHED("k_reconstruct");
  return EXL3_OK;
}

exl3_status launch_hadamard(const uint16_t *x16, const float *x32, int64_t rows, int n,
                            const PtrTable &s, int64_t rows_per_member, uint16_t *y,
                            hipStream_t st) {
  const int64_t waves = rows * (n / 128);
  if (waves == 0) return EXL3_OK;
  k_hadamard<<<(unsigned)((waves + 3) / 4), 256, 0, st>>>(x16, x32, rows, n, s, rows_per_member, y);
  EXL3_LAUNCHED("k_hadamard");
  return EXL3_OK;
}

template <int K, int CB, int PD>
static void qmv_go(dim3 grid, hipStream_t st, const PtrTable &tr, int tiles_n, int in, int out,
                   const uint16_t *xhat, int64_t xs, int64_t rows, int pass_rows, float *part,
                   const PtrTable *suh) {
  // the wave slots and pass_rows staged rows (at most 16 x 2 KB + 8 KB: under the 64 KB
  // that a launch gets without an attribute)
  static_assert((size_t)4 * slot_chunks(8) * 16 +
                    (size_t)kPassRows * (kMaxSliceSteps * kStepTiles * tile_words(true) + 4) * 4 <=
                64 * 1024,
                "k_qmv LDS");
  const size_t lds = (size_t)4 * slot_chunks(K) * 16 +
                     (size_t)pass_rows * staged_row_words(in / 16, dup_cb(CB)) * 4;
  k_qmv<K, CB, PD><<<grid, 256, lds, st>>>(tr, tiles_n, in, out, xhat, xs, rows, pass_rows, part,
                                           suh ? *suh : PtrTable{}, suh ? 1 : 0);
}

template <int K, int CB>
static void qmv_pd(int pd, dim3 grid, hipStream_t st, const PtrTable &tr, int tiles_n, int in,
                   int out, const uint16_t *xhat, int64_t xs, int64_t rows, int pass_rows,
                   float *part, const PtrTable *suh) {
  if (pd == 1)
    return qmv_go<K, CB, 1>(grid, st, tr, tiles_n, in, out, xhat, xs, rows, pass_rows, part, suh);
  if constexpr (K <= 4) {
    if (pd >= 4)
      return qmv_go<K, CB, 4>(grid, st, tr, tiles_n, in, out, xhat, xs, rows, pass_rows, part, suh);
  }
  qmv_go<K, CB, 2>(grid, st, tr, tiles_n, in, out, xhat, xs, rows, pass_rows, part, suh);
}

template <int K>
static void qmv_cb(int cb, int pd, dim3 grid, hipStream_t st, const PtrTable &tr, int tiles_n,
                   int in, int out, const uint16_t *xhat, int64_t xs, int64_t rows, int pass_rows,
                   float *part, const PtrTable *suh) {
  switch (cb) {
    case 0: qmv_pd<K, 0>(pd, grid, st, tr, tiles_n, in, out, xhat, xs, rows, pass_rows, part, suh); break;
    case 1: qmv_pd<K, 1>(pd, grid, st, tr, tiles_n, in, out, xhat, xs, rows, pass_rows, part, suh); break;
    case 2: qmv_pd<K, 2>(pd, grid, st, tr, tiles_n, in, out, xhat, xs, rows, pass_rows, part, suh); break;
    case 3: qmv_pd<K, 3>(pd, grid, st, tr, tiles_n, in, out, xhat, xs, rows, pass_rows, part, suh); break;
    default: qmv_pd<K, 4>(pd, grid, st, tr, tiles_n, in, out, xhat, xs, rows, pass_rows, part, suh); break;
  }
}

int qmv_pass_rows(int64_t rows) {
  const exl3_tuning tn = tuning();
  int pr = tn.rows_per_pass > 0 ? tn.rows_per_pass : kPassRows;
  if (pr > kPassRows) pr = kPassRows;
  return (int)std::min<int64_t>(pr, std::max<int64_t>(rows, 1));
}

int qmv_slices(int in) { return n_slices(in / 16); }

exl3_status launch_qmv(const exl3_trellis_desc &shape, const PtrTable &trellis, int n,
                       const uint16_t *xhat, int64_t x_member_stride, int64_t rows, float *part,
                       hipStream_t st, const PtrTable *suh) {
  const int in = shape.in_features, out = shape.out_features;
  const int k_tiles = in / 16;
  const int pr = qmv_pass_rows(rows);
  const int64_t gy = (int64_t)n_slices(k_tiles) * ((rows + pr - 1) / pr);
  if (gy > 65535 || n > 65535) return fail(EXL3_ERR_UNSUPPORTED, "linear launch too large");
  dim3 grid((unsigned)(out / 128), (unsigned)gy, (unsigned)n);
  const int tiles_n = out / 16, pd = prefetch_steps(k_tiles, shape.K);
  // the weight form of the process-wide tuning (the reference's f16 weights by default)
  const int kcb = kernel_cb(shape.codebook, tuning().weight_form);
  switch (shape.K) {
#define EXL3_K(KK)                                                                        \
  case KK:                                                                                \
    qmv_cb<KK>(kcb, pd, grid, st, trellis, tiles_n, in, out, xhat, x_member_stride, rows, \
               pr, part, suh);                                                            \
    break;
    EXL3_K(1) EXL3_K(2) EXL3_K(3) EXL3_K(4) EXL3_K(5) EXL3_K(6) EXL3_K(7) EXL3_K(8)
#undef EXL3_K
    default: return fail(EXL3_ERR_INVALID, "K out of range");
  }
  EXL3_LAUNCHED("k_qmv");
  return EXL3_OK;
}

exl3_status launch_qmv_finalize(int n, int n_sl, int64_t rows, int out, const float *part,
                                float *y32, uint16_t *y16, const PtrTable &svh, hipStream_t st) {
  const int64_t waves = (int64_t)n * rows * (out / 128);
  if (waves == 0) return EXL3_OK;
  k_qmv_finalize<<<(unsigned)((waves + 3) / 4), 256, 0, st>>>(n, n_sl, rows, out, part, y32,
                                                              y16, svh);
  EXL3_LAUNCHED("k_qmv_finalize");
  return EXL3_OK;
}

}  // namespace exl3h
