// Host-side internals shared by the library's translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "exl3_moe.h"

namespace exl3h {

// Thread-local last error (exl3_last_error).
void set_error(const std::string &msg);
exl3_status fail(exl3_status st, const std::string &msg);
exl3_status hip_check(hipError_t e, const char *what);

#define EXL3_HIP(call)                                          \
  do {                                                          \
    hipError_t e_ = (call);                                     \
    if (e_ != hipSuccess) return exl3h::hip_check(e_, #call);   \
  } while (0)

#define EXL3_LAUNCHED(what)                                     \
  do {                                                          \
    hipError_t e_ = hipGetLastError();                          \
    if (e_ != hipSuccess) return exl3h::hip_check(e_, what);    \
  } while (0)

inline hipStream_t stream_of(exl3_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// The k partition of a trellis GEMV, a function of the tensor's k-tile count only: the
// k range is cut into slices, each summed from zero by one wave, and an output is the
// in-order sum of its slice partials (device side: qmv_core.hpp).
int qmv_slices(int in);
// Token rows per MFMA pass of the standalone/grouped linear (rows_per_pass knob, <= 16).
int qmv_pass_rows(int64_t rows);

// Scheduling knobs (exl3_set_tuning) and their validation.
exl3_tuning tuning();
exl3_status check_tuning(const exl3_tuning *t);

// Validates a trellis descriptor for the Hadamard-based paths.
exl3_status check_desc(const exl3_trellis_desc *w, bool need_128);

// A small table of per-member device pointers passed by value in kernel arguments.
struct PtrTable {
  static constexpr int kMax = 128;
  const void *p[kMax];
};

// Launchers implemented in trellis_kernels.hip, used by the API layer.
exl3_status launch_decode(const exl3_trellis_desc &w, uint16_t *w_hat, hipStream_t st);
exl3_status launch_reconstruct(const exl3_trellis_desc &w, uint16_t *w_out, hipStream_t st);
// pre (x16) or post (x32) Hadamard over (rows, n); row r uses scale vector
// s.p[r / rows_per_member] (rows_per_member = rows when one vector is shared).
exl3_status launch_hadamard(const uint16_t *x16, const float *x32, int64_t rows, int n,
                            const PtrTable &s, int64_t rows_per_member, uint16_t *y,
                            hipStream_t st);

// xhat: (n, rows, in) f16 (member stride rows*in, or 0 when shared); part: f32
// (n, n_slices, rows, out). With suh (member m's scales in suh->p[m]), xhat is the raw
// x and the kernel applies the input Hadamard itself.
exl3_status launch_qmv(const exl3_trellis_desc &shape, const PtrTable &trellis, int n,
                       const uint16_t *xhat, int64_t x_member_stride, int64_t rows, float *part,
                       hipStream_t st, const PtrTable *suh = nullptr);
// Sums the slice partials in slice order into y32 (raw f32, (n, rows, out)) or, through
// the output Hadamard with member m's svh.p[m], into y16 (n, rows, out).
exl3_status launch_qmv_finalize(int n, int n_sl, int64_t rows, int out, const float *part,
                                float *y32, uint16_t *y16, const PtrTable &svh,
                                hipStream_t st);

// Hyper-connection prepare (csrc/hc.hip): site and shape checks, the partials' workspace,
// and the two launches (projection partials, then finalize with the optional RMSNorm).
exl3_status check_hc(const exl3_hc_site *hc, int D);
inline exl3_status check_hc_shape(int n, int D) {
  return (n < 1 || n > 8 || D <= 0 || D > 8192 || D % 2 || ((int64_t)n * D) % 64) ? EXL3_ERR_UNSUPPORTED : EXL3_OK;
}
size_t hc_part_bytes(int N, int D, int64_t P);
// Whether two buffers of n bytes each share a byte.
inline bool overlaps(const void *a, const void *b, size_t n) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return n && x < y + n && y < x + n;
}
exl3_status launch_hc_prepare(const exl3_hc_site *hc, const uint16_t *streams, int64_t P, int D,
                              const uint16_t *norm_w, float norm_eps, uint16_t *out, float *post,
                              float *comb, float *part, hipStream_t st);

// Hands device buffers made by the loader to a layer handle, which frees them at
// exl3_moe_layer_destroy; `in_place`/`repacked` count its trellis tensors.
void layer_adopt(exl3_moe_layer_t layer, const std::vector<void *> &bufs, int64_t in_place, int64_t repacked);
// The layer's hidden size.
int layer_hidden(exl3_moe_layer_t layer);

}  // namespace exl3h
