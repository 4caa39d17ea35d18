// C ABI: library state, errors, tuning and the single-tensor trellis entry points.
// Reference interface: src/trellis_gemm.h (muyouming/exl3-server).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <mutex>
#include <string>

#include "exl3_internal.hpp"
#include "exl3_moe.h"

namespace exl3h {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }

exl3_status fail(exl3_status st, const std::string &msg) {
  set_error(msg);
  return st;
}

exl3_status hip_check(hipError_t e, const char *what) {
  return fail(EXL3_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

static std::mutex g_tuning_mu;
static exl3_tuning g_tuning = {0, 16, 0, EXL3_FORM_REFERENCE};

exl3_tuning tuning() {
  std::lock_guard<std::mutex> lk(g_tuning_mu);
  return g_tuning;
}

exl3_status check_tuning(const exl3_tuning *t) {
  if (!t) return fail(EXL3_ERR_INVALID, "null tuning");
  if (t->weight_form != EXL3_FORM_REFERENCE && t->weight_form != EXL3_FORM_HALVES)
    return fail(EXL3_ERR_INVALID, "weight_form must be EXL3_FORM_REFERENCE or EXL3_FORM_HALVES");
  return EXL3_OK;
}

exl3_status check_desc(const exl3_trellis_desc *w, bool need_128) {
  if (!w) return fail(EXL3_ERR_INVALID, "null trellis descriptor");
  if (!w->trellis) return fail(EXL3_ERR_INVALID, "null trellis pointer");
  if (reinterpret_cast<uintptr_t>(w->trellis) % 4)
    return fail(EXL3_ERR_INVALID, "trellis base must be 4-byte aligned (use exl3_trellis_pack)");
  if (w->K < 1 || w->K > 8) return fail(EXL3_ERR_INVALID, "K must be in 1..8");
  if (w->codebook < 0 || w->codebook > 2) return fail(EXL3_ERR_INVALID, "codebook must be 0..2");
  const int m = need_128 ? 128 : 16;
  if (w->in_features <= 0 || w->out_features <= 0 || w->in_features % m || w->out_features % m)
    return fail(EXL3_ERR_INVALID, "in/out features must be positive multiples of " +
                                      std::to_string(m));
  if (need_128 && (!w->suh || !w->svh)) return fail(EXL3_ERR_INVALID, "null suh/svh");
  // the kernels address a tensor through 32-bit buffer offsets and park unused loads
  // at 1 GiB (past any tensor)
  if ((int64_t)w->in_features * w->out_features / 8 * w->K >= ((int64_t)1 << 30))
    return fail(EXL3_ERR_UNSUPPORTED, "trellis tensor of 1 GiB or more");
  return EXL3_OK;
}

}  // namespace exl3h

using namespace exl3h;

namespace {

// Workspace of the single/grouped linear: the slice partials (n, n_slices, rows, out) f32
// (the input Hadamard happens inside the QMV kernel).
struct LinearWs {
  size_t part_off, total;
};

LinearWs linear_ws(int in, int out, int64_t rows, int n) {
  LinearWs w;
  w.part_off = 0;
  w.total = align_up((size_t)n * qmv_slices(in) * rows * out * 4, 256);
  return w;
}

exl3_status check_ws(void *ws, size_t bytes, size_t need) {
  if (need && (!ws || bytes < need))
    return fail(EXL3_ERR_WORKSPACE, "workspace too small: need " + std::to_string(need) +
                                        " bytes, got " + std::to_string(bytes));
  if (reinterpret_cast<uintptr_t>(ws) % 256)
    return fail(EXL3_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return EXL3_OK;
}

// x (or xhat) -> partials -> (raw f32 | f16 via the output Hadamard), n members of one
// shape.
exl3_status linear_core(const exl3_trellis_desc *members, int n, const uint16_t *x,
                        int64_t rows, bool x_shared, bool x_is_xhat, const uint16_t *suh_stack,
                        const uint16_t *svh_stack, float *y32, uint16_t *y16, void *ws,
                        size_t ws_bytes, hipStream_t st) {
  const exl3_trellis_desc &w0 = members[0];
  const int in = w0.in_features, out = w0.out_features;
  const LinearWs lw = linear_ws(in, out, rows, n < PtrTable::kMax ? n : PtrTable::kMax);
  exl3_status rc = check_ws(ws, ws_bytes, lw.total);
  if (rc) return rc;
  float *part = reinterpret_cast<float *>((char *)ws + lw.part_off);
  const int n_sl = qmv_slices(in);
  for (int c0 = 0; c0 < n; c0 += PtrTable::kMax) {
    const int cn = std::min(PtrTable::kMax, n - c0);
    PtrTable tr{}, su{}, sv{};
    for (int i = 0; i < cn; ++i) {
      tr.p[i] = members[c0 + i].trellis;
      su.p[i] = suh_stack ? (const void *)(suh_stack + (int64_t)(c0 + i) * in)
                          : (const void *)members[c0 + i].suh;
      sv.p[i] = svh_stack ? (const void *)(svh_stack + (int64_t)(c0 + i) * out)
                          : (const void *)members[c0 + i].svh;
    }
    const uint16_t *xc = x + (x_shared ? 0 : (int64_t)c0 * rows * in);
    const int64_t x_stride = x_shared ? 0 : rows * in;
    // from x, the QMV kernel applies each member's input Hadamard while it stages rows
    rc = launch_qmv(w0, tr, cn, xc, x_stride, rows, part, st, x_is_xhat ? nullptr : &su);
    if (rc) return rc;
    rc = launch_qmv_finalize(cn, n_sl, rows, out, part,
                             y32 ? y32 + (int64_t)c0 * rows * out : nullptr,
                             y16 ? y16 + (int64_t)c0 * rows * out : nullptr, sv, st);
    if (rc) return rc;
  }
  return EXL3_OK;
}

}  // namespace

extern "C" {

const char *exl3_last_error(void) { return g_last_error.c_str(); }

int32_t exl3_abi_version(void) { return 2; }

exl3_status exl3_set_tuning(const exl3_tuning *t) {
  exl3_status rc = check_tuning(t);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(g_tuning_mu);
  g_tuning = *t;
  return EXL3_OK;
}

exl3_status exl3_get_tuning(exl3_tuning *t) {
  if (!t) return fail(EXL3_ERR_INVALID, "null tuning");
  *t = tuning();
  return EXL3_OK;
}

exl3_status exl3_trellis_path_info(const exl3_trellis_desc *w, int64_t rows,
                                   exl3_path_info *info) {
  exl3_status rc = check_desc(w, true);
  if (rc) return rc;
  if (!info || rows < 0) return fail(EXL3_ERR_INVALID, "bad path_info arguments");
  const exl3_tuning tn = tuning();
  const int mb = qmv_pass_rows(rows);
  // Every pass runs on the matrix cores; "staged" reports the reference's criterion
  // (a pass shared by at least mat_min_rows rows, trellis_gemm.cpp:800-812).
  info->staged = (tn.mat_min_rows > 0 && rows >= tn.mat_min_rows &&
                  (tn.mat_max_rows <= 0 || rows <= tn.mat_max_rows))
                     ? 1
                     : 0;
  info->rows_per_block = mb;
  info->pad_rows = (int32_t)((rows + mb - 1) / mb * mb);
  info->passes = (int32_t)((rows + mb - 1) / mb);
  info->splits = qmv_slices(w->in_features);
  info->tiles_per_workgroup = 32;
  return EXL3_OK;
}

exl3_status exl3_trellis_pack(const uint16_t *words16_host, int32_t k_tiles, int32_t n_tiles,
                              int32_t K, void *dst_device, exl3_stream_t stream) {
  if (!words16_host || !dst_device || k_tiles <= 0 || n_tiles <= 0 || K < 1 || K > 8)
    return fail(EXL3_ERR_INVALID, "exl3_trellis_pack: bad arguments");
  if (reinterpret_cast<uintptr_t>(dst_device) % 4)
    return fail(EXL3_ERR_INVALID, "exl3_trellis_pack: destination must be 4-byte aligned");
  const size_t bytes = (size_t)k_tiles * n_tiles * 32 * K;
  EXL3_HIP(hipMemcpyAsync(dst_device, words16_host, bytes, hipMemcpyHostToDevice,
                          stream_of(stream)));
  EXL3_HIP(hipStreamSynchronize(stream_of(stream)));
  return EXL3_OK;
}

exl3_status exl3_trellis_decode(const exl3_trellis_desc *w, uint16_t *w_hat,
                                exl3_stream_t stream) {
  exl3_status rc = check_desc(w, false);
  if (rc) return rc;
  if (!w_hat) return fail(EXL3_ERR_INVALID, "null output");
  return launch_decode(*w, w_hat, stream_of(stream));
}

exl3_status exl3_trellis_reconstruct(const exl3_trellis_desc *w, uint16_t *w_out,
                                     exl3_stream_t stream) {
  exl3_status rc = check_desc(w, true);
  if (rc) return rc;
  if (!w_out) return fail(EXL3_ERR_INVALID, "null output");
  return launch_reconstruct(*w, w_out, stream_of(stream));
}

exl3_status exl3_trellis_hadamard(const uint16_t *x_f16, const float *x_f32, int64_t rows,
                                  int32_t n, const uint16_t *s, int32_t stacked, uint16_t *y,
                                  exl3_stream_t stream) {
  if ((x_f16 == nullptr) == (x_f32 == nullptr))
    return fail(EXL3_ERR_INVALID, "exactly one of x_f16 / x_f32 must be given");
  if (!s || !y || rows < 0 || n <= 0 || n % 128 || stacked < 0)
    return fail(EXL3_ERR_INVALID, "exl3_trellis_hadamard: bad arguments");
  if (stacked > PtrTable::kMax)
    return fail(EXL3_ERR_UNSUPPORTED, "exl3_trellis_hadamard: at most 128 stacked vectors");
  if (stacked > 0 && rows % stacked)
    return fail(EXL3_ERR_INVALID, "rows must be a multiple of the stacked member count");
  PtrTable t{};
  int64_t rpm = rows > 0 ? rows : 1;
  if (stacked > 0) {
    for (int i = 0; i < stacked; ++i) t.p[i] = s + (int64_t)i * n;
    rpm = rows / stacked;
  } else {
    t.p[0] = s;
  }
  return launch_hadamard(x_f16, x_f32, rows, n, t, rpm, y, stream_of(stream));
}

size_t exl3_trellis_workspace_size(const exl3_trellis_desc *w, int64_t rows, int32_t n_members) {
  if (!w || rows < 0 || n_members <= 0) return 0;
  const int32_t chunk = n_members < PtrTable::kMax ? n_members : PtrTable::kMax;
  return linear_ws(w->in_features, w->out_features, rows, chunk).total;
}

exl3_status exl3_trellis_matmul_raw(const exl3_trellis_desc *w, const uint16_t *xhat,
                                    int64_t rows, float *yhat, void *workspace,
                                    size_t workspace_bytes, exl3_stream_t stream) {
  exl3_status rc = check_desc(w, true);
  if (rc) return rc;
  if (!xhat || !yhat || rows < 0) return fail(EXL3_ERR_INVALID, "bad matmul_raw arguments");
  if (rows == 0) return EXL3_OK;
  return linear_core(w, 1, xhat, rows, false, true, nullptr, nullptr, yhat, nullptr, workspace,
                     workspace_bytes, stream_of(stream));
}

exl3_status exl3_trellis_linear(const exl3_trellis_desc *w, const uint16_t *x, int64_t rows,
                                uint16_t *y, void *workspace, size_t workspace_bytes,
                                exl3_stream_t stream) {
  exl3_status rc = check_desc(w, true);
  if (rc) return rc;
  if (!x || !y || rows < 0) return fail(EXL3_ERR_INVALID, "bad linear arguments");
  if (rows == 0) return EXL3_OK;
  return linear_core(w, 1, x, rows, false, false, nullptr, nullptr, nullptr, y, workspace,
                     workspace_bytes, stream_of(stream));
}

exl3_status exl3_trellis_linear_grouped(const exl3_trellis_desc *members, int32_t n,
                                        const uint16_t *x, int64_t rows, int32_t x_shared,
                                        const uint16_t *suh_stack, const uint16_t *svh_stack,
                                        uint16_t *y, void *workspace, size_t workspace_bytes,
                                        exl3_stream_t stream) {
  if (!members || n <= 0) return fail(EXL3_ERR_INVALID, "no members");
  for (int i = 0; i < n; ++i) {
    exl3_status rc = check_desc(&members[i], true);
    if (rc) return rc;
    const exl3_trellis_desc &a = members[0], &b = members[i];
    if (a.in_features != b.in_features || a.out_features != b.out_features || a.K != b.K ||
        a.codebook != b.codebook)
      return fail(EXL3_ERR_INVALID, "grouped members must share shape, K and codebook");
  }
  if (!x || !y || rows < 0) return fail(EXL3_ERR_INVALID, "bad grouped arguments");
  if (rows == 0) return EXL3_OK;
  return linear_core(members, n, x, rows, x_shared != 0, false, suh_stack, svh_stack, nullptr, y,
                     workspace, workspace_bytes, stream_of(stream));
}

}  // extern "C"
