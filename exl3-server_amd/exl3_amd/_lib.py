"""ctypes binding of libexl3moe.so (the C ABI declared in include/exl3_moe.h).

There is no fallback: if the HIP library is not built, importing the entry points
raises. Every call checks the returned exl3_status and raises Exl3Error with the
library's exl3_last_error() text.
"""
from __future__ import annotations

import ctypes as C
import os
import re

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libexl3moe.so")
HEADER = os.path.join(os.path.dirname(os.path.dirname(PKG_DIR)), "include", "exl3_moe.h")

EXL3_OK, EXL3_ERR_INVALID, EXL3_ERR_UNSUPPORTED, EXL3_ERR_WORKSPACE, EXL3_ERR_HIP = range(5)


class Exl3Error(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"exl3 status {status}: {msg}")
        self.status = status


class TrellisDesc(C.Structure):
    _fields_ = [("trellis", C.c_void_p), ("suh", C.c_void_p), ("svh", C.c_void_p),
                ("in_features", C.c_int32), ("out_features", C.c_int32), ("K", C.c_int32),
                ("codebook", C.c_int32)]


class LinearDesc(C.Structure):
    _fields_ = [("tw", TrellisDesc), ("dense", C.c_void_p), ("in_features", C.c_int32),
                ("out_features", C.c_int32)]


class MoeConfig(C.Structure):
    _fields_ = [("hidden_size", C.c_int32), ("moe_intermediate_size", C.c_int32),
                ("n_routed_experts", C.c_int32), ("num_experts_per_tok", C.c_int32),
                ("n_group", C.c_int32), ("topk_group", C.c_int32),
                ("norm_topk_prob", C.c_int32), ("routed_scaling_factor", C.c_float),
                ("swiglu_limit", C.c_float)]


class StTensor(C.Structure):
    _fields_ = [("dtype", C.c_int32), ("ndim", C.c_int32), ("shape", C.c_int64 * 8),
                ("offset", C.c_int64), ("nbytes", C.c_int64), ("file_offset", C.c_int64)]


ST_DTYPES = {0: "F16", 1: "BF16", 2: "F32", 3: "I16", 4: "I32", 5: "U8", 6: "I8", 7: "I64", 8: "F64",
             9: "U16", 10: "U32", 11: "BOOL"}


class MoeLayerDesc(C.Structure):
    _fields_ = [("experts", C.POINTER(LinearDesc)), ("shared", C.POINTER(LinearDesc)),
                ("router_w", C.c_void_p), ("router_bias", C.c_void_p)]


# exl3_weight_form
FORM_REFERENCE = 0
FORM_HALVES = 1


class Tuning(C.Structure):
    _fields_ = [("rows_per_pass", C.c_int32), ("mat_min_rows", C.c_int32),
                ("mat_max_rows", C.c_int32), ("weight_form", C.c_int32)]


class PathInfo(C.Structure):
    _fields_ = [("staged", C.c_int32), ("rows_per_block", C.c_int32), ("pad_rows", C.c_int32),
                ("passes", C.c_int32), ("splits", C.c_int32),
                ("tiles_per_workgroup", C.c_int32)]


class MoeDiag(C.Structure):
    _fields_ = [("calls", C.c_int64), ("pairs", C.c_int64), ("runs", C.c_int64),
                ("distinct_experts", C.c_int64), ("staged_runs", C.c_int64),
                ("streamed_bytes", C.c_int64), ("shared_bytes", C.c_int64),
                ("run_hist", C.c_int64 * 65)]


class MoeTiming(C.Structure):
    _fields_ = [("calls", C.c_int64), ("router_ms", C.c_double), ("gate_up_ms", C.c_double),
                ("down_ms", C.c_double), ("combine_ms", C.c_double), ("total_ms", C.c_double),
                ("gate_up_trellis_bytes", C.c_int64), ("down_trellis_bytes", C.c_int64)]


class HcSite(C.Structure):
    _fields_ = [("mult", C.c_int32), ("sinkhorn_iters", C.c_int32), ("eps", C.c_float),
                ("fn", C.c_void_p), ("base", C.c_void_p), ("scale", C.c_void_p)]


vp, i32, i64, sz = C.c_void_p, C.c_int32, C.c_int64, C.c_size_t
P = C.POINTER

# name -> (restype, argtypes); restype int = exl3_status
SIGNATURES = {
    "exl3_last_error": (C.c_char_p, []),
    "exl3_abi_version": (i32, []),
    "exl3_set_tuning": (C.c_int, [P(Tuning)]),
    "exl3_get_tuning": (C.c_int, [P(Tuning)]),
    "exl3_trellis_path_info": (C.c_int, [P(TrellisDesc), i64, P(PathInfo)]),
    "exl3_trellis_pack": (C.c_int, [vp, i32, i32, i32, vp, vp]),
    "exl3_trellis_decode": (C.c_int, [P(TrellisDesc), vp, vp]),
    "exl3_trellis_reconstruct": (C.c_int, [P(TrellisDesc), vp, vp]),
    "exl3_trellis_hadamard": (C.c_int, [vp, vp, i64, i32, vp, i32, vp, vp]),
    "exl3_trellis_workspace_size": (sz, [P(TrellisDesc), i64, i32]),
    "exl3_trellis_matmul_raw": (C.c_int, [P(TrellisDesc), vp, i64, vp, vp, sz, vp]),
    "exl3_trellis_linear": (C.c_int, [P(TrellisDesc), vp, i64, vp, vp, sz, vp]),
    "exl3_trellis_linear_grouped": (C.c_int, [P(TrellisDesc), i32, vp, i64, i32, vp, vp, vp,
                                              vp, sz, vp]),
    "exl3_moe_layer_create": (C.c_int, [P(MoeLayerDesc), P(MoeConfig), P(vp)]),
    "exl3_moe_layer_destroy": (C.c_int, [vp]),
    "exl3_moe_workspace_size": (sz, [vp, i64]),
    "exl3_moe_route": (C.c_int, [vp, vp, i64, vp, vp, vp, sz, vp]),
    "exl3_moe_topk_route": (C.c_int, [vp, vp, i64, P(MoeConfig), vp, vp, vp]),
    "exl3_moe_layer": (C.c_int, [vp, vp, i64, i64, vp, vp, sz, vp]),
    "exl3_moe_layer_noalloc": (C.c_int, [vp, vp, i64, i64, vp, vp]),
    "exl3_moe_scratch_capacity": (sz, []),
    "exl3_moe_timing_enable": (C.c_int, [vp, i32]),
    "exl3_moe_timing_get": (C.c_int, [vp, P(MoeTiming)]),
    "exl3_moe_timing_reset": (C.c_int, [vp]),
    "exl3_moe_diag_enable": (C.c_int, [vp, i32]),
    "exl3_moe_diag_get": (C.c_int, [vp, P(MoeDiag)]),
    "exl3_moe_diag_reset": (C.c_int, [vp]),
    "exl3_moe_set_tuning": (C.c_int, [vp, P(Tuning)]),
    "exl3_st_open": (C.c_int, [C.c_char_p, P(vp)]),
    "exl3_st_close": (C.c_int, [vp]),
    "exl3_st_header_len": (i64, [vp]),
    "exl3_st_count": (i32, [vp]),
    "exl3_st_tensor_at": (C.c_int, [vp, i32, P(StTensor), P(C.c_char_p)]),
    "exl3_st_find": (C.c_int, [vp, C.c_char_p, P(StTensor)]),
    "exl3_st_data": (vp, [vp, C.c_char_p]),
    "exl3_moe_layer_load": (C.c_int, [P(C.c_char_p), i32, C.c_char_p, P(MoeConfig), P(vp), vp]),
    "exl3_moe_layer_load_info": (C.c_int, [vp, P(i64), P(i64)]),
    "exl3_moe_layer_load_block": (C.c_int, [vp, P(C.c_char_p), i32, C.c_char_p, P(HcSite), P(vp), vp]),
    "exl3_moe_get_tuning": (C.c_int, [vp, P(Tuning)]),
    "exl3_hc_workspace_size": (sz, [i32, i32, i64]),
    "exl3_hc_prepare": (C.c_int, [P(HcSite), vp, i64, i32, vp, C.c_float, vp, vp, vp, vp, sz, vp]),
    "exl3_rms_norm": (C.c_int, [vp, i64, i32, vp, C.c_float, vp, vp]),
    "exl3_hc_mix": (C.c_int, [vp, vp, vp, vp, i64, i32, i32, vp, vp]),
    "exl3_moe_block_workspace_size": (sz, [vp, i32, i64]),
    "exl3_moe_block": (C.c_int, [vp, P(HcSite), vp, C.c_float, vp, i64, vp, vp, sz, vp]),
}

_LIB = None


def header_symbols() -> list[str]:
    """Every exl3_* function declared in include/exl3_moe.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(exl3_[a-z0-9_]+)\s*\(", text)))


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP library not built: {LIB_PATH} (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(status: int) -> None:
    if status != EXL3_OK:
        msg = lib().exl3_last_error()
        raise Exl3Error(status, msg.decode() if msg else "")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
