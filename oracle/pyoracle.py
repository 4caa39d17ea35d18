"""ctypes binding of the CPU oracle (oracle/liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
checker / CPU baseline. The product (exl3-server_amd/) never imports this module.

Also binds oracle/_ref/libexl3ref.so (the reference's own src/exl3.cpp compiled in
the build container) when it is present; it is absent on the GPU box.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")


class OrLinear(C.Structure):
    _fields_ = [
        ("trellis", C.c_void_p),
        ("suh", C.c_void_p),
        ("svh", C.c_void_p),
        ("dense", C.c_void_p),
        ("in_", C.c_int32),
        ("out", C.c_int32),
        ("K", C.c_int32),
        ("cb", C.c_int32),
    ]


class OrMoeCfg(C.Structure):
    _fields_ = [
        ("hidden", C.c_int32),
        ("inter", C.c_int32),
        ("n_experts", C.c_int32),
        ("top_k", C.c_int32),
        ("n_group", C.c_int32),
        ("topk_group", C.c_int32),
        ("norm_topk_prob", C.c_int32),
        ("has_shared", C.c_int32),
        ("routed_scaling_factor", C.c_float),
        ("swiglu_limit", C.c_float),
    ]


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle not built: {path} (run __graft_entry__.build())")
        L = C.CDLL(path)
        L.or_f16_from_double.argtypes = [C.c_double]
        L.or_f16_from_double.restype = C.c_uint16
        L.or_f16_to_double.argtypes = [C.c_uint16]
        L.or_f16_to_double.restype = C.c_double
        L.or_codebook_value.argtypes = [C.c_uint16, C.c_int]
        L.or_codebook_value.restype = C.c_uint16
        L.or_codebook_lut.argtypes = [C.c_int, u16p]
        L.or_set_gemv_mode.argtypes = [C.c_int]
        L.or_get_gemv_mode.restype = C.c_int
        L.or_codebook_halves_sum.argtypes = [C.c_uint16, C.c_int]
        L.or_codebook_halves_sum.restype = C.c_float
        L.or_tile_state.argtypes = [u16p, C.c_int, C.c_int]
        L.or_tile_state.restype = C.c_uint16
        L.or_tile_state_bruteforce.argtypes = [u16p, C.c_int, C.c_int]
        L.or_tile_state_bruteforce.restype = C.c_uint16
        L.or_tile_perm.argtypes = [C.c_int]
        L.or_tile_perm.restype = C.c_int
        L.or_decode_inner.argtypes = [u16p, C.c_int64, C.c_int64, C.c_int, C.c_int, u16p, C.c_int]
        L.or_reconstruct.argtypes = [u16p, C.c_int64, C.c_int64, C.c_int, C.c_int, u16p, u16p,
                                     u16p, C.c_int]
        L.or_had_pre.argtypes = [u16p, C.c_int64, C.c_int64, u16p, u16p]
        L.or_had_post.argtypes = [f32p, C.c_int64, C.c_int64, u16p, u16p]
        L.or_had_post_f64.argtypes = [f64p, C.c_int64, C.c_int64, u16p, u16p]
        L.or_matmul_raw.argtypes = [u16p, C.c_int64, C.c_int64, C.c_int, C.c_int, u16p,
                                    C.c_int64, f64p, C.c_int]
        L.or_trellis_linear.argtypes = [u16p, C.c_int64, C.c_int64, C.c_int, C.c_int, u16p, u16p,
                                        u16p, C.c_int64, u16p, C.c_int]
        L.or_router_logits.argtypes = [u16p, C.c_int64, u16p, C.c_int, C.c_int, f64p]
        L.or_route.argtypes = [f64p, f32p, C.c_int64, C.POINTER(OrMoeCfg), i32p, f64p]
        L.or_moe_runs.argtypes = [i32p, C.c_int64, C.c_int] + [i32p] * 7
        L.or_moe_layer.argtypes = [C.POINTER(OrMoeCfg), C.POINTER(OrLinear), C.c_void_p, u16p,
                                   f32p, u16p, C.c_int64, u16p, i32p, f64p, C.c_int]
        L.or_moe_layer_routed.argtypes = [C.POINTER(OrMoeCfg), C.POINTER(OrLinear), C.c_void_p,
                                          u16p, C.c_int64, i32p, f64p, u16p, C.c_int]
        L.or_hc_prepare.argtypes = [u16p, C.c_int64, C.c_int, C.c_int, f32p, f32p, f32p, C.c_int,
                                    C.c_double, u16p, f64p, f64p]
        L.or_rms_norm.argtypes = [u16p, C.c_int64, C.c_int, u16p, C.c_double, u16p]
        L.or_hc_mix.argtypes = [u16p, f64p, f64p, u16p, C.c_int64, C.c_int, C.c_int, u16p]
        _LIB = L
    return _LIB


def ref_lib():
    """The reference's own codec, or None where it was not built (e.g. the GPU box)."""
    global _REF
    if _REF is None:
        path = os.path.join(_HERE, "_ref", "libexl3ref.so")
        if not os.path.exists(path):
            return None
        R = C.CDLL(path)
        R.ref_codebook_lut.argtypes = [C.c_int, u16p]
        R.ref_decode_inner.argtypes = [u16p, C.c_int64, C.c_int64, C.c_int, C.c_int, u16p, C.c_int]
        R.ref_decode_inner.restype = C.c_int
        R.ref_reconstruct.argtypes = [u16p, C.c_int64, C.c_int64, C.c_int, C.c_int, u16p, u16p,
                                      u16p, C.c_int]
        R.ref_reconstruct.restype = C.c_int
        _REF = R
    return _REF


def _threads(threads):
    # at most 16 workers: the GPU box grants one GPU's share of its host cores
    return threads if threads else min(16, os.cpu_count() or 1)


# --- thin numpy wrappers -------------------------------------------------------------

def codebook_lut(cb: int) -> np.ndarray:
    out = np.zeros(65536, np.uint16)
    lib().or_codebook_lut(cb, out)
    return out


def halves_sum_lut(cb: int) -> np.ndarray:
    """f32 exact sum of the two f16 halves of every state's masked hash word (mcg/3inst)."""
    L = lib()
    return np.array([L.or_codebook_halves_sum(s, cb) for s in range(65536)], np.float32)


class gemv_mode:
    """Context manager: the oracle's GEMV weights inside the block. exact_halves=True
    uses the unrounded lo + hi sum for mcg/3inst (the value the GPU's exact-halves form
    multiplies), False the reference's f16 weights (the default, and the GPU's default
    form)."""

    def __init__(self, exact_halves: bool):
        self.mode = 1 if exact_halves else 0

    def __enter__(self):
        self.prev = lib().or_get_gemv_mode()
        lib().or_set_gemv_mode(self.mode)
        return self

    def __exit__(self, *exc):
        lib().or_set_gemv_mode(self.prev)
        return False


def decode_inner(trellis: np.ndarray, in_f: int, out_f: int, K: int, cb: int, threads=0):
    w = np.zeros((in_f, out_f), np.uint16)
    rc = lib().or_decode_inner(np.ascontiguousarray(trellis, np.uint16).reshape(-1), in_f, out_f,
                               K, cb, w, _threads(threads))
    if rc:
        raise ValueError("or_decode_inner: bad geometry")
    return w


def reconstruct(trellis, in_f, out_f, K, cb, suh, svh, threads=0):
    w = np.zeros((in_f, out_f), np.uint16)
    rc = lib().or_reconstruct(np.ascontiguousarray(trellis, np.uint16).reshape(-1), in_f, out_f,
                              K, cb, np.ascontiguousarray(suh, np.uint16),
                              np.ascontiguousarray(svh, np.uint16), w, _threads(threads))
    if rc:
        raise ValueError("or_reconstruct: bad geometry")
    return w


def had_pre(x: np.ndarray, suh: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    rows, n = x.reshape(-1, x.shape[-1]).shape
    y = np.zeros_like(x)
    lib().or_had_pre(x.reshape(-1), rows, n, np.ascontiguousarray(suh, np.uint16), y.reshape(-1))
    return y


def had_post(yhat: np.ndarray, svh: np.ndarray) -> np.ndarray:
    yhat = np.ascontiguousarray(yhat, np.float32)
    rows, n = yhat.reshape(-1, yhat.shape[-1]).shape
    y = np.zeros(yhat.shape, np.uint16)
    lib().or_had_post(yhat.reshape(-1), rows, n, np.ascontiguousarray(svh, np.uint16),
                      y.reshape(-1))
    return y


def matmul_raw(trellis, in_f, out_f, K, cb, xhat, threads=0):
    xhat = np.ascontiguousarray(xhat, np.uint16).reshape(-1, in_f)
    rows = xhat.shape[0]
    y = np.zeros((rows, out_f), np.float64)
    rc = lib().or_matmul_raw(np.ascontiguousarray(trellis, np.uint16).reshape(-1), in_f, out_f, K,
                             cb, xhat.reshape(-1), rows, y.reshape(-1), _threads(threads))
    if rc:
        raise ValueError("or_matmul_raw: bad geometry")
    return y


def trellis_linear(trellis, in_f, out_f, K, cb, suh, svh, x, threads=0):
    x = np.ascontiguousarray(x, np.uint16).reshape(-1, in_f)
    rows = x.shape[0]
    y = np.zeros((rows, out_f), np.uint16)
    rc = lib().or_trellis_linear(np.ascontiguousarray(trellis, np.uint16).reshape(-1), in_f, out_f,
                                 K, cb, np.ascontiguousarray(suh, np.uint16),
                                 np.ascontiguousarray(svh, np.uint16), x.reshape(-1), rows,
                                 y.reshape(-1), _threads(threads))
    if rc:
        raise ValueError("or_trellis_linear: bad geometry")
    return y


def make_cfg(hidden, inter, n_experts, top_k, n_group=1, topk_group=1, norm_topk_prob=True,
             has_shared=True, routed_scaling_factor=1.0, swiglu_limit=10.0) -> OrMoeCfg:
    return OrMoeCfg(hidden, inter, n_experts, top_k, n_group, topk_group, int(norm_topk_prob),
                    int(has_shared), routed_scaling_factor, swiglu_limit)


def router_logits(h, router_w):
    h = np.ascontiguousarray(h, np.uint16)
    E, H = router_w.shape
    N = h.size // H
    out = np.zeros((N, E), np.float64)
    lib().or_router_logits(h.reshape(-1), N, np.ascontiguousarray(router_w, np.uint16).reshape(-1),
                           E, H, out.reshape(-1))
    return out


def route(logits, bias, cfg: OrMoeCfg):
    logits = np.ascontiguousarray(logits, np.float64)
    N = logits.shape[0]
    idx = np.zeros((N, cfg.top_k), np.int32)
    w = np.zeros((N, cfg.top_k), np.float64)
    rc = lib().or_route(logits.reshape(-1), np.ascontiguousarray(bias, np.float32), N,
                        C.byref(cfg), idx.reshape(-1), w.reshape(-1))
    if rc:
        raise ValueError("or_route: bad config")
    return idx, w


def moe_runs(idx: np.ndarray):
    idx = np.ascontiguousarray(idx, np.int32)
    N, K = idx.shape
    P = N * K
    bufs = [np.zeros(P, np.int32) for _ in range(7)]
    runs = lib().or_moe_runs(idx.reshape(-1), N, K, *bufs)
    se, sr, sk, perm, re, ro, rl = bufs
    return dict(sorted_expert=se, sorted_row=sr, sorted_rank=sk, perm=perm,
                run_expert=re[:runs].copy(), run_off=ro[:runs].copy(), run_len=rl[:runs].copy())


class LayerArrays:
    """Keeps the numpy arrays behind an or_linear table alive."""

    def __init__(self, linears):
        self.keep = []
        self.table = (OrLinear * len(linears))()
        for i, d in enumerate(linears):
            ent = self.table[i]
            if d.get("trellis") is not None:
                t = np.ascontiguousarray(d["trellis"], np.uint16)
                su = np.ascontiguousarray(d["suh"], np.uint16)
                sv = np.ascontiguousarray(d["svh"], np.uint16)
                self.keep += [t, su, sv]
                ent.trellis, ent.suh, ent.svh = t.ctypes.data, su.ctypes.data, sv.ctypes.data
                ent.dense = None
                ent.K, ent.cb = d["K"], d["cb"]
            else:
                w = np.ascontiguousarray(d["dense"], np.uint16)
                self.keep.append(w)
                ent.trellis = None
                ent.dense = w.ctypes.data
                ent.K, ent.cb = 0, 0
            ent.in_, ent.out = d["in"], d["out"]


def moe_layer(cfg: OrMoeCfg, experts, shared, router_w, bias, h, threads=0):
    """experts: list of 3*E dicts (gate, up, down per expert); shared: list of 3 or None."""
    ex = LayerArrays(experts)
    sh = LayerArrays(shared) if shared else None
    h = np.ascontiguousarray(h, np.uint16).reshape(-1, cfg.hidden)
    N = h.shape[0]
    out = np.zeros((N, cfg.hidden), np.uint16)
    idx = np.zeros((N, cfg.top_k), np.int32)
    w = np.zeros((N, cfg.top_k), np.float64)
    rc = lib().or_moe_layer(C.byref(cfg), ex.table, C.cast(sh.table, C.c_void_p) if sh else None,
                            np.ascontiguousarray(router_w, np.uint16).reshape(-1),
                            np.ascontiguousarray(bias, np.float32), h.reshape(-1), N,
                            out.reshape(-1), idx.reshape(-1), w.reshape(-1), _threads(threads))
    if rc:
        raise ValueError("or_moe_layer failed")
    return out, idx, w


def moe_layer_routed(cfg: OrMoeCfg, experts, shared, h, idx, weights, threads=0):
    ex = LayerArrays(experts)
    sh = LayerArrays(shared) if shared else None
    h = np.ascontiguousarray(h, np.uint16).reshape(-1, cfg.hidden)
    N = h.shape[0]
    out = np.zeros((N, cfg.hidden), np.uint16)
    rc = lib().or_moe_layer_routed(C.byref(cfg), ex.table,
                                   C.cast(sh.table, C.c_void_p) if sh else None, h.reshape(-1), N,
                                   np.ascontiguousarray(idx, np.int32).reshape(-1),
                                   np.ascontiguousarray(weights, np.float64).reshape(-1),
                                   out.reshape(-1), _threads(threads))
    if rc:
        raise ValueError("or_moe_layer_routed failed")
    return out


# --- hyper-connections and RMSNorm (glm5_hc.cpp, glm5_attn.cpp:12-22) ----------------------

def hc_prepare(streams, N, D, fn, base, scale, iters, eps):
    """streams: f16 bits (P, N, D). Returns (collapsed f16 bits (P, D), post (P, N), comb (P, N, N))."""
    st = np.ascontiguousarray(streams, np.uint16).reshape(-1)
    P = st.size // (N * D)
    coll = np.zeros((P, D), np.uint16)
    post = np.zeros((P, N), np.float64)
    comb = np.zeros((P, N, N), np.float64)
    lib().or_hc_prepare(st, P, N, D, np.ascontiguousarray(fn, np.float32).reshape(-1),
                        np.ascontiguousarray(base, np.float32), np.ascontiguousarray(scale, np.float32),
                        iters, eps, coll.reshape(-1), post.reshape(-1), comb.reshape(-1))
    return coll, post, comb


def rms_norm(x, w, eps):
    x = np.ascontiguousarray(x, np.uint16)
    P, D = x.shape
    y = np.zeros((P, D), np.uint16)
    lib().or_rms_norm(x.reshape(-1), P, D, np.ascontiguousarray(w, np.uint16), eps, y.reshape(-1))
    return y


def hc_mix(block_out, post, comb, residual):
    b = np.ascontiguousarray(block_out, np.uint16)
    P, D = b.shape
    N = post.shape[1]
    out = np.zeros((P, N, D), np.uint16)
    lib().or_hc_mix(b.reshape(-1), np.ascontiguousarray(post, np.float64).reshape(-1),
                    np.ascontiguousarray(comb, np.float64).reshape(-1),
                    np.ascontiguousarray(residual, np.uint16).reshape(-1), P, N, D, out.reshape(-1))
    return out


# --- the f32 -O3 threaded CPU baseline (oracle/cpu_layer.cpp) -------------------------

_CPU = None


def cpu_lib():
    """oracle/libcpulayer.so: bench.py's CPU baseline of the layer (measurement
    infrastructure; weights and routing bit-identical to the oracle's)."""
    global _CPU
    if _CPU is None:
        lib()  # the baseline links the oracle's routing and tables
        path = os.path.join(_HERE, "libcpulayer.so")
        if not os.path.exists(path):
            raise RuntimeError(f"CPU baseline not built: {path} (run __graft_entry__.build())")
        L = C.CDLL(path)
        L.cpu_decode.argtypes = [u16p, C.c_int64, C.c_int64, C.c_int, C.c_int, u16p, C.c_int]
        L.cpu_router_logits.argtypes = [u16p, C.c_int64, u16p, C.c_int, C.c_int, f64p, C.c_int]
        L.cpu_moe_layer.argtypes = [C.POINTER(OrMoeCfg), C.POINTER(OrLinear), C.c_void_p, u16p,
                                    f32p, u16p, C.c_int64, u16p, i32p, C.c_int]
        _CPU = L
    return _CPU


def cpu_threads():
    """Worker threads for the CPU baseline: the CPUs this process may run on, capped by
    OMP_NUM_THREADS where the host sets it (a GPU box grants one GPU's share of its
    cores that way)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = os.environ.get("OMP_NUM_THREADS")
    return max(1, min(n, int(cap))) if cap and cap.isdigit() else n


def cpu_decode(trellis, in_f, out_f, K, cb, threads=0):
    w = np.zeros((in_f, out_f), np.uint16)
    rc = cpu_lib().cpu_decode(np.ascontiguousarray(trellis, np.uint16).reshape(-1), in_f, out_f, K, cb, w,
                              threads or cpu_threads())
    if rc:
        raise ValueError("cpu_decode: bad geometry")
    return w


def cpu_router_logits(h, router_w, threads=0):
    h = np.ascontiguousarray(h, np.uint16)
    E, H = router_w.shape
    N = h.size // H
    out = np.zeros((N, E), np.float64)
    cpu_lib().cpu_router_logits(h.reshape(-1), N, np.ascontiguousarray(router_w, np.uint16).reshape(-1), E, H,
                                out.reshape(-1), threads or cpu_threads())
    return out


class CpuLayer:
    """A layer's tables for repeated cpu_moe_layer calls (the arrays stay referenced)."""

    def __init__(self, cfg: OrMoeCfg, experts, shared, router_w, bias):
        self.cfg = cfg
        self.ex = LayerArrays(experts)
        self.sh = LayerArrays(shared) if shared else None
        self.router_w = np.ascontiguousarray(router_w, np.uint16).reshape(-1)
        self.bias = np.ascontiguousarray(bias, np.float32)

    def __call__(self, h, threads=0):
        h = np.ascontiguousarray(h, np.uint16).reshape(-1, self.cfg.hidden)
        N = h.shape[0]
        out = np.zeros((N, self.cfg.hidden), np.uint16)
        idx = np.zeros((N, self.cfg.top_k), np.int32)
        rc = cpu_lib().cpu_moe_layer(C.byref(self.cfg), self.ex.table,
                                     C.cast(self.sh.table, C.c_void_p) if self.sh else None, self.router_w,
                                     self.bias, h.reshape(-1), N, out.reshape(-1), idx.reshape(-1),
                                     threads or cpu_threads())
        if rc:
            raise ValueError("cpu_moe_layer failed")
        return out, idx
