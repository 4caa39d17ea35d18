"""Host mirror of the reference's trellis_gemm.h over the C ABI (torch for device memory).

Names, argument meaning and error behaviour follow src/trellis_gemm.h of
muyouming/exl3-server: TrellisWeight, trellis_pack, trellis_linear, trellis_matmul_raw,
trellis_hadamard, trellis_linear_group{,_rows}{,_scaled}, trellis_set_tuning /
trellis_get_tuning, trellis_path_info. Shape errors raise ValueError (the reference
throws std::invalid_argument); library failures raise Exl3Error.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._lib import PathInfo, TrellisDesc, Tuning, call


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


@dataclass
class TrellisWeight:
    """One EXL3 trellis tensor on the device (trellis_gemm.h:21-48).

    packed: int16 words (in/16, out/16, 16*K) -- the on-disk layout; suh/svh: f16."""
    packed: torch.Tensor
    suh: torch.Tensor
    svh: torch.Tensor
    in_features: int
    out_features: int
    K: int
    codebook: int

    def desc(self) -> TrellisDesc:
        return TrellisDesc(self.packed.data_ptr(), self.suh.data_ptr(), self.svh.data_ptr(),
                           self.in_features, self.out_features, self.K, self.codebook)

    def bytes(self) -> int:
        return self.packed.numel() * 2 + 2 * (self.in_features + self.out_features)

    @property
    def device(self):
        return self.packed.device


def f16_from_bits(bits: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.float16)).to(device)


def trellis_pack(words16: np.ndarray, k_tiles: int, n_tiles: int, K: int,
                 device="cuda") -> torch.Tensor:
    """Copy on-disk words to a fresh device buffer (trellis_gemm.h:64)."""
    w = np.ascontiguousarray(words16, np.uint16).reshape(-1)
    if w.size != k_tiles * n_tiles * 16 * K:
        raise ValueError("trellis_pack: word count does not match the geometry")
    dst = torch.empty((k_tiles, n_tiles, 16 * K), dtype=torch.int16, device=device)
    call("exl3_trellis_pack", w.ctypes.data, k_tiles, n_tiles, K, dst.data_ptr(), _stream())
    return dst


def make_weight(words16, suh_bits, svh_bits, in_f, out_f, K, cb, device="cuda") -> TrellisWeight:
    packed = words16 if isinstance(words16, torch.Tensor) else trellis_pack(
        words16, in_f // 16, out_f // 16, K, device)
    return TrellisWeight(packed, f16_from_bits(suh_bits, device), f16_from_bits(svh_bits, device),
                         in_f, out_f, K, cb)


def _rows(x: torch.Tensor, in_f: int, what: str) -> int:
    if x.dtype != torch.float16 or not x.is_contiguous():
        raise ValueError(f"{what}: x must be a contiguous float16 tensor")
    if x.numel() % in_f:
        raise ValueError(f"{what}: input feature size mismatch")
    return x.numel() // in_f


def trellis_decode(w: TrellisWeight) -> torch.Tensor:
    out = torch.empty((w.in_features, w.out_features), dtype=torch.float16, device=w.device)
    call("exl3_trellis_decode", C.byref(w.desc()), out.data_ptr(), _stream())
    return out


def trellis_reconstruct(w: TrellisWeight) -> torch.Tensor:
    out = torch.empty((w.in_features, w.out_features), dtype=torch.float16, device=w.device)
    call("exl3_trellis_reconstruct", C.byref(w.desc()), out.data_ptr(), _stream())
    return out


def trellis_hadamard(x: torch.Tensor, s: torch.Tensor, pre: bool, stacked: int = 0) -> torch.Tensor:
    """pre: y = f16(H(x*s)/sqrt128) from f16 x; post: y = f16(H(f16(x))/sqrt128*s) from f32 x."""
    n = x.shape[-1]
    rows = x.numel() // n
    y = torch.empty(x.shape, dtype=torch.float16, device=x.device)
    if pre:
        if x.dtype != torch.float16:
            raise ValueError("trellis_hadamard(pre): x must be float16")
        call("exl3_trellis_hadamard", x.data_ptr(), None, rows, n, s.data_ptr(), stacked,
             y.data_ptr(), _stream())
    else:
        if x.dtype != torch.float32:
            raise ValueError("trellis_hadamard(post): x must be float32")
        call("exl3_trellis_hadamard", None, x.data_ptr(), rows, n, s.data_ptr(), stacked,
             y.data_ptr(), _stream())
    return y


def trellis_matmul_raw(w: TrellisWeight, xhat: torch.Tensor) -> torch.Tensor:
    rows = _rows(xhat, w.in_features, "trellis_matmul_raw")
    y = torch.empty((*xhat.shape[:-1], w.out_features), dtype=torch.float32, device=xhat.device)
    d = w.desc()
    ws = _workspace(_lib.lib().exl3_trellis_workspace_size(C.byref(d), rows, 1), xhat.device)
    call("exl3_trellis_matmul_raw", C.byref(d), xhat.data_ptr(), rows, y.data_ptr(),
         ws.data_ptr(), ws.numel(), _stream())
    return y


def trellis_linear(w: TrellisWeight, x: torch.Tensor) -> torch.Tensor:
    """y = x @ W in f16, x (..., in) -> (..., out) (trellis_gemm.h:51)."""
    rows = _rows(x, w.in_features, "trellis_linear")
    y = torch.empty((*x.shape[:-1], w.out_features), dtype=torch.float16, device=x.device)
    d = w.desc()
    ws = _workspace(_lib.lib().exl3_trellis_workspace_size(C.byref(d), rows, 1), x.device)
    call("exl3_trellis_linear", C.byref(d), x.data_ptr(), rows, y.data_ptr(), ws.data_ptr(),
         ws.numel(), _stream())
    return y


def _grouped(ws_list, x, rows, shared, suh_stack=None, svh_stack=None):
    n = len(ws_list)
    if n == 0:
        raise ValueError("trellis_linear_group: no members")
    w0 = ws_list[0]
    for w in ws_list:
        if (w.in_features, w.out_features, w.K, w.codebook) != (
                w0.in_features, w0.out_features, w0.K, w0.codebook):
            raise ValueError("trellis_linear_group: members must share their shape")
    descs = (TrellisDesc * n)(*[w.desc() for w in ws_list])
    y = torch.empty((n, rows, w0.out_features), dtype=torch.float16, device=x.device)
    wsz = _lib.lib().exl3_trellis_workspace_size(C.byref(descs[0]), rows, n)
    ws = _workspace(wsz, x.device)
    call("exl3_trellis_linear_grouped", descs, n, x.data_ptr(), rows, 1 if shared else 0,
         _ptr(suh_stack), _ptr(svh_stack), y.data_ptr(), ws.data_ptr(), ws.numel(), _stream())
    return y


def trellis_linear_group(ws_list, x: torch.Tensor) -> torch.Tensor:
    """n members on one shared (rows, in) activation -> (n, rows, out) (trellis_gemm.h:90)."""
    rows = _rows(x, ws_list[0].in_features, "trellis_linear_group")
    return _grouped(ws_list, x, rows, True)


def trellis_linear_group_rows(ws_list, x: torch.Tensor, rows: int) -> torch.Tensor:
    """x (n, rows, in), one block per member (trellis_gemm.h:91-92)."""
    if x.numel() != len(ws_list) * rows * ws_list[0].in_features:
        raise ValueError("trellis_linear_group_rows: activation size mismatch")
    return _grouped(ws_list, x, rows, False)


def trellis_linear_group_scaled(ws_list, x, suh_stack, svh_stack):
    rows = _rows(x, ws_list[0].in_features, "trellis_linear_group_scaled")
    return _grouped(ws_list, x, rows, True, suh_stack, svh_stack)


def trellis_linear_group_rows_scaled(ws_list, x, rows, suh_stack, svh_stack):
    if x.numel() != len(ws_list) * rows * ws_list[0].in_features:
        raise ValueError("trellis_linear_group_rows_scaled: activation size mismatch")
    return _grouped(ws_list, x, rows, False, suh_stack, svh_stack)


def trellis_set_tuning(rows_per_pass=0, mat_min_rows=16, mat_max_rows=0, weight_form=0) -> None:
    """Process-wide knobs of the single/grouped linear (exl3_set_tuning). weight_form:
    0 = the reference's f16 weights (default), 1 = exact halves (mcg/3inst only)."""
    call("exl3_set_tuning", C.byref(Tuning(rows_per_pass, mat_min_rows, mat_max_rows, weight_form)))


def trellis_get_tuning() -> dict:
    t = Tuning()
    call("exl3_get_tuning", C.byref(t))
    return {k: getattr(t, k) for k, _ in Tuning._fields_}


def trellis_path_info(w: TrellisWeight, rows: int) -> dict:
    info = PathInfo()
    call("exl3_trellis_path_info", C.byref(w.desc()), rows, C.byref(info))
    return {k: getattr(info, k) for k, _ in PathInfo._fields_}
