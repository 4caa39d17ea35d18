"""Host mirror of the reference's hyper-connection steps around the MoE (glm5_hc.h,
glm5_attn.cpp:12-22, glm5_forward.cpp:434-438) over the C ABI.

hc_prepare(streams, site, norm_w=None) -> (out, post, comb) is g5_hc_prepare (with the
following rms_norm fused when norm_w is given), rms_norm(x, w, eps), hc_mix(block_out,
post, comb, residual) is g5_hc_mix, and moe_block(layer, site, norm_w, eps, streams) is the
MLP sub-block of a GLM-5 MoE layer in one call. All tensors live on the device; there is no
host path.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._lib import HcSite, call
from .trellis import _stream, _workspace


@dataclass
class DeviceHcSite:
    """One hyper-connection site (G5Layer hc_*_fn / hc_*_base / hc_*_scale, glm5.h:79-82)
    on the device: fn (W, mult * hidden) f32 with W = (2 + mult) * mult, base (W), scale (3)."""
    mult: int
    sinkhorn_iters: int
    eps: float
    fn: torch.Tensor
    base: torch.Tensor
    scale: torch.Tensor

    @classmethod
    def from_numpy(cls, fn, base, scale, mult, iters=20, eps=1e-6, device="cuda"):
        dev = torch.device(device)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)  # noqa: E731
        return cls(mult, iters, eps, t(fn), t(base), t(scale))

    @property
    def hidden(self) -> int:
        return self.fn.shape[1] // self.mult

    def desc(self) -> HcSite:
        return HcSite(self.mult, self.sinkhorn_iters, self.eps, self.fn.data_ptr(), self.base.data_ptr(),
                      self.scale.data_ptr())


def _check_streams(streams: torch.Tensor, mult: int) -> tuple[int, int]:
    if streams.dtype != torch.float16 or not streams.is_contiguous() or streams.dim() < 2 or \
            streams.shape[-2] != mult:
        raise ValueError("streams must be a contiguous (..., mult, hidden) float16 tensor")
    D = streams.shape[-1]
    return streams.numel() // (mult * D), D


def hc_prepare(streams: torch.Tensor, site: DeviceHcSite, norm_w: torch.Tensor | None = None,
               norm_eps: float = 1e-5):
    """g5_hc_prepare (glm5_hc.cpp:242-340): streams (..., mult, hidden) f16 -> (out (...,
    hidden) f16, post (..., mult) f32, comb (..., mult, mult) f32); out is the collapsed
    stream, or rms_norm(collapsed) * norm_w when norm_w is given."""
    P, D = _check_streams(streams, site.mult)
    lead = streams.shape[:-2]
    out = torch.empty(lead + (D,), dtype=torch.float16, device=streams.device)
    post = torch.empty(lead + (site.mult,), dtype=torch.float32, device=streams.device)
    comb = torch.empty(lead + (site.mult, site.mult), dtype=torch.float32, device=streams.device)
    ws = _workspace(_lib.lib().exl3_hc_workspace_size(site.mult, D, P), streams.device)
    call("exl3_hc_prepare", C.byref(site.desc()), streams.data_ptr(), P, D,
         None if norm_w is None else norm_w.data_ptr(), norm_eps, out.data_ptr(), post.data_ptr(),
         comb.data_ptr(), ws.data_ptr(), ws.numel(), _stream())
    return out, post, comb


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """rms_norm (glm5_attn.cpp:12-22) over the last axis, f16 in and out."""
    if x.dtype != torch.float16 or not x.is_contiguous():
        raise ValueError("rms_norm: x must be a contiguous float16 tensor")
    D = x.shape[-1]
    y = torch.empty_like(x)
    call("exl3_rms_norm", x.data_ptr(), x.numel() // D, D, w.data_ptr(), eps, y.data_ptr(), _stream())
    return y


def hc_mix(block_out: torch.Tensor, post: torch.Tensor, comb: torch.Tensor,
           residual: torch.Tensor) -> torch.Tensor:
    """g5_hc_mix (glm5_hc.cpp:342-355): (..., hidden) block output and (..., mult, hidden)
    residual streams -> new streams (..., mult, hidden) f16."""
    mult = post.shape[-1]
    P, D = _check_streams(residual, mult)
    if block_out.dtype != torch.float16 or block_out.numel() != P * D or not block_out.is_contiguous():
        raise ValueError("hc_mix: block_out must be a contiguous float16 tensor of P * hidden elements")
    out = torch.empty_like(residual)
    call("exl3_hc_mix", block_out.data_ptr(), post.contiguous().data_ptr(), comb.contiguous().data_ptr(),
         residual.data_ptr(), P, mult, D, out.data_ptr(), _stream())
    return out


def moe_block(layer, site: DeviceHcSite, norm_w: torch.Tensor, norm_eps: float, streams: torch.Tensor,
              out: torch.Tensor | None = None, ws: torch.Tensor | None = None) -> torch.Tensor:
    """glm5_forward.cpp:434-438 for a MoE layer: hc_prepare -> rms_norm -> moe_layer_rows ->
    hc_mix in one call. layer is a DeviceMoeLayer; streams (..., mult, hidden) f16."""
    P, D = _check_streams(streams, site.mult)
    if D != layer.cfg.hidden:
        raise ValueError("moe_block: streams' hidden size differs from the layer's")
    if out is None:
        out = torch.empty_like(streams)
    need = _lib.lib().exl3_moe_block_workspace_size(layer.handle, site.mult, P)
    if ws is None or ws.numel() < need:
        ws = _workspace(need, streams.device)
    call("exl3_moe_block", layer.handle, C.byref(site.desc()), norm_w.data_ptr(), norm_eps,
         streams.data_ptr(), P, out.data_ptr(), ws.data_ptr(), ws.numel(), _stream())
    return out
