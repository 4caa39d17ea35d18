"""Host mirror of the reference's glm5_moe.h over the C ABI.

moe_topk_route(logits, bias, n_group, topk_group, top_k, norm_topk_prob,
routed_scaling_factor) and a device-resident layer (DeviceMoeLayer) whose __call__ is
moe_layer / moe_layer_rows: h (B, L, hidden) f16 -> (B, L, hidden) f16, with routing,
dispatch and every expert launch on the device. MoeRowsDiag is exposed as diag().
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib, synth
from ._lib import LinearDesc, MoeConfig, MoeDiag, MoeLayerDesc, MoeTiming, TrellisDesc, Tuning, call
from .trellis import TrellisWeight, _stream, _workspace, f16_from_bits


def moe_config(cfg: synth.MoeConfig) -> MoeConfig:
    return MoeConfig(cfg.hidden, cfg.inter, cfg.n_experts, cfg.top_k, cfg.n_group,
                     cfg.topk_group, int(cfg.norm_topk_prob), cfg.routed_scaling_factor,
                     cfg.swiglu_limit)


def moe_topk_route(logits: torch.Tensor, bias: torch.Tensor, n_group: int, topk_group: int,
                   top_k: int, norm_topk_prob: bool, routed_scaling_factor: float):
    """Returns (weights (N, top_k) f32, indices (N, top_k) i32) (glm5_moe.h:29-31)."""
    if logits.dtype != torch.float32 or logits.dim() != 2:
        raise ValueError("moe_topk_route: logits must be (N, E) float32")
    N, E = logits.shape
    cfg = MoeConfig(0, 0, E, top_k, n_group, topk_group, int(norm_topk_prob),
                    routed_scaling_factor, 0.0)
    w = torch.empty((N, top_k), dtype=torch.float32, device=logits.device)
    ids = torch.empty((N, top_k), dtype=torch.int32, device=logits.device)
    call("exl3_moe_topk_route", logits.contiguous().data_ptr(),
         bias.to(torch.float32).contiguous().data_ptr(), N, C.byref(cfg), w.data_ptr(),
         ids.data_ptr(), _stream())
    return w, ids


# --- on-device synthetic tensors (same splitmix64 stream as synth.u64_stream) ----------

def _s64(v: int) -> int:
    v &= 0xFFFFFFFFFFFFFFFF
    return v - (1 << 64) if v >= (1 << 63) else v


_GAMMA = _s64(0x9E3779B97F4A7C15)
_M1 = _s64(0xBF58476D1CE4E5B9)
_M2 = _s64(0x94D049BB133111EB)


def _lsr(z: torch.Tensor, n: int) -> torch.Tensor:
    return (z >> n) & ((1 << (64 - n)) - 1)


def u64_stream_torch(key: int, n: int, device) -> torch.Tensor:
    i = torch.arange(1, n + 1, dtype=torch.int64, device=device)
    z = i * _GAMMA + _s64(key)
    z = (z ^ _lsr(z, 30)) * _M1
    z = (z ^ _lsr(z, 27)) * _M2
    return z ^ _lsr(z, 31)


def trellis_words_torch(seed: int, name: str, in_f: int, out_f: int, K: int,
                        device) -> torch.Tensor:
    """Device int16 words, bit-identical to synth.trellis_words (uniform random int16)."""
    n = (in_f // 16) * (out_f // 16) * 16 * K
    out = torch.empty(n, dtype=torch.int16, device=device)
    key = synth.tensor_key(seed, name)
    chunk = 1 << 26
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        i = torch.arange(s + 1, s + m + 1, dtype=torch.int64, device=device)
        z = i * _GAMMA + _s64(key)
        z = (z ^ _lsr(z, 30)) * _M1
        z = (z ^ _lsr(z, 27)) * _M2
        z = z ^ _lsr(z, 31)
        out[s:s + m] = (_lsr(z, 48) - ((_lsr(z, 48) >> 15) << 16)).to(torch.int16)
    return out.view(in_f // 16, out_f // 16, 16 * K)


class DeviceLinear:
    def __init__(self, lin: synth.Linear, device, words: torch.Tensor | None = None):
        self.in_f, self.out_f = lin.in_f, lin.out_f
        self.dense = None
        self.tw = None
        if lin.quantized or words is not None:
            packed = words
            if packed is None:
                packed = torch.from_numpy(lin.trellis.view(np.int16)).to(device)
            self.tw = TrellisWeight(packed, f16_from_bits(lin.suh, device),
                                    f16_from_bits(lin.svh, device), lin.in_f, lin.out_f, lin.K,
                                    lin.cb)
        else:
            self.dense = f16_from_bits(lin.dense, device)

    def desc(self) -> LinearDesc:
        d = LinearDesc()
        if self.tw is not None:
            d.tw = self.tw.desc()
            d.dense = None
        else:
            d.tw = TrellisDesc()
            d.dense = self.dense.data_ptr()
        d.in_features, d.out_features = self.in_f, self.out_f
        return d


class DeviceMoeLayer:
    """A layer's tensors on the device plus its library handle (G5Layer + G5MoePrep)."""

    def __init__(self, layer: synth.MoeLayer, device="cuda", words=None):
        """words: optional {expert linear index: device int16 words} overriding
        layer.experts[i].trellis (used for full-size layers generated on the device)."""
        self.cfg = layer.cfg
        self.device = torch.device(device)
        words = words or {}
        self.experts = [DeviceLinear(l, self.device, words.get(i))
                        for i, l in enumerate(layer.experts)]
        self.shared = None
        if layer.shared is not None:
            self.shared = [DeviceLinear(l, self.device, words.get(("shared", j)))
                           for j, l in enumerate(layer.shared)]
        self.router_w = f16_from_bits(layer.router_w, self.device)
        self.bias = torch.from_numpy(np.ascontiguousarray(layer.bias, np.float32)).to(self.device)
        ex = (LinearDesc * len(self.experts))(*[l.desc() for l in self.experts])
        sh = (LinearDesc * 3)(*[l.desc() for l in self.shared]) if self.shared else None
        desc = MoeLayerDesc(ex, sh, self.router_w.data_ptr(), self.bias.data_ptr())
        self._cfg = moe_config(self.cfg)
        h = C.c_void_p()
        call("exl3_moe_layer_create", C.byref(desc), C.byref(self._cfg), C.byref(h))
        self.handle = h
        self._ws = None

    def close(self):
        if self.handle:
            call("exl3_moe_layer_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def workspace_bytes(self, rows: int) -> int:
        return _lib.lib().exl3_moe_workspace_size(self.handle, rows)

    def workspace(self, rows: int) -> torch.Tensor:
        need = self.workspace_bytes(rows)
        if self._ws is None or self._ws.numel() < need:
            self._ws = _workspace(need, self.device)
        return self._ws

    def __call__(self, h: torch.Tensor, out: torch.Tensor | None = None,
                 ws: torch.Tensor | None = None) -> torch.Tensor:
        if h.dtype != torch.float16 or h.shape[-1] != self.cfg.hidden or not h.is_contiguous():
            raise ValueError("moe_layer: h must be a contiguous (B, L, hidden) float16 tensor")
        B = h.shape[0] if h.dim() >= 2 else 1
        L = h.numel() // (B * self.cfg.hidden)
        if out is None:
            out = torch.empty_like(h)
        ws = self.workspace(B * L) if ws is None else ws
        call("exl3_moe_layer", self.handle, h.data_ptr(), B, L, out.data_ptr(), ws.data_ptr(),
             ws.numel(), _stream())
        return out

    def route(self, h: torch.Tensor):
        rows = h.numel() // self.cfg.hidden
        w = torch.empty((rows, self.cfg.top_k), dtype=torch.float32, device=h.device)
        ids = torch.empty((rows, self.cfg.top_k), dtype=torch.int32, device=h.device)
        ws = self.workspace(rows)
        call("exl3_moe_route", self.handle, h.data_ptr(), rows, w.data_ptr(), ids.data_ptr(),
             ws.data_ptr(), ws.numel(), _stream())
        return w, ids

    def timing_enable(self, on=True):
        call("exl3_moe_timing_enable", self.handle, 1 if on else 0)

    def timing_reset(self):
        call("exl3_moe_timing_reset", self.handle)

    def timing(self) -> dict:
        t = MoeTiming()
        call("exl3_moe_timing_get", self.handle, C.byref(t))
        return {k: getattr(t, k) for k, _ in MoeTiming._fields_}

    def set_tuning(self, rows_per_pass=0, mat_min_rows=16, mat_max_rows=0, weight_form=0):
        """This handle's tuning knobs (exl3_moe_set_tuning). Only weight_form moves output
        bits: 0 = the reference's f16 weights (default), 1 = exact halves (mcg/3inst)."""
        call("exl3_moe_set_tuning", self.handle,
             C.byref(Tuning(rows_per_pass, mat_min_rows, mat_max_rows, weight_form)))

    def tuning(self) -> dict:
        t = Tuning()
        call("exl3_moe_get_tuning", self.handle, C.byref(t))
        return {k: getattr(t, k) for k, _ in Tuning._fields_}

    def diag_enable(self, on=True):
        call("exl3_moe_diag_enable", self.handle, 1 if on else 0)

    def diag_reset(self):
        call("exl3_moe_diag_reset", self.handle)

    def diag(self) -> dict:
        d = MoeDiag()
        call("exl3_moe_diag_get", self.handle, C.byref(d))
        out = {k: getattr(d, k) for k, _ in MoeDiag._fields_ if k != "run_hist"}
        out["run_hist"] = {r: int(d.run_hist[r]) for r in range(65) if d.run_hist[r]}
        return out
