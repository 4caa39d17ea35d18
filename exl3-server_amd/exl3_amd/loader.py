"""EXL3 safetensors shards and the MoE layer loader (ctypes binding of exl3_st_*,
exl3_moe_layer_load and exl3_moe_layer_load_block). Mirrors the reference's
SafetensorsFile (safetensors.h:23-70), the MoE part of load_glm5 (glm5.cpp:284-376,
503-518) and the MLP sub-block's own tensors of load_decoder_layer (glm5.cpp:409-415)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib, synth
from ._lib import HcSite, ST_DTYPES, StTensor, call
from .moe import DeviceMoeLayer, moe_config
from .trellis import _stream

_NP = {"F16": np.uint16, "BF16": np.uint16, "F32": np.float32, "I16": np.int16, "I32": np.int32,
       "U8": np.uint8, "I8": np.int8, "I64": np.int64, "F64": np.float64, "U16": np.uint16,
       "U32": np.uint32, "BOOL": np.bool_}


class Shard:
    """A parsed, mapped safetensors file (host only)."""

    def __init__(self, path: str):
        h = C.c_void_p()
        call("exl3_st_open", path.encode(), C.byref(h))
        self.handle = h
        self.path = path

    @property
    def header_len(self) -> int:
        return _lib.lib().exl3_st_header_len(self.handle)

    def tensors(self) -> dict:
        out = {}
        for i in range(_lib.lib().exl3_st_count(self.handle)):
            t, name = StTensor(), C.c_char_p()
            call("exl3_st_tensor_at", self.handle, i, C.byref(t), C.byref(name))
            out[name.value.decode()] = {"dtype": ST_DTYPES[t.dtype], "shape": tuple(t.shape[:t.ndim]),
                                        "offset": t.offset, "nbytes": t.nbytes,
                                        "file_offset": t.file_offset}
        return out

    def data(self, name: str) -> np.ndarray:
        t = StTensor()
        call("exl3_st_find", self.handle, name.encode(), C.byref(t))
        p = _lib.lib().exl3_st_data(self.handle, name.encode())
        raw = (C.c_uint8 * t.nbytes).from_address(p)
        arr = np.frombuffer(bytes(raw), dtype=_NP[ST_DTYPES[t.dtype]])
        return arr.reshape(tuple(t.shape[:t.ndim]))

    def close(self):
        if self.handle:
            call("exl3_st_close", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class LoadedMoeLayer(DeviceMoeLayer):
    """A MoE layer whose device memory the library loaded from shards (and owns)."""

    def __init__(self, paths, prefix: str, cfg: synth.MoeConfig, device="cuda"):
        self.cfg = cfg
        self.device = torch.device(device)
        self.experts = self.shared = None
        self._cfg = moe_config(cfg)
        arr = (C.c_char_p * len(paths))(*[p.encode() for p in paths])
        h = C.c_void_p()
        with torch.cuda.device(self.device):
            call("exl3_moe_layer_load", arr, len(paths), prefix.encode(), C.byref(self._cfg), C.byref(h),
                 _stream())
        self.handle = h
        self._ws = None

    def load_info(self) -> dict:
        a, b = C.c_int64(), C.c_int64()
        call("exl3_moe_layer_load_info", self.handle, C.byref(a), C.byref(b))
        return {"in_place": a.value, "repacked": b.value}

    def load_block(self, paths, layer_prefix: str, mult: int, sinkhorn_iters: int = 20,
                   eps: float = 1e-6) -> "LoadedBlock":
        """The MLP sub-block's own tensors of this layer's decoder layer
        (exl3_moe_layer_load_block): post_attention_layernorm.weight and hc_ffn_*, held by
        this layer's handle."""
        arr = (C.c_char_p * len(paths))(*[p.encode() for p in paths])
        site = HcSite(mult, sinkhorn_iters, eps, None, None, None)
        nw = C.c_void_p()
        with torch.cuda.device(self.device):
            call("exl3_moe_layer_load_block", self.handle, arr, len(paths), layer_prefix.encode(),
                 C.byref(site), C.byref(nw), _stream())
        return LoadedBlock(site, nw.value, self.cfg.hidden)


class _DevicePtr:
    """A device address the library owns, in the form the bindings read (data_ptr())."""

    def __init__(self, p: int):
        self.p = p

    def data_ptr(self) -> int:
        return self.p


class LoadedBlock:
    """A hyper-connection site and RMSNorm weight loaded into layer-owned device memory:
    the block itself goes to exl3_amd.hc.moe_block / hc_prepare in place of a DeviceHcSite,
    and `norm_w` in place of a norm weight tensor."""

    def __init__(self, site: HcSite, norm_w: int, hidden: int):
        self._site = site
        self.mult, self.sinkhorn_iters, self.eps = site.mult, site.sinkhorn_iters, site.eps
        self.hidden = hidden
        self.norm_w = _DevicePtr(norm_w)

    def desc(self) -> HcSite:
        return self._site

    def arrays(self) -> dict:
        """Host copies of the loaded tensors: fn, base, scale (f32) and norm_w (f16 bits)."""
        # the HIP runtime the library itself links (its own allocations): dlsym through the
        # library's handle resolves the symbol in its dependencies
        hip = C.CDLL(_lib.lib()._name)
        hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        hip.hipMemcpy.restype = C.c_int
        torch.cuda.synchronize()
        N, D = self.mult, self.hidden
        W = (2 + N) * N

        def get(ptr, n, dt):
            out = np.empty(n, dt)
            if hip.hipMemcpy(out.ctypes.data, ptr, out.nbytes, 2) != 0:  # device to host
                raise RuntimeError("hipMemcpy failed")
            return out
        return {"fn": get(self._site.fn, W * N * D, np.float32).reshape(W, N * D),
                "base": get(self._site.base, W, np.float32), "scale": get(self._site.scale, 3, np.float32),
                "norm_w": get(self.norm_w.p, D, np.uint16)}
