"""EXL3 safetensors shards and the MoE layer loader (ctypes binding of exl3_st_* and
exl3_moe_layer_load). Mirrors the reference's SafetensorsFile (safetensors.h:23-70) and
the MoE part of load_glm5 (glm5.cpp:284-376, 503-518)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib, synth
from ._lib import ST_DTYPES, StTensor, call
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
