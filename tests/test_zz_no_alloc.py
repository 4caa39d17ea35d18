"""GPU test of the allocation-free layer entry point (exl3_moe_layer_noalloc), called
through the C ABI: its output equals exl3_moe_layer's (same kernels, so bit for bit) on
two calls in a row, the second with fewer rows than the first, so that the shared scratch
array still holds the first call's contents when the second one runs; a call whose
workspace exceeds the scratch capacity is refused with an error and leaves the output
untouched."""
import ctypes as C

import numpy as np
import pytest
import torch

from exl3_amd import _lib, synth
from exl3_amd._lib import Exl3Error, call
from exl3_amd.moe import DeviceMoeLayer
from exl3_amd.trellis import _stream
from test_gpu_moe import glm5_layer_on_device

pytestmark = pytest.mark.gpu


def noalloc(d, x, B):
    out = torch.empty(B, 1, x.shape[-1], dtype=torch.float16, device=x.device)
    call("exl3_moe_layer_noalloc", d.handle, x.data_ptr(), B, 1, out.data_ptr(), _stream())
    return out


def rows(seed, name, B, H, dev):
    return torch.from_numpy(synth.activations(seed, name, B, H).view(np.float16)).to(dev).view(B, 1, H)


@pytest.mark.parametrize("shared_K", [-1, 0, 3])
def test_noalloc_equals_workspace_call(dev, shared_K):
    # shared_K: -1 none, 0 f16 shared expert, 3 trellis shared expert
    cfg = synth.MoeConfig(hidden=512, inter=256, n_experts=16, top_k=4, routed_scaling_factor=1.5,
                          gate_up_K=4, gate_up_cb=1, down_K=3, down_cb=2,
                          shared_inter=0 if shared_K < 0 else 256, shared_K=max(shared_K, 0), shared_cb=0)
    layer = synth.make_layer(cfg, 91)
    d = DeviceMoeLayer(layer, dev)
    H = cfg.hidden
    cap = _lib.lib().exl3_moe_scratch_capacity()
    assert cap == 32 << 20
    for B in (24, 5):  # second call smaller than the first
        assert d.workspace_bytes(B) <= cap
        x = rows(91, f"noalloc.{shared_K}.{B}", B, H, dev)
        got = noalloc(d, x, B)
        want = d(x)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), B
        assert torch.count_nonzero(want.float()).item() > 0
    d.close()


def test_noalloc_glm5_b8(dev):
    # the GLM-5-shaped decode call (configs[2]'s shape at B=8), twice, then B=3
    layer, words = glm5_layer_on_device(dev, 92, "na")
    cfg = layer.cfg
    d = DeviceMoeLayer(layer, dev, words=words)
    for i, B in enumerate((8, 8, 3)):
        x = rows(92, f"noalloc.glm5.{i}", B, cfg.hidden, dev)
        got = noalloc(d, x, B)
        want = d(x)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (i, B)
    d.close()


def test_noalloc_rejects_beyond_capacity(dev):
    layer, words = glm5_layer_on_device(dev, 93, "nb")
    cfg = layer.cfg
    d = DeviceMoeLayer(layer, dev, words=words)
    cap = _lib.lib().exl3_moe_scratch_capacity()
    B = 31  # the first row count whose GLM-5 workspace exceeds 32 MiB
    assert d.workspace_bytes(30) <= cap < d.workspace_bytes(B)
    x = rows(93, "noalloc.big", B, cfg.hidden, dev)
    out = torch.full((B, 1, cfg.hidden), 7.0, dtype=torch.float16, device=dev)
    with pytest.raises(Exl3Error, match="scratch"):
        call("exl3_moe_layer_noalloc", d.handle, x.data_ptr(), B, 1, out.data_ptr(), _stream())
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)
    # and the largest call that fits still works, bit-identical to the workspace call
    x30 = x[:30].contiguous()
    got = noalloc(d, x30, 30)
    want = d(x30)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    d.close()
