"""GPU: calls over zero token rows through the C ABI. Every compute entry point
(exl3_moe_layer with B = 0 or L = 0, exl3_moe_route, exl3_moe_topk_route,
exl3_moe_block, exl3_trellis_linear, exl3_trellis_linear_grouped,
exl3_trellis_matmul_raw, exl3_trellis_hadamard, exl3_hc_prepare, exl3_rms_norm,
exl3_hc_mix) returns EXL3_OK and writes nothing: the outputs keep a sentinel. The
workspace queries answer 0 bytes for zero rows, as the header states, and the handles
give the same bytes afterwards as before."""
import ctypes as C

import numpy as np
import pytest
import torch

from exl3_amd import _lib, synth
from exl3_amd.hc import DeviceHcSite, hc_prepare
from exl3_amd.moe import DeviceMoeLayer

pytestmark = pytest.mark.gpu

SENT = 7.0


def sentinel(shape, dtype, dev):
    return torch.full(shape, SENT if dtype.is_floating_point else 7, dtype=dtype, device=dev)


def unchanged(t):
    return bool((t == (SENT if t.dtype.is_floating_point else 7)).all())


def test_zero_row_calls_write_nothing(dev):
    L = _lib.lib()
    cfg = synth.config_small()
    d = DeviceMoeLayer(synth.make_layer(cfg, 71), dev)
    H = cfg.hidden
    x = torch.from_numpy(synth.activations(74, "zr", 4, H).view(np.float16)).to(dev).view(4, 1, H)
    y_before = d(x).clone()
    assert L.exl3_moe_workspace_size(d.handle, 0) == 0

    out = sentinel((4, 1, H), torch.float16, dev)
    ws = torch.empty(d.workspace_bytes(4), dtype=torch.uint8, device=dev)
    for B, Lq in ((0, 1), (1, 0), (0, 0)):
        st = L.exl3_moe_layer(d.handle, x.data_ptr(), B, Lq, out.data_ptr(), ws.data_ptr(), ws.numel(), None)
        assert st == _lib.EXL3_OK, (B, Lq, L.exl3_last_error())
    # no workspace at all is enough for zero rows
    assert L.exl3_moe_layer(d.handle, x.data_ptr(), 0, 1, out.data_ptr(), None, 0, None) == _lib.EXL3_OK

    w = sentinel((4, cfg.top_k), torch.float32, dev)
    ids = sentinel((4, cfg.top_k), torch.int32, dev)
    assert L.exl3_moe_route(d.handle, x.data_ptr(), 0, w.data_ptr(), ids.data_ptr(), ws.data_ptr(),
                            ws.numel(), None) == _lib.EXL3_OK
    logits = torch.zeros(4, cfg.n_experts, device=dev)
    assert L.exl3_moe_topk_route(logits.data_ptr(), d.bias.data_ptr(), 0, C.byref(d._cfg), w.data_ptr(),
                                 ids.data_ptr(), None) == _lib.EXL3_OK

    # the hyper-connection steps and the block
    N = 4
    rng = np.random.default_rng(72)
    W = (2 + N) * N
    site = DeviceHcSite.from_numpy((rng.normal(size=(W, N * H)) / np.sqrt(N * H)).astype(np.float32),
                                   rng.normal(size=W).astype(np.float32), np.array([1.0, 1.0, 1.0], np.float32),
                                   N, 20, 1e-6, dev)
    streams = torch.from_numpy(rng.normal(size=(4, N, H)).astype(np.float16)).to(dev)
    nw = torch.ones(H, dtype=torch.float16, device=dev)
    assert L.exl3_moe_block_workspace_size(d.handle, N, 0) == 0
    s_out = sentinel((4, N, H), torch.float16, dev)
    assert L.exl3_moe_block(d.handle, C.byref(site.desc()), nw.data_ptr(), 1e-5, streams.data_ptr(), 0,
                            s_out.data_ptr(), None, 0, None) == _lib.EXL3_OK
    coll = sentinel((4, H), torch.float16, dev)
    post = sentinel((4, N), torch.float32, dev)
    comb = sentinel((4, N, N), torch.float32, dev)
    assert L.exl3_hc_prepare(C.byref(site.desc()), streams.data_ptr(), 0, H, None, 1e-5, coll.data_ptr(),
                             post.data_ptr(), comb.data_ptr(), None, 0, None) == _lib.EXL3_OK
    assert L.exl3_rms_norm(streams.data_ptr(), 0, H, nw.data_ptr(), 1e-5, coll.data_ptr(), None) == _lib.EXL3_OK
    pf = torch.ones(4, N, device=dev)
    cf = torch.eye(N, device=dev).expand(4, N, N).contiguous()
    assert L.exl3_hc_mix(x.data_ptr(), pf.data_ptr(), cf.data_ptr(), streams.data_ptr(), 0, N, H,
                         s_out.data_ptr(), None) == _lib.EXL3_OK

    # the linear entry points on one expert's gate projection
    tw = d.experts[0].tw
    desc = tw.desc()
    lin_ws = torch.empty(max(1, L.exl3_trellis_workspace_size(C.byref(desc), 4, 2)), dtype=torch.uint8,
                         device=dev)
    y = sentinel((4, cfg.inter), torch.float16, dev)
    assert L.exl3_trellis_linear(C.byref(desc), x.data_ptr(), 0, y.data_ptr(), lin_ws.data_ptr(),
                                 lin_ws.numel(), None) == _lib.EXL3_OK
    yg = sentinel((2, 4, cfg.inter), torch.float16, dev)
    members = (_lib.TrellisDesc * 2)(desc, desc)
    assert L.exl3_trellis_linear_grouped(members, 2, x.data_ptr(), 0, 1, None, None, yg.data_ptr(),
                                         lin_ws.data_ptr(), lin_ws.numel(), None) == _lib.EXL3_OK
    yh = sentinel((4, cfg.inter), torch.float32, dev)
    assert L.exl3_trellis_matmul_raw(C.byref(desc), x.data_ptr(), 0, yh.data_ptr(), lin_ws.data_ptr(),
                                     lin_ws.numel(), None) == _lib.EXL3_OK
    xr = sentinel((4, H), torch.float16, dev)
    assert L.exl3_trellis_hadamard(x.data_ptr(), None, 0, H, tw.suh.data_ptr(), 0, xr.data_ptr(),
                                   None) == _lib.EXL3_OK

    torch.cuda.synchronize()
    for t in (out, w, ids, s_out, coll, post, comb, y, yg, yh, xr):
        assert unchanged(t)
    # the handles work as before
    assert torch.equal(d(x), y_before)
    c1, p1, m1 = hc_prepare(streams, site)
    assert torch.isfinite(c1.float()).all() and torch.isfinite(p1).all() and torch.isfinite(m1).all()
    d.close()
