"""The layer call under graph capture and from several host threads.

Captured into a HIP graph, the layer call replays to the eager call's bytes.

A caller may capture whole decode steps (the reference's engine runs a layer per MLX
graph evaluation). The layer call is stream-ordered work only: kernel launches, and
in long-run calls with a trellis shared expert an event fork to the layer's second
stream and a join back, with no host synchronisation, allocation or memset. Each
replay runs after eager work of its own on the same layer and is checked bit for
bit against the eager result. Two host threads calling one layer on their own
streams and workspaces get the eager bytes too.
"""
import numpy as np
import pytest
import torch

from exl3_amd import synth
from exl3_amd.moe import DeviceMoeLayer

pytestmark = pytest.mark.gpu


def small_cfg():
    # trellis shared expert, so that 70-row calls fork it onto the layer's second stream
    return synth.MoeConfig(hidden=256, inter=128, n_experts=8, top_k=3, routed_scaling_factor=1.5,
                           gate_up_K=4, gate_up_cb=1, down_K=3, down_cb=2, shared_inter=128,
                           shared_K=3, shared_cb=0)


@pytest.mark.parametrize("B", [8, 40, 70])
def test_layer_graph_replays_equal_eager(dev, B):
    cfg = small_cfg()
    d = DeviceMoeLayer(synth.make_layer(cfg, 21), dev)
    H = cfg.hidden
    x = torch.from_numpy(synth.activations(21, f"graph.{B}", B, H).view(np.float16)).to(dev).view(B, 1, H)
    x2 = torch.from_numpy(synth.activations(22, f"graph2.{B}", B, H).view(np.float16)).to(dev).view(B, 1, H)
    out = torch.empty_like(x)
    ws = torch.empty(d.workspace_bytes(B), dtype=torch.uint8, device=dev)
    eager = d(x, out=out, ws=ws).clone()
    other = d(x2).clone()  # the layer's own workspace, not the captured one
    assert not torch.equal(eager, other)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on a non-default stream before capture
        d(x, out=out, ws=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        d(x, out=out, ws=ws)
    torch.cuda.synchronize()
    for i in range(3):
        out.fill_(0)
        # eager work between replays: a call on other rows, then a sync
        assert torch.equal(d(x2), other), i
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
    del g
    d.close()


def test_layer_two_threads_two_streams(dev):
    # calls on distinct streams with distinct workspaces may run concurrently, from two
    # host threads on one layer handle; at 70 rows both fork the trellis shared expert
    # onto the layer's second stream (the handle's lock orders the forks)
    import threading
    cfg = small_cfg()
    d = DeviceMoeLayer(synth.make_layer(cfg, 31), dev)
    H, B = cfg.hidden, 70
    xs = [torch.from_numpy(synth.activations(31 + t, f"thr.{t}", B, H).view(np.float16)).to(dev).view(B, 1, H)
          for t in range(2)]
    want = [d(x).clone() for x in xs]
    torch.cuda.synchronize()
    got = [[None] * 5 for _ in range(2)]
    errors = []

    def run(t):
        try:
            s = torch.cuda.Stream()
            ws = torch.empty(d.workspace_bytes(B), dtype=torch.uint8, device=dev)
            out = [torch.empty_like(xs[t]) for _ in range(5)]
            with torch.cuda.stream(s):
                for i in range(5):
                    d(xs[t], out=out[i], ws=ws)
            s.synchronize()
            got[t] = out
        except Exception as e:  # reported on the main thread
            errors.append(e)

    th = [threading.Thread(target=run, args=(t,)) for t in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errors, errors
    for t in range(2):
        for i in range(5):
            assert torch.equal(got[t][i], want[t]), (t, i)
    d.close()
