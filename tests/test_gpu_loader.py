"""GPU test of the EXL3 MoE layer loader (exl3_moe_layer_load) on the committed
two-shard fixture (tests/golden/moe_shard_{a,b}.safetensors): trellis tensors at
4-byte-aligned file positions are used in place and the others repacked on the device;
the loaded layer's output equals, bit for bit, the same layer built from the generator's
arrays (exl3_moe_layer_create), and the oracle within the north-star tolerance."""
import os
import sys

import numpy as np
import pytest
import torch

from exl3_amd._lib import Exl3Error
from exl3_amd.loader import LoadedMoeLayer, Shard
from exl3_amd.moe import DeviceMoeLayer
from exl3_amd import synth
from test_gpu_moe import check_out, check_routing, ocfg_of, to_dev

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_shard  # noqa: E402

SHARDS = [os.path.join(GOLDEN, f"moe_shard_{x}.safetensors") for x in "ab"]


def test_loaded_layer_equals_built_layer_and_oracle(oracle, dev):
    cfg = make_shard.SHARD_CFG
    lay = make_shard.layer()
    loaded = LoadedMoeLayer(SHARDS, make_shard.PREFIX, cfg, dev)
    # in place exactly where the file position is 4-byte aligned
    aligned = 0
    total = 0
    for p in SHARDS:
        s = Shard(p)
        for name, t in s.tensors().items():
            if name.endswith(".trellis"):
                total += 1
                aligned += t["file_offset"] % 4 == 0
        s.close()
    info = loaded.load_info()
    assert info == {"in_place": aligned, "repacked": total - aligned}
    assert 0 < aligned < total
    built = DeviceMoeLayer(lay, dev)
    oc = ocfg_of(oracle, cfg, True)
    for B in (1, 5, 17):
        h = synth.activations(707, f"loader.x.{B}", B, cfg.hidden)
        x = to_dev(h, dev, B, 1, cfg.hidden)
        y = loaded(x)
        yb = built(x)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), yb.view(torch.int16)), B
        _, ids = loaded.route(x)
        logits = oracle.router_logits(h, lay.router_w)
        idx, w, _ = check_routing(oracle, logits, lay.bias, ids.cpu().numpy(), oc)
        want = oracle.moe_layer_routed(oc, [l.oracle_dict() for l in lay.experts],
                                       [l.oracle_dict() for l in lay.shared], h, idx, w)
        check_out(y, want)
    loaded.close()
    built.close()


def test_loader_errors(dev):
    cfg = make_shard.SHARD_CFG
    with pytest.raises(Exl3Error, match="missing linear"):
        LoadedMoeLayer(SHARDS[:1], make_shard.PREFIX, cfg, dev)  # experts 3-5 are in shard b
    with pytest.raises(Exl3Error, match="missing linear model.layers.1.mlp.experts.0.gate_proj"):
        LoadedMoeLayer(SHARDS, "model.layers.1.mlp.", cfg, dev)
    with pytest.raises(Exl3Error, match="cannot open"):
        LoadedMoeLayer(SHARDS + ["/nonexistent.safetensors"], make_shard.PREFIX, cfg, dev)
