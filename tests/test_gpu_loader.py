"""GPU test of the EXL3 MoE layer loader (exl3_moe_layer_load, exl3_moe_layer_load_block)
on the committed shard fixtures (tests/golden/moe_shard_{a,b,c}.safetensors): trellis
tensors at 4-byte-aligned file positions are used in place and the others repacked on the
device; a loaded layer's output equals, bit for bit, the same layer built from the
generator's arrays (exl3_moe_layer_create), and the oracle within the north-star
tolerance. Layer 1 (shard c) takes the codebook fallback for marker-less tensors (3inst,
glm5.cpp:303) for routed and trellis shared experts, and its MLP sub-block tensors come
back converted as the reference's load_any (glm5.cpp:205-281) does."""
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
SHARD_C = os.path.join(GOLDEN, "moe_shard_c.safetensors")


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


def test_layer1_markerless_3inst_and_trellis_shared(oracle, dev):
    # layer 1 of shard c (the loader also sees shards a and b, holding layer 0's keys):
    # gate/up and the trellis shared expert have no codebook marker, so they load as 3inst
    import dataclasses
    cfg = make_shard.SHARD_CFG_1
    lay = make_shard.layer1()
    loaded = LoadedMoeLayer(SHARDS + [SHARD_C], make_shard.PREFIX_1, cfg, dev)
    built = DeviceMoeLayer(lay, dev)
    # the same tensors read as mcg (the codebook a wrong fallback would pick)
    wrong = dataclasses.replace(cfg, gate_up_cb=synth.CB_MCG, shared_cb=synth.CB_MCG)
    lay_w = synth.make_layer(wrong, make_shard.SHARD_SEED_1, tag="layer1")
    built_w = DeviceMoeLayer(lay_w, dev)
    oc = ocfg_of(oracle, cfg, True)
    for B in (2, 9, 70):
        h = synth.activations(717, f"loader1.x.{B}", B, cfg.hidden)
        x = to_dev(h, dev, B, 1, cfg.hidden)
        y = loaded(x)
        assert torch.equal(y.view(torch.int16), built(x).view(torch.int16)), B
        assert not torch.equal(y.view(torch.int16), built_w(x).view(torch.int16)), B
        _, ids = loaded.route(x)
        idx, w, _ = check_routing(oracle, oracle.router_logits(h, lay.router_w), lay.bias,
                                  ids.cpu().numpy(), oc)
        want = oracle.moe_layer_routed(oc, [l.oracle_dict() for l in lay.experts],
                                       [l.oracle_dict() for l in lay.shared], h, idx, w)
        check_out(y, want)
    for d in (loaded, built, built_w):
        d.close()


def test_block_tensors_load_and_drive_the_block(dev):
    # exl3_moe_layer_load_block: the norm weight (BF16 on disk) to f16 and the hc site
    # (F32 fn, BF16 base, F16 scale) to f32, as load_any converts them; the block run from
    # the loaded tensors equals, bit for bit, the block run from the same values uploaded
    # from numpy
    from exl3_amd.hc import DeviceHcSite, moe_block
    cfg = make_shard.SHARD_CFG_1
    loaded = LoadedMoeLayer([SHARD_C], make_shard.PREFIX_1, cfg, dev)
    blk = loaded.load_block([SHARD_C], make_shard.LAYER_PREFIX_1, make_shard.HC_MULT, 20, 1e-6)
    got = blk.arrays()
    nw_bf, fn, base_bf, scale_f16 = make_shard.block1()
    widen = lambda b: (b.astype(np.uint32) << 16).view(np.float32)  # noqa: E731
    want_nw = widen(nw_bf).astype(np.float16)          # bf16 -> f32 -> f16, one RNE
    want_base = widen(base_bf).astype(np.float16).astype(np.float32)  # through f16
    want_scale = scale_f16.view(np.float16).astype(np.float32)
    assert np.array_equal(got["norm_w"], want_nw.view(np.uint16))
    assert np.array_equal(got["fn"], fn)
    assert np.array_equal(got["base"], want_base) and np.array_equal(got["scale"], want_scale)
    # the subnormal norm values did round: bf16 keeps bits that f16 cannot
    assert not np.array_equal(widen(nw_bf)[[3, 70, 141]], want_nw[[3, 70, 141]].astype(np.float32))
    site = DeviceHcSite.from_numpy(fn, want_base, want_scale, make_shard.HC_MULT, 20, 1e-6, dev)
    nw_t = torch.from_numpy(want_nw).to(dev)
    P, N, D = 9, make_shard.HC_MULT, cfg.hidden
    st = torch.from_numpy(np.random.default_rng(5).normal(size=(P, N, D)).astype(np.float16)).to(dev)
    a = moe_block(loaded, blk, blk.norm_w, 1e-5, st)
    b = moe_block(loaded, site, nw_t, 1e-5, st)
    torch.cuda.synchronize()
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    with pytest.raises(Exl3Error, match="missing tensor"):
        loaded.load_block([SHARD_C], "model.layers.0.", make_shard.HC_MULT)
    with pytest.raises(Exl3Error, match="hc_ffn_fn must be"):
        loaded.load_block([SHARD_C], make_shard.LAYER_PREFIX_1, 2)
    loaded.close()
