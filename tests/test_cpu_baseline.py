"""The CPU baseline (oracle/cpu_layer.cpp, timed by bench.py's cpu_baseline leg) against
the oracle: decoded weights and router logits bit-identical, routing identical, and the
layer within the north-star tolerance (max |err| <= 2e-2 * rms, cosine >= 0.9999) -- the
baseline accumulates in f32 where the oracle uses f64."""
import numpy as np
import pytest

from exl3_amd import synth


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_cpu_decode_bit_identical(oracle, K, cb):
    rng = np.random.default_rng(K * 3 + cb)
    t = rng.integers(0, 1 << 16, size=(128 // 16) * (96 // 16) * 16 * K, dtype=np.uint16)
    assert np.array_equal(oracle.cpu_decode(t, 128, 96, K, cb, threads=3),
                          oracle.decode_inner(t, 128, 96, K, cb))


def test_cpu_router_logits_bit_identical(oracle):
    rng = np.random.default_rng(1)
    h = rng.normal(size=(5, 384)).astype(np.float16).view(np.uint16)
    w = (rng.normal(size=(24, 384)) * 0.02).astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.cpu_router_logits(h, w, threads=4), oracle.router_logits(h, w))


def _check(got, want):
    a = got.view(np.float16).astype(np.float64)
    b = want.view(np.float16).astype(np.float64)
    rms = np.sqrt(np.mean(b ** 2))
    assert np.max(np.abs(a - b)) <= 2e-2 * rms
    assert (a * b).sum() / np.sqrt((a ** 2).sum() * (b ** 2).sum()) >= 0.9999


@pytest.mark.parametrize("shared_K", [None, 0, 3])
@pytest.mark.parametrize("B", [1, 6])
def test_cpu_layer_vs_oracle(oracle, shared_K, B):
    cfg = synth.MoeConfig(hidden=256, inter=128, n_experts=12, top_k=3, routed_scaling_factor=2.5,
                          shared_inter=0 if shared_K is None else 128, gate_up_K=4, gate_up_cb=1,
                          down_K=3, down_cb=2, shared_K=shared_K or 0, shared_cb=0)
    layer = synth.make_layer(cfg, 77)
    h = synth.activations(77, f"cpu.{B}", B, cfg.hidden)
    has_shared = layer.shared is not None
    oc = oracle.make_cfg(cfg.hidden, cfg.inter, cfg.n_experts, cfg.top_k, cfg.n_group, cfg.topk_group,
                         cfg.norm_topk_prob, has_shared, cfg.routed_scaling_factor, cfg.swiglu_limit)
    ex = [l.oracle_dict() for l in layer.experts]
    sh = [l.oracle_dict() for l in layer.shared] if has_shared else None
    want, widx, _ = oracle.moe_layer(oc, ex, sh, layer.router_w, layer.bias, h)
    cl = oracle.CpuLayer(oc, ex, sh, layer.router_w, layer.bias)
    for threads in (1, 5):
        got, gidx = cl(h, threads)
        assert np.array_equal(gidx, widx)
        _check(got, want)


def test_cpu_layer_many_rows_per_run(oracle):
    # 40 rows over 4 experts (runs of ~30 rows: the baseline's 16-row accumulator blocks)
    cfg = synth.MoeConfig(hidden=128, inter=128, n_experts=4, top_k=3, routed_scaling_factor=1.5,
                          gate_up_K=3, gate_up_cb=2, down_K=3, down_cb=2, shared_inter=128, shared_K=0)
    layer = synth.make_layer(cfg, 5)
    h = synth.activations(5, "cpu.rows", 40, 128)
    oc = oracle.make_cfg(128, 128, 4, 3, 1, 1, True, True, 1.5, cfg.swiglu_limit)
    ex = [l.oracle_dict() for l in layer.experts]
    sh = [l.oracle_dict() for l in layer.shared]
    want, widx, _ = oracle.moe_layer(oc, ex, sh, layer.router_w, layer.bias, h)
    got, gidx = oracle.CpuLayer(oc, ex, sh, layer.router_w, layer.bias)(h, 4)
    assert np.array_equal(gidx, widx)
    _check(got, want)
