#!/usr/bin/env python3
"""bench.py -- EXL3 MoE decode layer on one MI355X.

Metric: MoE-layer decode tokens/s + achieved HBM GB/s on trellis bytes,
B=8, 1 MI355X. Workload: GLM-5-shaped layer -- hidden 4096, expert
intermediate 1024, 288 experts, top-8 sigmoid routing with a selection-only correction
bias, routed_scaling_factor 2.5, swiglu_limit 10, gate/up K4 mcg, down K5 mcg, fp16
shared expert (intermediate 1024). Seeded synthetic weights and N(0,1) activations.

A step is one full layer call (router, dispatch, routed experts, shared expert,
combine) on one batch of 8 token rows. Steps rotate over --layers distinct layer
instances (default 8, ~15.7 GB of trellis) with their own inputs, so consecutive steps
stream different experts and the 256 MB MALL cannot serve a repeated working set.

--workload picks the run: glm5_moe_decode_b8 (the default and the metric's workload),
glm5_moe_decode_b1..b4 (the same layer at 1-4 rows: decode and the multi-row verify /
MTP regime), glm5_moe_staged_b64 (configs[3]: 48 identical rows + 16 independent rows,
B=64), glm5_moe_prefill_2048 (configs[4]: 2048 rows, gate/up K4 3inst, down K5 mul1, K6
mcg shared expert, 8 hot experts taking about a quarter of the selections), small_b1
(configs[0]: hidden 512, 16 experts, top-2, K4 mcg, one row) or trellis_linear
(configs[1]).

Clock settle: before its W warmup steps, each run keeps the GPU busy with untimed
steps of the same workload for --settle-ms (default 300 ms; reported in the line as
`settle`). MI355X raises its clocks over the first ~100-200 ms of sustained load: at
W=5 and K=20 right after the layers are built, a B=8 step measured ~0.14 ms, against
~0.12 ms for the same 20 steps once the clocks have settled. The timed region is still
exactly K full steps.

Output: one JSON line. `value` = 8 rows / (wall time per step) with inputs resident in
HBM. `roofline` = the routed gate|up kernel (the dominant kernel): algorithmic trellis
bytes of the distinct experts it streams per launch / its average launch time (HIP
events on the call's stream). `cpu_baseline` (glm5_moe_decode_b8 and small_b1) = the
f32 -O3 CPU restatement of the same layer (oracle/cpu_layer.cpp: on-the-fly table
decode, AVX2/FMA, one worker per CPU granted to the process; routing and decoded
weights checked bit-identical to the oracle first), median of timed calls after
warm-up on a bounded sample of the same workload, plus one call on one thread.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "exl3-server_amd"))

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16 matrix peak
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "moe_decode_glm5_b8_traffic.md")


def settle(step, ms):
    """Untimed steps of the workload until `ms` of wall time has passed (checked every 16
    steps, each check waits for the GPU): the clocks reach their sustained level before
    the warmup and the timed steps. Returns {"ms": elapsed, "steps": steps run}."""
    import torch
    n, t0 = 0, time.perf_counter()
    while ms > 0:
        for _ in range(16):
            step(n)
            n += 1
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= ms:
            break
    return {"ms": round((time.perf_counter() - t0) * 1e3, 1), "steps": n}


def measured_traffic(kernel):
    """HBM bytes per dispatch of `kernel` (FETCH_SIZE + WRITE_SIZE, copy-calibrated) from the
    committed rocprofv3 counter summary of this same workload, or None."""
    import re
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    m = re.search(rf"^{kernel} HBM bytes per dispatch \(read \+ write\): (\d+)$", text, re.M)
    return int(m.group(1)) if m else None


WORKLOADS = {
    # name: (synth config, token rows per step, description)
    "glm5_moe_decode_b8": ("glm5", 8, "configs[2]: GLM-5-shaped layer, decode batch 8"),
    **{f"glm5_moe_decode_b{b}": ("glm5", b, f"configs[2]'s layer at B={b}: decode (1) and the multi-row "
                                            "verify / MTP regime (2-4)") for b in (1, 2, 3, 4)},
    "glm5_moe_staged_b64": ("glm5", 64, "configs[3]: 48 identical rows + 16 independent rows"),
    "glm5_moe_prefill_2048": ("prefill", 2048, "configs[4]: 2048-token prefill, gate/up K4 3inst, "
                                               "down K5 mul1, shared K6 mcg, 8 hot experts"),
    "small_b1": ("small", 1, "configs[0]: small EXL3 MoE layer (hidden 512, 16 experts, top-2, K4 mcg), "
                             "batch-1 decode"),
    "glm5_moe_block_b8": ("block", 8, "the MLP sub-block of the B=8 layer: hyper-connection prepare (4 streams), "
                                      "RMSNorm, the MoE, hyper-connection mix"),
    "trellis_linear": ("linear", 1, "configs[1]: one trellis linear at rows=1 (in 4096), K=1..8 x 3 codebooks"),
}


def bench_linear(args):
    """exl3_trellis_linear at rows = 1: in 4096 x out 24576 (the reference's headline GEMV
    shape, perf.md:75) at K=4 mcg is the line's value, plus the K=1..8 x {3inst, mcg, mul1}
    sweep at 4096 x 4096. Each shape rotates over enough distinct copies
    (>= 512 MB) that the MALL cannot serve them; the time is HIP events around the timed
    calls."""
    import ctypes as C
    import numpy as np
    import torch
    from exl3_amd import synth
    from exl3_amd.moe import trellis_words_torch
    from exl3_amd.trellis import TrellisWeight, f16_from_bits, call, _lib

    dev = torch.device("cuda:0")

    def run(in_f, out_f, K, steps, warmup, cb=1, settle_ms=50.0):
        nbytes = in_f * out_f // 256 * 32 * K
        copies = max(2, -(-(512 << 20) // nbytes))
        su = f16_from_bits(synth.normal_f16(1, "lin.suh", (in_f,), 1.0, 0.05), dev)
        sv = f16_from_bits(synth.normal_f16(1, "lin.svh", (out_f,), 1.0, 0.05), dev)
        ws = [TrellisWeight(trellis_words_torch(args.seed, f"lin.{K}.{i}", in_f, out_f, K, dev), su, sv,
                            in_f, out_f, K, cb) for i in range(copies)]
        x = torch.from_numpy(synth.activations(1, "lin.x", 1, in_f).view(np.float16)).to(dev)
        y = torch.empty((1, out_f), dtype=torch.float16, device=dev)
        d0 = ws[0].desc()
        wsb = torch.empty(max(256, int(_lib.lib().exl3_trellis_workspace_size(C.byref(d0), 1, 1))),
                          dtype=torch.uint8, device=dev)
        descs = [w.desc() for w in ws]
        st = torch.cuda.current_stream().cuda_stream

        def step(i):
            call("exl3_trellis_linear", C.byref(descs[i % copies]), x.data_ptr(), 1, y.data_ptr(),
                 wsb.data_ptr(), wsb.numel(), st)
        settled = settle(step, min(settle_ms, args.settle_ms))
        for i in range(warmup):
            step(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            step(i)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        del ws
        torch.cuda.empty_cache()
        run.settled = settled
        return ms, nbytes / (ms * 1e-3) / 1e9

    steps = args.steps if args.steps is not None else 400
    warmup = args.warmup if args.warmup is not None else 40
    ms, gbps = run(4096, 24576, 4, steps, warmup, settle_ms=args.settle_ms)
    settled = run.settled
    # the reference's headline tensor classes (tests/glm5_gemv_nt_test.cpp:147-171) at rows = 1
    classes = {}
    for name, (i_f, o_f, K, cb) in (("lm_head 4096x154880 K6 mcg", (4096, 154880, 6, 1)),
                                    ("kda qkv 4096x24576 K4 mul1", (4096, 24576, 4, 2)),
                                    ("mla o_proj 16384x4096 K6 mcg", (16384, 4096, 6, 1)),
                                    ("kda o_proj 8192x4096 K4 mcg", (8192, 4096, 4, 1)),
                                    ("expert gate 4096x2048 K3 mul1", (4096, 2048, 3, 2)),
                                    ("expert gate 4096x2048 K2 mul1", (4096, 2048, 2, 2))):
        kms, kg = run(i_f, o_f, K, max(50, steps // 4), max(5, warmup // 4), cb)
        classes[name] = {"ms": round(kms, 5), "GBps": round(kg, 1)}
    sweep = {}
    for cb, name in ((0, "3inst"), (1, "mcg"), (2, "mul1")):
        for K in range(1, 9):
            kms, kg = run(4096, 4096, K, steps, warmup, cb)
            sweep[f"{name}_K{K}"] = {"ms": round(kms, 5), "GBps": round(kg, 1)}
    line = {
        "metric": "trellis linear GB/s on trellis bytes, rows=1, 1 MI355X", "value": round(gbps, 1),
        "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup, "settle": settled,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "trellis_linear", "in": 4096, "out": 24576, "K": 4, "codebook": "mcg",
                   "rows": 1, "weight_form": args.weight_form, "parallelism": "none (one GPU)"},
        "roofline": {"kernel": "exl3_trellis_linear (QMV with the input Hadamard, finalize)", "bound": "hbm",
                     "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None},
        "sweep_4096x4096": sweep, "classes_rows1": classes, "cpu_baseline": None,
    }
    print(json.dumps(line))
HOT_BIAS = 0.23  # bias tilt that sends about a quarter of the selections to 8 hot experts


VALU_PROFILE = os.path.join(ROOT, "profiles", "moe_decode_glm5_b8_valu.md")


def bench_block(args):
    """exl3_moe_block at B=8 on the GLM-5 layer (glm5_forward.cpp:434-438): g5_hc_prepare of
    4 residual streams (RMS over 16384 values, 24 projections, 20 Sinkhorn iterations) with
    the RMSNorm fused, the MoE layer, and g5_hc_mix fused into its combine; seeded synthetic
    hyper-connection weights. The same layer instances' plain exl3_moe_layer calls are
    timed in the same run, so hc_overhead_ms is what the steps either side cost."""
    import numpy as np
    import torch
    from exl3_amd import synth
    from exl3_amd.hc import DeviceHcSite, moe_block

    steps = args.steps if args.steps is not None else 400
    warmup = args.warmup if args.warmup is not None else 40
    n_layers = args.layers if args.layers is not None else 8
    dev = torch.device("cuda:0")
    cfg, layers = build_layers(n_layers, args.seed, dev, "glm5")
    for _, _, d in layers:
        d.set_tuning(weight_form=1 if args.weight_form == "halves" else 0)
    H, B, NS = cfg.hidden, 8, 4
    rng = np.random.default_rng(args.seed)
    W = (2 + NS) * NS
    sites, norms, streams, outs, wss, xs, ys = [], [], [], [], [], [], []
    for li, (_, _, d) in enumerate(layers):
        fn = (rng.normal(size=(W, NS * H)) / np.sqrt(NS * H)).astype(np.float32)
        base = (rng.normal(size=W) * 0.5).astype(np.float32)
        sites.append(DeviceHcSite.from_numpy(fn, base, np.ones(3, np.float32), NS, 20, 1e-6, dev))
        norms.append(torch.from_numpy(rng.normal(1.0, 0.05, H).astype(np.float16)).to(dev))
        streams.append(torch.from_numpy(rng.normal(size=(B, NS, H)).astype(np.float16)).to(dev))
        outs.append(torch.empty_like(streams[-1]))
        wss.append(torch.empty(max(256, d.workspace_bytes(B) * 2 + (64 << 20)), dtype=torch.uint8, device=dev))
        xs.append(streams[-1][:, 0].contiguous().view(B, 1, H))
        ys.append(torch.empty_like(xs[-1]))

    def block(i):
        li = i % n_layers
        moe_block(layers[li][2], sites[li], norms[li], 1e-5, streams[li], out=outs[li], ws=wss[li])

    def layer(i):
        li = i % n_layers
        layers[li][2](xs[li], out=ys[li], ws=wss[li])

    settled = []

    def timed(fn):
        settled.append(settle(fn, args.settle_ms if not settled else min(50.0, args.settle_ms)))
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        t = time.perf_counter()
        for i in range(steps):
            fn(i)
        torch.cuda.synchronize()
        return (time.perf_counter() - t) * 1e3 / steps

    block_ms = timed(block)
    layer_ms = timed(layer)
    block_ms2 = timed(block)
    ms = min(block_ms, block_ms2)
    line = {
        "metric": "MoE MLP sub-block tokens/s (hc prepare + RMSNorm + MoE + hc mix), B=8, 1 MI355X",
        "value": round(B / (ms / 1e3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "settle": settled[0],
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "glm5_moe_block_b8", "batch": B, "hidden": H, "hc_mult": NS, "sinkhorn_iters": 20,
                   "experts": cfg.n_experts, "top_k": cfg.top_k, "layer_instances": n_layers,
                   "parallelism": "none (one GPU)"},
        "layer_only_ms_per_step": round(layer_ms, 5),
        "hc_overhead_ms": round(ms - layer_ms, 5),
        "roofline": None, "cpu_baseline": None,
    }
    for _, _, d in layers:
        d.close()
    print(json.dumps(line))


def profiled_valu_busy(kernel):
    """VALU issue fraction of `kernel` from the committed rocprofv3 counter summary of
    the B=8 decode workload (the expert kernels are bound by decode VALU, not HBM), or None."""
    import re
    try:
        text = open(VALU_PROFILE).read()
    except OSError:
        return None
    m = re.search(rf"^{kernel} VALU busy: ([0-9.]+)$", text, re.M)
    return float(m.group(1)) if m else None


def build_layers(n_layers, seed, device, kind="glm5"):
    import numpy as np  # noqa: F401
    from exl3_amd import synth
    from exl3_amd.moe import DeviceMoeLayer, trellis_words_torch

    if kind == "small":
        cfg = synth.config_small()
        layers = [synth.make_layer(cfg, seed + li, f"bench.small{li}") for li in range(n_layers)]
        return cfg, [(layer, {}, DeviceMoeLayer(layer, device)) for layer in layers]
    cfg = synth.config_glm5() if kind == "glm5" else synth.config_prefill()
    H, I, E = cfg.hidden, cfg.inter, cfg.n_experts
    hot = list(range(0, E, E // 8)) if kind == "prefill" else []
    out = []
    for li in range(n_layers):
        tag = f"bench.layer{li}"
        bias = synth.normal_f32(seed, f"{tag}.gate.e_score_correction_bias", (E,), 0, cfg.bias_std)
        if hot:
            bias = bias.copy()
            bias[hot] += np.float32(HOT_BIAS)
        layer = synth.MoeLayer(cfg, [], None,
                               synth.normal_f16(seed, f"{tag}.gate.weight", (E, H), 0, cfg.router_std),
                               bias)
        words = {}
        for e in range(E):
            for j, (nm, i_f, o_f, K, cb) in enumerate((("gate_proj", H, I, cfg.gate_up_K, cfg.gate_up_cb),
                                                       ("up_proj", H, I, cfg.gate_up_K, cfg.gate_up_cb),
                                                       ("down_proj", I, H, cfg.down_K, cfg.down_cb))):
                p = f"{tag}.experts.{e}.{nm}"
                layer.experts.append(synth.Linear(
                    i_f, o_f, suh=synth.normal_f16(seed, p + ".suh", (i_f,), 1, 0.05),
                    svh=synth.normal_f16(seed, p + ".svh", (o_f,), 1, 0.05), K=K, cb=cb))
                words[3 * e + j] = trellis_words_torch(seed, p + ".trellis", i_f, o_f, K, device)
        SI = cfg.shared_inter
        dims = ((f"{tag}.shared_experts.gate_proj", H, SI), (f"{tag}.shared_experts.up_proj", H, SI),
                (f"{tag}.shared_experts.down_proj", SI, H))
        if cfg.shared_K == 0:
            layer.shared = [synth.make_dense_linear(seed, p, i_f, o_f) for p, i_f, o_f in dims]
        else:
            layer.shared = []
            for j, (p, i_f, o_f) in enumerate(dims):
                layer.shared.append(synth.Linear(
                    i_f, o_f, suh=synth.normal_f16(seed, p + ".suh", (i_f,), 1, 0.05),
                    svh=synth.normal_f16(seed, p + ".svh", (o_f,), 1, 0.05), K=cfg.shared_K,
                    cb=cfg.shared_cb))
                words[("shared", j)] = trellis_words_torch(seed, p + ".trellis", i_f, o_f, cfg.shared_K,
                                                           device)
        out.append((layer, words, DeviceMoeLayer(layer, device, words=words)))
    return cfg, out


def make_inputs(workload, seed, li, B, H):
    import numpy as np
    from exl3_amd import synth
    if workload == "glm5_moe_staged_b64":
        same = synth.activations(seed, f"bench.same{li}", 1, H)
        rest = synth.activations(seed, f"bench.rest{li}", B - 48, H)
        return np.concatenate([np.repeat(same, 48, 0), rest], 0)
    return synth.activations(seed, f"bench.x{li}", B, H)


def cpu_model():
    """The host CPU's model string and logical CPU count (/proc/cpuinfo)."""
    model, n = None, 0
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                n += 1
                model = model or ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return model, n or os.cpu_count()


def cpu_baseline(layer, words, h_list, budget_s, gpu_out=None):
    """The f32 -O3 CPU restatement of the layer (oracle/cpu_layer.cpp: router, on-the-fly
    table decode, Hadamards, f32 GEMV, SwiGLU, combine, shared expert), one worker per
    host CPU granted to this process: two warm-up calls, then calls on distinct inputs
    until the budget (at least 5), median; one call on one thread. Before timing, the
    sampled call's routing is checked equal to the oracle's (f64 logits, or_route) and
    the decoded weights of its first experts bit-equal to the oracle's decode."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle

    cfg = layer.cfg
    experts = []
    for i, lin in enumerate(layer.experts):
        t = lin.trellis if lin.trellis is not None else words[i].cpu().numpy().view(np.uint16)
        experts.append(dict(trellis=t, suh=lin.suh, svh=lin.svh, K=lin.K, cb=lin.cb,
                            **{"in": lin.in_f, "out": lin.out_f}))
    shared = [l.oracle_dict() for l in layer.shared] if layer.shared else None
    ocfg = pyoracle.make_cfg(cfg.hidden, cfg.inter, cfg.n_experts, cfg.top_k, cfg.n_group,
                             cfg.topk_group, cfg.norm_topk_prob, shared is not None,
                             cfg.routed_scaling_factor, cfg.swiglu_limit)
    cl = pyoracle.CpuLayer(ocfg, experts, shared, layer.router_w, layer.bias)
    threads = pyoracle.cpu_threads()
    # identity with the oracle on the sampled call
    out0, idx0 = cl(h_list[0], threads)
    oidx, _ = pyoracle.route(pyoracle.router_logits(h_list[0], layer.router_w), layer.bias, ocfg)
    routing_equal = bool(np.array_equal(idx0, oidx))
    checked = sorted(set(idx0.reshape(-1).tolist()))[:4]
    weights_equal = all(
        np.array_equal(pyoracle.cpu_decode(experts[3 * e + j]["trellis"], experts[3 * e + j]["in"],
                                           experts[3 * e + j]["out"], experts[3 * e + j]["K"],
                                           experts[3 * e + j]["cb"], threads),
                       pyoracle.decode_inner(experts[3 * e + j]["trellis"], experts[3 * e + j]["in"],
                                             experts[3 * e + j]["out"], experts[3 * e + j]["K"],
                                             experts[3 * e + j]["cb"], threads))
        for e in checked for j in range(3))
    if not (routing_equal and weights_equal):
        raise RuntimeError(f"CPU baseline differs from the oracle: routing {routing_equal}, "
                           f"weights {weights_equal}")
    vs_gpu = None
    if gpu_out is not None:
        a = out0.view(np.float16).astype(np.float64)
        b = gpu_out.view(np.float16).astype(np.float64).reshape(a.shape)
        vs_gpu = float(np.max(np.abs(a - b)) / np.sqrt(np.mean(b ** 2)))
    cl(h_list[1 % len(h_list)], threads)  # second warm-up call
    times, nbytes = [], []
    t_start = time.time()
    i = 0
    while i < 5 or (time.time() - t_start < budget_s and i < 1000):
        h = h_list[i % len(h_list)]
        t0 = time.perf_counter()
        _, idx = cl(h, threads)
        times.append(time.perf_counter() - t0)
        nbytes.append(sum(layer.expert_trellis_bytes(e) if layer.experts[3 * e].trellis is not None
                          else sum(words[3 * e + j].numel() * 2 for j in range(3))
                          for e in set(idx.reshape(-1).tolist())))
        i += 1
    med = float(np.median(times))
    rows = h_list[0].shape[0]
    t0 = time.perf_counter()
    cl(h_list[0], 1)
    t1 = time.perf_counter() - t0
    model, ncpu = cpu_model()
    return {"value": round(rows / med, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{len(times)} timed calls (after 2 warm-up calls) of one {cfg.hidden}-hidden, "
                      f"{cfg.n_experts}-expert layer at B={rows} on {len(h_list)} distinct inputs, median "
                      f"{med * 1e3:.2f} ms/call; oracle/cpu_layer.cpp (f32, -O3 AVX2/FMA/F16C), "
                      f"{threads} threads; one call on 1 thread: {t1 * 1e3:.1f} ms",
            "value_1thread": round(rows / t1, 3),
            "trellis_GBps": round(float(np.median(nbytes)) / med / 1e9, 3),
            "cpu_model": model, "host_logical_cpus": ncpu,
            "routing_equal_oracle": routing_equal, "weights_equal_oracle": weights_equal,
            "weights_checked": f"{3 * len(checked)} tensors of experts {checked}",
            "max_err_rel_vs_gpu": vs_gpu}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[1])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="glm5_moe_decode_b8",
                    help="the bench line's workload (default: the metric's B=8 decode); the "
                         "others are measurement runs of configs[0], [1], [3], [4] and of the "
                         "B=8 layer at 1-4 rows")
    ap.add_argument("--steps", type=int, default=None, help="default 400 (prefill: 20)")
    ap.add_argument("--warmup", type=int, default=None, help="default 40 (prefill: 3)")
    ap.add_argument("--layers", type=int, default=None,
                    help="distinct layer instances rotated (default 8; prefill: 2)")
    ap.add_argument("--settle-ms", type=float, default=300.0,
                    help="untimed steps of the workload for this long before the warmup, so "
                         "that the GPU clocks settle (0: none)")
    ap.add_argument("--seed", type=int, default=20261201)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--weight-form", choices=("reference", "halves"), default="reference",
                    help="mcg/3inst GEMV weights: the reference's f16 values (default) or the "
                         "opt-in exact halves (exl3_tuning.weight_form)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after the timed steps, run one plain device copy of 256 MiB (the "
                         "known-size kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not run here "
              "(across GPUs the layer would shard by expert, each GPU holding E/G experts, "
              "which is not built)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    from exl3_amd import synth

    kind, B, _ = WORKLOADS[args.workload]
    form = 1 if args.weight_form == "halves" else 0
    from exl3_amd.trellis import trellis_set_tuning
    trellis_set_tuning(weight_form=form)
    if kind == "linear":
        bench_linear(args)
        return
    if kind == "block":
        bench_block(args)
        return
    prefill = kind == "prefill"
    args.steps = args.steps if args.steps is not None else (20 if prefill else 400)
    args.warmup = args.warmup if args.warmup is not None else (3 if prefill else 40)
    args.layers = args.layers if args.layers is not None else (2 if prefill else 8)
    dev = torch.device("cuda:0")
    t0 = time.time()
    cfg, layers = build_layers(args.layers, args.seed, dev, kind)
    for _, _, d in layers:
        d.set_tuning(weight_form=form)
    H = cfg.hidden
    xs = [torch.from_numpy(make_inputs(args.workload, args.seed, li, B, H).view(np.float16))
          .to(dev).view(B, 1, H) for li in range(args.layers)]
    outs = [torch.empty_like(x) for x in xs]
    wss = [d.workspace(B) for _, _, d in layers]
    torch.cuda.synchronize()
    print(f"[bench] built {args.layers} layers in {time.time() - t0:.1f}s", file=sys.stderr)

    def step(i):
        li = i % args.layers
        layers[li][2](xs[li], out=outs[li], ws=wss[li])

    settled = settle(step, args.settle_ms)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    ev0.record()
    for i in range(args.steps):
        step(i)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = wall * 1e3 / args.steps
    value = B / (ms_per_step / 1e3)

    if args.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # Per-stage kernel time (HIP events inside the library, on the same stream) over one
    # more rotation of every layer instance, several times.
    for _, _, d in layers:
        d.timing_reset()
        d.timing_enable(True)
    for i in range(args.layers * (2 if prefill else 8)):
        step(i)
    torch.cuda.synchronize()
    tm = {k: 0.0 for k in ("calls", "router_ms", "gate_up_ms", "down_ms", "combine_ms", "total_ms",
                           "gate_up_trellis_bytes", "down_trellis_bytes")}
    for _, _, d in layers:
        d.timing_enable(False)
        for k, v in d.timing().items():
            tm[k] += v
    calls = tm["calls"]
    gu_bytes = tm["gate_up_trellis_bytes"] / calls
    dn_bytes = tm["down_trellis_bytes"] / calls
    gu_ms = tm["gate_up_ms"] / calls
    dn_ms = tm["down_ms"] / calls
    gu_gbps = gu_bytes / (gu_ms * 1e-3) / 1e9
    dn_gbps = dn_bytes / (dn_ms * 1e-3) / 1e9
    routed_gbps = (gu_bytes + dn_bytes) / ((gu_ms + dn_ms) * 1e-3) / 1e9
    expert_bytes = (2 * H * cfg.inter * cfg.gate_up_K + cfg.inter * H * cfg.down_K) // 8
    distinct = (gu_bytes + dn_bytes) / expert_bytes

    # f16 MFMA work of the routed gate/up launch: 2 flops per weight and routed pair
    gu_flops = 2.0 * 2 * H * cfg.inter * B * cfg.top_k
    gu_tflops = gu_flops / (gu_ms * 1e-3) / 1e12
    shared = ("none" if not cfg.shared_inter else
              f"fp16 {cfg.shared_inter}" if cfg.shared_K == 0 else f"K{cfg.shared_K} trellis {cfg.shared_inter}")
    cbn = {0: "3inst", 1: "mcg", 2: "mul1"}
    metric = ("MoE-layer decode tokens/s + achieved HBM GB/s on trellis bytes, B=8, 1 MI355X"
              if args.workload == "glm5_moe_decode_b8" else
              f"MoE-layer tokens/s + achieved HBM GB/s on trellis bytes, {args.workload}, 1 MI355X")
    line = {
        "metric": metric,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup, "settle": settled,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": args.workload, "batch": B, "hidden": H,
                   "moe_intermediate": cfg.inter, "experts": cfg.n_experts, "top_k": cfg.top_k,
                   "gate_up": f"K{cfg.gate_up_K} {cbn[cfg.gate_up_cb]}",
                   "down": f"K{cfg.down_K} {cbn[cfg.down_cb]}", "shared_expert": shared,
                   "layer_instances": args.layers, "weight_form": args.weight_form,
                   "parallelism": "none (one GPU)"},
        "roofline": {"kernel": "k_moe_gate_up", "bound": "hbm", "achieved": round(gu_gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gu_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic("k_moe_gate_up") if args.workload == "glm5_moe_decode_b8" else None,
                     "algorithmic_bytes_per_launch": round(gu_bytes),
                     "avg_launch_ms": round(gu_ms, 5),
                     "valu_busy_profiled": profiled_valu_busy("k_moe_gate_up") if args.workload == "glm5_moe_decode_b8" else None},
        "roofline_down": {"kernel": "k_moe_down", "achieved": round(dn_gbps, 1),
                          "frac": round(dn_gbps / HBM_PEAK_GBPS, 4),
                          "traffic": measured_traffic("k_moe_down") if args.workload == "glm5_moe_decode_b8" else None,
                          "algorithmic_bytes_per_launch": round(dn_bytes), "avg_launch_ms": round(dn_ms, 5),
                          "valu_busy_profiled": profiled_valu_busy("k_moe_down") if args.workload == "glm5_moe_decode_b8" else None},
        "routed_trellis_GBps": round(routed_gbps, 1),
        "distinct_experts_per_step": round(distinct, 2),
        "stages_ms": {k: round(tm[k] / calls, 5) for k in ("router_ms", "gate_up_ms", "down_ms",
                                                           "combine_ms", "total_ms")},
        "gpu_ms_per_step_events": round(gpu_ms / args.steps, 5),
    }
    if prefill:
        # prefill streams every expert once and is compute-heavy: the MFMA roofline of the
        # routed gate/up launch (f16 dense peak) next to its HBM one
        line["roofline"] = {"kernel": "k_moe_gate_up", "bound": "mfma", "achieved": round(gu_tflops, 2),
                            "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                            "frac": round(gu_tflops / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None,
                            "algorithmic_flops_per_launch": gu_flops, "avg_launch_ms": round(gu_ms, 5),
                            "hbm_GBps": round(gu_gbps, 1), "hbm_frac": round(gu_gbps / HBM_PEAK_GBPS, 4)}
    if args.workload not in ("glm5_moe_decode_b8", "small_b1"):
        args.no_cpu_baseline = True  # the CPU leg is sampled on configs[0] and configs[2]
    if not args.no_cpu_baseline:
        layer, words, d0 = layers[0]
        h_list = [synth.activations(args.seed, f"bench.cpu.x{i}", B, H) for i in range(8)]
        y0 = d0(torch.from_numpy(h_list[0].view(np.float16)).to(dev).view(B, 1, H))
        line["cpu_baseline"] = cpu_baseline(layer, words, h_list, args.cpu_seconds,
                                            y0.cpu().numpy().view(np.uint16))
    else:
        line["cpu_baseline"] = None
    for _, _, d in layers:
        d.close()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
