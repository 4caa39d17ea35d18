"""Seeded MoE layer configurations shared by the GPU parity tests and the oracle's own
CPU tests (not a test module)."""
import dataclasses

import numpy as np

from exl3_amd import synth


def random_cfgs(n, seed):
    """n seeded layer configurations over the shape space the kernels take: hidden and
    intermediate multiples of 128, E up to 64 with optional group-limited routing,
    top-k up to 8, every K and codebook, no / trellis / f16 shared expert."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        E = int(rng.choice([4, 8, 12, 16, 40, 64]))
        groups = [g for g in (1, 2, 4) if E % g == 0 and E // g >= 2]
        ng = int(rng.choice(groups))
        tg = int(rng.integers(1, ng + 1))
        topk = int(rng.integers(1, min(8, E * tg // ng) + 1))
        shared = int(rng.integers(0, 3))  # 0 none, 1 trellis, 2 f16
        out.append(synth.MoeConfig(
            hidden=128 * int(rng.integers(1, 6)), inter=128 * int(rng.integers(1, 4)), n_experts=E,
            top_k=topk, n_group=ng, topk_group=tg, norm_topk_prob=bool(rng.integers(0, 2)),
            routed_scaling_factor=float(rng.choice([1.0, 1.5, 2.5])),
            swiglu_limit=float(rng.choice([0.5, 7.0, 10.0])),
            shared_inter=128 * int(rng.integers(1, 3)) if shared else 0,
            gate_up_K=int(rng.integers(1, 9)), gate_up_cb=int(rng.integers(0, 3)),
            down_K=int(rng.integers(1, 9)), down_cb=int(rng.integers(0, 3)),
            shared_K=int(rng.integers(1, 9)) if shared == 1 else 0, shared_cb=int(rng.integers(0, 3))))
    return out


# (seed, config index, rows) of random_cfgs layers at a SwiGLU limit of 0.5 where the
# oracle's two weight forms differ by more than the north-star bound: large gate/up
# outputs clipped to +-0.5 leave a small output for the weights' f16 rounding to move
# (tests/test_oracle.py checks that these cases separate the forms)
LIMIT_HALF_CASES = [(7, 3, 17), (7, 4, 17), (8, 5, 17), (9, 1, 17), (28, 2, 3)]


def limit_half_case(seed, i, B):
    cfg = dataclasses.replace(random_cfgs(6, seed)[i], swiglu_limit=0.5)
    layer = synth.make_layer(cfg, seed * 10 + i)
    h = synth.activations(seed * 10 + i, f"lim.x.{i}", B, cfg.hidden)
    return cfg, layer, h
