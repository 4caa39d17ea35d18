"""Seeded synthetic inputs for the EXL3 MoE layer (numpy, no torch).

Every tensor of a configuration is drawn from a counter-based generator so that any
tensor can be regenerated on its own from (base seed, tensor name):

  key      = splitmix64(base_seed ^ fnv1a64(name))
  u64[i]   = splitmix64(key + (i + 1) * 0x9E3779B97F4A7C15)
  uniform  = ((u64 >> 11) + 0.5) / 2^53                      in (0, 1)
  normal   = Box-Muller on consecutive uniform pairs (f64), cos branch
  f16      = round-to-nearest-even of the f64 value (numpy's float16 cast is RNE)
  trellis  = u64 >> 48 as uint16 words (uniform random int16)

The configurations are the five workloads of the benchmark contract (small CPU layer,
single-linear sweep, GLM-5-shaped B=8 decode, B=64 staged decode, 2048-token prefill).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)

CB_3INST, CB_MCG, CB_MUL1 = 0, 1, 2
CB_NAMES = {CB_3INST: "3inst", CB_MCG: "mcg", CB_MUL1: "mul1"}


def _mix(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def splitmix64_scalar(x: int) -> int:
    x = (x + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
    z = x
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
    return z ^ (z >> 31)


def fnv1a64(s: str) -> int:
    h = 0xCBF29CE484222325
    for b in s.encode():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def tensor_key(seed: int, name: str) -> int:
    return splitmix64_scalar((seed ^ fnv1a64(name)) & 0xFFFFFFFFFFFFFFFF)


def u64_stream(key: int, n: int, start: int = 0) -> np.ndarray:
    i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix(np.uint64(key) + i * GAMMA)


def uniform01(key: int, n: int) -> np.ndarray:
    u = u64_stream(key, n) >> np.uint64(11)
    return (u.astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)


def normal(seed: int, name: str, shape, mean=0.0, std=1.0) -> np.ndarray:
    n = int(np.prod(shape))
    u = uniform01(tensor_key(seed, name), 2 * n).reshape(n, 2)
    z = np.sqrt(-2.0 * np.log(u[:, 0])) * np.cos(2.0 * np.pi * u[:, 1])
    return (mean + std * z).reshape(shape)


def normal_f16(seed: int, name: str, shape, mean=0.0, std=1.0) -> np.ndarray:
    """f16 bit patterns (uint16) of N(mean, std) draws, RNE-rounded."""
    return normal(seed, name, shape, mean, std).astype(np.float16).view(np.uint16)


def normal_f32(seed: int, name: str, shape, mean=0.0, std=1.0) -> np.ndarray:
    return normal(seed, name, shape, mean, std).astype(np.float32)


def trellis_words(seed: int, name: str, in_f: int, out_f: int, K: int) -> np.ndarray:
    """Uniform random int16 words, on-disk layout (in/16, out/16, 16*K) as uint16."""
    n = (in_f // 16) * (out_f // 16) * 16 * K
    w = (u64_stream(tensor_key(seed, name), n) >> np.uint64(48)).astype(np.uint16)
    return w.reshape(in_f // 16, out_f // 16, 16 * K)


@dataclass
class Linear:
    """One linear: an EXL3 trellis (trellis/suh/svh/K/cb) or a plain f16 (in, out) weight."""
    in_f: int
    out_f: int
    trellis: np.ndarray | None = None  # uint16 (in/16, out/16, 16K)
    suh: np.ndarray | None = None      # f16 bits [in]
    svh: np.ndarray | None = None      # f16 bits [out]
    K: int = 0
    cb: int = CB_MCG
    dense: np.ndarray | None = None    # f16 bits (in, out)

    @property
    def quantized(self) -> bool:
        return self.trellis is not None

    def trellis_bytes(self) -> int:
        return 0 if self.trellis is None else self.trellis.size * 2

    def oracle_dict(self) -> dict:
        if self.quantized:
            return dict(trellis=self.trellis, suh=self.suh, svh=self.svh, K=self.K, cb=self.cb,
                        **{"in": self.in_f, "out": self.out_f})
        return dict(dense=self.dense, **{"in": self.in_f, "out": self.out_f})


def make_trellis_linear(seed, name, in_f, out_f, K, cb, scale_std=0.05) -> Linear:
    return Linear(in_f, out_f, trellis=trellis_words(seed, name + ".trellis", in_f, out_f, K),
                  suh=normal_f16(seed, name + ".suh", (in_f,), 1.0, scale_std),
                  svh=normal_f16(seed, name + ".svh", (out_f,), 1.0, scale_std), K=K, cb=cb)


def make_dense_linear(seed, name, in_f, out_f) -> Linear:
    # N(0, 1/sqrt(in)) keeps the projection's output at unit scale.
    return Linear(in_f, out_f, dense=normal_f16(seed, name + ".weight", (in_f, out_f), 0.0,
                                                 1.0 / np.sqrt(in_f)))


@dataclass
class MoeConfig:
    hidden: int
    inter: int
    n_experts: int
    top_k: int
    n_group: int = 1
    topk_group: int = 1
    norm_topk_prob: bool = True
    routed_scaling_factor: float = 1.0
    swiglu_limit: float = 10.0
    shared_inter: int = 0            # 0 = no shared expert
    gate_up_K: int = 4
    gate_up_cb: int = CB_MCG
    down_K: int = 4
    down_cb: int = CB_MCG
    shared_K: int = 0                # 0 = fp16 shared expert
    shared_cb: int = CB_MCG
    bias_std: float = 0.01
    router_std: float = 0.02


@dataclass
class MoeLayer:
    cfg: MoeConfig
    experts: list                    # 3*E Linear (gate, up, down per expert)
    shared: list | None              # 3 Linear or None
    router_w: np.ndarray             # f16 bits (E, H)
    bias: np.ndarray                 # f32 (E,)
    meta: dict = field(default_factory=dict)

    def expert_trellis_bytes(self, e: int) -> int:
        return sum(self.experts[3 * e + j].trellis_bytes() for j in range(3))


def make_layer(cfg: MoeConfig, seed: int, tag: str = "layer0", hot_experts=None,
               hot_bias=0.0) -> MoeLayer:
    H, I, E = cfg.hidden, cfg.inter, cfg.n_experts
    experts = []
    for e in range(E):
        p = f"{tag}.experts.{e}"
        experts.append(make_trellis_linear(seed, p + ".gate_proj", H, I, cfg.gate_up_K, cfg.gate_up_cb))
        experts.append(make_trellis_linear(seed, p + ".up_proj", H, I, cfg.gate_up_K, cfg.gate_up_cb))
        experts.append(make_trellis_linear(seed, p + ".down_proj", I, H, cfg.down_K, cfg.down_cb))
    shared = None
    if cfg.shared_inter > 0:
        p = f"{tag}.shared_experts"
        SI = cfg.shared_inter
        if cfg.shared_K > 0:
            shared = [make_trellis_linear(seed, p + ".gate_proj", H, SI, cfg.shared_K, cfg.shared_cb),
                      make_trellis_linear(seed, p + ".up_proj", H, SI, cfg.shared_K, cfg.shared_cb),
                      make_trellis_linear(seed, p + ".down_proj", SI, H, cfg.shared_K, cfg.shared_cb)]
        else:
            shared = [make_dense_linear(seed, p + ".gate_proj", H, SI),
                      make_dense_linear(seed, p + ".up_proj", H, SI),
                      make_dense_linear(seed, p + ".down_proj", SI, H)]
    router_w = normal_f16(seed, f"{tag}.gate.weight", (E, H), 0.0, cfg.router_std)
    bias = normal_f32(seed, f"{tag}.gate.e_score_correction_bias", (E,), 0.0, cfg.bias_std)
    if hot_experts is not None:
        bias = bias.copy()
        bias[np.asarray(hot_experts)] += np.float32(hot_bias)
    return MoeLayer(cfg, experts, shared, router_w, bias)


def activations(seed: int, name: str, rows: int, hidden: int) -> np.ndarray:
    return normal_f16(seed, name, (rows, hidden), 0.0, 1.0)


# --- the benchmark contract's configurations ----------------------------------------

def config_small() -> MoeConfig:
    """hidden 512, inter 256, 16 experts, top-2, K4 mcg, no shared expert."""
    return MoeConfig(hidden=512, inter=256, n_experts=16, top_k=2, routed_scaling_factor=1.0,
                     gate_up_K=4, gate_up_cb=CB_MCG, down_K=4, down_cb=CB_MCG, shared_inter=0)


def config_glm5(shared_K: int = 0) -> MoeConfig:
    """configs[2]/[3]: GLM-5-shaped layer (gate/up K4 mcg, down K5 mcg, fp16 shared expert)."""
    return MoeConfig(hidden=4096, inter=1024, n_experts=288, top_k=8, routed_scaling_factor=2.5,
                     swiglu_limit=10.0, shared_inter=1024, gate_up_K=4, gate_up_cb=CB_MCG,
                     down_K=5, down_cb=CB_MCG, shared_K=shared_K)


def config_prefill() -> MoeConfig:
    """gate/up K4 3inst, down K5 mul1, shared expert K6 mcg."""
    return MoeConfig(hidden=4096, inter=1024, n_experts=288, top_k=8, routed_scaling_factor=2.5,
                     swiglu_limit=10.0, shared_inter=1024, gate_up_K=4, gate_up_cb=CB_3INST,
                     down_K=5, down_cb=CB_MUL1, shared_K=6, shared_cb=CB_MCG)
