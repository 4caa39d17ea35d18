"""Writes tests/golden/moe_shard_{a,b,c}.safetensors for the loader tests, from the seeded
generator (exl3_amd.synth): one small EXL3 MoE layer split over shards a and b, and in
shard c a second layer and its MLP sub-block's own tensors.

The layer is SHARD_CFG at seed SHARD_SEED (synth.make_layer, tag "layer0"); its tensors
are stored under the reference's key names (glm5.cpp:503-518, exl3.h:4-9):

  model.layers.0.mlp.gate.weight                         F16 (E, hidden)
  model.layers.0.mlp.gate.e_score_correction_bias        F32 (E)
  model.layers.0.mlp.experts.{e}.{gate,up,down}_proj.trellis   I16 (in/16, out/16, 16K)
  ...                                            .suh / .svh     F16 (in) / (out)
  ...                                            .mcg | .mul1    I32 scalar marker
  model.layers.0.mlp.shared_experts.{gate,up,down}_proj.weight F16 (out, in)

Byte placement is chosen so that the loader meets every case a real checkpoint has: the
headers' lengths are 2 and 1 mod 4 (11 of the 13 real shards have header_len % 4 != 0,
docs/perf.md:105), and small filler tensors of 1 to 3 bytes shift later tensors, so that
trellis tensors sit at file positions congruent to 0, 1, 2 and 3 mod 4: those at 0 are
used in place, the others are repacked on the device.

Shard c holds layer 1 (SHARD_CFG_1 at SHARD_SEED_1, tag "layer1"): gate/up in the 3inst
codebook, which has no marker tensor (the loader's fallback, glm5.cpp:303), down in mcg,
and a trellis shared expert (K3 3inst, no markers either); plus the decoder layer's MLP
sub-block tensors (glm5.cpp:409-415) in the dtypes load_any converts:

  model.layers.1.post_attention_layernorm.weight   BF16 (hidden)   (a few values in f16's
                                                                    subnormal range)
  model.layers.1.hc_ffn_fn                         F32 (24, 4 * hidden)
  model.layers.1.hc_ffn_base                       BF16 (24)
  model.layers.1.hc_ffn_scale                      F16 (3)

Run from the repository root: python tests/golden/make_shard.py
"""
from __future__ import annotations

import json
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "exl3-server_amd"))

from exl3_amd import synth  # noqa: E402

SHARD_SEED = 606
SHARD_CFG = synth.MoeConfig(hidden=256, inter=128, n_experts=6, top_k=2, routed_scaling_factor=1.5,
                            swiglu_limit=10.0, shared_inter=128, gate_up_K=3, gate_up_cb=synth.CB_MCG,
                            down_K=2, down_cb=synth.CB_MUL1, shared_K=0)
PREFIX = "model.layers.0.mlp."
SHARD_SEED_1 = 616
SHARD_CFG_1 = synth.MoeConfig(hidden=256, inter=128, n_experts=4, top_k=2, routed_scaling_factor=2.5,
                              swiglu_limit=10.0, shared_inter=128, gate_up_K=2, gate_up_cb=synth.CB_3INST,
                              down_K=3, down_cb=synth.CB_MCG, shared_K=3, shared_cb=synth.CB_3INST)
LAYER_PREFIX_1 = "model.layers.1."
PREFIX_1 = LAYER_PREFIX_1 + "mlp."
HC_MULT = 4
MARKER = {synth.CB_MCG: "mcg", synth.CB_MUL1: "mul1"}
PROJ = ("gate_proj", "up_proj", "down_proj")


def layer():
    return synth.make_layer(SHARD_CFG, SHARD_SEED)


def layer1():
    return synth.make_layer(SHARD_CFG_1, SHARD_SEED_1, tag="layer1")


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def block1():
    """Layer 1's MLP sub-block tensors as stored: norm weight (bf16 bits), fn (f32), base
    (bf16 bits), scale (f16 bits)."""
    D, N = SHARD_CFG_1.hidden, HC_MULT
    W = (2 + N) * N
    nw = synth.normal(SHARD_SEED_1, "layer1.post_norm", (D,), 1.0, 0.2).astype(np.float32)
    # values below f16's smallest normal (2^-14): bf16 keeps more bits there than f16 does,
    # so the conversion rounds
    nw[[3, 70, 141, 200]] = np.array([1.3e-5, -2.71e-6, 4.4e-7, 5.9e-5], np.float32)
    fn = synth.normal(SHARD_SEED_1, "layer1.hc_ffn_fn", (W, N * D), 0.0, 1.0 / np.sqrt(N * D)).astype(np.float32)
    base = synth.normal(SHARD_SEED_1, "layer1.hc_ffn_base", (W,), 0.0, 0.5).astype(np.float32)
    scale = np.array([1.3, 0.7, 2.1], np.float16).view(np.uint16)
    return bf16_bits(nw), fn, bf16_bits(base), scale


def linear_tensors(key, lin):
    out = [(key + ".trellis", "I16", lin.trellis.astype("<u2")),
           (key + ".suh", "F16", lin.suh.astype("<u2")),
           (key + ".svh", "F16", lin.svh.astype("<u2"))]
    if lin.cb in MARKER:
        out.append((key + "." + MARKER[lin.cb], "I32", np.zeros((), "<i4")))
    return out


def expert_tensors(lay, e, prefix=PREFIX):
    out = []
    for j, nm in enumerate(PROJ):
        out += linear_tensors(f"{prefix}experts.{e}.{nm}", lay.experts[3 * e + j])
    return out


def filler(name, nbytes):
    return (name, "U8", np.arange(nbytes, dtype=np.uint8))


def write(path, tensors, header_mod4):
    """tensors: [(name, dtype, array)] in data order; pads the JSON with spaces so that
    the header length (8 + JSON) is header_mod4 mod 4."""
    meta, off = {}, 0
    for name, dt, arr in tensors:
        nb = arr.nbytes
        meta[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + nb]}
        off += nb
    meta["__metadata__"] = {"format": "pt", "note": "synthetic EXL3 MoE layer for loader tests"}
    js = json.dumps(meta, separators=(",", ":"))
    while (8 + len(js)) % 4 != header_mod4:
        js += " "
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(js)))
        f.write(js.encode())
        for _, _, arr in tensors:
            f.write(np.ascontiguousarray(arr).tobytes())


def main():
    lay = layer()
    E = SHARD_CFG.n_experts
    # shard a: header 2 mod 4; a 2-byte filler makes experts 0-1 4-byte aligned, a second
    # one puts expert 2 and the router 2 bytes off
    a = [filler(f"{PREFIX}pad.a0", 2)] + expert_tensors(lay, 0) + expert_tensors(lay, 1)
    a += [filler(f"{PREFIX}pad.a1", 2)] + expert_tensors(lay, 2)
    a += [(f"{PREFIX}gate.weight", "F16", lay.router_w.astype("<u2")),
          (f"{PREFIX}gate.e_score_correction_bias", "F32", lay.bias.astype("<f4"))]
    write(os.path.join(HERE, "moe_shard_a.safetensors"), a, 2)
    # shard b: header 1 mod 4; a 2-byte filler puts expert 3 three bytes off, another one
    # expert 4 one byte off, a 3-byte one aligns expert 5, and the shared expert follows
    # (a 1-byte filler leaves it one byte off)
    b = [filler(f"{PREFIX}pad.b0", 2)] + expert_tensors(lay, 3) + [filler(f"{PREFIX}pad.b1", 2)]
    b += expert_tensors(lay, 4) + [filler(f"{PREFIX}pad.b2", 3)] + expert_tensors(lay, 5)
    b += [filler(f"{PREFIX}pad.b3", 1)]
    for j, nm in enumerate(PROJ):
        w = lay.shared[j].dense  # (in, out) f16 bits
        b.append((f"{PREFIX}shared_experts.{nm}.weight", "F16", np.ascontiguousarray(w.T).astype("<u2")))
    write(os.path.join(HERE, "moe_shard_b.safetensors"), b, 1)
    assert E == 6
    # shard c: header 3 mod 4; layer 1 and its block tensors
    l1 = layer1()
    c = [filler(f"{PREFIX_1}pad.c0", 1)]
    for e in range(SHARD_CFG_1.n_experts):
        c += expert_tensors(l1, e, PREFIX_1)
    for j, nm in enumerate(PROJ):
        c += linear_tensors(f"{PREFIX_1}shared_experts.{nm}", l1.shared[j])
    c += [(f"{PREFIX_1}gate.weight", "F16", l1.router_w.astype("<u2")),
          (f"{PREFIX_1}gate.e_score_correction_bias", "F32", l1.bias.astype("<f4"))]
    nw, fn, base, scale = block1()
    c += [(f"{LAYER_PREFIX_1}post_attention_layernorm.weight", "BF16", nw.astype("<u2")),
          (f"{LAYER_PREFIX_1}hc_ffn_fn", "F32", fn.astype("<f4")),
          (f"{LAYER_PREFIX_1}hc_ffn_base", "BF16", base.astype("<u2")),
          (f"{LAYER_PREFIX_1}hc_ffn_scale", "F16", scale.astype("<u2"))]
    write(os.path.join(HERE, "moe_shard_c.safetensors"), c, 3)


if __name__ == "__main__":
    main()
