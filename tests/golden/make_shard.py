"""Writes tests/golden/moe_shard_{a,b}.safetensors: one small EXL3 MoE layer split over
two safetensors shards, from the seeded generator (exl3_amd.synth), for the loader tests.

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
MARKER = {synth.CB_MCG: "mcg", synth.CB_MUL1: "mul1"}
PROJ = ("gate_proj", "up_proj", "down_proj")


def layer():
    return synth.make_layer(SHARD_CFG, SHARD_SEED)


def expert_tensors(lay, e):
    out = []
    for j, nm in enumerate(PROJ):
        lin = lay.experts[3 * e + j]
        key = f"{PREFIX}experts.{e}.{nm}"
        out.append((key + ".trellis", "I16", lin.trellis.astype("<u2")))
        out.append((key + ".suh", "F16", lin.suh.astype("<u2")))
        out.append((key + ".svh", "F16", lin.svh.astype("<u2")))
        if lin.cb in MARKER:
            out.append((key + "." + MARKER[lin.cb], "I32", np.zeros((), "<i4")))
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


if __name__ == "__main__":
    main()
