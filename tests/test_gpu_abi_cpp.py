"""The layer called from C++ through include/exl3_moe.h alone.

tests/abi_c/moe_cpp_probe.cpp is the binding a C++ engine would write: hipMalloc'd
tensors, exl3_linear_desc arrays for the experts and the shared expert, layer create,
the workspace query, one exl3_moe_layer call on the default stream, destroy. Its
output equals the Python binding's call on the same layer bit for bit, and the oracle
within the layer tolerance.
"""
import os
import shutil
import subprocess

import numpy as np
import pytest
import torch

from exl3_amd import _lib, synth
from exl3_amd.moe import DeviceMoeLayer
from test_gpu_moe import check_out, check_routing, ocfg_of, to_dev

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def build_probe(tmp_path):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    libdir = os.path.dirname(_lib.LIB_PATH)
    exe = tmp_path / "moe_cpp_probe"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
                    "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROCM, "include"),
                    os.path.join(ROOT, "tests", "abi_c", "moe_cpp_probe.cpp"),
                    "-L", libdir, "-lexl3moe", f"-Wl,-rpath,{libdir}",
                    "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}",
                    "-o", str(exe)], check=True)
    return exe


def write_layer(path, layer, h, B):
    cfg = layer.cfg
    kind = 0 if layer.shared is None else (1 if layer.shared[0].quantized else 2)
    sh = layer.shared[0] if layer.shared else None
    hdr = np.array([cfg.hidden, cfg.inter, cfg.n_experts, cfg.top_k, cfg.n_group, cfg.topk_group,
                    int(cfg.norm_topk_prob), kind, cfg.shared_inter if kind else 0,
                    cfg.gate_up_K, cfg.gate_up_cb, cfg.down_K, cfg.down_cb,
                    sh.K if kind == 1 else 0, sh.cb if kind == 1 else 0, B], dtype="<i4")
    parts = [hdr.tobytes(), np.array([cfg.routed_scaling_factor, cfg.swiglu_limit], "<f4").tobytes()]
    for lin in layer.experts + (layer.shared or []):
        if lin.quantized:
            parts += [lin.trellis.astype("<u2").tobytes(), lin.suh.astype("<u2").tobytes(),
                      lin.svh.astype("<u2").tobytes()]
        else:
            parts.append(lin.dense.astype("<u2").tobytes())
    parts += [layer.router_w.astype("<u2").tobytes(), layer.bias.astype("<f4").tobytes(),
              h.astype("<u2").tobytes()]
    path.write_bytes(b"".join(parts))


@pytest.mark.parametrize("shared_K,B", [(0, 8), (3, 8), (3, 70), (-1, 40)])
def test_cpp_binding_equals_python_and_oracle(oracle, dev, tmp_path, shared_K, B):
    # shared_K: 0 f16 shared expert, 3 trellis (at 70 rows on the layer's second
    # stream), -1 none
    cfg = synth.MoeConfig(hidden=256, inter=128, n_experts=8, top_k=3, routed_scaling_factor=1.5,
                          gate_up_K=4, gate_up_cb=1, down_K=3, down_cb=2,
                          shared_inter=0 if shared_K < 0 else 128, shared_K=max(shared_K, 0),
                          shared_cb=0)
    layer = synth.make_layer(cfg, 41)
    H = cfg.hidden
    h = synth.activations(41, f"cpp.{shared_K}.{B}", B, H)
    exe = build_probe(tmp_path)
    write_layer(tmp_path / "layer.bin", layer, h, B)
    print(f"moe_cpp_probe shared_K={shared_K} B={B}", flush=True)
    r = subprocess.run([str(exe), str(tmp_path / "layer.bin"), str(tmp_path / "out.bin")],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.returncode, r.stdout, r.stderr)
    got = np.fromfile(tmp_path / "out.bin", dtype="<u2").reshape(B, H)

    d = DeviceMoeLayer(layer, dev)
    x = to_dev(h, dev, B, 1, H)
    y = d(x)
    _, ids = d.route(x)
    torch.cuda.synchronize()
    assert np.array_equal(got, y.view(torch.int16).cpu().numpy().reshape(B, H).view(np.uint16))

    oc = ocfg_of(oracle, cfg, layer.shared is not None)
    logits = oracle.router_logits(h, layer.router_w)
    idx, w, _ = check_routing(oracle, logits, layer.bias, ids.cpu().numpy(), oc)
    want = oracle.moe_layer_routed(oc, [l.oracle_dict() for l in layer.experts],
                                   None if layer.shared is None else
                                   [l.oracle_dict() for l in layer.shared], h, idx, w)
    check_out(torch.from_numpy(got.view(np.float16)), want)
    d.close()
