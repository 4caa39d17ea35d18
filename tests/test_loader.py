"""CPU tests of the safetensors shard reader (exl3_st_*, host-only C ABI) on the
committed EXL3 fixtures (tests/golden/moe_shard_{a,b,c}.safetensors, written by
tests/golden/make_shard.py from the seeded generator): the header parse, the tensor table,
every tensor's bytes against the generator, the alignment cases, and the reference's
consistency checks on malformed files (safetensors.cpp:52-102)."""
import os
import struct

import numpy as np
import pytest

from exl3_amd import synth
from exl3_amd._lib import Exl3Error

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
import sys  # noqa: E402
sys.path.insert(0, GOLDEN)
import make_shard  # noqa: E402

SHARDS = [os.path.join(GOLDEN, f"moe_shard_{x}.safetensors") for x in "ab"]


@pytest.fixture(scope="module")
def shards():
    from exl3_amd.loader import Shard
    s = [Shard(p) for p in SHARDS]
    yield s
    for x in s:
        x.close()


def test_fixture_is_what_the_script_writes(tmp_path, monkeypatch):
    # regenerating the fixture gives the committed bytes
    monkeypatch.setattr(make_shard, "HERE", str(tmp_path))
    make_shard.main()
    for x in "abc":
        with open(os.path.join(tmp_path, f"moe_shard_{x}.safetensors"), "rb") as f, \
                open(os.path.join(GOLDEN, f"moe_shard_{x}.safetensors"), "rb") as g:
            assert f.read() == g.read()


def test_header_and_table(shards):
    a, b = shards
    assert a.header_len % 4 == 2 and b.header_len % 4 == 1
    ta, tb = a.tensors(), b.tensors()
    P = make_shard.PREFIX
    assert ta[P + "gate.weight"]["dtype"] == "F16" and ta[P + "gate.weight"]["shape"] == (6, 256)
    assert ta[P + "gate.e_score_correction_bias"]["dtype"] == "F32"
    t = tb[P + "experts.3.gate_proj.trellis"]
    assert t["dtype"] == "I16" and t["shape"] == (16, 8, 48) and t["nbytes"] == 16 * 8 * 48 * 2
    assert t["file_offset"] == b.header_len + t["offset"]
    assert tb[P + "experts.3.down_proj.mul1"]["shape"] == () and tb[P + "experts.3.gate_proj.mcg"]["nbytes"] == 4
    assert tb[P + "shared_experts.down_proj.weight"]["shape"] == (256, 128)  # (out, in)
    assert "__metadata__" not in ta
    # trellis tensors at every file alignment mod 4
    mods = {v["file_offset"] % 4 for tab in (ta, tb) for k, v in tab.items() if k.endswith(".trellis")}
    assert mods == {0, 1, 2, 3}


def test_shard_c_table():
    # layer 1: 3inst gate/up and shared expert without marker tensors, mcg down with its
    # marker; the MLP sub-block tensors in the dtypes the block loader converts
    from exl3_amd.loader import Shard
    c = Shard(os.path.join(GOLDEN, "moe_shard_c.safetensors"))
    try:
        assert c.header_len % 4 == 3
        t = c.tensors()
        P, LP = make_shard.PREFIX_1, make_shard.LAYER_PREFIX_1
        for e in range(make_shard.SHARD_CFG_1.n_experts):
            for nm in ("gate_proj", "up_proj"):
                assert P + f"experts.{e}.{nm}.trellis" in t
                assert not any(P + f"experts.{e}.{nm}.{m}" in t for m in ("mcg", "mul1"))
            assert P + f"experts.{e}.down_proj.mcg" in t
        assert t[P + "shared_experts.down_proj.trellis"]["shape"] == (128 // 16, 256 // 16, 48)
        assert not any(k.startswith(P + "shared_experts") and k.endswith((".mcg", ".mul1")) for k in t)
        assert (t[LP + "post_attention_layernorm.weight"]["dtype"], t[LP + "hc_ffn_fn"]["dtype"],
                t[LP + "hc_ffn_base"]["dtype"], t[LP + "hc_ffn_scale"]["dtype"]) == ("BF16", "F32", "BF16", "F16")
        assert t[LP + "hc_ffn_fn"]["shape"] == (24, 4 * 256)
        nw, fn, base, scale = make_shard.block1()
        assert np.array_equal(c.data(LP + "post_attention_layernorm.weight"), nw)
        assert np.array_equal(c.data(LP + "hc_ffn_fn"), fn)
    finally:
        c.close()


def test_bf16_helper_rounds_to_nearest_even():
    # the fixture's f32 -> bf16 rounding against an exact f64 restatement on edge cases
    x = np.array([1.0, 1.00390625, 1.005859375, 1.0078125 * (1 + 2 ** -9), -3.14159, 65504.0,
                  1e-5, 2.0 ** -130], np.float32)
    b = make_shard.bf16_bits(x)
    back = (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    for xi, bi in zip(x.astype(np.float64), back):
        e = np.floor(np.log2(abs(xi)))
        ulp = 2.0 ** (max(e, -126) - 7)
        assert abs(bi - xi) <= ulp / 2


def test_bytes_equal_the_generator(shards):
    lay = make_shard.layer()
    P = make_shard.PREFIX
    by_name = {}
    for s in shards:
        for name in s.tensors():
            by_name[name] = s
    for e in range(make_shard.SHARD_CFG.n_experts):
        for j, nm in enumerate(make_shard.PROJ):
            lin = lay.experts[3 * e + j]
            key = f"{P}experts.{e}.{nm}"
            assert np.array_equal(by_name[key + ".trellis"].data(key + ".trellis").view(np.uint16), lin.trellis)
            assert np.array_equal(by_name[key + ".suh"].data(key + ".suh"), lin.suh)
            assert np.array_equal(by_name[key + ".svh"].data(key + ".svh"), lin.svh)
    assert np.array_equal(shards[0].data(P + "gate.weight"), lay.router_w)
    assert np.array_equal(shards[0].data(P + "gate.e_score_correction_bias"), lay.bias)
    for j, nm in enumerate(make_shard.PROJ):
        assert np.array_equal(shards[1].data(f"{P}shared_experts.{nm}.weight"), lay.shared[j].dense.T)


def _write(path, header: bytes, data: bytes, n=None):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(header) if n is None else n))
        f.write(header)
        f.write(data)
    return str(path)


@pytest.mark.parametrize("case", ["bad_json", "inconsistent", "past_end", "huge_len", "bad_dtype", "truncated"])
def test_malformed_files_are_refused(tmp_path, case):
    from exl3_amd.loader import Shard
    ok = b'{"x":{"dtype":"F16","shape":[2,2],"data_offsets":[0,8]}}'
    p = {
        "bad_json": lambda: _write(tmp_path / "f", b'{"x":{"dtype":"F16",', b"\0" * 8),
        "inconsistent": lambda: _write(tmp_path / "f", ok.replace(b"[2,2]", b"[2,3]"), b"\0" * 8),
        "past_end": lambda: _write(tmp_path / "f", ok, b"\0" * 4),
        "huge_len": lambda: _write(tmp_path / "f", ok, b"\0" * 8, n=1 << 40),
        "bad_dtype": lambda: _write(tmp_path / "f", ok.replace(b"F16", b"Q7"), b"\0" * 8),
        "truncated": lambda: str(open(tmp_path / "f", "wb").write(b"\1\2\3") and tmp_path / "f"),
    }[case]()
    with pytest.raises(Exl3Error):
        Shard(p)
    # and the well-formed file opens
    s = Shard(_write(tmp_path / "g", ok, b"\1\0\2\0\3\0\4\0"))
    assert s.data("x").tolist() == [[1, 2], [3, 4]]
    s.close()
