"""CPU tests of the C ABI boundary: the library loads, exports every symbol the header
declares, and host-side validation answers without touching a GPU."""
import ctypes as C
import os

import numpy as np
import pytest

from exl3_amd import _lib
from exl3_amd._lib import TrellisDesc


def test_library_exports_every_header_symbol():
    L = _lib.lib()
    syms = _lib.header_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(L, s), s
    # the Python binding declares a signature for each of them
    assert sorted(_lib.SIGNATURES) == syms


def test_abi_version_and_tuning_roundtrip():
    L = _lib.lib()
    assert L.exl3_abi_version() == 2
    t0 = _lib.Tuning()
    _lib.call("exl3_get_tuning", C.byref(t0))
    # the reference's f16 weights by default
    assert t0.mat_min_rows == 16 and t0.weight_form == _lib.FORM_REFERENCE
    _lib.call("exl3_set_tuning", C.byref(_lib.Tuning(2, 0, 0, _lib.FORM_HALVES)))
    t1 = _lib.Tuning()
    _lib.call("exl3_get_tuning", C.byref(t1))
    assert (t1.rows_per_pass, t1.mat_min_rows, t1.weight_form) == (2, 0, _lib.FORM_HALVES)
    # a weight form outside the enum is refused and leaves the knobs as they were
    for bad in (2, -1):
        assert L.exl3_set_tuning(C.byref(_lib.Tuning(0, 16, 0, bad))) == 1
        assert b"weight_form" in L.exl3_last_error()
    t2 = _lib.Tuning()
    _lib.call("exl3_get_tuning", C.byref(t2))
    assert t2.weight_form == _lib.FORM_HALVES
    _lib.call("exl3_set_tuning", C.byref(t0))


def fake_desc(in_f=4096, out_f=1024, K=4, cb=1, base=0x10000):
    # never dereferenced: only host-side validation runs in these tests
    return TrellisDesc(base, base + 0x100000, base + 0x200000, in_f, out_f, K, cb)


def test_validation_errors_without_gpu():
    L = _lib.lib()
    info = _lib.PathInfo()
    for bad in (fake_desc(K=0), fake_desc(K=9), fake_desc(cb=3), fake_desc(in_f=100),
                fake_desc(out_f=0), fake_desc(base=0x10002)):
        st = L.exl3_trellis_path_info(C.byref(bad), 1, C.byref(info))
        assert st == _lib.EXL3_ERR_INVALID
        assert L.exl3_last_error()
    with pytest.raises(_lib.Exl3Error) as ei:
        _lib.call("exl3_trellis_linear", C.byref(fake_desc(K=11)), 0x1000, 1, 0x2000, None, 0,
                  None)
    assert ei.value.status == _lib.EXL3_ERR_INVALID
    assert b"K must be" in L.exl3_last_error()


def test_path_info_and_workspace_query():
    L = _lib.lib()
    info = _lib.PathInfo()
    d = fake_desc()
    _lib.call("exl3_trellis_path_info", C.byref(d), 8, C.byref(info))
    # one MFMA pass serves up to 16 token rows
    assert info.staged == 0 and info.rows_per_block == 8 and info.passes == 1
    assert info.splits == 8  # 256 k-tiles: 8 slices of 8 wave steps of 4 k-tiles
    _lib.call("exl3_trellis_path_info", C.byref(d), 40, C.byref(info))
    assert info.staged == 1 and info.rows_per_block == 16 and info.passes == 3
    ws1 = L.exl3_trellis_workspace_size(C.byref(d), 1, 1)
    ws8 = L.exl3_trellis_workspace_size(C.byref(d), 8, 3)
    assert 0 < ws1 < ws8
    assert ws1 >= 8 * 1024 * 4  # 8 slice planes of f32 partials


def test_workspace_too_small_is_reported_before_launch():
    L = _lib.lib()
    d = fake_desc()
    st = L.exl3_trellis_linear(C.byref(d), 0x1000, 1, 0x2000, 0x100000, 16, None)
    assert st == _lib.EXL3_ERR_WORKSPACE


def test_topk_route_rejects_bad_config():
    L = _lib.lib()
    cfg = _lib.MoeConfig(0, 0, 5, 6, 1, 1, 1, 1.0, 0.0)  # top_k > E
    st = L.exl3_moe_topk_route(0x1000, 0x2000, 1, C.byref(cfg), 0x3000, 0x4000, None)
    assert st == _lib.EXL3_ERR_INVALID
    cfg = _lib.MoeConfig(0, 0, 2048, 8, 1, 1, 1, 1.0, 0.0)  # too many experts
    assert L.exl3_moe_topk_route(0x1000, 0x2000, 1, C.byref(cfg), 0x3000, 0x4000,
                                 None) == _lib.EXL3_ERR_UNSUPPORTED


def test_synth_generator_is_counter_based():
    from exl3_amd import synth
    a = synth.trellis_words(1, "t", 32, 64, 3)
    b = synth.trellis_words(1, "t", 32, 64, 3)
    c = synth.trellis_words(1, "u", 32, 64, 3)
    assert a.shape == (2, 4, 48) and np.array_equal(a, b) and not np.array_equal(a, c)
    # uniform 16-bit words: mean near 32767.5
    assert abs(a.astype(np.float64).mean() - 32767.5) < 2000
    x = synth.normal(2, "n", (100000,))
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1) < 0.02


@pytest.mark.parametrize("compiler,std", [("gcc", "-std=c11"), ("g++", "-std=c++17")])
def test_header_compiles_and_links(tmp_path, compiler, std):
    # include/exl3_moe.h as a C and as a C++ translation unit, linked against the
    # library, calling host-only entry points (the binding a C or C++ engine would add)
    import shutil
    import subprocess
    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} not available")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    libdir = os.path.dirname(_lib.LIB_PATH)
    exe = tmp_path / "abi_probe"
    src = os.path.join(root, "tests", "abi_c", "abi_probe.c")
    lang = ["-x", "c++"] if compiler == "g++" else []
    subprocess.run([compiler, std, "-Wall", "-Wextra", "-Werror", "-I", os.path.join(root, "include"),
                    *lang, src, "-x", "none", "-L", libdir, "-lexl3moe", f"-Wl,-rpath,{libdir}",
                    "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True)
    assert out.stdout.strip() == "ok"


def test_cpp_layer_probe_compiles_and_links(tmp_path):
    # the C++ layer caller (run on a GPU by test_gpu_abi_cpp) builds against the header,
    # the library and the HIP runtime; without arguments it prints its usage only
    import shutil
    import subprocess
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    if shutil.which("g++") is None or not os.path.exists(os.path.join(rocm, "include", "hip")):
        pytest.skip("g++ or the HIP headers not available")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    libdir = os.path.dirname(_lib.LIB_PATH)
    exe = tmp_path / "moe_cpp_probe"
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
                    "-I", os.path.join(root, "include"), "-I", os.path.join(rocm, "include"),
                    os.path.join(root, "tests", "abi_c", "moe_cpp_probe.cpp"),
                    "-L", libdir, "-lexl3moe", f"-Wl,-rpath,{libdir}",
                    "-L", os.path.join(rocm, "lib"), "-lamdhip64", "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 2 and "usage" in out.stderr
