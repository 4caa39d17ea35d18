"""GPU parity tests of the trellis tensor path through the C ABI.

Bit-exact against the oracle: decode (W_hat), reconstruct (W), the Hadamard steps.
Tolerance (stated per test) against the oracle's f64 GEMV: matmul_raw and linear. The
default weight form multiplies the reference's f16 weights (trellis_gemm.cpp:348-356),
the same values the oracle's default mode multiplies, so the tight f32-accumulation
bounds hold against it. The opt-in exact-halves form (exl3_tuning.weight_form = 1,
mcg/3inst) multiplies lo + hi unrounded and is held to the same tight bounds against
the oracle's exact-halves mode (oracle.gemv_mode(True)).
Bit-exact invariants of the reference (tests/glm5_gemv_nt_test.cpp, moe_test.cpp):
the row-block knob moves no byte, grouped == per-member, rows == single rows.
"""
import contextlib

import numpy as np
import pytest
import torch

from exl3_amd import synth
from exl3_amd.trellis import (TrellisWeight, f16_from_bits, trellis_decode, trellis_hadamard,
                              trellis_linear, trellis_linear_group, trellis_linear_group_rows,
                              trellis_linear_group_rows_scaled, trellis_matmul_raw,
                              trellis_pack, trellis_reconstruct, trellis_set_tuning)

pytestmark = pytest.mark.gpu
SEED = 77


@contextlib.contextmanager
def weight_form(oracle, form):
    """The process-wide weight form of the linear and the matching oracle mode."""
    trellis_set_tuning(weight_form=form)
    try:
        with oracle.gemv_mode(form == 1):
            yield
    finally:
        trellis_set_tuning()


def make(dev, in_f, out_f, K, cb, name, scale_std=0.05):
    words = synth.trellis_words(SEED, name, in_f, out_f, K)
    su = synth.normal_f16(SEED, name + ".suh", (in_f,), 1.0, scale_std)
    sv = synth.normal_f16(SEED, name + ".svh", (out_f,), 1.0, scale_std)
    w = TrellisWeight(trellis_pack(words, in_f // 16, out_f // 16, K, dev),
                      f16_from_bits(su, dev), f16_from_bits(sv, dev), in_f, out_f, K, cb)
    return w, words, su, sv


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().numpy().view(np.uint16)


def x_f16(dev, rows, n, name):
    return torch.from_numpy(synth.activations(SEED, name, rows, n).view(np.float16)).to(dev)


@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_decode_bit_exact(oracle, dev, K, cb):
    # 4096 x 4096 at every K and codebook
    w, words, _, _ = make(dev, 4096, 4096, K, cb, f"dec.{K}.{cb}")
    got = bits(trellis_decode(w))
    want = oracle.decode_inner(words, 4096, 4096, K, cb)
    assert np.array_equal(got, want)


def test_decode_small_and_ragged_shapes(oracle, dev):
    for (i, o, K, cb) in [(16, 16, 1, 0), (16, 48, 8, 2), (48, 16, 5, 1), (160, 272, 3, 0)]:
        w, words, _, _ = make(dev, i, o, K, cb, f"decs.{i}.{o}")
        assert np.array_equal(bits(trellis_decode(w)), oracle.decode_inner(words, i, o, K, cb))


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 6, 7, 8])
def test_reconstruct_bit_exact(oracle, dev, K):
    for cb in range(3):
        w, words, su, sv = make(dev, 512, 640, K, cb, f"rec.{K}.{cb}")
        got = bits(trellis_reconstruct(w))
        assert np.array_equal(got, oracle.reconstruct(words, 512, 640, K, cb, su, sv))


def test_hadamard_bit_exact(oracle, dev):
    x = synth.activations(SEED, "had.x", 7, 1024)
    s = synth.normal_f16(SEED, "had.s", (1024,), 1.0, 0.05)
    got = bits(trellis_hadamard(torch.from_numpy(x.view(np.float16)).to(dev),
                                f16_from_bits(s, dev), pre=True))
    assert np.array_equal(got, oracle.had_pre(x, s))
    y = synth.normal_f32(SEED, "had.y", (7, 1024), 0.0, 30.0)
    got = bits(trellis_hadamard(torch.from_numpy(y).to(dev), f16_from_bits(s, dev), pre=False))
    assert np.array_equal(got, oracle.had_post(y, s))
    # stacked: 3 members x 2 rows, one scale vector per member
    st = synth.normal_f16(SEED, "had.st", (3, 1024), 1.0, 0.05)
    x6 = synth.activations(SEED, "had.x6", 6, 1024)
    got = bits(trellis_hadamard(torch.from_numpy(x6.view(np.float16)).to(dev),
                                f16_from_bits(st, dev), pre=True, stacked=3))
    for m in range(3):
        assert np.array_equal(got[2 * m:2 * m + 2], oracle.had_pre(x6[2 * m:2 * m + 2], st[m]))


def gemv_bound(xhat_bits, what_bits):
    """Per-output bound for f32 accumulation against the f64 sum: 64 f32 ulps of
    sum_k |x_k w_kn| (a wrong decode or layout is off by O(|w| |x|) ~ 1)."""
    x = np.abs(xhat_bits.view(np.float16).astype(np.float64))
    w = np.abs(what_bits.view(np.float16).astype(np.float64))
    return 64 * 2.0 ** -24 * (x @ w)


def north_star(got_bits, want_bits):
    g = got_bits.view(np.float16).astype(np.float64).reshape(-1)
    r = want_bits.view(np.float16).astype(np.float64).reshape(-1)
    rms = np.sqrt(np.mean(r ** 2))
    cos = (g * r).sum() / np.sqrt((g ** 2).sum() * (r ** 2).sum())
    assert np.max(np.abs(g - r)) <= 2e-2 * rms and cos >= 0.9999, (np.max(np.abs(g - r)), rms, cos)


MM_CASES = [(1, 2, 0), (2, 0, 0), (3, 1, 0), (4, 1, 0), (5, 1, 0), (6, 0, 0), (8, 2, 0),
            (2, 0, 1), (4, 1, 1), (5, 1, 1), (7, 0, 1)]


@pytest.mark.parametrize("K,cb,form", MM_CASES)
def test_matmul_raw_vs_f64(oracle, dev, K, cb, form):
    in_f, out_f, rows = 4096, 1024, 3
    w, words, _, _ = make(dev, in_f, out_f, K, cb, f"mm.{K}.{cb}")
    xh = synth.normal_f16(SEED, f"mm.x.{K}", (rows, in_f), 0.0, 1.0)
    what = oracle.decode_inner(words, in_f, out_f, K, cb)
    bound = gemv_bound(xh, what)
    with weight_form(oracle, form):
        got = trellis_matmul_raw(w, torch.from_numpy(xh.view(np.float16)).to(dev)).cpu().numpy()
        want = oracle.matmul_raw(words, in_f, out_f, K, cb, xh)
    assert np.all(np.abs(got - want) <= bound)
    if form == 1:
        # against the reference's f16 weights: the f32 bound plus each weight's f16
        # rounding (at most 2^-11 of it)
        ref = oracle.matmul_raw(words, in_f, out_f, K, cb, xh)
        x = np.abs(xh.view(np.float16).astype(np.float64))
        extra = 2.0 ** -11 * (x @ np.abs(what.view(np.float16).astype(np.float64)))
        assert np.all(np.abs(got - ref) <= bound + extra)
        assert not np.array_equal(got, ref.astype(np.float32))


# f16 output tolerance of one linear: the f32-vs-f64 GEMV difference can move the f16
# rounding of yhat by one ulp before the output Hadamard mixes 128 of them.
LIN_TOL_RMS = 2e-3


def check_linear_tight(got, want):
    g = got.view(np.float16).astype(np.float64)
    r = want.view(np.float16).astype(np.float64).reshape(g.shape)
    rms = np.sqrt(np.mean(r ** 2))
    assert np.isfinite(g).all() and rms > 0.1
    assert np.max(np.abs(g - r)) <= LIN_TOL_RMS * rms
    assert np.mean(got.reshape(-1) == want.reshape(-1)) > 0.9


@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_linear_sweep_4096(oracle, dev, K, cb):
    # in = out = 4096, rows = 1, the default form against the reference's
    # f16 weights
    w, words, su, sv = make(dev, 4096, 4096, K, cb, f"lin.{K}.{cb}")
    x = synth.activations(SEED, f"lin.x.{K}.{cb}", 1, 4096)
    got = bits(trellis_linear(w, torch.from_numpy(x.view(np.float16)).to(dev)))
    want = oracle.trellis_linear(words, 4096, 4096, K, cb, su, sv, x)
    north_star(got, want)
    check_linear_tight(got, want)


@pytest.mark.parametrize("K", [1, 4, 5, 8])
@pytest.mark.parametrize("cb", [0, 1])
def test_linear_sweep_4096_halves_form(oracle, dev, K, cb):
    # the opt-in exact-halves form on configs[1] against the oracle's exact-halves mode
    w, words, su, sv = make(dev, 4096, 4096, K, cb, f"lin.{K}.{cb}")
    x = synth.activations(SEED, f"lin.x.{K}.{cb}", 1, 4096)
    with weight_form(oracle, 1):
        got = bits(trellis_linear(w, torch.from_numpy(x.view(np.float16)).to(dev)))
        want = oracle.trellis_linear(words, 4096, 4096, K, cb, su, sv, x)
    check_linear_tight(got, want)
    # and it is a different form: some outputs differ from the default form's
    assert not np.array_equal(got, bits(trellis_linear(w, torch.from_numpy(x.view(np.float16)).to(dev))))


def test_rows_invariance_and_row_block_knob(dev):
    w, *_ = make(dev, 2048, 1024, 3, 2, "inv")
    x = x_f16(dev, 13, 2048, "inv.x")
    base = bits(trellis_linear(w, x))
    for r in range(13):
        assert np.array_equal(bits(trellis_linear(w, x[r:r + 1].contiguous())), base[r:r + 1])
    try:
        for mb in (1, 2, 4, 5, 16):
            trellis_set_tuning(rows_per_pass=mb)
            assert np.array_equal(bits(trellis_linear(w, x)), base)
    finally:
        trellis_set_tuning()


def test_grouped_equals_members(dev):
    ws = [make(dev, 1024, 512, 4, 1, f"grp.{i}")[0] for i in range(5)]
    x = x_f16(dev, 2, 1024, "grp.x")
    g = bits(trellis_linear_group(ws, x))
    for i, w in enumerate(ws):
        assert np.array_equal(g[i], bits(trellis_linear(w, x)))
    xr = x_f16(dev, 5 * 3, 1024, "grp.xr").view(5, 3, 1024)
    gr = bits(trellis_linear_group_rows(ws, xr, 3))
    for i, w in enumerate(ws):
        assert np.array_equal(gr[i], bits(trellis_linear(w, xr[i].contiguous())))
    # scale-stack form with the members' own scales is bit-identical
    suh = torch.stack([w.suh for w in ws])
    svh = torch.stack([w.svh for w in ws])
    gs = bits(trellis_linear_group_rows_scaled(ws, xr, 3, suh, svh))
    assert np.array_equal(gs, gr)


def test_many_members_beyond_one_launch(dev):
    # more members than one kernel-argument table holds: chunked launches, same bytes
    w, words, su, sv = make(dev, 128, 128, 2, 0, "many")
    ws = [w] * 130
    x = x_f16(dev, 1, 128, "many.x")
    g = bits(trellis_linear_group(ws, x))
    one = bits(trellis_linear(w, x))
    assert all(np.array_equal(g[i], one) for i in range(130))


@pytest.mark.parametrize("K,cb", [(1, 0), (4, 1), (5, 2), (8, 1)])
def test_dword_aligned_base(dev, K, cb):
    # the ABI requires a 4-byte-aligned base (not 16): a copy at base + 4 bytes gives
    # the same bits as the 256-byte-aligned original
    w, *_ = make(dev, 1024, 512, K, cb, f"al.{K}.{cb}")
    big = torch.empty(w.packed.numel() + 2, dtype=torch.int16, device=dev)
    big[2:].copy_(w.packed.reshape(-1))
    moved = TrellisWeight(big[2:].view(w.packed.shape), w.suh, w.svh, w.in_features,
                          w.out_features, K, cb)
    assert moved.packed.data_ptr() % 16 == 4
    x = x_f16(dev, 3, 1024, f"al.x.{K}")
    assert np.array_equal(bits(trellis_linear(moved, x)), bits(trellis_linear(w, x)))
    assert np.array_equal(bits(trellis_decode(moved)), bits(trellis_decode(w)))


@pytest.mark.parametrize("i", range(12))
def test_linear_random_shapes(oracle, dev, i):
    # seeded random linears (in and out multiples of 128 up to 1280, every K and
    # codebook, 1..70 rows), in each weight form against the oracle's f64 linear in the
    # same form within the f16 bound below (the default form also at the north-star
    # tolerance), one row equal to that row alone, and the grouped call (this member
    # twice) equal to the single call
    rng = np.random.default_rng(9000 + i)
    in_f, out_f = 128 * int(rng.integers(1, 11)), 128 * int(rng.integers(1, 11))
    K, cb = int(rng.integers(1, 9)), int(rng.integers(0, 3))
    rows = int(rng.choice([1, 2, 5, 16, 17, 33, 70]))
    w, words, su, sv = make(dev, in_f, out_f, K, cb, f"rnd.{i}")
    xb = synth.activations(SEED, f"rnd.x.{i}", rows, in_f)
    x = torch.from_numpy(xb.view(np.float16)).to(dev)
    for form in ((0, 1) if cb != 2 else (0,)):
        with weight_form(oracle, form):
            got = bits(trellis_linear(w, x))
            want = oracle.trellis_linear(words, in_f, out_f, K, cb, su, sv, xb)
            if form == 0:
                north_star(got, want)
            g = got.view(np.float16).astype(np.float64)
            r = want.view(np.float16).astype(np.float64).reshape(g.shape)
            rms = np.sqrt(np.mean(r ** 2))
            assert np.isfinite(g).all() and rms > 0.01, (in_f, out_f, K, cb, rows)
            # yhat is rounded to f16 before the output Hadamard (trellis_gemm.cpp:397-399):
            # where the f32 GEMV lands within its error of an f16 rounding boundary that
            # yhat moves by one ulp, and the outputs of its 128-block move by at most one
            # ulp of their own. So: within 2 ulps of the largest output, and almost all
            # outputs bit-identical.
            ulp = 2.0 ** (np.floor(np.log2(np.abs(r).max())) - 10)
            err = np.max(np.abs(g - r))
            assert err <= 2 * ulp, (in_f, out_f, K, cb, rows, form, err, ulp)
            assert np.mean(got.reshape(-1) != want.reshape(-1)) <= 0.1, (in_f, out_f, K, cb, rows, form)
            j = rows // 2
            assert np.array_equal(bits(trellis_linear(w, x[j:j + 1].contiguous())), got[j:j + 1])
            grp = bits(trellis_linear_group([w, w], x))
            assert np.array_equal(grp[0], got) and np.array_equal(grp[1], got)
