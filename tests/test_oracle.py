"""CPU tests that pin the oracle (oracle/exl3_oracle.c) -- no GPU.

Each oracle function is checked against something other than its own formula:
golden vectors written from the reference's src/exl3.cpp (tests/golden/), numpy's
float16 as a second f16 implementation, bit-by-bit brute force, explicit Sylvester
matrices, the reference test's router known answers (tests/moe_test.cpp (a)/(b)),
and an independent numpy f64 restatement of the layer on dequantised weights.
"""
import hashlib
import json
import os

import numpy as np
import pytest

from exl3_amd import synth
from layer_cases import LIMIT_HALF_CASES, limit_half_case

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a, np.uint16).astype("<u2").tobytes()).hexdigest()


# --- f16 rounding (reference fp16.h:18-64) ------------------------------------------------

def test_f16_roundtrip_exhaustive(oracle):
    # every one of the 65,536 f16 patterns: f16 -> f64 equals numpy's widening, and
    # f64 -> f16 returns the same pattern (NaNs to the canonical quiet NaN)
    L = oracle.lib()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = bits.view(np.float16).astype(np.float64)
    back = np.array([L.or_f16_from_double(float(v)) for v in vals], np.uint32)
    wide = np.array([L.or_f16_to_double(int(b)) for b in bits], np.float64)
    nan = np.isnan(vals)
    assert np.array_equal(back[~nan], bits[~nan].astype(np.uint32))
    assert np.all(back[nan] == 0x7E00)
    assert np.array_equal(wide[~nan], vals[~nan])
    assert np.all(np.isnan(wide[nan]))


def test_f16_ties_to_even_vs_numpy(oracle):
    L = oracle.lib()
    # midpoints between every pair of adjacent finite positive f16 values, plus
    # points a quarter ulp either side: numpy's float16 cast is RNE from f64.
    pos = np.arange(0, 0x7C00, dtype=np.uint16)
    lo = pos[:-1].view(np.float16).astype(np.float64)
    hi = pos[1:].view(np.float16).astype(np.float64)
    probe = np.concatenate([(lo + hi) / 2, lo + (hi - lo) / 4, hi - (hi - lo) / 4])
    probe = np.concatenate([probe, -probe])
    want = probe.astype(np.float16).view(np.uint16)
    got = np.array([L.or_f16_from_double(float(x)) for x in probe], np.uint16)
    assert np.array_equal(got, want)


def test_f16_edges(oracle):
    L = oracle.lib()
    assert L.or_f16_from_double(65504.0) == 0x7BFF
    assert L.or_f16_from_double(65519.99) == 0x7BFF
    assert L.or_f16_from_double(65520.0) == 0x7C00        # rounds up to inf
    assert L.or_f16_from_double(-1e9) == 0xFC00
    assert L.or_f16_from_double(2.0 ** -25) == 0x0000     # tie to even -> 0
    assert L.or_f16_from_double(2.0 ** -25 * 1.0001) == 0x0001
    assert L.or_f16_from_double(-0.0) == 0x8000
    assert L.or_f16_from_double(float("nan")) == 0x7E00


# --- codebooks (reference exl3.cpp:21-42) ---------------------------------------------------

@pytest.mark.parametrize("cb", [0, 1, 2])
def test_codebook_golden(oracle, cb):
    g = json.load(open(os.path.join(GOLDEN, "codebooks.json")))[str(cb)]
    lut = oracle.codebook_lut(cb)
    assert sha(lut) == g["sha256"]
    for s, v in g["samples"]:
        assert int(lut[s]) == v
    vals = lut.view(np.float16).astype(np.float64)
    assert np.isfinite(vals).all()
    assert vals.min() == g["min"] and vals.max() == g["max"]


@pytest.mark.parametrize("cb", [0, 1])
def test_halves_sum_rounds_to_reference(oracle, cb):
    # the exact-halves GEMV weight is the reference weight before its one f16 rounding:
    # RNE of it is the reference's (golden-pinned) value for every state, and it lies
    # within half an f16 ulp of that value
    exact = oracle.halves_sum_lut(cb).astype(np.float64)
    ref_bits = oracle.codebook_lut(cb)
    assert np.array_equal(exact.astype(np.float16).view(np.uint16), ref_bits)
    ref = ref_bits.view(np.float16).astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(exact - ref) <= ulp / 2)
    assert np.any(exact != ref)  # the rounding does move some weights
    # and it is the sum of the two halves by hand for a few states
    C = 0xCBAC1FED if cb == 1 else 89226354
    for st in (0, 1, 12345, 65535):
        x = (st * C + (0 if cb == 1 else 64248484)) & 0xFFFFFFFF
        x = (x & 0x8FFF8FFF) ^ 0x3B603B60
        lo = np.array([x & 0xFFFF], np.uint16).view(np.float16)[0]
        hi = np.array([x >> 16], np.uint16).view(np.float16)[0]
        assert exact[st] == float(lo) + float(hi)


def test_gemv_mode_switches_weights(oracle):
    # mode 1 changes the mcg GEMV by at most the weight rounding, and mul1 not at all
    rng = np.random.default_rng(5)
    in_f, out_f, K = 256, 128, 3
    tr = rng.integers(0, 65536, size=(in_f // 16, out_f // 16, 16 * K), dtype=np.uint16)
    x = rng.normal(size=(2, in_f)).astype(np.float16).view(np.uint16)
    for cb in (1, 2):
        a = oracle.matmul_raw(tr, in_f, out_f, K, cb, x)
        with oracle.gemv_mode(True):
            b = oracle.matmul_raw(tr, in_f, out_f, K, cb, x)
        w = oracle.decode_inner(tr, in_f, out_f, K, cb).view(np.float16).astype(np.float64)
        bound = (np.abs(x.view(np.float16).astype(np.float64)) @ np.abs(w)) * 2.0 ** -11
        if cb == 2:
            assert np.array_equal(a, b)
        else:
            assert np.all(np.abs(a - b) <= bound) and not np.array_equal(a, b)
    assert oracle.lib().or_get_gemv_mode() == 0


def test_codebook_closed_form_ranges(oracle):
    # mul1: f16(0x6400 + bytesum) is an integer in [1024, 2044]; the fma maps it
    # monotonically into [1024*inv + bias, 2044*inv + bias].
    inv = float(np.uint16(0x1EEE).view(np.float16))
    bias = float(np.uint16(0xC931).view(np.float16))
    v = oracle.codebook_lut(2).view(np.float16).astype(np.float64)
    assert v.min() >= np.float16(1024 * inv + bias) - 1e-3
    assert v.max() <= np.float16(2044 * inv + bias) + 1e-3
    # mcg / 3inst: each half has exponent field in 12..15 (values in [1/8, 2)), so the
    # sum's magnitude is below 4 and above 0 unless the halves cancel exactly.
    for cb in (0, 1):
        v = oracle.codebook_lut(cb).view(np.float16).astype(np.float64)
        assert np.abs(v).max() < 4.0


def test_codebook_value_matches_hash_by_hand(oracle):
    # one state by hand per codebook
    s = 0x1234
    x = (s * 0xCBAC1FED) & 0xFFFFFFFF
    x = (x & 0x8FFF8FFF) ^ 0x3B603B60
    want = np.float16(float(np.uint16(x & 0xFFFF).view(np.float16)) +
                      float(np.uint16(x >> 16).view(np.float16)))
    assert oracle.lib().or_codebook_value(s, 1) == int(want.view(np.uint16))
    x = (s * 89226354 + 64248484) & 0xFFFFFFFF
    x = (x & 0x8FFF8FFF) ^ 0x3B603B60
    want = np.float16(float(np.uint16(x & 0xFFFF).view(np.float16)) +
                      float(np.uint16(x >> 16).view(np.float16)))
    assert oracle.lib().or_codebook_value(s, 0) == int(want.view(np.uint16))
    x = (s * 0x83DCD12D) & 0xFFFFFFFF
    bsum = sum((x >> (8 * i)) & 0xFF for i in range(4))
    val = float(np.uint16(0x6400 + bsum).view(np.float16))
    want = np.float16(val * float(np.uint16(0x1EEE).view(np.float16)) +
                      float(np.uint16(0xC931).view(np.float16)))
    assert oracle.lib().or_codebook_value(s, 2) == int(want.view(np.uint16))


# --- ring windows and permutation (reference exl3.cpp:55-107) -------------------------------

@pytest.mark.parametrize("K", range(1, 9))
def test_tile_state_bruteforce(oracle, K):
    L = oracle.lib()
    for trial in range(3):
        t = synth.trellis_words(5 + trial, f"bf.{K}", 16, 16, K).reshape(-1)
        for p in range(256):
            assert L.or_tile_state(t, K, p) == L.or_tile_state_bruteforce(t, K, p)


def test_tile_perm_is_bijection(oracle):
    L = oracle.lib()
    seen = sorted(L.or_tile_perm(p) for p in range(256))
    assert seen == list(range(256))
    # reference lane 0's first four positions are rows {0,1,8,9} of column 0
    assert [L.or_tile_perm(p) for p in range(4)] == [0, 16, 128, 144]
    assert L.or_tile_perm(4) == 8  # i = 4 -> column 8


def test_state_window_by_hand(oracle):
    # K = 1, all words zero except the very first ring bit: position p's window ends at
    # bit p+1, so ring bit 0 is the LSB of p=0 and bit 15 of p=15 (the MSB), and no
    # other position sees it except through the ring wrap of the last 15 positions.
    t = np.zeros(16, np.uint16)
    t[1] = 0x8000  # ring word 0 = s[0] | s[1] << 16 -> bit 31 set = ring bit 0
    L = oracle.lib()
    assert L.or_tile_state(t, 1, 0) == 1
    assert L.or_tile_state(t, 1, 15) == 1 << 15
    assert L.or_tile_state(t, 1, 16) == 0
    assert L.or_tile_state(t, 1, 255) == 0  # window = ring bits 240..255
    assert L.or_tile_state(t, 1, 14) == 1 << 14


# --- decode / reconstruct golden (reference exl3.cpp:109-209) ---------------------------------

def test_decode_golden_small(oracle):
    z = np.load(os.path.join(GOLDEN, "decode.npz"))
    for K in range(1, 9):
        for cb in range(3):
            w = oracle.decode_inner(z[f"words_{K}_{cb}"], 32, 32, K, cb)
            assert np.array_equal(w, z[f"what_{K}_{cb}"]), (K, cb)


def test_decode_golden_hash(oracle):
    g = json.load(open(os.path.join(GOLDEN, "decode.json")))
    for key, c in g["cases"].items():
        K, cb = map(int, key.split("_"))
        words = synth.trellis_words(g["seed"], c["name"], 128, 256, K)
        w = oracle.decode_inner(words, 128, 256, K, cb)
        assert sha(w) == c["sha256"], key
        flat = w.reshape(-1)
        assert all(int(flat[i]) == v for i, v in c["samples"])


def test_reconstruct_golden(oracle):
    g = json.load(open(os.path.join(GOLDEN, "reconstruct.json")))
    z = np.load(os.path.join(GOLDEN, "reconstruct.npz"))
    for key, c in g["cases"].items():
        K, cb = map(int, key.split("_"))
        words = synth.trellis_words(g["seed"], c["name"], 256, 384, K)
        w = oracle.reconstruct(words, 256, 384, K, cb, z[f"suh_{key}"], z[f"svh_{key}"])
        assert sha(w) == c["sha256"], key
    for cb in range(3):
        w = oracle.reconstruct(z[f"full_words_{cb}"], 128, 128, 4, cb, z[f"full_suh_{cb}"],
                               z[f"full_svh_{cb}"])
        assert np.array_equal(w, z[f"full_w_{cb}"])


def test_reference_lib_agrees_when_present(oracle):
    R = oracle.ref_lib()
    if R is None:
        pytest.skip("reference codec not built here (it is built in the build container only)")
    for K in (1, 3, 6, 8):
        for cb in range(3):
            words = synth.trellis_words(99, f"xref.{K}.{cb}", 256, 128, K)
            ref = np.zeros((256, 128), np.uint16)
            R.ref_decode_inner(words.reshape(-1), 256, 128, K, cb, ref, 2)
            assert np.array_equal(oracle.decode_inner(words, 256, 128, K, cb), ref)


def sylvester(n=128):
    H = np.array([[1.0]])
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H


def test_sylvester_identity_and_reconstruct(oracle):
    H = sylvester()
    assert np.array_equal(H @ H, 128 * np.eye(128))
    # reconstruct == f16(diag(suh) H W_hat H diag(svh) / 128) up to f32 rounding
    K, cb = 4, 1
    words = synth.trellis_words(3, "syl", 128, 128, K)
    # widely spread scales so that swapping them is visible
    su = np.abs(synth.normal(3, "syl.suh", (128,), 1.0, 0.6)).astype(np.float16).view(np.uint16)
    sv = np.abs(synth.normal(3, "syl.svh", (128,), 1.0, 0.6)).astype(np.float16).view(np.uint16)
    what = oracle.decode_inner(words, 128, 128, K, cb).view(np.float16).astype(np.float64)
    s_u = su.view(np.float16).astype(np.float64)
    s_v = sv.view(np.float16).astype(np.float64)
    want = (s_u[:, None] * (H @ what @ H) * s_v[None, :]) / 128.0
    got = oracle.reconstruct(words, 128, 128, K, cb, su, sv).view(np.float16).astype(np.float64)
    assert np.max(np.abs(got - want)) <= 2e-3 * np.max(np.abs(want))
    # a transposed operand or a missing scale is off by O(1)
    for wrong in ((s_v[:, None] * (H @ what @ H) * s_u[None, :]) / 128.0,
                  (s_u[:, None] * (H @ what.T @ H) * s_v[None, :]) / 128.0,
                  (s_u[:, None] * (what @ H) * s_v[None, :]) / 128.0 * np.sqrt(128)):
        assert np.max(np.abs(got - wrong)) > 0.1 * np.max(np.abs(want))


def test_had_pre_post_vs_sylvester(oracle):
    H = sylvester()
    # exact small integers: the butterflies are exact, so only the stated rounding
    # points remain (f32 scale multiply, one f16 rounding)
    rng = np.random.default_rng(0)
    x = rng.integers(-8, 9, size=(3, 256)).astype(np.float16)
    s = np.ones(256, np.float16)
    got = oracle.had_pre(x.view(np.uint16), s.view(np.uint16)).view(np.float16)
    scale = np.float32(1.0) / np.float32(11.313708498984761)
    for r in range(3):
        for b in range(2):
            blk = (H @ x[r, b * 128:(b + 1) * 128].astype(np.float64)).astype(np.float32)
            want = (blk * scale).astype(np.float16)
            assert np.array_equal(got[r, b * 128:(b + 1) * 128], want)
    sv = rng.uniform(0.5, 1.5, 256).astype(np.float16)
    y = rng.integers(-8, 9, size=(2, 256)).astype(np.float32)
    got = oracle.had_post(y, sv.view(np.uint16)).view(np.float16)
    for r in range(2):
        for b in range(2):
            blk = (H @ y[r, b * 128:(b + 1) * 128].astype(np.float64)).astype(np.float32)
            want = ((blk * scale) * sv[b * 128:(b + 1) * 128].astype(np.float32)).astype(np.float16)
            assert np.array_equal(got[r, b * 128:(b + 1) * 128], want)


def test_trellis_linear_vs_dense(oracle):
    # trellis_linear(x) == x @ reconstruct-in-f64 within f16 rounding
    K, cb, n_in, n_out = 5, 2, 256, 384
    words = synth.trellis_words(4, "lin", n_in, n_out, K)
    su = synth.normal_f16(4, "lin.suh", (n_in,), 1.0, 0.05)
    sv = synth.normal_f16(4, "lin.svh", (n_out,), 1.0, 0.05)
    x = synth.normal_f16(4, "lin.x", (3, n_in))
    y = oracle.trellis_linear(words, n_in, n_out, K, cb, su, sv, x).view(np.float16).astype(np.float64)
    H = sylvester()
    what = oracle.decode_inner(words, n_in, n_out, K, cb).view(np.float16).astype(np.float64)
    Hi = np.kron(np.eye(n_in // 128), H)
    Ho = np.kron(np.eye(n_out // 128), H)
    W = (su.view(np.float16).astype(np.float64)[:, None] * (Hi @ what @ Ho) *
         sv.view(np.float16).astype(np.float64)[None, :]) / 128.0
    want = x.view(np.float16).astype(np.float64) @ W
    rms = np.sqrt(np.mean(want ** 2))
    assert np.max(np.abs(y - want)) <= 2e-2 * rms


# --- router (reference glm5_moe.cpp:16-60; tests/moe_test.cpp:225-275) ----------------------

def test_router_logits_vs_numpy(oracle):
    # logits = f32(h) . f32(router_w)^T with router_w (E, H) row-major as on disk
    # (reference glm5_moe.cpp:127-128, glm5.cpp:506). A non-square layer, so that reading
    # the weight as (H, E), or contracting the wrong axis, cannot pass.
    rng = np.random.default_rng(11)
    N, E, H = 5, 24, 384
    h = rng.normal(size=(N, H)).astype(np.float16)
    w = (rng.normal(size=(E, H)) * 0.02).astype(np.float16)
    got = oracle.router_logits(h.view(np.uint16), w.view(np.uint16))
    want = h.astype(np.float64) @ w.astype(np.float64).T
    assert got.shape == (N, E)
    assert np.max(np.abs(got - want)) <= 1e-12 * np.max(np.abs(want))
    # the transposed layout (the same bytes read as (H, E)) is far off
    wt = w.reshape(-1).reshape(H, E).astype(np.float64)
    wrong = h.astype(np.float64) @ wt
    assert np.max(np.abs(wrong - want)) > 0.1 * np.max(np.abs(want))
    # row t of the logits depends on row t of h only
    got2 = oracle.router_logits(h[2:3].view(np.uint16), w.view(np.uint16))
    assert np.array_equal(got2[0], got[2])


def test_router_known_answer_bias_flips(oracle):
    cfg = oracle.make_cfg(2, 3, 5, 2, 1, 1, True, True, 2.5, 10.0)
    logits = np.array([[2.0, 1.0, 0.5, -2.0, -3.0]])
    bias = np.array([0.0, 0.0, 0.0, 0.8, 0.75], np.float32)
    idx, w = oracle.route(logits, bias, cfg)
    assert sorted(idx[0].tolist()) == [0, 3]
    got = dict(zip(idx[0].tolist(), w[0].tolist()))
    assert abs(got[0] - 2.201993) < 1e-4
    assert abs(got[3] - 0.298008) < 1e-4


def test_router_known_answer_group_limit(oracle):
    cfg = oracle.make_cfg(2, 3, 4, 2, 2, 1, False, True, 1.0, 10.0)
    idx, _ = oracle.route(np.array([[1.0, 0.9, 2.0, -1.0]]), np.zeros(4, np.float32), cfg)
    assert sorted(idx[0].tolist()) == [0, 1]


def test_router_bruteforce_subsets(oracle):
    # tiny E: the top-k set is the k-subset with the largest biased scores
    rng = np.random.default_rng(1)
    E, K = 7, 3
    cfg = oracle.make_cfg(8, 8, E, K, 1, 1, True, True, 1.7, 10.0)
    for _ in range(50):
        lg = rng.normal(size=(1, E))
        b = rng.normal(scale=0.1, size=E).astype(np.float32)
        idx, w = oracle.route(lg, b, cfg)
        sc = 1 / (1 + np.exp(-lg[0]))
        sfc = sc + b.astype(np.float64)
        best = np.argsort(-sfc, kind="stable")[:K]
        assert set(idx[0].tolist()) == set(best.tolist())
        assert list(idx[0]) == list(best)  # descending order
        ww = sc[best] / (sc[best].sum() + 1e-20) * np.float32(1.7)
        assert np.allclose(w[0], ww, rtol=1e-12)


# --- dispatch (reference glm5_moe.cpp:158-255) ----------------------------------------------

def test_runs_by_hand(oracle):
    idx = np.array([[3, 1], [1, 0], [3, 2]], np.int32)  # 3 rows, top-2
    r = oracle.moe_runs(idx)
    # stable by expert, pair order (row, rank): e0:(1,1) e1:(0,1),(1,0) e2:(2,1) e3:(0,0),(2,0)
    assert r["sorted_expert"].tolist() == [0, 1, 1, 2, 3, 3]
    assert r["sorted_row"].tolist() == [1, 0, 1, 2, 0, 2]
    assert r["sorted_rank"].tolist() == [1, 1, 0, 1, 0, 0]
    assert r["run_expert"].tolist() == [0, 1, 2, 3]
    assert r["run_len"].tolist() == [1, 2, 1, 2]
    assert r["run_off"].tolist() == [0, 1, 3, 4]
    # perm[rank * N + row] = sorted position
    assert r["perm"].tolist() == [4, 2, 5, 1, 0, 3]


def test_runs_chunked_geometry(oracle):
    # the reference's (h) case: 11 rows x 3 ranks over 4 experts
    rng = np.random.default_rng(7)
    idx = np.stack([rng.permutation(4)[:3] for _ in range(11)]).astype(np.int32)
    r = oracle.moe_runs(idx)
    assert r["run_len"].sum() == 33
    P = 33
    for pos in range(P):
        row, rank = r["sorted_row"][pos], r["sorted_rank"][pos]
        assert idx[row, rank] == r["sorted_expert"][pos]
        assert r["perm"][rank * 11 + row] == pos
    assert np.all(np.diff(r["sorted_expert"]) >= 0)


# --- the layer ---------------------------------------------------------------------------

def numpy_layer(layer, h_bits, idx, w, oracle):
    """Independent f64 restatement on dequantised weights (no intermediate f16 rounding
    except the f16 inputs); the oracle must agree to f16 tolerance."""
    cfg = layer.cfg

    def W(lin):
        if lin.quantized:
            return oracle.reconstruct(lin.trellis, lin.in_f, lin.out_f, lin.K, lin.cb, lin.suh,
                                      lin.svh).view(np.float16).astype(np.float64)
        return lin.dense.view(np.float16).astype(np.float64)

    def swiglu(ls, x):
        g = x @ W(ls[0])
        u = x @ W(ls[1])
        g = np.minimum(g, cfg.swiglu_limit)
        u = np.clip(u, -cfg.swiglu_limit, cfg.swiglu_limit)
        return (g / (1 + np.exp(-g)) * u) @ W(ls[2])

    x = h_bits.view(np.float16).astype(np.float64)
    out = np.zeros_like(x)
    for b in range(x.shape[0]):
        for k in range(cfg.top_k):
            e = idx[b, k]
            out[b] += w[b, k] * swiglu(layer.experts[3 * e:3 * e + 3], x[b:b + 1])[0]
    if layer.shared is not None:
        out += swiglu(layer.shared, x)
    return out


def test_oracle_layer_small_vs_numpy(oracle):
    cfg = synth.MoeConfig(hidden=256, inter=128, n_experts=6, top_k=2, routed_scaling_factor=1.5,
                          shared_inter=128, gate_up_K=3, gate_up_cb=2, down_K=4, down_cb=1)
    layer = synth.make_layer(cfg, 11)
    h = synth.activations(11, "x", 5, cfg.hidden)
    ocfg = oracle.make_cfg(cfg.hidden, cfg.inter, cfg.n_experts, cfg.top_k, 1, 1, True, True,
                           cfg.routed_scaling_factor, cfg.swiglu_limit)
    out, idx, w = oracle.moe_layer(ocfg, [l.oracle_dict() for l in layer.experts],
                                   [l.oracle_dict() for l in layer.shared], layer.router_w,
                                   layer.bias, h)
    want = numpy_layer(layer, h, idx, w, oracle)
    got = out.view(np.float16).astype(np.float64)
    rms = np.sqrt(np.mean(want ** 2))
    assert rms > 1e-3
    assert np.max(np.abs(got - want)) <= 2e-2 * rms
    cos = (got * want).sum() / np.sqrt((got ** 2).sum() * (want ** 2).sum())
    assert cos >= 0.9999
    # a routing mistake (dropping the second expert) is far outside that bound
    w2 = w.copy()
    w2[:, 1] = 0
    wrong = numpy_layer(layer, h, idx, w2, oracle)
    assert np.max(np.abs(got - wrong)) > 2e-2 * rms


def test_oracle_layer_rows_equal_single_rows(oracle):
    cfg = synth.MoeConfig(hidden=128, inter=128, n_experts=4, top_k=3, routed_scaling_factor=1.5,
                          gate_up_K=3, gate_up_cb=2, down_K=3, down_cb=2)
    layer = synth.make_layer(cfg, 5)
    ocfg = oracle.make_cfg(128, 128, 4, 3, 1, 1, True, False, 1.5, 10.0)
    h = synth.activations(5, "rows", 11, 128)
    ex = [l.oracle_dict() for l in layer.experts]
    out, _, _ = oracle.moe_layer(ocfg, ex, None, layer.router_w, layer.bias, h)
    for b in range(11):
        one, _, _ = oracle.moe_layer(ocfg, ex, None, layer.router_w, layer.bias, h[b:b + 1])
        assert np.array_equal(one[0], out[b])


def test_oracle_swiglu_clip_like_mlx(oracle):
    # mx::clip(gate, none, L) and mx::clip(up, -L, L) apply whatever L is
    # (glm5_moe.cpp:70-71): L = 0 zeroes the layer output; a small L bounds every
    # SwiGLU value by L * silu(L)
    for limit in (0.0, 0.25):
        cfg = synth.MoeConfig(hidden=256, inter=128, n_experts=6, top_k=2, swiglu_limit=limit,
                              shared_inter=128, gate_up_K=3, gate_up_cb=2, down_K=4, down_cb=1)
        layer = synth.make_layer(cfg, 12)
        h = synth.activations(12, "lim", 4, cfg.hidden)
        ocfg = oracle.make_cfg(cfg.hidden, cfg.inter, cfg.n_experts, cfg.top_k, 1, 1, True, True,
                               cfg.routed_scaling_factor, cfg.swiglu_limit)
        out, idx, w = oracle.moe_layer(ocfg, [l.oracle_dict() for l in layer.experts],
                                       [l.oracle_dict() for l in layer.shared], layer.router_w,
                                       layer.bias, h)
        got = out.view(np.float16).astype(np.float64)
        want = numpy_layer(layer, h, idx, w, oracle)
        if limit == 0.0:
            assert not np.any(got) and not np.any(want)
        else:
            rms = np.sqrt(np.mean(want ** 2))
            assert rms > 1e-4 and np.max(np.abs(got - want)) <= 2e-2 * rms


@pytest.mark.parametrize("seed,i,B", LIMIT_HALF_CASES)
def test_limit_half_cases_separate_the_forms(oracle, seed, i, B):
    # the GPU parity cases at a SwiGLU limit of 0.5 (tests/layer_cases.py): the oracle on
    # the reference's f16 weights and the oracle on exact halves differ by more than the
    # north-star bound (2e-2 of the RMS), so a GEMV that multiplied the exact halves could
    # not pass the reference-weight check there, and the other way round
    cfg, layer, h = limit_half_case(seed, i, B)
    has = cfg.shared_inter > 0
    oc = oracle.make_cfg(cfg.hidden, cfg.inter, cfg.n_experts, cfg.top_k, cfg.n_group, cfg.topk_group,
                         cfg.norm_topk_prob, has, cfg.routed_scaling_factor, cfg.swiglu_limit)
    ex = [l.oracle_dict() for l in layer.experts]
    sh = [l.oracle_dict() for l in layer.shared] if has else None
    ref, _, _ = oracle.moe_layer(oc, ex, sh, layer.router_w, layer.bias, h)
    with oracle.gemv_mode(True):
        exact, _, _ = oracle.moe_layer(oc, ex, sh, layer.router_w, layer.bias, h)
    a = ref.view(np.float16).astype(np.float64)
    b = exact.view(np.float16).astype(np.float64)
    assert np.max(np.abs(a - b)) > 2e-2 * np.sqrt(np.mean(a ** 2))
