"""exl3_trellis_linear at the reference's real tensor classes (tests/glm5_gemv_nt_test.cpp
:143-172: the 25 (in, out, K) classes of the GLM-5 checkpoint's text tower, lm_head
4096x154880 K6 to mla kv_a 4096x512 K4) and row counts {1, 2, 3, 4, 13, 26} (:323-387).

Per class, on uniform random trellis words with N(1, 0.05) scales (the reference's
make_trellis, :60-76; mul1 as there, plus mcg and 3inst on three classes):
  - parity: sampled 128-column blocks (the first, a seeded one, the last) against the
    oracle's f64 linear on the sub-tensor of those columns (a column block of a trellis
    tensor is itself a trellis tensor: its tiles (tk, tn) for tn in the block, with the
    block's svh), at the north-star bound (max |err| <= 2e-2 * rms, cosine >= 0.9999)
    and within 2 output ulps (the bound of test_linear_random_shapes) of the oracle on
    the reference's f16 weights; the mcg/3inst classes also in the opt-in exact-halves
    weight form against the oracle's exact-halves mode. At most a quarter of the sampled
    outputs of a class may differ from the oracle at all: a yhat element within f32
    round-off of an f16 rounding boundary (about 0.5% of them) moves every output of its
    128-block by about 1/8 ulp through the output Hadamard, so about half the blocks carry
    such a move and about an eighth of their outputs round differently;
  - the reference's invariance: a row of a multi-row call equals that row alone, and the
    row-block knob (rows_per_pass) moves no byte.
"""
import numpy as np
import pytest
import torch

from exl3_amd import synth
from exl3_amd.moe import trellis_words_torch
from exl3_amd.trellis import TrellisWeight, f16_from_bits, trellis_linear, trellis_set_tuning

pytestmark = pytest.mark.gpu
SEED = 4242

# (name, in, out, K, codebook): glm5_gemv_nt_test.cpp:147-171, mul1 as its make_trellis
REAL_SHAPES = [
    ("lm_head", 4096, 154880, 6, 2),
    ("kda_qkv_proj", 4096, 24576, 4, 2),
    ("mla_o_proj_k6", 16384, 4096, 6, 2),
    ("mla_o_proj_k4", 16384, 4096, 4, 2),
    ("mtp_eh_proj", 8192, 4096, 5, 2),
    ("dense_down", 12288, 4096, 3, 2),
    ("dense_gate_up", 4096, 12288, 3, 2),
    ("mla_q_b_k6", 1536, 16384, 6, 2),
    ("kda_o_proj", 8192, 4096, 4, 2),
    ("mla_q_b_k4", 1536, 16384, 4, 2),
    ("shared_down_k6", 2048, 4096, 6, 2),
    ("shared_gate_up_k6", 4096, 2048, 6, 2),
    ("indexer_wq_b_1536x4096_k6", 1536, 4096, 6, 2),
    ("indexer_wq_b_4096x1536_k6", 4096, 1536, 6, 2),
    ("shared_down_k4", 2048, 4096, 4, 2),
    ("shared_gate_up_k4", 4096, 2048, 4, 2),
    ("exp_down_k3", 2048, 4096, 3, 2),
    ("exp_gate_up_k3", 4096, 2048, 3, 2),
    ("indexer_wq_b_1536x4096_k4", 1536, 4096, 4, 2),
    ("indexer_wq_b_4096x1536_k4", 4096, 1536, 4, 2),
    ("exp_down_k2", 2048, 4096, 2, 2),
    ("exp_gate_up_k2", 4096, 2048, 2, 2),
    ("mla_kv_a_k6", 4096, 512, 6, 2),
    ("mla_kv_a_k5", 4096, 512, 5, 2),
    ("mla_kv_a_k4", 4096, 512, 4, 2),
    # mcg and 3inst on four classes
    ("kda_qkv_proj_mcg", 4096, 24576, 4, 1),
    ("mla_o_proj_k6_3inst", 16384, 4096, 6, 0),
    ("exp_gate_up_k4_3inst", 4096, 2048, 4, 0),
    ("lm_head_mcg", 4096, 154880, 6, 1),
]
ROWS = (1, 2, 3, 4, 13, 26)
ORACLE_ROWS = (1, 3, 26)


def bits(t):
    return t.detach().contiguous().cpu().numpy().view(np.uint16)


def north_star(g, r):
    rms = np.sqrt(np.mean(r ** 2))
    cos = (g * r).sum() / np.sqrt((g ** 2).sum() * (r ** 2).sum())
    assert np.max(np.abs(g - r)) <= 2e-2 * rms and cos >= 0.9999, (np.max(np.abs(g - r)), rms, cos)


@pytest.mark.parametrize("name,in_f,out_f,K,cb", REAL_SHAPES, ids=[s[0] for s in REAL_SHAPES])
def test_real_shape_class(oracle, dev, name, in_f, out_f, K, cb):
    words = trellis_words_torch(SEED, f"cls.{name}", in_f, out_f, K, dev)
    su = synth.normal_f16(SEED, f"cls.{name}.suh", (in_f,), 1.0, 0.05)
    sv = synth.normal_f16(SEED, f"cls.{name}.svh", (out_f,), 1.0, 0.05)
    w = TrellisWeight(words, f16_from_bits(su, dev), f16_from_bits(sv, dev), in_f, out_f, K, cb)
    n_cb = out_f // 128
    rng = np.random.default_rng(in_f * 7 + out_f + K)
    blocks = sorted({0, int(rng.integers(0, n_cb)), n_cb - 1})
    tiles = words.view(in_f // 16, out_f // 16, 16 * K)
    subs = {b: tiles[:, 8 * b:8 * b + 8, :].contiguous().cpu().numpy().view(np.uint16) for b in blocks}
    differ, checked = 0, 0
    for form in ((0, 1) if cb != 2 else (0,)):
        trellis_set_tuning(weight_form=form)
        try:
            d, c = _class_rows(oracle, dev, w, subs, blocks, name, in_f, K, cb, su, sv, form)
        finally:
            trellis_set_tuning()
        differ += d
        checked += c
    assert differ <= 0.25 * checked, (differ, checked)
    del w, words
    torch.cuda.empty_cache()


def _class_rows(oracle, dev, w, subs, blocks, name, in_f, K, cb, su, sv, form):
    differ, checked = 0, 0
    for rows in ROWS:
        xb = synth.activations(SEED, f"cls.{name}.x{rows}", rows, in_f)
        x = torch.from_numpy(xb.view(np.float16)).to(dev)
        got = bits(trellis_linear(w, x))
        assert np.isfinite(got.view(np.float16)).all()
        # a row of the call equals the row alone (first, middle, last)
        for r in sorted({0, rows // 2, rows - 1}):
            assert np.array_equal(bits(trellis_linear(w, x[r:r + 1].contiguous())), got[r:r + 1]), (rows, r)
        if rows in (4, 26):
            for mb in (1, 3, 16):
                trellis_set_tuning(rows_per_pass=mb, weight_form=form)
                assert np.array_equal(bits(trellis_linear(w, x)), got), (rows, mb)
            trellis_set_tuning(weight_form=form)
        if rows not in ORACLE_ROWS:
            continue
        for b in blocks:
            cols = slice(128 * b, 128 * b + 128)
            g = got[:, cols].view(np.float16).astype(np.float64)
            with oracle.gemv_mode(form == 1):
                want = oracle.trellis_linear(subs[b], in_f, 128, K, cb, su, sv[cols], xb)
            r = want.view(np.float16).astype(np.float64).reshape(g.shape)
            north_star(g, r)
            # yhat is rounded to f16 before the output Hadamard: within 2 ulps of the
            # block's largest output
            ulp = 2.0 ** (np.floor(np.log2(np.abs(r).max())) - 10)
            assert np.max(np.abs(g - r)) <= 2 * ulp, (rows, b, form, np.max(np.abs(g - r)), ulp)
            differ += int(np.sum(got[:, cols].reshape(-1) != want.reshape(-1)))
            checked += want.size
    return differ, checked
