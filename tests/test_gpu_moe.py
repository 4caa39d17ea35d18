"""GPU parity tests of the MoE layer through the C ABI.

Routing: top-k id sets equal to the oracle's f64 routing, except where the k-th and
(k+1)-th biased scores are closer than NEAR_TIE (reported, then the GPU's routing is
used to check the experts' arithmetic). Layer output: the north-star tolerance,
max |err| <= 2e-2 * rms(reference) and cosine >= 0.9999, against the oracle on the
reference's f16 weights (the default weight form). The opt-in exact-halves form
(exl3_tuning.weight_form = 1) is held to the same bound against the oracle's
exact-halves mode (check_out_forms); the limit-0.5 cases are layers where the two
forms differ by more than that bound, so each form must match its own oracle.
Invariants of the reference (moe_test.cpp (g)/(h)): an N-row call equals N single-row
calls bit for bit; the run grouping equals the oracle's.
"""
import numpy as np
import pytest
import torch

from exl3_amd import synth
from exl3_amd.moe import DeviceMoeLayer, moe_topk_route, trellis_words_torch
from layer_cases import LIMIT_HALF_CASES, limit_half_case, random_cfgs

pytestmark = pytest.mark.gpu

NEAR_TIE = 1e-6
TOL_RMS = 2e-2
COS_MIN = 0.9999


def ocfg_of(oracle, cfg, has_shared):
    return oracle.make_cfg(cfg.hidden, cfg.inter, cfg.n_experts, cfg.top_k, cfg.n_group,
                           cfg.topk_group, cfg.norm_topk_prob, has_shared,
                           cfg.routed_scaling_factor, cfg.swiglu_limit)


def to_dev(h_bits, dev, B, L, H):
    return torch.from_numpy(h_bits.view(np.float16)).to(dev).view(B, L, H)


def check_out(got_t, want_bits, tol=TOL_RMS):
    got = got_t.float().cpu().numpy().astype(np.float64).reshape(want_bits.shape)
    ref = want_bits.view(np.float16).astype(np.float64)
    rms = np.sqrt(np.mean(ref ** 2))
    err = np.max(np.abs(got - ref))
    cos = (got * ref).sum() / np.sqrt((got ** 2).sum() * (ref ** 2).sum())
    assert np.isfinite(got).all() and rms > 1e-3
    assert err <= tol * rms, (err, rms, tol)
    assert cos >= COS_MIN, cos
    return err / rms, cos


LONG_ROWS = 65        # calls of this many rows or more take the long-run kernels
LONG_PASS_ROWS = 64   # rows per weight pass of the long-run kernels


def check_row_alone(d, x, y_rows, r, B):
    """Row r of a B-row call against the same row alone. Short-run calls (< LONG_ROWS):
    bit-identical, the reference's rows-path invariant (moe_test.cpp (g)). Long-run calls
    accumulate each output over the whole k range in one MFMA chain instead of summing k
    slices, the counterpart of the reference's staged path, which is held to 1% of the
    largest |value| against its QMV (glm5_gemv_nt_test.cpp:221-247): that bound here."""
    alone = d(x[r:r + 1].contiguous()).view(-1).cpu()
    row = y_rows[r].reshape(-1).cpu()
    if B < LONG_ROWS:
        assert torch.equal(alone, row), (B, r)
    else:
        a, b = alone.double(), row.double()
        assert torch.isfinite(b).all() and (a - b).abs().max() <= 1e-2 * a.abs().max(), (B, r)


def _masked_choice_scores(sfc, n_group, topk_group):
    """scores_for_choice after the group limit (oracle or_route: group score = sum of the
    group's top-2), and the gap between the last kept and the first dropped group score."""
    E = sfc.shape[0]
    ng = max(n_group, 1)
    tg = min(max(topk_group, 1), ng)
    if ng == 1:
        return sfc, np.inf
    g = sfc.reshape(ng, E // ng)
    top2 = np.sort(g, 1)[:, ::-1][:, :min(2, g.shape[1])].sum(1)
    order = np.argsort(-top2, kind="stable")
    keep = np.zeros(ng, bool)
    keep[order[:tg]] = True
    gap = top2[order[tg - 1]] - top2[order[tg]] if tg < ng else np.inf
    return np.where(np.repeat(keep, E // ng), sfc, -np.inf), gap


def check_out_forms(oracle, d, x, got_t, routed_args):
    """The layer in both weight forms against the matching oracle mode, each at the
    got_t (the default form: the reference's f16 weights) against the
    reference-rounded oracle, then the handle's exact-halves form against the oracle's
    exact-halves mode. Returns the default form's (err/rms, cosine)."""
    res = check_out(got_t, oracle.moe_layer_routed(*routed_args))
    d.set_tuning(weight_form=1)
    try:
        y_h = d(x)
    finally:
        d.set_tuning()
    with oracle.gemv_mode(True):
        check_out(y_h, oracle.moe_layer_routed(*routed_args))
    return res


def check_routing(oracle, logits, bias, ids_gpu, cfg):
    """Set equality per row, allowing only near-tie flips: at the k-th boundary of the
    group-masked scores_for_choice, or between the last kept and first dropped group
    score. Returns the routing to check the experts against: the oracle's, except on a
    flipped row, where it is the GPU's ids with their f64 weights (so the layer output is
    still compared with the selection the GPU made)."""
    idx, w = oracle.route(logits, bias, cfg)
    sc = 1 / (1 + np.exp(-logits))
    sfc = sc + bias.astype(np.float64)[None, :]
    K = cfg.top_k
    flips = 0
    idx = idx.copy()
    w = w.copy()
    for b in range(idx.shape[0]):
        if set(ids_gpu[b].tolist()) == set(idx[b].tolist()):
            continue
        masked, ggap = _masked_choice_scores(sfc[b], cfg.n_group, cfg.topk_group)
        s = np.sort(masked)[::-1]
        assert s[K - 1] - s[K] < NEAR_TIE or ggap < NEAR_TIE, \
            f"row {b}: routing differs without a near tie"
        flips += 1
        g = ids_gpu[b].astype(np.int64)
        wg = sc[b][g]
        if cfg.norm_topk_prob:
            wg = wg / (wg.sum() + 1e-20)
        idx[b] = g
        w[b] = wg * np.float64(np.float32(cfg.routed_scaling_factor))
    return idx, w, flips


def test_topk_route_known_answers(dev):
    # tests/moe_test.cpp:225-254: bias flips the selection to {0, 3}
    logits = torch.tensor([[2.0, 1.0, 0.5, -2.0, -3.0]], device=dev)
    bias = torch.tensor([0.0, 0.0, 0.0, 0.8, 0.75], device=dev)
    w, ids = moe_topk_route(logits, bias, 1, 1, 2, True, 2.5)
    got = dict(zip(ids[0].tolist(), w[0].tolist()))
    assert sorted(got) == [0, 3]
    assert abs(got[0] - 2.201993) < 1e-4 and abs(got[3] - 0.298008) < 1e-4
    # tests/moe_test.cpp:256-275: group limit selects {0, 1}
    w, ids = moe_topk_route(torch.tensor([[1.0, 0.9, 2.0, -1.0]], device=dev),
                            torch.zeros(4, device=dev), 2, 1, 2, False, 1.0)
    assert sorted(ids[0].tolist()) == [0, 1]


def _sigmoid_f32(x):
    return (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)


@pytest.mark.parametrize("E,K,levels", [(288, 8, 1), (288, 8, 3), (288, 8, 16), (288, 8, 60),
                                        (16, 2, 2), (1024, 16, 24), (1024, 16, 200),
                                        (64, 64, 3), (40, 40, 2), (100, 64, 5), (130, 1, 1)])
def test_topk_route_ties_to_lower_ids(dev, E, K, levels):
    # scores drawn from a few levels (logits -1 .. 7, whose f32 sigmoids all differ), so
    # many experts tie, also across the K-th place (glm5_moe.cpp:16-60: top_k by biased
    # score, ties to the lower expert id); the ids in pick order and the weights (un-biased
    # scores, normalised in pick order, scaled) against numpy. The first row ties every
    # expert; the second puts 40 experts at logit 30, whose sigmoid rounds to exactly 1 in
    # f32. Up to 16 levels put more than 64 experts at or above the K-th place's score.
    # K = E (every expert picked), K = 64 (the largest top-k) and K = 1 over full ties
    # take the threshold's edge cases.
    rng = np.random.default_rng(E * 1000 + levels)
    N = 24
    lv = rng.integers(0, levels, size=(N, E))
    lg = (lv.astype(np.float32) * np.float32(8.0 / levels) - np.float32(1.0)).astype(np.float32)
    lg[0] = 0.5
    lg[1, rng.choice(E, size=min(40, E), replace=False)] = 30.0
    b = np.zeros(E, np.float32)
    w, ids = moe_topk_route(torch.from_numpy(lg).to(dev), torch.from_numpy(b).to(dev), 1, 1, K,
                            True, 2.5)
    ids, w = ids.cpu().numpy(), w.cpu().numpy()
    sig = _sigmoid_f32(lg)
    assert sig[1].max() == 1.0 and (sig[1] == 1.0).sum() == min(40, E)
    for r in range(N):
        order = sorted(range(E), key=lambda e: (-sig[r, e], e))[:K]
        assert ids[r].tolist() == order, (r, ids[r].tolist(), order)
        sc = _sigmoid_f32(lg[r, order])
        denom = np.float32(0.0)
        for v in sc:
            denom = np.float32(denom + v)
        want = sc / (denom + np.float32(1e-20)) * np.float32(2.5)
        assert np.allclose(w[r], want, rtol=2e-6, atol=0), (r, w[r], want)


def test_topk_route_vs_oracle_many_rows(oracle, dev):
    rng = np.random.default_rng(3)
    E, K = 288, 8
    lg = rng.normal(scale=0.5, size=(300, E)).astype(np.float32)
    b = rng.normal(scale=0.01, size=E).astype(np.float32)
    w, ids = moe_topk_route(torch.from_numpy(lg).to(dev), torch.from_numpy(b).to(dev), 1, 1, K,
                            True, 2.5)
    cfg = oracle.make_cfg(16, 16, E, K, 1, 1, True, False, 2.5, 10.0)
    idx, ow, flips = check_routing(oracle, lg.astype(np.float64), b, ids.cpu().numpy(), cfg)
    assert flips == 0
    # weights in the oracle's order, f32 vs f64
    got = np.take_along_axis(w.cpu().numpy(), np.argsort(ids.cpu().numpy(), 1), 1)
    want = np.take_along_axis(ow, np.argsort(idx, 1), 1)
    assert np.allclose(got, want, rtol=2e-6, atol=1e-7)
    # groups: 8 groups of 36, keep 4
    cfg_g = oracle.make_cfg(16, 16, E, K, 8, 4, True, False, 2.5, 10.0)
    w, ids = moe_topk_route(torch.from_numpy(lg).to(dev), torch.from_numpy(b).to(dev), 8, 4, K,
                            True, 2.5)
    idx, _ = oracle.route(lg.astype(np.float64), b, cfg_g)
    assert np.array_equal(np.sort(ids.cpu().numpy(), 1), np.sort(idx, 1))


@pytest.mark.parametrize("B", [1, 4, 8, 17])
def test_small_layer_vs_oracle(oracle, dev, B):
    # configs[0]'s layer (hidden 512, 16 experts, top-2, K4 mcg, no shared expert)
    cfg = synth.config_small()
    layer = synth.make_layer(cfg, 2024)
    h = synth.activations(2024, f"small.x.{B}", B, cfg.hidden)
    d = DeviceMoeLayer(layer, dev)
    y = d(to_dev(h, dev, B, 1, cfg.hidden))
    _, ids = d.route(to_dev(h, dev, B, 1, cfg.hidden))
    oc = ocfg_of(oracle, cfg, False)
    logits = oracle.router_logits(h, layer.router_w)
    idx, w, _ = check_routing(oracle, logits, layer.bias, ids.cpu().numpy(), oc)
    want = oracle.moe_layer_routed(oc, [l.oracle_dict() for l in layer.experts], None, h, idx, w)
    check_out(y, want)
    d.close()


def test_long_passes_every_block_count(oracle, dev):
    # long-run calls (>= 65 rows) on configs[0]'s layer (16 experts, top-2): 100 rows give
    # runs of 5-22 rows (passes of one or two 16-row MFMA blocks), 300 rows 27-53 (two to
    # four blocks), 700 rows 66-132 (a full 64-row pass of four blocks, then a shorter
    # one); each pass computes only its occupied blocks. Every row against the oracle.
    cfg = synth.config_small()
    layer = synth.make_layer(cfg, 2025)
    d = DeviceMoeLayer(layer, dev)
    oc = ocfg_of(oracle, cfg, False)
    seen = set()
    for B in (100, 300, 700):
        h = synth.activations(2025, f"small.long.{B}", B, cfg.hidden)
        x = to_dev(h, dev, B, 1, cfg.hidden)
        y = d(x)
        _, ids = d.route(x)
        logits = oracle.router_logits(h, layer.router_w)
        idx, w, _ = check_routing(oracle, logits, layer.bias, ids.cpu().numpy(), oc)
        for ln in oracle.moe_runs(idx)["run_len"].tolist():
            for p0 in range(0, ln, LONG_PASS_ROWS):
                seen.add((min(LONG_PASS_ROWS, ln - p0) + 15) // 16)
        want = oracle.moe_layer_routed(oc, [l.oracle_dict() for l in layer.experts], None, h, idx, w)
        check_out(y, want)
    assert seen == {1, 2, 3, 4}, seen
    d.close()


def test_layer_with_shared_experts(oracle, dev):
    # trellis shared expert (configs[4]'s mix, small) and an f16 shared expert
    for shared_K in (6, 0):
        cfg = synth.MoeConfig(hidden=512, inter=256, n_experts=24, top_k=4, routed_scaling_factor=2.5,
                              shared_inter=384, gate_up_K=4, gate_up_cb=0, down_K=5, down_cb=2,
                              shared_K=shared_K, shared_cb=1)
        layer = synth.make_layer(cfg, 99)
        B = 6
        h = synth.activations(99, "sh.x", B, cfg.hidden)
        d = DeviceMoeLayer(layer, dev)
        y = d(to_dev(h, dev, B, 1, cfg.hidden))
        _, ids = d.route(to_dev(h, dev, B, 1, cfg.hidden))
        oc = ocfg_of(oracle, cfg, True)
        logits = oracle.router_logits(h, layer.router_w)
        idx, w, _ = check_routing(oracle, logits, layer.bias, ids.cpu().numpy(), oc)
        want = oracle.moe_layer_routed(oc, [l.oracle_dict() for l in layer.experts],
                                       [l.oracle_dict() for l in layer.shared], h, idx, w)
        check_out(y, want)
        d.close()


def _moe_test_g_linear(in_f, out_f, byte):
    # tests/moe_test.cpp:524-545 (mkqg): K3 mul1, every ring word 0x0101 * byte, suh and
    # svh from the reference's formulas (f32, then f16)
    K = 3
    words = np.full(((in_f // 16) * (out_f // 16) * 16 * K,), 0x0101 * (byte & 0xFF), np.uint16)
    i_in, i_out = np.arange(in_f, dtype=np.uint64), np.arange(out_f, dtype=np.uint64)
    sc = (np.float32(0.5) + np.float32(0.01) * ((i_in * 13 + byte) % 17).astype(np.float32)).astype(np.float16)
    sv = (np.float32(0.25) + np.float32(0.01) * ((i_out * 7 + byte) % 13).astype(np.float32)).astype(np.float16)
    return synth.Linear(in_f, out_f, trellis=words.reshape(in_f // 16, out_f // 16, 16 * K),
                        suh=sc.view(np.uint16), svh=sv.view(np.uint16), K=K, cb=synth.CB_MUL1)


def test_moe_test_g_h_fixture(oracle, dev):
    # tests/moe_test.cpp:513-653, sections (g) and (h), on their own fixture: hidden and
    # intermediate 128, 4 experts, top-3, K3 mul1 tensors of byte-uniform ring words
    # (bytes {9, 31, ..., 199} in turn, the shared expert 9, 31, 49), scaling 1.5, limit
    # 10, norm_topk_prob; inputs h4[i] = 0.03 ((29 i + 7) mod 31) - 0.4 and
    # h11[i] = 0.05 ((13 i + 5) mod 37) - 0.7. The router weights follow the test's
    # formula 0.2 (r mod 100) / 100 - 0.1 on a seeded generator here, not its mt19937
    # stream. Checks as there: outputs finite and non-zero, the 4- and 11-row calls (33
    # pairs over 4 experts) equal to single-row calls bit for bit; and, beyond the
    # reference, the layer against the oracle.
    GB = (9, 31, 49, 62, 75, 89, 110, 128, 155, 173, 186, 199)
    H = I = 128
    E, K = 4, 3
    cfg = synth.MoeConfig(hidden=H, inter=I, n_experts=E, top_k=K, routed_scaling_factor=1.5,
                          swiglu_limit=10.0, shared_inter=I, gate_up_K=3, gate_up_cb=synth.CB_MUL1,
                          down_K=3, down_cb=synth.CB_MUL1, shared_K=3, shared_cb=synth.CB_MUL1)
    experts = []
    for e in range(E):
        for w in range(3):
            b = GB[(e * 3 + w) % 12]
            experts.append(_moe_test_g_linear(I, H, b) if w == 2 else _moe_test_g_linear(H, I, b))
    shared = [_moe_test_g_linear(H, I, 9), _moe_test_g_linear(H, I, 31), _moe_test_g_linear(I, H, 49)]
    rng = np.random.default_rng(5)
    gw = (np.float32(0.2) * (rng.integers(0, 1 << 32, E * H) % 100).astype(np.float32) / np.float32(100)
          - np.float32(0.1)).astype(np.float16).reshape(E, H)
    gb = (np.float32(0.05) * (rng.integers(0, 1 << 32, E) % 100).astype(np.float32) / np.float32(100))
    layer = synth.MoeLayer(cfg, experts, shared, gw.view(np.uint16), gb.astype(np.float32))
    d = DeviceMoeLayer(layer, dev)
    oc = ocfg_of(oracle, cfg, True)
    for B, a, m, c, mod in ((4, 0.03, 29, 7, 31), (11, 0.05, 13, 5, 37)):
        i = np.arange(B * H, dtype=np.int64)
        hv = (np.float32(a) * ((i * m + c) % mod).astype(np.float32) - np.float32(0.4 if B == 4 else 0.7))
        h = hv.astype(np.float16).view(np.uint16).reshape(B, H)
        x = to_dev(h, dev, B, 1, H)
        yb = d(x)
        yf = yb.float().cpu()
        assert torch.isfinite(yf).all() and yf.abs().max() > 1e-3, B
        for b in range(B):
            assert torch.equal(d(x[b:b + 1].contiguous()).cpu().view(-1), yb.cpu()[b].view(-1)), (B, b)
        _, ids = d.route(x)
        logits = oracle.router_logits(h, layer.router_w)
        idx, w, _ = check_routing(oracle, logits, layer.bias, ids.cpu().numpy(), oc)
        want = oracle.moe_layer_routed(oc, [l.oracle_dict() for l in experts],
                                       [l.oracle_dict() for l in shared], h, idx, w)
        check_out(yb, want)
    d.close()


def test_rows_path_equals_single_rows(dev):
    # moe_test.cpp (g)/(h): 128-wide fixture, 4 experts, top-3, 11 rows (33 pairs,
    # every expert selected several times); the batch equals single-row calls
    cfg = synth.MoeConfig(hidden=128, inter=128, n_experts=4, top_k=3, routed_scaling_factor=1.5,
                          gate_up_K=3, gate_up_cb=2, down_K=3, down_cb=2, shared_inter=128,
                          shared_K=3, shared_cb=2)
    layer = synth.make_layer(cfg, 5)
    d = DeviceMoeLayer(layer, dev)
    for B in (4, 11, 40, 100):  # 40: pre-rotated rows; 100: the long-run path (runs of ~75 rows)
        h = synth.activations(5, f"rows.{B}", B, 128)
        x = to_dev(h, dev, B, 1, 128)
        yb = d(x).cpu()
        assert torch.isfinite(yb.float()).all() and yb.float().abs().max() > 1e-3
        for b in range(B):
            check_row_alone(d, x, yb.view(B, -1), b, B)
    d.close()


def test_repeat_calls_are_deterministic(dev):
    cfg = synth.config_small()
    layer = synth.make_layer(cfg, 7)
    d = DeviceMoeLayer(layer, dev)
    h = synth.activations(7, "det", 8, cfg.hidden)
    x = to_dev(h, dev, 8, 1, cfg.hidden)
    y0 = d(x).clone()
    for _ in range(5):
        assert torch.equal(d(x), y0)
    d.close()


@pytest.mark.parametrize("H,E", [(384, 72), (512, 64), (1280, 130), (4096, 96), (8192, 40), (4096, 288)])
def test_tiled_router_logits_equal_single_row(dev, H, E):
    # calls of 256 rows or more compute the router logits in 64 x 64 tiles (k splits of
    # 1, 4, 2, 8, 8 and 8 here; 1280 ends a quarter on a partial staging round, 8192
    # takes two rounds per quarter; 130 and 288 experts end on partial expert tiles);
    # the routing weights, f32 functions of the logits, equal the single-row (untiled)
    # calls' bit for bit, and the rows past the last full 64-row tile are routed like
    # the rest
    cfg = synth.MoeConfig(hidden=H, inter=128, n_experts=E, top_k=4, routed_scaling_factor=2.5)
    d = DeviceMoeLayer(synth.make_layer(cfg, 61, tag=f"tile{H}"), dev)
    N = 300
    x = to_dev(synth.activations(61, f"tile.x.{H}", N, H), dev, N, 1, H)
    w, ids = d.route(x)
    for r in (0, 1, 63, 64, 127, 128, 130, 255, 256, 299):
        w1, i1 = d.route(x[r:r + 1].contiguous())
        assert torch.equal(i1.view(-1), ids[r].view(-1)), r
        assert torch.equal(w1.view(-1), w[r].view(-1)), r
    d.close()


def test_layer_rejects_too_many_rows_before_launch(dev):
    # B * L beyond one call's limit (2^24 / top_k rows), including a product that would
    # overflow int64, is refused on the host; the workspace query answers 0 for it
    from exl3_amd import _lib
    cfg = synth.config_small()
    d = DeviceMoeLayer(synth.make_layer(cfg, 8), dev)
    L = _lib.lib()
    limit = (1 << 24) // cfg.top_k
    assert d.workspace_bytes(limit) > 0 and d.workspace_bytes(limit + 1) == 0
    x = to_dev(synth.activations(8, "lim", 1, cfg.hidden), dev, 1, 1, cfg.hidden)
    out = torch.empty_like(x)
    for B, Lq in ((limit + 1, 1), (1 << 40, 1 << 40), (1 << 62, 4)):
        st = L.exl3_moe_layer(d.handle, x.data_ptr(), B, Lq, out.data_ptr(), x.data_ptr(), 1, None)
        assert st == _lib.EXL3_ERR_UNSUPPORTED, (B, Lq)
        assert b"too many rows" in L.exl3_last_error()
    # the handle still works
    y = d(x).clone()
    assert torch.equal(d(x), y)
    d.close()


def glm5_layer_on_device(dev, seed, tag, cfg=None, hot_experts=None, hot_bias=0.0):
    """Full-size GLM-5 layer: small tensors from numpy, trellis words on the device."""
    cfg = cfg or synth.config_glm5()
    H, I, E = cfg.hidden, cfg.inter, cfg.n_experts
    bias = synth.normal_f32(seed, f"{tag}.gate.e_score_correction_bias", (E,), 0, 0.01)
    if hot_experts is not None:
        bias = bias.copy()
        bias[np.asarray(hot_experts)] += np.float32(hot_bias)
    layer = synth.MoeLayer(cfg, [], None, synth.normal_f16(seed, f"{tag}.gate.weight", (E, H), 0, 0.02),
                           bias)
    words = {}
    for e in range(E):
        for j, (nm, i_f, o_f, K) in enumerate((("gate_proj", H, I, cfg.gate_up_K),
                                               ("up_proj", H, I, cfg.gate_up_K),
                                               ("down_proj", I, H, cfg.down_K))):
            p = f"{tag}.experts.{e}.{nm}"
            lin = synth.Linear(i_f, o_f, trellis=None, suh=synth.normal_f16(seed, p + ".suh", (i_f,), 1, 0.05),
                               svh=synth.normal_f16(seed, p + ".svh", (o_f,), 1, 0.05), K=K,
                               cb=cfg.gate_up_cb if j < 2 else cfg.down_cb)
            layer.experts.append(lin)
            words[3 * e + j] = trellis_words_torch(seed, p + ".trellis", i_f, o_f, K, dev)
    SI = cfg.shared_inter
    dims = ((f"{tag}.shared_experts.gate_proj", H, SI), (f"{tag}.shared_experts.up_proj", H, SI),
            (f"{tag}.shared_experts.down_proj", SI, H))
    if cfg.shared_K == 0:
        layer.shared = [synth.make_dense_linear(seed, p, i_f, o_f) for p, i_f, o_f in dims]
    else:
        layer.shared = []
        for j, (p, i_f, o_f) in enumerate(dims):
            layer.shared.append(synth.Linear(i_f, o_f, trellis=None,
                                             suh=synth.normal_f16(seed, p + ".suh", (i_f,), 1, 0.05),
                                             svh=synth.normal_f16(seed, p + ".svh", (o_f,), 1, 0.05),
                                             K=cfg.shared_K, cb=cfg.shared_cb))
            words[("shared", j)] = trellis_words_torch(seed, p + ".trellis", i_f, o_f, cfg.shared_K, dev)
    return layer, words


def oracle_linear(lin, w):
    if lin.trellis is not None or w is None:
        return lin.oracle_dict()
    return dict(trellis=w.cpu().numpy().view(np.uint16), suh=lin.suh, svh=lin.svh, K=lin.K,
                cb=lin.cb, **{"in": lin.in_f, "out": lin.out_f})


def oracle_experts(layer, words, used):
    out = []
    dummy = dict(trellis=np.zeros(16, np.uint16), suh=np.zeros(1, np.uint16),
                 svh=np.zeros(1, np.uint16), K=1, cb=0, **{"in": 16, "out": 16})
    for i, lin in enumerate(layer.experts):
        out.append(oracle_linear(lin, words.get(i)) if i // 3 in used else dummy)
    return out


def oracle_shared(layer, words):
    return [oracle_linear(l, words.get(("shared", j))) for j, l in enumerate(layer.shared)]


def test_glm5_layer_b8_vs_oracle(oracle, dev):
    # GLM-5-shaped layer at batch 8
    layer, words = glm5_layer_on_device(dev, 31, "glm5")
    cfg = layer.cfg
    d = DeviceMoeLayer(layer, dev, words=words)
    h = synth.activations(31, "glm5.x", 8, cfg.hidden)
    x = to_dev(h, dev, 8, 1, cfg.hidden)
    d.diag_enable()
    y = d(x)
    _, ids = d.route(x)
    oc = ocfg_of(oracle, cfg, True)
    logits = oracle.router_logits(h, layer.router_w)
    idx, w, flips = check_routing(oracle, logits, layer.bias, ids.cpu().numpy(), oc)
    used = set(idx.reshape(-1).tolist())
    want = oracle.moe_layer_routed(oc, oracle_experts(layer, words, used),
                                   oracle_shared(layer, words), h, idx, w)
    rel, cos = check_out(y, want)
    dg = d.diag()
    assert dg["calls"] == 1 and dg["pairs"] == 64 and dg["distinct_experts"] == len(used)
    hist = {}
    for r in oracle.moe_runs(idx)["run_len"].tolist():
        hist[min(r, 64)] = hist.get(min(r, 64), 0) + 1
    assert dg["run_hist"] == hist
    print(f"\nglm5 B=8: distinct experts {len(used)}, max|err|/rms {rel:.3g}, cos {cos:.7f}, "
          f"near-tie flips {flips}")
    d.close()


@pytest.fixture(scope="module")
def glm5_verify_layer(dev):
    layer, words = glm5_layer_on_device(dev, 61, "glm5v")
    d = DeviceMoeLayer(layer, dev, words=words)
    yield layer, words, d
    d.close()


@pytest.mark.parametrize("B", [1, 2, 3, 4])
def test_glm5_layer_verify_rows_vs_oracle(oracle, dev, glm5_verify_layer, B):
    # rows 1-4 at GLM-5 shape: decode and the multi-row verify / MTP regime
    # (glm5_mtp.cpp:55: the draft block calls the MoE on 2-4 rows); against the oracle at
    # the north-star bound, and the B-row call equal to B single-row calls bit for bit
    layer, words, d = glm5_verify_layer
    cfg = layer.cfg
    h = synth.activations(61, f"glm5v.x{B}", B, cfg.hidden)
    x = to_dev(h, dev, B, 1, cfg.hidden)
    y = d(x)
    _, ids = d.route(x)
    oc = ocfg_of(oracle, cfg, True)
    idx, w, flips = check_routing(oracle, oracle.router_logits(h, layer.router_w), layer.bias,
                                  ids.cpu().numpy(), oc)
    used = set(idx.reshape(-1).tolist())
    want = oracle.moe_layer_routed(oc, oracle_experts(layer, words, used), oracle_shared(layer, words),
                                   h, idx, w)
    rel, cos = check_out(y, want)
    for b in range(B):
        assert torch.equal(d(x[b:b + 1].contiguous()), y[b:b + 1])
    print(f"\nglm5 B={B}: distinct experts {len(used)}, max|err|/rms {rel:.3g}, cos {cos:.7f}, flips {flips}")


def check_diag_bytes(dg, run_len, cfg, pass_rows, mat_min_rows=16):
    """MoeRowsDiag semantics (reference glm5_moe.cpp:265-287): runs in the staged window,
    and each run's expert bytes once per weight pass (passes of pass_rows rows), from the
    oracle's run table."""
    run_len = [int(r) for r in run_len]
    eb = cfg.hidden * cfg.inter * (2 * cfg.gate_up_K + cfg.down_K) // 8
    assert dg["staged_runs"] == sum(1 for r in run_len if r >= mat_min_rows)
    assert dg["streamed_bytes"] == sum(eb * -(-r // pass_rows) for r in run_len)
    assert dg["shared_bytes"] == eb * len(run_len)
    assert dg["distinct_experts"] == len(run_len)


def test_glm5_b64_run_grouping(oracle, dev):
    # 48 of 64 rows identical -> 8 runs of >= 48 rows; 16 independent rows
    layer, words = glm5_layer_on_device(dev, 41, "glm5b")
    cfg = layer.cfg
    d = DeviceMoeLayer(layer, dev, words=words)
    same = synth.activations(41, "b64.same", 1, cfg.hidden)
    rest = synth.activations(41, "b64.rest", 16, cfg.hidden)
    h = np.concatenate([np.repeat(same, 48, 0), rest], 0)
    x = to_dev(h, dev, 64, 1, cfg.hidden)
    d.diag_enable()
    y = d(x)
    oc = ocfg_of(oracle, cfg, True)
    logits = oracle.router_logits(h, layer.router_w)
    _, ids = d.route(x)
    idx, w, _ = check_routing(oracle, logits, layer.bias, ids.cpu().numpy(), oc)
    runs = oracle.moe_runs(idx)
    hist = {}
    for r in runs["run_len"].tolist():
        hist[min(r, 64)] = hist.get(min(r, 64), 0) + 1
    dg = d.diag()
    assert dg["run_hist"] == hist
    assert sum(1 for r in runs["run_len"] if r >= 48) >= 8
    check_diag_bytes(dg, runs["run_len"], cfg, 16)
    # the handle's own staged window: only the diagnostics' staged count moves
    assert d.tuning()["mat_min_rows"] == 16
    d.set_tuning(mat_min_rows=50)
    d.diag_reset()
    y2 = d(x)
    assert torch.equal(y2.cpu(), y.cpu())
    check_diag_bytes(d.diag(), runs["run_len"], cfg, 16, mat_min_rows=50)
    used = set(idx.reshape(-1).tolist())
    want = oracle.moe_layer_routed(oc, oracle_experts(layer, words, used),
                                   oracle_shared(layer, words), h, idx, w)
    check_out(y, want)
    # the 48 identical rows give identical outputs
    yc = y.view(64, -1).cpu()
    assert all(torch.equal(yc[i], yc[0]) for i in range(48))
    d.close()


def test_prefill_2048_config5(oracle, dev):
    # 2048 token rows; gate/up K4 3inst, down K5 mul1, shared expert K6 mcg;
    # 8 hot experts take about a quarter of the selections (bias tilt 0.23)
    cfg = synth.config_prefill()
    hot = list(range(0, cfg.n_experts, cfg.n_experts // 8))
    layer, words = glm5_layer_on_device(dev, 51, "pf", cfg, hot, 0.23)
    N, H = 2048, cfg.hidden
    h = synth.activations(51, "pf.x", N, H)
    x = to_dev(h, dev, N, 1, H)
    d = DeviceMoeLayer(layer, dev, words=words)
    d.diag_enable()
    y = d(x).view(N, H)
    _, ids = d.route(x)
    oc = ocfg_of(oracle, cfg, True)
    logits = oracle.router_logits(h, layer.router_w)
    idx, w, flips = check_routing(oracle, logits, layer.bias, ids.cpu().numpy(), oc)
    hot_frac = np.isin(idx, hot).mean()
    assert 0.2 < hot_frac < 0.3, hot_frac
    runs = oracle.moe_runs(idx)
    hist = {}
    for r in runs["run_len"].tolist():
        hist[min(r, 64)] = hist.get(min(r, 64), 0) + 1
    assert d.diag()["run_hist"] == hist
    check_diag_bytes(d.diag(), runs["run_len"], cfg, LONG_PASS_ROWS)
    # checked rows: in every hot expert's run, the rows either side of each weight-pass
    # boundary and the run's last row (each hot run spans several passes), plus rows spread
    # over the call; each within the staged-path bound of the same row alone (the decode
    # path) and, all together, within the north-star bound of the oracle
    rows = set(range(0, N, 61)) | {N - 1}
    for e in hot:
        k = int(np.nonzero(runs["run_expert"] == e)[0][0])
        off, ln = int(runs["run_off"][k]), int(runs["run_len"][k])
        assert ln > 2 * LONG_PASS_ROWS, (e, ln)
        for q in sorted({0, LONG_PASS_ROWS - 1, LONG_PASS_ROWS, 3 * LONG_PASS_ROWS, ln - 1}):
            rows.add(int(runs["sorted_row"][off + min(q, ln - 1)]))
    rows = sorted(rows)
    assert len(rows) >= 64
    yc = y.cpu()
    for r in rows:
        check_row_alone(d, x, yc, r, N)
    used = set(idx[rows].reshape(-1).tolist())
    want = oracle.moe_layer_routed(oc, oracle_experts(layer, words, used), oracle_shared(layer, words),
                                   h[rows], idx[rows], w[rows])
    rel, cos = check_out(yc[rows], want)
    print(f"\nprefill 2048: hot fraction {hot_frac:.3f}, runs {len(runs['run_len'])}, "
          f"max run {max(runs['run_len'])}, sampled max|err|/rms {rel:.3g}, cos {cos:.7f}, flips {flips}")
    d.close()


@pytest.mark.parametrize("N", [2600, 8500])
def test_dispatch_many_pairs(oracle, dev, N):
    # the counting sort over several workgroups: 2600 rows x top-8 = 20800 pairs in 21
    # chunks of 1024 (the last one ragged, 320 pairs); 8500 rows = 68000 pairs, past 64
    # chunks of 1024, in 34 chunks of 2048 (two rounds of 64 pairs per wave); hot experts
    # whose runs span chunks and need several 64-row passes; small tensors keep it quick
    cfg = synth.MoeConfig(hidden=256, inter=128, n_experts=64, top_k=8, routed_scaling_factor=2.0,
                          shared_inter=128, gate_up_K=3, gate_up_cb=1, down_K=2, down_cb=2, shared_K=0)
    hot = [3, 17, 40]
    layer, words = glm5_layer_on_device(dev, 61, "many", cfg, hot, 0.3)
    H = cfg.hidden
    h = synth.activations(61, "many.x", N, H)
    x = to_dev(h, dev, N, 1, H)
    d = DeviceMoeLayer(layer, dev, words=words)
    d.diag_enable()
    y = d(x).view(N, H)
    _, ids = d.route(x)
    oc = ocfg_of(oracle, cfg, True)
    logits = oracle.router_logits(h, layer.router_w)
    idx, w, _ = check_routing(oracle, logits, layer.bias, ids.cpu().numpy(), oc)
    runs = oracle.moe_runs(idx)
    assert max(runs["run_len"]) > 2 * LONG_PASS_ROWS
    hist = {}
    for r in runs["run_len"].tolist():
        hist[min(r, 64)] = hist.get(min(r, 64), 0) + 1
    assert d.diag()["run_hist"] == hist
    check_diag_bytes(d.diag(), runs["run_len"], cfg, LONG_PASS_ROWS)
    rows = sorted(set(list(range(0, N, 157 if N < 4000 else 421)) + [N - 1]))
    yc = y.cpu()
    for r in rows:
        check_row_alone(d, x, yc, r, N)
    used = set(idx[rows].reshape(-1).tolist())
    want = oracle.moe_layer_routed(oc, oracle_experts(layer, words, used), oracle_shared(layer, words),
                                   h[rows], idx[rows], w[rows])
    check_out(yc[rows], want)
    d.close()


def test_dispatch_over_a_million_pairs(oracle, dev):
    # 131,200 rows x top-8 = 1,049,600 pairs: 64 chunks of 17,408 pairs, 17 rounds of 64
    # pairs per wave, so each wave takes its pairs' experts in two batches of loads (the
    # 16-round batch, then one more). The rows repeat with period 4,100: the oracle routes
    # the first 4,100, and every copy of a row must get that row's routing and, bit for
    # bit, its output (a row's long-run output depends only on its own input), wherever
    # its pairs fall among the chunks
    cfg = synth.MoeConfig(hidden=256, inter=128, n_experts=64, top_k=8, routed_scaling_factor=2.0,
                          shared_inter=128, gate_up_K=3, gate_up_cb=1, down_K=2, down_cb=2, shared_K=0)
    layer, words = glm5_layer_on_device(dev, 62, "mill", cfg, [3, 17, 40], 0.3)
    R, reps, H = 4100, 32, cfg.hidden
    N = R * reps
    base = synth.activations(62, "mill.x", R, H)
    x = to_dev(np.tile(base, (reps, 1)), dev, N, 1, H)
    d = DeviceMoeLayer(layer, dev, words=words)
    d.diag_enable()
    y = d(x).view(N, H)
    _, ids = d.route(x)
    ids = ids.cpu().numpy().reshape(N, -1)
    assert (ids.reshape(reps, R, -1) == ids[None, :R]).all()
    oc = ocfg_of(oracle, cfg, True)
    idx, w, _ = check_routing(oracle, oracle.router_logits(base, layer.router_w), layer.bias, ids[:R], oc)
    runs = oracle.moe_runs(np.tile(idx, (reps, 1)))
    hist = {}
    for r in runs["run_len"].tolist():
        hist[min(r, 64)] = hist.get(min(r, 64), 0) + 1
    assert d.diag()["run_hist"] == hist
    check_diag_bytes(d.diag(), runs["run_len"], cfg, LONG_PASS_ROWS)
    yc = y.cpu()
    yr = yc.view(reps, R, H)
    assert torch.equal(yr, yr[:1].expand(reps, R, H).contiguous())
    rows = [0, 1, 2175, 2176, R // 2, R - 1]
    for r in rows:
        check_row_alone(d, x, yc, r, N)
    used = set(idx[rows].reshape(-1).tolist())
    want = oracle.moe_layer_routed(oc, oracle_experts(layer, words, used), oracle_shared(layer, words),
                                   base[rows], idx[rows], w[rows])
    check_out(yc[rows], want)
    d.close()


@pytest.mark.parametrize("gu_K,gu_cb,dn_K,dn_cb", [(1, 0, 2, 1), (2, 2, 3, 0), (3, 1, 6, 2), (5, 0, 7, 1),
                                                   (6, 2, 8, 0), (7, 1, 1, 2), (8, 0, 4, 1)])
def test_layer_k_codebook_sweep(oracle, dev, gu_K, gu_cb, dn_K, dn_cb):
    # every K and codebook through the MoE expert kernels (gate/up and down), with a
    # trellis shared expert; B=5 (short runs) and B=70 (the long-run kernels)
    cfg = synth.MoeConfig(hidden=256, inter=384, n_experts=12, top_k=3, routed_scaling_factor=1.5,
                          shared_inter=256, gate_up_K=gu_K, gate_up_cb=gu_cb, down_K=dn_K,
                          down_cb=dn_cb, shared_K=dn_K, shared_cb=gu_cb)
    layer = synth.make_layer(cfg, 300 + gu_K)
    d = DeviceMoeLayer(layer, dev)
    oc = ocfg_of(oracle, cfg, True)
    for B in (5, 70):
        h = synth.activations(300 + gu_K, f"kcb.x.{B}", B, cfg.hidden)
        x = to_dev(h, dev, B, 1, cfg.hidden)
        y = d(x)
        _, ids = d.route(x)
        logits = oracle.router_logits(h, layer.router_w)
        idx, w, _ = check_routing(oracle, logits, layer.bias, ids.cpu().numpy(), oc)
        want = oracle.moe_layer_routed(oc, [l.oracle_dict() for l in layer.experts],
                                       [l.oracle_dict() for l in layer.shared], h, idx, w)
        check_out(y, want)
        if B == 70:  # long-run path against the decode path
            yc = y.view(B, -1).cpu()
            for r in (0, 33, 69):
                check_row_alone(d, x, yc, r, B)
    d.close()


def test_layer_many_experts_grouped(oracle, dev):
    # E = 1024 (the largest routing table), 8 groups keeping 4, top-16, f16 shared expert
    cfg = synth.MoeConfig(hidden=256, inter=128, n_experts=1024, top_k=16, n_group=8, topk_group=4,
                          routed_scaling_factor=2.0, shared_inter=128, gate_up_K=2, gate_up_cb=1,
                          down_K=3, down_cb=1, shared_K=0)
    layer = synth.make_layer(cfg, 1024)
    d = DeviceMoeLayer(layer, dev)
    oc = ocfg_of(oracle, cfg, True)
    # 48 pairs: one-wave dispatch; 320 pairs: the one-workgroup counting sort; 2080 pairs:
    # the counting sort over 3 workgroups (every expert's count read from each chunk)
    for B in (3, 20, 130):
        h = synth.activations(1024, f"many.x.{B}", B, cfg.hidden)
        x = to_dev(h, dev, B, 1, cfg.hidden)
        d.diag_reset()
        d.diag_enable()
        y = d(x)
        _, ids = d.route(x)
        logits = oracle.router_logits(h, layer.router_w)
        idx, w, _ = check_routing(oracle, logits, layer.bias, ids.cpu().numpy(), oc)
        hist = {}
        for r in oracle.moe_runs(idx)["run_len"].tolist():
            hist[min(r, 64)] = hist.get(min(r, 64), 0) + 1
        assert d.diag()["run_hist"] == hist
        want = oracle.moe_layer_routed(oc, [l.oracle_dict() for l in layer.experts],
                                       [l.oracle_dict() for l in layer.shared], h, idx, w)
        check_out(y, want)
    d.close()


@pytest.mark.parametrize("B", [8, 9, 16, 17, 64, 65])
def test_dispatch_boundaries_rows_invariance(dev, B):
    # the dispatch and routing paths change at 64 pairs, 16 rows and 65 rows: every
    # batch row equals the same row alone (bit for bit below 65 rows, within the
    # staged-path bound from 65)
    cfg = synth.MoeConfig(hidden=128, inter=128, n_experts=20, top_k=8, routed_scaling_factor=1.0,
                          gate_up_K=4, gate_up_cb=1, down_K=5, down_cb=1, shared_inter=0)
    layer = synth.make_layer(cfg, 77)
    d = DeviceMoeLayer(layer, dev)
    h = synth.activations(77, f"bnd.{B}", B, 128)
    x = to_dev(h, dev, B, 1, 128)
    yb = d(x).view(B, -1).cpu()
    assert torch.isfinite(yb.float()).all()
    for r in sorted({0, B // 2, B - 1}):
        check_row_alone(d, x, yb, r, B)
    d.close()


def test_layer_large_hidden_many_slices(oracle, dev):
    # hidden 8192 (16 gate/up k slices, the activation kernel's long slice sum) and
    # intermediate 2048 (4 down slices, the combine's long slice sum); short and long runs
    cfg = synth.MoeConfig(hidden=8192, inter=2048, n_experts=6, top_k=2, routed_scaling_factor=1.0,
                          gate_up_K=2, gate_up_cb=1, down_K=2, down_cb=2, shared_inter=0)
    layer = synth.make_layer(cfg, 8192)
    d = DeviceMoeLayer(layer, dev)
    oc = ocfg_of(oracle, cfg, False)
    for B in (3, 66):
        h = synth.activations(8192, f"big.x.{B}", B, cfg.hidden)
        x = to_dev(h, dev, B, 1, cfg.hidden)
        y = d(x)
        _, ids = d.route(x)
        logits = oracle.router_logits(h, layer.router_w)
        idx, w, _ = check_routing(oracle, logits, layer.bias, ids.cpu().numpy(), oc)
        rows = list(range(B)) if B < 8 else [0, 31, 65]
        want = oracle.moe_layer_routed(oc, [l.oracle_dict() for l in layer.experts], None, h[rows],
                                       idx[rows], w[rows])
        check_out(y.view(B, -1)[rows], want)
        if B == 66:
            check_row_alone(d, x, y.view(B, -1).cpu(), 31, B)
    d.close()


@pytest.mark.parametrize("i", range(24))
def test_layer_random_shapes(oracle, dev, i):
    # seeded random configurations at a row count each that walks the dispatch and path
    # boundaries: the oracle's output within tolerance, and (for the batch) one row
    # equal to the same row alone, bit for bit
    cfg = random_cfgs(24, 4321)[i]
    B = (1, 3, 8, 17, 40, 70)[i % 6]
    layer = synth.make_layer(cfg, 4400 + i)
    d = DeviceMoeLayer(layer, dev)
    h = synth.activations(4400 + i, f"rand.x.{i}", B, cfg.hidden)
    x = to_dev(h, dev, B, 1, cfg.hidden)
    y = d(x)
    _, ids = d.route(x)
    has_shared = cfg.shared_inter > 0
    oc = ocfg_of(oracle, cfg, has_shared)
    logits = oracle.router_logits(h, layer.router_w)
    idx, w, _ = check_routing(oracle, logits, layer.bias, ids.cpu().numpy(), oc)
    args = (oc, [l.oracle_dict() for l in layer.experts],
            [l.oracle_dict() for l in layer.shared] if has_shared else None, h, idx, w)
    check_out_forms(oracle, d, x, y, args)
    check_row_alone(d, x, y.view(B, -1).cpu(), B // 2, B)
    d.close()


@pytest.mark.parametrize("seed,i,B", LIMIT_HALF_CASES)
def test_layer_limit_half_each_form_its_oracle(oracle, dev, seed, i, B):
    cfg, layer, h = limit_half_case(seed, i, B)
    d = DeviceMoeLayer(layer, dev)
    x = to_dev(h, dev, B, 1, cfg.hidden)
    y = d(x)
    _, ids = d.route(x)
    has_shared = cfg.shared_inter > 0
    oc = ocfg_of(oracle, cfg, has_shared)
    idx, w, _ = check_routing(oracle, oracle.router_logits(h, layer.router_w), layer.bias,
                              ids.cpu().numpy(), oc)
    args = (oc, [l.oracle_dict() for l in layer.experts],
            [l.oracle_dict() for l in layer.shared] if has_shared else None, h, idx, w)
    check_out_forms(oracle, d, x, y, args)
    d.close()


def test_swiglu_limit_zero_clips_everything(oracle, dev):
    # the reference clips gate to <= L and up to [-L, L] whatever L is (glm5_moe.cpp:
    # 70-71), so a limit of 0 (its default when a checkpoint has none, model.cpp:143)
    # zeroes every expert's SwiGLU output and the layer output is exactly zero
    cfg = synth.MoeConfig(hidden=256, inter=128, n_experts=8, top_k=2, swiglu_limit=0.0,
                          shared_inter=128, shared_K=3, shared_cb=1)
    layer = synth.make_layer(cfg, 77)
    d = DeviceMoeLayer(layer, dev)
    for B in (3, 70):
        h = synth.activations(77, f"lim0.{B}", B, cfg.hidden)
        y = d(to_dev(h, dev, B, 1, cfg.hidden))
        assert torch.count_nonzero(y.float()).item() == 0, B
    oc = ocfg_of(oracle, cfg, True)
    h = synth.activations(77, "lim0.3", 3, cfg.hidden)
    want, _, _ = oracle.moe_layer(oc, [l.oracle_dict() for l in layer.experts],
                                  [l.oracle_dict() for l in layer.shared], layer.router_w, layer.bias, h)
    assert not np.any(want.view(np.float16).astype(np.float64))
    d.close()
