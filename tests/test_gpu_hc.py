"""GPU parity tests of the hyper-connection steps around the MoE (exl3_hc_prepare,
exl3_rms_norm, exl3_hc_mix, exl3_moe_block; reference glm5_hc.cpp:242-355,
glm5_attn.cpp:12-22, glm5_forward.cpp:434-438) through the C ABI.

The device computes in f32 (the reference's mx arrays are f32 for the prepare's statistics
and f16 for the streams, with f32 accumulation inside its matmuls); the oracle computes in
f64 with the reference's f16 rounding points. Tolerances, written per check:
  post, comb           |gpu - oracle| <= 2e-5 (f32 round-off through a 16384-term dot
                       product, a sigmoid/softmax and 20 Sinkhorn iterations)
  f16 outputs          every element within `ulps` f16 ulps of the oracle's plus, for the
                       collapsed stream sum_n pre[n] * s[n], COND * sum_n |s[n]| (f32
                       round-off of the terms, which cancellation can make several ulps of
                       a small sum; scaled by r * |w| behind the RMSNorm), and at most
                       MISMATCH_FRAC of the elements differ at all (a difference needs the
                       f64 value within f32 round-off of an f16 rounding boundary)
  the block            bit-identical to the separate calls prepare -> layer -> mix, and the
                       chain against the oracle's at the north-star bound
                       (max |err| <= 2e-2 * rms, cosine >= 0.9999).
"""
import numpy as np
import pytest
import torch

from exl3_amd import _lib, synth
from exl3_amd.hc import DeviceHcSite, hc_mix, hc_prepare, moe_block, rms_norm
from exl3_amd.moe import DeviceMoeLayer

pytestmark = pytest.mark.gpu

EPS = 1e-6           # GLM-5 hc_eps
NORM_EPS = 1e-5      # GLM-5 rms_norm_eps
MISMATCH_FRAC = 1e-2
COND = 1e-6          # f32 round-off of pre[n] and of the N-term sum, relative to the terms
TOL_RMS = 2e-2
COS_MIN = 0.9999


def make_site(seed, N, D, fn_std=None):
    """fn with unit-variance projections of an RMS-normalised input (std 1/sqrt(N*D)) so
    that pre, post and comb spread over the sigmoid's and softmax's range."""
    rng = np.random.default_rng(seed)
    W = (2 + N) * N
    fn = (rng.normal(size=(W, N * D)) * (fn_std or 1 / np.sqrt(N * D))).astype(np.float32)
    base = (rng.normal(size=W) * 0.5).astype(np.float32)
    scale = np.array([1.3, 0.7, 2.1], np.float32)
    return fn, base, scale


def streams_of(seed, P, N, D, scale=1.0):
    rng = np.random.default_rng(seed)
    return (rng.normal(size=(P, N, D)) * scale).astype(np.float16).view(np.uint16)


def dev_f16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.float16)).to(dev)


def check_f16(got_t, want_bits, ulps, extra=0.0):
    got = got_t.cpu().numpy().view(np.uint16).reshape(want_bits.shape)
    g = got.view(np.float16).astype(np.float64)
    w = want_bits.view(np.float16).astype(np.float64)
    assert np.isfinite(g).all()
    spacing = np.abs(np.spacing(want_bits.view(np.float16))).astype(np.float64)
    bound = ulps * spacing + extra
    assert np.all(np.abs(g - w) <= bound), np.max(np.abs(g - w) / bound)
    frac = np.mean(got != want_bits)
    assert frac <= MISMATCH_FRAC, frac
    return frac


def collapse_cond(st_bits):
    """COND * sum_n |s[n]| per (position, d)."""
    return COND * np.abs(st_bits.view(np.float16).astype(np.float64)).sum(1)


# (positions, streams, hidden): GLM-5's 4 streams, fewer, and 5..8 (the wide kernels:
# an 8 x 8 Sinkhorn layout and up to 80 projections)
SHAPES = [(8, 4, 4096), (3, 4, 512), (5, 2, 384), (17, 1, 256), (1, 3, 256), (40, 4, 1024),
          (4, 5, 512), (3, 6, 1024), (6, 8, 4096), (9, 7, 256)]


@pytest.mark.parametrize("P,N,D", SHAPES)
@pytest.mark.parametrize("norm", [False, True])
def test_hc_prepare_vs_oracle(oracle, dev, P, N, D, norm):
    fn, base, scale = make_site(10 * N + D, N, D)
    st = streams_of(P * 7 + N, P, N, D)
    site = DeviceHcSite.from_numpy(fn, base, scale, N, 20, EPS, dev)
    nw_bits = (np.random.default_rng(D).normal(1.0, 0.2, size=D)).astype(np.float16).view(np.uint16)
    nw = dev_f16(nw_bits, dev) if norm else None
    out, post, comb = hc_prepare(dev_f16(st, dev), site, nw, NORM_EPS)
    coll, opost, ocomb = oracle.hc_prepare(st, N, D, fn, base, scale, 20, EPS)
    assert np.max(np.abs(post.cpu().numpy() - opost)) <= 2e-5
    assert np.max(np.abs(comb.cpu().numpy() - ocomb)) <= 2e-5
    if norm:
        # the fused norm equals the separate RMSNorm of the unnormalised prepare, whose
        # collapsed stream is checked against the oracle's; the norm itself against the
        # oracle's RMSNorm of that same collapsed stream (two f16 roundings: 2 ulps)
        plain, _, _ = hc_prepare(dev_f16(st, dev), site, None)
        check_f16(plain, coll, ulps=1, extra=collapse_cond(st))
        assert torch.equal(out, rms_norm(plain, nw, NORM_EPS))
        check_f16(out, oracle.rms_norm(plain.cpu().numpy().view(np.uint16), nw_bits, NORM_EPS), ulps=2)
    else:
        check_f16(out, coll, ulps=1, extra=collapse_cond(st))


def test_hc_prepare_glm5_scale_streams(oracle, dev):
    # streams of large magnitude (late-layer residuals reach hundreds): the RMS factor
    # scales them back, so pre/post/comb must match as for unit streams
    P, N, D = 4, 4, 4096
    fn, base, scale = make_site(77, N, D)
    st = streams_of(78, P, N, D, scale=300.0)
    site = DeviceHcSite.from_numpy(fn, base, scale, N, 20, EPS, dev)
    out, post, comb = hc_prepare(dev_f16(st, dev), site)
    coll, opost, ocomb = oracle.hc_prepare(st, N, D, fn, base, scale, 20, EPS)
    assert np.max(np.abs(post.cpu().numpy() - opost)) <= 2e-5
    assert np.max(np.abs(comb.cpu().numpy() - ocomb)) <= 2e-5
    check_f16(out, coll, ulps=1, extra=collapse_cond(st))


@pytest.mark.parametrize("eps", [1e-3, 0.05])
@pytest.mark.parametrize("iters", [1, 3, 4, 20])
@pytest.mark.parametrize("N", [4, 8])
def test_hc_prepare_large_eps_and_iteration_count(oracle, dev, eps, iters, N):
    # At hc_eps 1e-6 a dropped eps (in the rsqrt, pre, the softmax or any Sinkhorn
    # denominator) moves post/comb by ~1e-6, inside the 2e-5 bound; at 1e-3 and 0.05 it
    # moves them by far more. The oracle's iteration count is pinned on the CPU, and 3 and 4
    # iterations differ by more than the bound for these logits, so matching it at each
    # count pins the device's count too.
    P, D = 5, 1024
    fn, base, scale = make_site(90 + iters + N, N, D)
    base[2 * N:] = np.random.default_rng(91).uniform(-3, 3, size=N * N).astype(np.float32)
    st = streams_of(92, P, N, D)
    site = DeviceHcSite.from_numpy(fn, base, scale, N, iters, eps, dev)
    out, post, comb = hc_prepare(dev_f16(st, dev), site)
    coll, opost, ocomb = oracle.hc_prepare(st, N, D, fn, base, scale, iters, eps)
    assert np.max(np.abs(post.cpu().numpy() - opost)) <= 2e-5
    assert np.max(np.abs(comb.cpu().numpy() - ocomb)) <= 2e-5
    check_f16(out, coll, ulps=1, extra=collapse_cond(st))


@pytest.mark.parametrize("N", [1, 2, 3, 5, 6, 7])
def test_hc_prepare_zero_eps_fewer_streams(oracle, dev, N):
    # hc_mult below 4 (or 5..7) leaves entries of the device's 4 x 4 (8 x 8) Sinkhorn
    # layout outside N x N; at hc_eps 0 their rows and columns sum to 0, and the reference
    # (which has no such entries) stays finite: so must the device, and match the oracle
    P, D = 3, 512
    fn, base, scale = make_site(300 + N, N, D)
    st = streams_of(301 + N, P, N, D)
    site = DeviceHcSite.from_numpy(fn, base, scale, N, 20, 0.0, dev)
    out, post, comb = hc_prepare(dev_f16(st, dev), site)
    coll, opost, ocomb = oracle.hc_prepare(st, N, D, fn, base, scale, 20, 0.0)
    assert np.isfinite(comb.cpu().numpy()).all() and np.isfinite(post.cpu().numpy()).all()
    assert np.max(np.abs(post.cpu().numpy() - opost)) <= 2e-5
    assert np.max(np.abs(comb.cpu().numpy() - ocomb)) <= 2e-5
    check_f16(out, coll, ulps=1, extra=collapse_cond(st))


def test_hc_mix_identity_roundtrip(dev):
    # the reference's expand -> mix identity: streams that are copies of x, post = 1 and
    # comb = I give out[n] = f16(bo + x) exactly (1 * bo and 1 * x are exact, the sum is
    # rounded once)
    P, N, D = 6, 4, 512
    rng = np.random.default_rng(93)
    x = rng.normal(size=(P, D)).astype(np.float16)
    bo = rng.normal(size=(P, D)).astype(np.float16)
    st = np.ascontiguousarray(np.broadcast_to(x[:, None, :], (P, N, D)))
    comb = np.broadcast_to(np.eye(N, dtype=np.float32), (P, N, N)).copy()
    out = hc_mix(torch.from_numpy(bo).to(dev), torch.ones(P, N, device=dev), torch.from_numpy(comb).to(dev),
                 torch.from_numpy(st).to(dev)).cpu().numpy()
    want = (bo.astype(np.float32) + x.astype(np.float32)).astype(np.float16)
    assert np.array_equal(out, np.broadcast_to(want[:, None, :], (P, N, D)))


@pytest.mark.parametrize("P,D", [(7, 4096), (3, 1000), (2, 8192), (33, 6144)])
def test_rms_norm_vs_oracle(oracle, dev, P, D):
    rng = np.random.default_rng(P + D)
    x = (rng.normal(size=(P, D)) * 3).astype(np.float16).view(np.uint16)
    w = rng.normal(1.0, 0.2, size=D).astype(np.float16).view(np.uint16)
    y = rms_norm(dev_f16(x, dev), dev_f16(w, dev), NORM_EPS)
    check_f16(y, oracle.rms_norm(x, w, NORM_EPS), ulps=2)


@pytest.mark.parametrize("P,N,D", [(8, 4, 4096), (5, 3, 256), (2, 1, 130), (4, 8, 512), (3, 6, 256)])
def test_hc_mix_vs_oracle(oracle, dev, P, N, D):
    rng = np.random.default_rng(P * N + D)
    b = rng.normal(size=(P, D)).astype(np.float16).view(np.uint16)
    res = (rng.normal(size=(P, N, D)) * 4).astype(np.float16).view(np.uint16)
    post = rng.uniform(0, 2, size=(P, N)).astype(np.float32)
    comb = rng.dirichlet(np.ones(N), size=(P, N)).astype(np.float32)
    out = hc_mix(dev_f16(b, dev), torch.from_numpy(post).to(dev), torch.from_numpy(comb).to(dev),
                 dev_f16(res, dev))
    want = oracle.hc_mix(b, post.astype(np.float64), comb.astype(np.float64), res)
    # out = f16(a + f16(r)), r = sum_m comb[m][n] * res[m] summed in f32 on the device and
    # in f64 by the oracle: f16(r) may differ by one ulp of r, which a cancelling a
    # turns into many ulps of out
    r = np.einsum("pmn,pmd->pnd", comb.astype(np.float64), res.view(np.float16).astype(np.float64))
    check_f16(out, want, ulps=1, extra=np.abs(np.spacing(r.astype(np.float16))).astype(np.float64))


def test_hc_mix_transposes_comb(oracle, dev):
    # comb = a permutation matrix P[m][n] = 1 iff n = pi(m): stream n receives residual
    # stream pi^-1(n) (the reference's comb^T @ residual), post = 0 leaves only that term
    P, N, D = 2, 4, 256
    pi = np.array([2, 0, 3, 1])
    comb = np.zeros((P, N, N), np.float32)
    comb[:, np.arange(N), pi] = 1
    res = np.random.default_rng(1).normal(size=(P, N, D)).astype(np.float16)
    out = hc_mix(torch.zeros(P, D, dtype=torch.float16, device=dev), torch.zeros(P, N, device=dev),
                 torch.from_numpy(comb).to(dev), torch.from_numpy(res).to(dev)).cpu().numpy()
    inv = np.argsort(pi)
    assert np.array_equal(out, res[:, inv, :])


def _block_layer(hidden, seed):
    cfg = synth.MoeConfig(hidden=hidden, inter=256, n_experts=16, top_k=4, routed_scaling_factor=2.5,
                          shared_inter=256, gate_up_K=4, gate_up_cb=0, down_K=3, down_cb=2, shared_K=0)
    return cfg, synth.make_layer(cfg, seed)


@pytest.mark.parametrize("P,N", [(1, 4), (8, 4), (37, 4), (5, 8), (3, 6), (100, 4), (70, 8)])
def test_moe_block_equals_separate_calls(dev, P, N):
    # P >= 65: the long-run kernels, whose combine variant carries the fused mix
    D = 512
    cfg, layer = _block_layer(D, 31)
    d = DeviceMoeLayer(layer, dev)
    fn, base, scale = make_site(32, N, D)
    site = DeviceHcSite.from_numpy(fn, base, scale, N, 20, EPS, dev)
    nw = dev_f16(np.random.default_rng(33).normal(1, 0.2, D).astype(np.float16).view(np.uint16), dev)
    st = dev_f16(streams_of(34 + P, P, N, D, scale=2.0), dev)
    got = moe_block(d, site, nw, NORM_EPS, st)
    h, post, comb = hc_prepare(st, site, nw, NORM_EPS)
    y = d(h.view(P, 1, D))
    want = hc_mix(y.view(P, D), post, comb, st)
    assert torch.equal(got, want)
    # a second call with fewer rows (workspace reused) equals its own separate calls
    st1 = st[-1:].contiguous()
    got1 = moe_block(d, site, nw, NORM_EPS, st1)
    h1, post1, comb1 = hc_prepare(st1, site, nw, NORM_EPS)
    assert torch.equal(got1, hc_mix(d(h1.view(1, 1, D)).view(1, D), post1, comb1, st1))
    d.close()


@pytest.mark.parametrize("N", [4, 8])
def test_moe_block_vs_oracle_chain(oracle, dev, N):
    # oracle chain: hc_prepare -> rms_norm -> the MoE on the device's h and routing ->
    # hc_mix; the MoE part at the north-star bound, the final streams too
    from test_gpu_moe import check_out, check_routing, ocfg_of
    P, D = 6, 512
    cfg, layer = _block_layer(D, 41)
    d = DeviceMoeLayer(layer, dev)
    fn, base, scale = make_site(42, N, D)
    site = DeviceHcSite.from_numpy(fn, base, scale, N, 20, EPS, dev)
    nw_bits = np.random.default_rng(43).normal(1, 0.2, D).astype(np.float16).view(np.uint16)
    st_bits = streams_of(44, P, N, D, scale=2.0)
    st = dev_f16(st_bits, dev)
    got = moe_block(d, site, dev_f16(nw_bits, dev), NORM_EPS, st)
    h, post, comb = hc_prepare(st, site, dev_f16(nw_bits, dev), NORM_EPS)
    coll, opost, ocomb = oracle.hc_prepare(st_bits, N, D, fn, base, scale, 20, EPS)
    plain, _, _ = hc_prepare(st, site, None)
    check_f16(plain, coll, ulps=1, extra=collapse_cond(st_bits))
    check_f16(h, oracle.rms_norm(plain.cpu().numpy().view(np.uint16), nw_bits, NORM_EPS), ulps=2)
    h_bits = h.cpu().numpy().view(np.uint16)
    _, ids = d.route(h.view(P, 1, D))
    oc = ocfg_of(oracle, cfg, True)
    idx, w, _ = check_routing(oracle, oracle.router_logits(h_bits, layer.router_w), layer.bias,
                              ids.cpu().numpy(), oc)
    moe_want = oracle.moe_layer_routed(oc, [l.oracle_dict() for l in layer.experts],
                                       [l.oracle_dict() for l in layer.shared], h_bits, idx, w)
    check_out(d(h.view(P, 1, D)), moe_want)
    want = oracle.hc_mix(moe_want, opost, ocomb, st_bits)
    check_out(got, want)
    d.close()


def test_moe_block_glm5_hidden(dev):
    # GLM-5's hidden 4096 and hc_mult 4 through the block, bit-identical to separate calls
    P, N, D = 8, 4, 4096
    cfg, layer = _block_layer(D, 51)
    d = DeviceMoeLayer(layer, dev)
    fn, base, scale = make_site(52, N, D)
    site = DeviceHcSite.from_numpy(fn, base, scale, N, 20, EPS, dev)
    nw = dev_f16(np.random.default_rng(53).normal(1, 0.2, D).astype(np.float16).view(np.uint16), dev)
    st = dev_f16(streams_of(54, P, N, D, scale=2.0), dev)
    got = moe_block(d, site, nw, NORM_EPS, st)
    h, post, comb = hc_prepare(st, site, nw, NORM_EPS)
    want = hc_mix(d(h.view(P, 1, D)).view(P, D), post, comb, st)
    assert torch.equal(got, want)
    assert torch.isfinite(got.float()).all()
    d.close()


def test_block_argument_errors(dev):
    N, D = 4, 512
    cfg, layer = _block_layer(D, 61)
    d = DeviceMoeLayer(layer, dev)
    fn, base, scale = make_site(62, N, D)
    site = DeviceHcSite.from_numpy(fn, base, scale, N, 20, EPS, dev)
    nw = torch.ones(D, dtype=torch.float16, device=dev)
    st = torch.zeros(3, N, D, dtype=torch.float16, device=dev)
    with pytest.raises(_lib.Exl3Error, match="overlap"):
        moe_block(d, site, nw, NORM_EPS, st, out=st)
    bad = DeviceHcSite(9, 20, EPS, site.fn, site.base, site.scale)
    with pytest.raises(_lib.Exl3Error, match="hc_mult"):
        hc_prepare(torch.zeros(1, 9, D, dtype=torch.float16, device=dev), bad)
    odd = DeviceHcSite(3, 20, EPS, site.fn, site.base, site.scale)
    with pytest.raises(_lib.Exl3Error, match="multiple of 64"):
        hc_prepare(torch.zeros(1, 3, 200, dtype=torch.float16, device=dev), odd)
    # zero positions: nothing to do
    assert moe_block(d, site, nw, NORM_EPS, st[:0]).numel() == 0
    d.close()
