"""CPU pins of the oracle's hyper-connection and RMSNorm restatements (or_hc_prepare,
or_rms_norm, or_hc_mix; reference glm5_hc.cpp:242-355, glm5_attn.cpp:12-22). MLX is
absent, so there are no golden vectors for these; each check below is a property the
reference's formulas fix and that a plausible mistake (a softmax or Sinkhorn on the wrong
axis, fn read as (in, out), a missing RMS factor, comb not transposed in the mix) breaks."""
import numpy as np
import pytest

from exl3_amd import synth

EPS = 1e-6


def make(seed, P, N, D, fn_std=0.02):
    rng = np.random.default_rng(seed)
    W = (2 + N) * N
    streams = rng.normal(size=(P, N, D)).astype(np.float16).view(np.uint16)
    fn = (rng.normal(size=(W, N * D)) * fn_std).astype(np.float32)
    base = rng.normal(size=W).astype(np.float32) * 0.5
    scale = np.array([1.3, 0.7, 2.1], np.float32)
    return streams, fn, base, scale


def test_sinkhorn_columns_sum_to_one_and_rows_converge(oracle):
    streams, fn, base, scale = make(1, 5, 4, 64)
    _, post, comb = oracle.hc_prepare(streams, 4, 64, fn, base, scale, 20, EPS)
    assert np.all(np.abs(comb.sum(1) - 1) < 1e-5)        # the last step normalises columns
    assert np.all(np.abs(comb.sum(2) - 1) < 1e-3)        # 20 iterations: rows close too
    assert np.all((post > 0) & (post < 2))


def test_softmax_axis_and_base_layout(oracle):
    # fn = 0, so w = 0 and the comb logits are base: make them constant along j and varying
    # along i. A softmax over j (the reference's axis -1) gives a uniform matrix, which
    # stays uniform under Sinkhorn; a softmax over i would not.
    N, D = 4, 32
    streams, fn, base, scale = make(2, 1, N, D)
    fn[:] = 0
    a = np.array([0.3, -1.2, 2.0, 0.7], np.float32)
    base[2 * N:] = np.repeat(a, N)
    _, post, comb = oracle.hc_prepare(streams, N, D, fn, base, scale, 1, EPS)
    assert np.max(np.abs(comb - comb.mean())) < 1e-12
    # and the pre/post blocks come first: post = 2 sigmoid(base[N:2N]) with w = 0
    assert np.allclose(post[0], 2 / (1 + np.exp(-base[N:2 * N].astype(np.float64))), rtol=1e-12)


def test_stream_permutation_equivariance(oracle):
    # relabelling the streams (and fn's input blocks, pre/post entries and comb rows and
    # columns with them) permutes every output and leaves the collapsed stream unchanged
    P, N, D = 3, 4, 48
    streams, fn, base, scale = make(3, P, N, D)
    pi = np.array([2, 0, 3, 1])
    st2 = streams.reshape(P, N, D)[:, pi, :].copy()
    fnb = fn.reshape(-1, N, D)[:, pi, :].reshape(-1, N * D)
    rows = np.concatenate([pi, N + pi, (2 * N + (pi[:, None] * N + pi[None, :])).reshape(-1)])
    fn2 = fnb[rows].copy()
    base2 = base[rows].copy()
    c1, p1, m1 = oracle.hc_prepare(streams, N, D, fn, base, scale, 20, EPS)
    c2, p2, m2 = oracle.hc_prepare(st2, N, D, fn2, base2, scale, 20, EPS)
    assert np.allclose(p2, p1[:, pi], rtol=1e-12, atol=0)
    assert np.allclose(m2, m1[:, pi][:, :, pi], rtol=1e-9, atol=1e-15)
    assert np.array_equal(c1, c2) or np.max(np.abs(c1.view(np.float16).astype(float) - c2.view(np.float16).astype(float))) <= \
        np.abs(c1.view(np.float16).astype(float)).max() * 2 ** -10


@pytest.mark.parametrize("eps", [EPS, 1e-3])
def test_rms_factor_and_fn_orientation(oracle, eps):
    # eps 1e-3 makes the eps inside the rsqrt visible (sqrt(ms + eps) vs sqrt(ms) + eps
    # differ by ~5e-4 at ms ~ 1). fn one-hot: output j reads element i_j of the flattened (N, D) streams, times the
    # RMS factor; with scale 1 and base 0, pre = sigmoid(s[i_j] * rms) + eps
    P, N, D = 2, 2, 40
    streams, fn, base, scale = make(4, P, N, D)
    W = (2 + N) * N
    fn[:] = 0
    idx = np.array([5, 77, 3, 60, 11, 44, 19, 70])[:W]
    fn[np.arange(W), idx] = 1
    base[:] = 0
    scale[:] = 1
    _, post, _ = oracle.hc_prepare(streams, N, D, fn, base, scale, 20, eps)
    s = streams.reshape(P, N * D).view(np.float16).astype(np.float64)
    rms = 1 / np.sqrt((s ** 2).mean(1) + eps)
    want_post = 2 / (1 + np.exp(-(s[:, idx[N:2 * N]] * rms[:, None])))
    assert np.allclose(post, want_post, rtol=1e-12)
    # scaling the streams by 2 (exact in f16) leaves post/comb unchanged and doubles the
    # collapsed stream exactly
    streams, fn, base, scale = make(5, P, 4, 64)
    c1, p1, m1 = oracle.hc_prepare(streams, 4, 64, fn, base, scale, 20, EPS)
    s2 = (streams.view(np.float16) * np.float16(2)).view(np.uint16)
    c2, p2, m2 = oracle.hc_prepare(s2, 4, 64, fn, base, scale, 20, EPS)
    # (not exact: the eps inside the rsqrt weighs 4x less after the scaling)
    assert np.allclose(p1, p2, rtol=1e-5) and np.allclose(m1, m2, rtol=1e-5)
    assert np.array_equal(c2.view(np.float16), c1.view(np.float16) * np.float16(2))


def test_scale_index_closed_form(oracle):
    # fn one-hot (projection j reads element idx[j] of the flattened streams), a random
    # base and three distinct scale entries: scale[0] acts on the pre logits, scale[1] on
    # post, scale[2] on comb (glm5_hc.cpp:313-315). The closed form below builds each
    # output from the one element its projection reads; a swapped scale index moves post,
    # comb or the collapsed stream far outside the bounds (checked: every swap fails).
    P, N, D = 3, 3, 40
    streams, fn, base, _ = make(8, P, N, D)
    W = (2 + N) * N
    rng = np.random.default_rng(9)
    idx = rng.choice(N * D, size=W, replace=False)
    fn[:] = 0
    fn[np.arange(W), idx] = 1
    base[:] = rng.normal(size=W).astype(np.float32)
    scale = np.array([1.7, 0.45, 2.6], np.float32)
    coll, post, comb = oracle.hc_prepare(streams, N, D, fn, base, scale, 4, EPS)
    s = streams.reshape(P, N * D).view(np.float16).astype(np.float64)
    rms = 1 / np.sqrt((s ** 2).mean(1) + EPS)
    b = base.astype(np.float64)
    sig = lambda v: 1 / (1 + np.exp(-v))  # noqa: E731

    def closed(sc):
        w = s[:, idx] * rms[:, None]                       # (P, W)
        pre = sig(w[:, :N] * sc[0] + b[:N]) + EPS
        pst = 2 * sig(w[:, N:2 * N] * sc[1] + b[N:2 * N])
        z = (w[:, 2 * N:] * sc[2] + b[2 * N:]).reshape(P, N, N)
        c = np.exp(z - z.max(2, keepdims=True))
        c = c / c.sum(2, keepdims=True) + EPS
        c = c / (c.sum(1, keepdims=True) + EPS)
        for _ in range(3):
            c = c / (c.sum(2, keepdims=True) + EPS)
            c = c / (c.sum(1, keepdims=True) + EPS)
        col = (pre[:, :, None] * s.reshape(P, N, D)).sum(1)
        return col, pst, c

    sc = scale.astype(np.float64)
    col, pst, c = closed(sc)
    g = coll.view(np.float16).astype(np.float64).reshape(P, D)
    assert np.all(np.abs(g - col) <= np.abs(np.spacing(col.astype(np.float16))).astype(np.float64))
    assert np.allclose(post, pst, rtol=1e-12) and np.allclose(comb, c, rtol=1e-10)
    for perm in ([1, 0, 2], [2, 1, 0], [0, 2, 1], [1, 2, 0], [2, 0, 1]):
        col2, pst2, c2 = closed(sc[perm])
        assert (np.max(np.abs(g - col2)) > 0.01 or np.max(np.abs(post - pst2)) > 0.01
                or np.max(np.abs(comb - c2)) > 0.01), perm


@pytest.mark.parametrize("eps", [EPS, 1e-3, 0.05])
def test_n1_closed_form(oracle, eps):
    P, D = 3, 32
    streams, fn, base, scale = make(6, P, 1, D)
    fn[:] = 0
    coll, post, comb = oracle.hc_prepare(streams, 1, D, fn, base, scale, 20, eps)
    pre = 1 / (1 + np.exp(-float(base[0]))) + eps
    c = 1.0 + eps                       # softmax of one element, plus eps
    c = c / (c + eps)                   # column normalisation
    for _ in range(19):
        c = c / (c + eps)
        c = c / (c + eps)
    assert np.allclose(comb, c, rtol=1e-14) and np.allclose(post, 2 / (1 + np.exp(-float(base[1]))), rtol=1e-14)
    want = (streams.reshape(P, D).view(np.float16).astype(np.float64) * pre).astype(np.float16)
    assert np.array_equal(coll, want.view(np.uint16))


def test_rms_norm_properties(oracle):
    rng = np.random.default_rng(7)
    x = (rng.normal(size=(4, 256)) * 3).astype(np.float16)
    ones = np.ones(256, np.float16).view(np.uint16)
    y = oracle.rms_norm(x.view(np.uint16), ones, 1e-6).view(np.float16).astype(np.float64)
    assert np.all(np.abs((y ** 2).mean(1) - 1) < 2e-3)   # unit mean square before the weight
    y2 = oracle.rms_norm((x * np.float16(4)).view(np.uint16), ones, 1e-6)
    assert np.array_equal(y2.view(np.float16).astype(np.float64), y)   # scale invariant
    w = rng.normal(size=256).astype(np.float16)
    yw = oracle.rms_norm(x.view(np.uint16), w.view(np.uint16), 1e-6).view(np.float16)
    assert np.array_equal(yw, (y.astype(np.float16) * w))  # then an f16 multiply by the weight


def test_hc_mix_transpose_and_closed_form(oracle):
    rng = np.random.default_rng(8)
    P, N, D = 2, 4, 64
    b = rng.normal(size=(P, D)).astype(np.float16)
    res = rng.normal(size=(P, N, D)).astype(np.float16)
    post = rng.uniform(0, 2, size=(P, N))
    # comb a permutation matrix: comb[m][n] = 1 if n == pi[m]. comb^T @ residual gives
    # out[n] = residual[pi^-1(n)]; the untransposed product would give residual[pi(n)].
    pi = np.array([1, 3, 0, 2])
    comb = np.zeros((P, N, N))
    comb[:, np.arange(N), pi] = 1
    out = oracle.hc_mix(b.view(np.uint16), post, comb, res.view(np.uint16)).view(np.float16)
    inv = np.argsort(pi)
    pb = (post.astype(np.float16)[:, :, None] * b[:, None, :])      # f16 product
    want = pb + res[:, inv, :]
    assert np.array_equal(out, want)
    # linear: doubling both inputs doubles the output exactly
    comb2 = rng.uniform(0, 0.5, size=(P, N, N))
    o1 = oracle.hc_mix(b.view(np.uint16), post, comb2, res.view(np.uint16)).view(np.float16)
    o2 = oracle.hc_mix((b * np.float16(2)).view(np.uint16), post, comb2, (res * np.float16(2)).view(np.uint16))
    assert np.array_equal(o2.view(np.float16), o1 * np.float16(2))


def sinkhorn_rank1(v, N, iters, eps):
    """Sinkhorn on a matrix whose N rows all equal v: the column sums are N * v_j and every
    row sums to sum(v), so the matrix keeps equal rows and the iteration is a recursion on
    v alone: columns, then (iters - 1) x (rows, columns), each denominator + eps."""
    v = v / (N * v + eps)
    for _ in range(iters - 1):
        v = v / (v.sum() + eps)
        v = v / (N * v + eps)
    return v


@pytest.mark.parametrize("eps", [EPS, 1e-3, 0.05])
@pytest.mark.parametrize("iters", [1, 2, 3, 20])
def test_sinkhorn_equal_rows_closed_form(oracle, eps, iters):
    # fn = 0, so the comb logits are base[2N + i*N + j]: make them vary along j only. The
    # softmax over j gives every row the same v = softmax(a) + eps, and Sinkhorn reduces to
    # the recursion above. At iters = 1 (columns only) the entries are ~1/N; normalising
    # rows first would leave them ~softmax(a). Each eps is visible at eps >= 1e-3, and each
    # iteration changes v by more than the tolerance while it is far from 1/N.
    N, D = 4, 32
    streams, fn, base, scale = make(9, 2, N, D)
    fn[:] = 0
    a = np.array([1.7, -0.9, 0.4, -2.2], np.float32)
    base[2 * N:] = np.tile(a, N)
    _, _, comb = oracle.hc_prepare(streams, N, D, fn, base, scale, iters, eps)
    z = a.astype(np.float64)
    v = np.exp(z - z.max())
    v = v / v.sum() + eps
    want = sinkhorn_rank1(v, N, iters, eps)
    assert np.allclose(comb, np.broadcast_to(want, comb.shape), rtol=1e-13, atol=0)


def test_sinkhorn_iteration_count_is_load_bearing(oracle):
    # softmax + eps matrices from logits spread over [-3, 3] (the reference hc_test's
    # kind 1): one iteration leaves the row sums far from 1, 3 and 4 iterations differ,
    # and 20 leave the columns at 1 (the last step) and the rows much closer to 1 than 4
    # do (how close depends on the matrix: 8e-4 for this one, 1e-6 after 100)
    N, D, P = 4, 32, 2
    streams, fn, base, scale = make(10, P, N, D)
    fn[:] = 0
    base[2 * N:] = np.random.default_rng(11).uniform(-3, 3, size=N * N).astype(np.float32)
    out = {k: oracle.hc_prepare(streams, N, D, fn, base, scale, k, EPS)[2] for k in (1, 3, 4, 20)}
    assert np.max(np.abs(out[1].sum(2) - 1)) > 1e-3
    assert np.max(np.abs(out[3] - out[4])) > 1e-4
    assert np.max(np.abs(out[20].sum(1) - 1)) <= 1e-5
    rows4, rows20 = (np.max(np.abs(out[k].sum(2) - 1)) for k in (4, 20))
    assert rows20 <= 1e-3 and rows20 < rows4 / 10
