"""Host-only models of the streamed row body's one-read pairs (layernorm's
mean and variance; softmax's max and exp-sum, below): the device's order of operations restated in float32
numpy, so the bound the GPU tests hold the device to (helpers.
assert_layernorm_close) is shown to pass for the right arithmetic and to
fail for plausible mistakes in it.

Per lane of a 1024-lane row (4-wide vectors; lane l owns vectors l, l +
1024, ...): its first vector, then groups of 4 vectors (16 values), then
single vectors, each folded as the group's sum, mean (an exact power-of-two
scaling) and centred sum of squares, then merged into the lane's (S, M2, n)
with Chan, Golub & LeVeque's pairwise update in its commutative form
(tca::hip::chan_merge_present: the two M2 add first, the means and the
weight by reciprocals). The lanes of a wave meet in a butterfly (offsets
32 .. 1), the 16 waves in wave order. The finish takes the mean a = S inv_n
and sum (x - a)^2 = M2 + n (S / n - a)^2."""
import numpy as np
import pytest

from helpers import assert_layernorm_close
from tcacomp_amd import inputs

F = np.float32


def _rcp(v):
    return (F(1) / v).astype(np.float32)


def _merge(s, m2, n, sb, m2b, nb, mistake=None):
    """chan_merge_present over lane arrays (a lane with n = 0 takes the
    other's triple; the arithmetic computed for it is discarded)."""
    with np.errstate(divide="ignore", invalid="ignore"):
        d = (sb * _rcp(nb) - s * _rcp(n)).astype(np.float32)
        w = nb if mistake == "weight" else (n * nb * _rcp(n + nb)).astype(np.float32)
        between = F(0) if mistake == "between" else (d * d * w).astype(np.float32)
        m2_new = ((m2 + m2b) + between).astype(np.float32)
    first = n == 0
    return (np.where(first, sb, s + sb).astype(np.float32), np.where(first, m2b, m2_new).astype(np.float32),
            np.where(first, nb, n + nb).astype(np.float32))


def _add(s, m2, n, vals, ok, mistake=None):
    """chan_add_n over the values vals [lanes, N] of the lanes where ok."""
    N = vals.shape[1]
    gs = vals[:, 0].copy()
    for i in range(1, N):
        gs = (gs + vals[:, i]).astype(np.float32)
    gm = (gs * F(1.0 / (4 if mistake == "group_mean" else N))).astype(np.float32)
    g2 = np.zeros_like(gs)
    for i in range(N):
        d = (vals[:, i] - gm).astype(np.float32)
        g2 = (np.float64(d) * d + g2).astype(np.float32)  # fma: one rounding
    ns, nm2, nn = _merge(s, m2, n, gs, g2, np.full_like(gs, F(N)), mistake)
    return np.where(ok, ns, s), np.where(ok, nm2, m2), np.where(ok, nn, n)


def model_row(x, inv_n, mistake=None):
    """(mean, var) of one f32 row as the streamed body computes them."""
    S, V = 1024, 4
    vecs = x.shape[0] // V
    xv = x.reshape(vecs, V)
    nlane = -(-vecs // S)
    lane = np.arange(S)
    s = np.zeros(S, F)
    m2 = np.zeros(S, F)
    n = np.zeros(S, F)

    def vec(k):
        v = lane + k * S
        ok = v < vecs
        return xv[np.minimum(v, vecs - 1)], ok

    first, ok0 = vec(0)
    s, m2, n = _add(s, m2, n, first, ok0, mistake)
    k = 1
    while k + 3 < nlane:
        group = [vec(k + u) for u in range(4)]
        vals = np.concatenate([g[0] for g in group], axis=1)
        all_ok = group[3][1]
        s1, m21, n1 = _add(s, m2, n, vals, all_ok, mistake)
        for u in range(4):  # lanes whose last vector is past the row: vector by vector
            part = ~all_ok & group[u][1]
            s2, m22, n2 = _add(s, m2, n, group[u][0], part, mistake)
            s, m2, n = np.where(part, s2, s), np.where(part, m22, m2), np.where(part, n2, n)
        s, m2, n = np.where(all_ok, s1, s), np.where(all_ok, m21, m2), np.where(all_ok, n1, n)
        k += 4
    while k < nlane:
        v, ok = vec(k)
        s, m2, n = _add(s, m2, n, v, ok, mistake)
        k += 1
    # butterfly within each wave of 64 lanes
    off = 32
    while off:
        partner = lane ^ off
        s, m2, n = _merge(s, m2, n, s[partner], m2[partner], n[partner], mistake)
        off >>= 1
    ws, wm2, wn = s[::64], m2[::64], n[::64]
    cs, cm, cn = ws[:1], wm2[:1], wn[:1]
    for w in range(1, S // 64):
        cs, cm, cn = _merge(cs, cm, cn, ws[w:w + 1], wm2[w:w + 1], wn[w:w + 1], mistake)
    mean = F(cs[0] * F(inv_n))
    pd = F(cs[0] / cn[0] - mean)
    total = F(cm[0] + cn[0] * pd * pd)
    return mean, F(total * F(inv_n))


def _layernorm(x, g, b, inv_n, eps, mistake=None):
    y = np.empty_like(x)
    for r in range(x.shape[0]):
        mean, var = model_row(x[r], inv_n, mistake)
        rs = F(1.0 / np.sqrt(np.float64(F(var + F(eps)))))
        y[r] = ((x[r] - mean) * rs * g + b).astype(np.float32)
    return y


def _reference(x, g, b, inv_n, eps):
    xd = x.astype(np.float64)
    mean = xd.sum(1, keepdims=True) * inv_n
    var = ((xd - mean) ** 2).sum(1, keepdims=True) * inv_n
    return (xd - mean) / np.sqrt(var + eps) * g.astype(np.float64) + b.astype(np.float64)


def _rows(C):
    x = inputs.normal((3, C), 1.0, 21)
    x[1] += 1000.0  # far from zero: the sum of squares must be about the chunks' own means
    x[2, : C // 2] -= 5.0  # a step between the halves: the between-chunk terms carry the variance
    x[2, C // 2:] += 5.0
    return x


@pytest.mark.parametrize("C", [40000, 40004, 65540])
def test_streamed_pair_model_within_the_gpu_bound(C):
    """The right arithmetic stays within the bound the GPU tests use."""
    x = _rows(C)
    g, b = inputs.uniform((C,), 0.5, 1.5, 1), inputs.uniform((C,), -0.1, 0.1, 2)
    inv_n, eps = float(np.float32(1.0 / C)), 1e-5
    got = _layernorm(x, g, b, inv_n, eps)
    assert_layernorm_close(got, _reference(x, g, b, inv_n, eps), x, g, b, eps, "model C=%d" % C)


@pytest.mark.parametrize("mistake", ["between", "weight", "group_mean"])
def test_streamed_pair_model_mistakes_fail_the_bound(mistake):
    """A dropped between-group term, the pair weight taken as the second
    count, or a group of 16 values centred on a quarter of its sum (the
    count of one vector's values) each break the bound."""
    C = 40000
    x = _rows(C)
    g, b = inputs.uniform((C,), 0.5, 1.5, 1), inputs.uniform((C,), -0.1, 0.1, 2)
    inv_n, eps = float(np.float32(1.0 / C)), 1e-5
    got = _layernorm(x, g, b, inv_n, eps, mistake)
    with pytest.raises(AssertionError):
        assert_layernorm_close(got, _reference(x, g, b, inv_n, eps), x, g, b, eps, "model with " + mistake)


# The softmax pair: each lane's online (m, s) over groups of 16 values
# (tca::hip::online_expsum_add: the group's max, a rescale when it grows,
# then the group's terms about the running max; -inf for values past the
# row), the butterfly and the waves merging (m, s) pairs
# (tca::hip::online_expsum_merge), then the exp-sum about the row's max a
# as s e^(m - a). The terms take float64 exp rounded to float32 (the device's
# v_exp_f32 is within 2.7e-6 relative, far inside the tolerance).

def _exp(v):
    with np.errstate(invalid="ignore"):
        return np.exp(v.astype(np.float64)).astype(np.float32)


def _online_add(m, s, vals, mistake=None):
    g = vals.max(axis=1)
    grow = g > m
    scale = np.where(grow, _exp(m - np.where(grow, g, m)), F(1))
    s = np.where(grow & (mistake != "no_rescale"), (s * scale).astype(np.float32), s)
    m_old = m
    m = np.where(grow, g, m)
    sh = np.where((m_old if mistake == "stale_shift" else m) == -np.inf, F(0), m_old if mistake == "stale_shift" else m)
    for i in range(vals.shape[1]):
        s = (s + _exp(vals[:, i] - sh)).astype(np.float32)
    return m, s


def _online_merge(m, s, m2, s2):
    M = np.maximum(m, m2)
    a = np.where(m == M, s, (s * _exp(m - M)).astype(np.float32))
    b = np.where(m2 == M, s2, (s2 * _exp(m2 - M)).astype(np.float32))
    return M, (a + b).astype(np.float32)


def model_softmax_row(x, mistake=None):
    """(max, exp-sum about it) of one f32 row as the streamed body computes them."""
    S, V = 1024, 4
    vecs = x.shape[0] // V
    xv = x.reshape(vecs, V)
    nlane = -(-vecs // S)
    lane = np.arange(S)
    m = np.full(S, -np.inf, F)
    s = np.zeros(S, F)

    def vec(k):
        v = lane + k * S
        return np.where((v < vecs)[:, None], xv[np.minimum(v, vecs - 1)], F(-np.inf))

    m, s = _online_add(m, s, vec(0), mistake)
    k = 1
    while k + 3 < nlane:
        m, s = _online_add(m, s, np.concatenate([vec(k + u) for u in range(4)], axis=1), mistake)
        k += 4
    while k < nlane:
        m, s = _online_add(m, s, vec(k), mistake)
        k += 1
    off = 32
    while off:
        partner = lane ^ off
        m, s = _online_merge(m, s, m[partner], s[partner])
        off >>= 1
    wm, wsum = m[::64], s[::64]
    cm, cs = wm[:1], wsum[:1]
    for w in range(1, S // 64):
        cm, cs = _online_merge(cm, cs, wm[w:w + 1], wsum[w:w + 1])
    a = F(max(F(-np.inf), cm[0]))
    return a, F(cs[0] * _exp(np.array([cm[0] - a], F))[0])


def _softmax_rows(C):
    x = inputs.normal((3, C), 2.0, 22)
    x[1, -1] = 40.0  # the maximum last: every earlier partial rescales
    x[2, : C // 2] += 30.0  # the large values first: later groups add small terms
    return x


@pytest.mark.parametrize("C", [40000, 40004, 65540])
def test_streamed_softmax_model_within_the_gpu_bound(C):
    """The right arithmetic stays within the relative bound the GPU softmax
    tests use (reduce_tol), for the exp-sum and so for every output."""
    from helpers import reduce_tol
    x = _softmax_rows(C)
    for r in range(x.shape[0]):
        a, den = model_softmax_row(x[r])
        xd = x[r].astype(np.float64)
        assert a == np.float32(x[r].max())
        d64 = np.exp(xd - a).sum()
        assert abs(den - d64) <= reduce_tol(C) * d64, (r, den, d64)


@pytest.mark.parametrize("mistake", ["no_rescale", "stale_shift"])
def test_streamed_softmax_model_mistakes_fail_the_bound(mistake):
    """A running sum not rescaled when the max grows, or a group's terms
    taken about the max before the group, break the bound."""
    from helpers import reduce_tol
    C = 40000
    x = _softmax_rows(C)
    worst = 0.0
    for r in range(x.shape[0]):
        a, den = model_softmax_row(x[r], mistake)
        d64 = np.exp(x[r].astype(np.float64) - a).sum()
        worst = max(worst, abs(den - d64) / d64 / reduce_tol(C) if np.isfinite(den) else np.inf)
    assert worst > 1.0, worst
