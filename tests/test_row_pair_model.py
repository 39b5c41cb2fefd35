"""Host-only model of the streamed row body's one-read mean and variance
(layernorm's pair): the device's order of operations restated in float32
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
