"""Host-only model of the column family's one-read mean and variance (the
fused lowering of a mean followed by a centred sum of squares over the
reduced axis): the device kernels' order of operations restated in float32
numpy, row slot by row slot and chunk by chunk, so the error bound the GPU
test holds the device to is checked here against exact arithmetic, and
plausible mistakes in the update formula are shown to break it.

Per thread: rows r_lo + s + k STEP, a first group of 4, groups of 16 while
whole ones fit, then groups of 4; each group's sum, mean and centred sum of
squares from its rows, merged into the thread's running (S, M2, n) with
Chan, Golub & LeVeque's pairwise update. Slots merge in slot order, chunks
in wave order (16 waves, chunk w, w + 16, ...), and the finish takes
sum (x - m)^2 = M2 + n (S / n - m)^2 with m = S * inv_n.

The bound (helpers.fused_var_bound): each merge adds non-negative terms,
each with a few roundings relative to itself, plus one rounding of the
running sum, and a merge's difference of means carries an absolute error of
a few u times the mean (Chan, Golub & LeVeque, "Algorithms for computing
the sample variance", 1983: relative error O(depth * kappa * u), kappa^2 =
1 + n mean^2 / T). With D bounding the merges along any chain of the fold
(groups of a thread, row slots, chunks, waves), 2 (D + 16) kappa u T; plus
the sum's own rounding, which moves S / n away from the exact mean by at
most gamma_R sum|x| / n and enters as n (S / n - m)^2; plus the final
multiply's rounding."""
import numpy as np
import pytest

from helpers import fused_var_bound

F = np.float32
U = 2.0 ** -24


def _fma(a, b, c):
    return F(np.float64(a) * np.float64(b) + np.float64(c))


def _chan(s, m2, n, sb, m2b, nb, drop_between=False, weight_nb=False):
    d = F(F(sb / nb) - F(s / n))
    w = F(nb) if weight_nb else F(F(n * nb) / F(n + nb))
    add = F(0) if drop_between else F(F(d * d) * w)
    return F(s + sb), F(m2 + F(m2b + add)), F(n + nb)


def model(x, step, P, inv_n, **mistake):
    """Float32 model of the fused kernels over x [R] (one column)."""
    R = x.shape[0]
    if R == 0:
        return F(0) * inv_n, F(0) * inv_n
    chunks = []
    for p in range(P):
        r_lo, r_hi = p * R // P, (p + 1) * R // P
        slots = []
        for s in range(min(step, r_hi - r_lo)):
            S = m2 = F(0)
            cn = F(0)
            r = r_lo + s
            first = True
            while r < r_hi:
                rows = 16 if (not first and r + 15 * step < r_hi) else 4
                e = [x[r + u * step] for u in range(rows) if r + u * step < r_hi]
                nu = F(len(e))
                gs = e[0]
                for v in e[1:]:
                    gs = F(gs + v)
                gm = F(gs * F(1.0 / nu))
                g2 = F(F(e[0] - gm) * F(e[0] - gm))
                for v in e[1:]:
                    g2 = _fma(F(v - gm), F(v - gm), g2)
                if first:
                    m2 = g2
                else:
                    dl = F(gm - F(S * F(1.0 / cn)))
                    w = nu if mistake.get("weight_nb") else F(F(cn * nu) / F(cn + nu))
                    add = F(0) if mistake.get("drop_between") else F(F(dl * dl) * w)
                    m2 = F(m2 + F(g2 + add))
                for i, v in enumerate(e):
                    S = v if (first and i == 0) else F(S + v)
                cn = F(cn + nu)
                r += rows * step
                first = False
            slots.append((S, m2, cn))
        S, m2, n = slots[0]
        for sb, m2b, nb in slots[1:]:
            S, m2, n = _chan(S, m2, n, sb, m2b, nb, **mistake)
        chunks.append((S, m2, n))
    waves = []
    for w in range(min(P, 16)):
        S, m2, n = chunks[w]
        for k in range(w + 16, P, 16):
            S, m2, n = _chan(S, m2, n, *chunks[k], **mistake)
        waves.append((S, m2, n))
    S, m2, n = waves[0]
    for wv in waves[1:]:
        S, m2, n = _chan(S, m2, n, *wv, **mistake)
    m = F(F(F(0) + S) * inv_n)
    dm = F(F(S * F(1.0 / n)) - m)
    tot = F(m2 + F(n * F(dm * dm)))
    return m, F(F(F(0) + tot) * inv_n)


def bound(x, m, inv_n):
    """(exact variance as the program defines it, the fused path's bound)
    for one column: the GPU test's bound (helpers.fused_var_bound)."""
    exact, b = fused_var_bound(x[:, None], np.array([m]), inv_n)
    return float(exact[0]), float(b[0])


CASES = [  # (R, step, P, data)
    (1, 8, 1, "int"), (5, 8, 1, "int"), (37, 8, 1, "int"), (64, 8, 1, "int"), (100, 1, 1, "int"),
    (1000, 8, 16, "int"), (3000, 8, 16, "int"), (8192, 8, 16, "int"), (65536, 8, 16, "int"),
    (4097, 4, 64, "offset"), (20000, 8, 16, "offset"), (333, 2, 5, "normal"), (8192, 8, 16, "drift"),
]


def _data(R, kind, seed):
    rng = np.random.default_rng(seed)
    if kind == "int":
        return rng.integers(-8, 9, size=R).astype(F)
    if kind == "offset":
        return (100.0 + rng.standard_normal(R)).astype(F)
    if kind == "drift":  # a column whose mean moves along the rows
        return (np.linspace(0.0, 50.0, R) + rng.standard_normal(R)).astype(F)
    return rng.standard_normal(R).astype(F)


@pytest.mark.parametrize("R,step,P,kind", CASES)
def test_fused_model_within_bound(R, step, P, kind):
    for seed in range(3):
        x = _data(R, kind, seed * 7 + R)
        inv_n = F(1.0 / R)
        m, var = model(x, step, P, inv_n)
        want_m = F(F(x.astype(np.float64).sum()) * inv_n) if kind == "int" else None
        if want_m is not None:
            assert m == want_m  # integer data: the sum is exact in any order
        exact, b = bound(x, m, inv_n)
        assert abs(float(var) - exact) <= b, (R, kind, seed, float(var), exact, b)


@pytest.mark.parametrize("mistake", ["drop_between", "weight_nb"])
@pytest.mark.parametrize("R,step,P,kind", [(1000, 8, 16, "int"), (8192, 8, 16, "int"), (20000, 8, 16, "offset"),
                                           (64, 8, 1, "int")])
def test_fused_model_mistakes_break_the_bound(R, step, P, kind, mistake):
    """A dropped between-group term or a wrong pair weight leaves the bound:
    the GPU test's bound is tight enough to see either."""
    x = _data(R, kind, R)
    inv_n = F(1.0 / R)
    m, var = model(x, step, P, inv_n, **{mistake: True})
    exact, b = bound(x, m, inv_n)
    assert abs(float(var) - exact) > b, (R, kind, mistake)


def test_fused_model_constant_and_empty():
    x = np.full(5000, 3.0, F)
    m, var = model(x, 8, 16, F(1.0 / 5000))
    assert m == F(3.0) and var == F(0.0)
    m, var = model(np.zeros(0, F), 8, 1, F(1.0))
    assert var == F(0.0)
