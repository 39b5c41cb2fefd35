"""The column family on the device: reductions over a non-contiguous axis
(As(C, R) drops R; the reference's middle-axis reductions,
testing/kernels/runtime/row_sum.tca), at shapes that reach every path:
no rows or no columns, narrow rows (several rows per wave step), every
vector width, one row chunk (the partial kernel stores) and many (partials,
then the merge), several batch indices.

Expected values: integer-valued f32 inputs keep every sum exact (partial
sums below 2^24), so the device matches the float64 sum rounded once, bit
for bit, in any fold order; max is exact; u8 -> u32 sums are exact;
col_mean_bf16's piped map is one rounded multiply and one rounded add on
both sides.

col_mean_var (a variance reading its mean: one column nest of two passes)
runs in both lowerings: fused into one read (the default: each partial
keeps the sum and the centred sum of squares, merged pairwise) and pass by
pass (EMIT_NO_PASS_FUSION: the whole-column kernel at <= 64 rows or more
than 512 column blocks, otherwise a partial + merge pair per pass), at
shapes that reach one chunk and many. Its mean is an exact sum times
f32(1 / R), one rounded multiply: bit for bit. Pass by pass, its variance
sums f32 terms (x - mean)^2, each rounded once on both sides, in an order of
the device's choosing: within the fold's rounding bound, gamma_(R-1)
sum|terms| (gamma_n = n u / (1 - n u), u = 2^-24), plus the final
multiply's rounding. Fused, within helpers.fused_var_bound around the exact
sum of (x - mean)^2 (the pairwise update's bound, pinned on a float32 model
of the kernels in tests/test_col_fused_model.py)."""
import sys

import numpy as np
import pytest

from helpers import CANARY, compiled, fused_var_bound, run, to_dev
from tcacomp_amd.compiler import TensorDesc
from tcacomp_amd.pkg import EMIT_NO_PASS_FUSION

pytestmark = pytest.mark.gpu

U32 = 4

SHAPES = [(0, 5), (5, 0), (1, 1), (3, 7), (100, 3), (1000, 16), (64, 8192), (8192, 8192), (65536, 1024),
          (2, 1 << 20), (300, 1022), (4097, 513), (70000, 12)]


def _ints(shape, bound, seed):
    return np.random.default_rng(seed).integers(-bound, bound + 1, size=shape).astype(np.float32)


@pytest.mark.parametrize("R,C", SHAPES)
def test_col_sum_max(gpu, R, C):
    print("col_sum_max", R, C, flush=True)
    sys.stdout.flush()
    x = _ints((R, C), 8, R * 7 + C)
    s = to_dev(np.full(C, CANARY, np.float32), gpu)
    m = to_dev(np.full(C, CANARY, np.float32), gpu)
    run(compiled("col_sum_max_dyn"), [to_dev(x, gpu), s, m])
    assert np.abs(x).sum(axis=0).max(initial=0) < 2 ** 24  # exact sums
    want_s = x.astype(np.float64).sum(axis=0).astype(np.float32)
    want_m = np.max(x, axis=0, initial=-np.inf).astype(np.float32)
    np.testing.assert_array_equal(s.cpu().numpy(), want_s)
    np.testing.assert_array_equal(m.cpu().numpy(), want_m)


# The most elements a tensor may hold: the u32 index domain less the
# kernels' index headroom (2^16).
TOP = 2 ** 32 - 2 ** 16 - 1


@pytest.mark.parametrize("R,C", [(TOP, 1), (TOP // 4, 4)], ids=["V1", "V4"])
def test_col_reductions_at_the_element_limit(gpu, R, C):
    """Columns as long as a tensor may be (17 GB of f32; the row loops step
    within 2^16 of 2^32): zeros with marks 1, 2, 4 in the last column at the
    first, the middle and the last row. Column sum + max must be exactly 7
    and 4 there and 0 elsewhere; with 4 columns, the one-read mean and
    variance must give 7 inv_n and (21 - 14 m + R m^2) inv_n (m the stored
    mean) there, 0 elsewhere."""
    import torch
    print("col reductions at the element limit", R, C, flush=True)
    sys.stdout.flush()
    x = torch.zeros((R, C), device=gpu)
    x[0, C - 1], x[R // 2, C - 1], x[R - 1, C - 1] = 1.0, 2.0, 4.0
    s = torch.full((C,), CANARY, device=gpu)
    m = torch.full((C,), CANARY, device=gpu)
    run(compiled("col_sum_max_dyn"), [x, s, m])
    want_s, want_m = np.zeros(C, np.float32), np.zeros(C, np.float32)
    want_s[-1], want_m[-1] = 7.0, 4.0
    np.testing.assert_array_equal(s.cpu().numpy(), want_s)
    np.testing.assert_array_equal(m.cpu().numpy(), want_m)
    if C == 1:
        return
    inv_n = float(np.float32(1.0 / R))
    mean = torch.full((1, C), CANARY, device=gpu)
    var = torch.full((1, C), CANARY, device=gpu)
    run(compiled("col_mean_var_dyn"), [x.view(1, R, C), mean, var], scalars=[inv_n])
    gm, gv = mean.cpu().numpy()[0].astype(np.float64), var.cpu().numpy()[0].astype(np.float64)
    assert np.all(gm[:-1] == 0.0) and np.all(gv[:-1] == 0.0), (gm, gv)
    assert abs(gm[-1] - 7.0 * inv_n) <= 1e-6 * 7.0 * inv_n, gm
    wv = (21.0 - 14.0 * gm[-1] + R * gm[-1] ** 2) * inv_n
    assert abs(gv[-1] - wv) <= 1e-4 * wv, (gv, wv)
    del x
    torch.cuda.empty_cache()


@pytest.mark.parametrize("B,R,C", [(1, 1, 8), (2, 1000, 520), (3, 5, 8), (4, 300, 4100), (2, 0, 16),
                                   (5, 2000, 6), (1, 20000, 2048)])
def test_col_mean_bf16(gpu, B, R, C):
    import torch
    print("col_mean_bf16", B, R, C, flush=True)
    sys.stdout.flush()
    x = _ints((B, R, C), 8, B * 31 + R * 7 + C)  # small integers: exact in bf16
    g = _ints((C,), 3, 1) * np.float32(0.5)
    scale = 0.125
    out = to_dev(np.full((B, C), CANARY, np.float32), gpu)
    xd = torch.from_numpy(x).to(gpu).to(torch.bfloat16)
    run(compiled("col_mean_bf16"), [xd, to_dev(g, gpu), out], scalars=[scale])
    ssum = x.astype(np.float64).sum(axis=1).astype(np.float32)
    want = ssum * np.float32(scale) + g[None, :]
    np.testing.assert_array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("R,C", [(1, 16), (7, 33), (5000, 4096), (300, 1000), (100000, 48), (3, 1 << 20),
                                 (0, 64)])
def test_col_sum_u8(gpu, R, C):
    import torch
    print("col_sum_u8", R, C, flush=True)
    sys.stdout.flush()
    x = np.random.default_rng(R + C).integers(0, 256, size=(R, C), dtype=np.uint8)
    o = torch.full((C,), 0x5A5A5A5A, dtype=torch.int32, device=gpu)
    run(compiled("col_sum_u8"), [to_dev(x, gpu), TensorDesc(o.data_ptr(), (C,), U32)])
    want = (x.astype(np.uint64).sum(axis=0) % (1 << 32)).astype(np.uint32)
    np.testing.assert_array_equal(o.cpu().numpy().view(np.uint32), want)


FUSED = pytest.mark.parametrize("flags", [0, EMIT_NO_PASS_FUSION], ids=["one_read", "passes"])


def _passes_bound(x, want_mean, inv_n):
    """(exact, bound) of the per-pass lowering: f32 terms (x - mean)^2, each
    rounded once as on the device, summed in an order of the device's
    choosing (gamma_(R-1) sum|terms|), plus the final multiply's rounding."""
    R = x.shape[1]
    d = x - want_mean[:, None, :]
    terms = (d * d).astype(np.float64)
    exact = terms.sum(axis=1)
    nu = max(R - 1, 0) * 2.0 ** -24
    bound = nu / (1 - nu) * np.abs(terms).sum(axis=1) * float(inv_n) + np.abs(exact * float(inv_n)) * 2.0 ** -23
    return exact * float(inv_n), bound


@FUSED
@pytest.mark.parametrize("name", ["col_mean_var_dyn", "col_mean_var_l_dyn"])
@pytest.mark.parametrize("B,R,C", [(1, 0, 8), (1, 1, 1), (3, 64, 1000), (2, 37, 6), (1, 100, 140000),
                                   (1, 1000, 1000), (2, 3000, 65), (4, 300, 4100), (1, 65536, 256)])
def test_col_mean_var(gpu, name, B, R, C, flags):
    print(name, B, R, C, flags, flush=True)
    sys.stdout.flush()
    x = _ints((B, R, C), 8, B * 131 + R * 7 + C)
    inv_n = np.float32(1.0 / max(R, 1))
    mean = to_dev(np.full((B, C), CANARY, np.float32), gpu)
    var = to_dev(np.full((B, C), CANARY, np.float32), gpu)
    args = [to_dev(x, gpu)] + ([mean] if name == "col_mean_var_dyn" else []) + [var]
    run(compiled(name, flags), args, scalars=[float(inv_n)])
    ssum = x.astype(np.float64).sum(axis=1).astype(np.float32)  # exact: |sums| < 2^24
    want_mean = ssum * inv_n
    if name == "col_mean_var_dyn":
        np.testing.assert_array_equal(mean.cpu().numpy(), want_mean)
    if flags:
        want, bound = _passes_bound(x, want_mean, inv_n)
    else:
        want, bound = fused_var_bound(x, want_mean, inv_n)
    got = var.cpu().numpy().astype(np.float64)
    err = np.abs(got - want)
    assert np.all(err <= bound), (name, B, R, C, float(err.max()), float(bound[err > bound].min(initial=0)))


@FUSED
@pytest.mark.parametrize("B,R,C", [(1, 0, 16), (1, 1, 8), (2, 37, 24), (3, 64, 1000), (1, 1000, 4096), (2, 3000, 72),
                                   (1, 65536, 256), (1, 100, 140000), (1, 500, 1004), (1, 700, 1002), (2, 300, 1001)])
def test_col_mean_var_bf16(gpu, B, R, C, flags):
    """bf16 columns (16-byte vectors of 8, or 4 / 2 / 1 at other widths),
    small integers exact in bf16: the mean bit for bit, the variance within
    its lowering's bound."""
    import torch
    print("col_mean_var_bf16", B, R, C, flags, flush=True)
    sys.stdout.flush()
    x = _ints((B, R, C), 8, B * 17 + R * 5 + C)
    inv_n = np.float32(1.0 / max(R, 1))
    mean = to_dev(np.full((B, C), CANARY, np.float32), gpu)
    var = to_dev(np.full((B, C), CANARY, np.float32), gpu)
    xd = torch.from_numpy(x).to(gpu).to(torch.bfloat16)
    run(compiled("col_mean_var_bf16", flags), [xd, mean, var], scalars=[float(inv_n)])
    want_mean = x.astype(np.float64).sum(axis=1).astype(np.float32) * inv_n
    np.testing.assert_array_equal(mean.cpu().numpy(), want_mean)
    if flags:
        want, bound = _passes_bound(x, want_mean, inv_n)
    else:
        want, bound = fused_var_bound(x, want_mean, inv_n)
    err = np.abs(var.cpu().numpy().astype(np.float64) - want)
    assert np.all(err <= bound), (B, R, C, float(err.max()), float(bound[err > bound].min(initial=0)))


@FUSED
@pytest.mark.parametrize("kind", ["offset", "drift"])
@pytest.mark.parametrize("B,R,C", [(1, 5000, 1000), (2, 300, 4100), (1, 100000, 48), (1, 64, 4096), (3, 7, 33)])
def test_col_mean_var_float(gpu, kind, B, R, C, flags):
    """Non-integer columns far from zero mean (normal around 100) and with a
    mean that moves along the rows: the mean within the sequential sum's
    bound of the float64 mean, the variance within its lowering's bound
    around the device's own mean."""
    print("col_mean_var_float", kind, B, R, C, flags, flush=True)
    sys.stdout.flush()
    rng = np.random.default_rng(B * 7 + R + C)
    x = rng.standard_normal((B, R, C))
    x += 100.0 if kind == "offset" else np.linspace(0.0, 50.0, R)[None, :, None]
    x = x.astype(np.float32)
    inv_n = np.float32(1.0 / R)
    mean = to_dev(np.full((B, C), CANARY, np.float32), gpu)
    var = to_dev(np.full((B, C), CANARY, np.float32), gpu)
    run(compiled("col_mean_var_dyn", flags), [to_dev(x, gpu), mean, var], scalars=[float(inv_n)])
    m = mean.cpu().numpy()
    x64 = x.astype(np.float64)
    g = R * 2.0 ** -24 / (1 - R * 2.0 ** -24)
    mean_bound = (g * np.abs(x64).sum(axis=1) + np.abs(x64.sum(axis=1)) * 2.0 ** -23) * float(inv_n)
    assert np.all(np.abs(m - x64.sum(axis=1) * float(inv_n)) <= mean_bound)
    if flags:
        want, bound = _passes_bound(x, m, inv_n)
    else:
        want, bound = fused_var_bound(x, m, inv_n)
    err = np.abs(var.cpu().numpy().astype(np.float64) - want)
    assert np.all(err <= bound), (kind, B, R, C, float(err.max()), float(bound[err > bound].min(initial=0)))
