"""The streaming row family (row length a run-time dim) against the CPU
oracle. Same tolerances as test_gpu_configs.py: max bit-identical, sums
within 1e-5*sqrt(K)*||terms||_2, softmax/layernorm relative 1e-5*sqrt(K).
Row lengths cover every variant the launch guards choose between (vector
width 4 / 2 / 1 by C mod 4; register-cached in 256-lane blocks up to 1024
vectors per row, in 1024-lane blocks up to 4096, streamed beyond), both
sides of each boundary, empty rows (the output is
init), short rows packed many to a wave, and rows long enough for the
cross-wave LDS meeting (up to 16 waves per row)."""
import sys

import numpy as np
import pytest

import oracle
from helpers import (CANARY, assert_layernorm_close, assert_reduce_close, canaries, compiled, host, out_dev, reduce_tol,
                     run, to_dev)
from tcacomp_amd import inputs
from tcacomp_amd.pkg import EMIT_NO_PASS_FUSION

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("C", [0, 1, 3, 6, 7, 64, 1000, 1023, 1025, 2046, 2050, 4096, 4099, 4100, 8190, 8192,
                               10002, 16384, 16388, 50000])
@pytest.mark.parametrize("R", [1, 7, 300])
def test_stream_row_sum_max(gpu, R, C):
    _say("stream C2", R, C)
    x = inputs.normal((R, C), 1.0, 0)
    ws, wm = oracle.row_sum_max(x)
    s, m = out_dev((R,), gpu), out_dev((R,), gpu)
    run(compiled("row_sum_max_dyn"), [to_dev(x, gpu), s, m])
    gs, gm = host(s), host(m)
    assert canaries(gs) == 0 and canaries(gm) == 0
    assert np.array_equal(gm.view(np.uint32), wm.view(np.uint32)), "row max is not bit-identical"
    if C == 0:
        assert np.all(gs == 0.0) and np.all(np.isneginf(gm))  # empty rows: the inits
    assert_reduce_close(gs, ws, np.sqrt((x.astype(np.float64) ** 2).sum(1)), C, "stream row sum")


def test_stream_matches_register_family(gpu):
    R, C = 64, 8192
    x = inputs.normal((R, C), 1.0, 3)
    outs = []
    for name in ("row_sum_max_dyn", "row_sum_max_8192"):
        s, m = out_dev((R,), gpu), out_dev((R,), gpu)
        run(compiled(name), [to_dev(x, gpu), s, m])
        outs.append((host(s), host(m)))
    assert np.array_equal(outs[0][1].view(np.uint32), outs[1][1].view(np.uint32))
    assert_reduce_close(outs[0][0], outs[1][0].astype(np.float32),
                        2 * np.sqrt((x.astype(np.float64) ** 2).sum(1)), C, "stream vs row")


# Row lengths on both sides of every guard of the f32 variants: 4-vector cache
# (V 4: C <= 16384, V 2: <= 8192, V 1: <= 4096), 8-vector cache (V 4: <= 32768,
# V 2: <= 16384, V 1: <= 8192), streamed beyond.
STREAM_MULTIPASS_C = [1, 5, 200, 4096, 4097, 4098, 8193, 9001, 12002, 16384, 16386, 20000, 20002, 32768, 32772,
                      40000]


@pytest.mark.parametrize("C", STREAM_MULTIPASS_C)
@pytest.mark.parametrize("R", [1, 37])
def test_stream_softmax(gpu, R, C):
    _say("stream C3", R, C)
    x = inputs.normal((R, C), 2.0, 0)
    want = oracle.softmax(x)
    y = out_dev((R, C), gpu)
    run(compiled("softmax_dyn"), [to_dev(x, gpu), y])
    got = host(y)
    assert canaries(got) == 0
    rel = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want.astype(np.float64)), 1e-30)
    assert rel.max() <= reduce_tol(C), "softmax relative error %g" % rel.max()
    assert np.abs(got.astype(np.float64).sum(1) - 1.0).max() <= reduce_tol(C)


@pytest.mark.parametrize("C", [3, 96, 1024, 5000, 8194] + STREAM_MULTIPASS_C[4:])
@pytest.mark.parametrize("R", [1, 37])
def test_stream_layernorm(gpu, R, C):
    _say("stream C4", R, C)
    x = inputs.normal((R, C), 1.0, 0)
    g, b = inputs.uniform((C,), 0.5, 1.5, 1), inputs.uniform((C,), -0.1, 0.1, 2)
    inv_n, eps = float(np.float32(1.0 / C)), 1e-5
    want = oracle.layernorm(x, g, b, inv_n, eps)
    y = out_dev((R, C), gpu)
    run(compiled("layernorm_dyn"), [to_dev(x, gpu), to_dev(g, gpu), to_dev(b, gpu), y], scalars=[inv_n, eps])
    got = host(y)
    assert canaries(got) == 0
    assert_layernorm_close(got, want, x, g, b, eps, "stream C4 R=%d C=%d" % (R, C))


@pytest.mark.parametrize("R,C", [(1, 16388), (3, 1_000_000), (7, 4097), (255, 8194), (2, 4_000_002),
                                 (1, 50_000_000)])
def test_split_rows(gpu, R, C):
    """Few long rows: each row split over many blocks (partial folds into an
    HBM scratch, then a merge); every vector width."""
    _say("split C2", R, C)
    x = inputs.normal((R, C), 1.0, 7)
    ws, wm = oracle.row_sum_max(x)
    s, m = out_dev((R,), gpu), out_dev((R,), gpu)
    run(compiled("row_sum_max_dyn"), [to_dev(x, gpu), s, m])
    gs, gm = host(s), host(m)
    assert np.array_equal(gm.view(np.uint32), wm.view(np.uint32)), "row max is not bit-identical"
    assert_reduce_close(gs, ws, np.sqrt((x.astype(np.float64) ** 2).sum(1)), C, "split row sum")


@pytest.mark.parametrize("N", [16388, 1_000_004, 64 * 1024 * 1024 + 2])
def test_full_reduction(gpu, N):
    """sum and max of a whole vector into rank-0 outputs."""
    _say("full reduction", N)
    x = inputs.normal((1, N), 1.0, 9)
    ws, wm = oracle.row_sum_max(x)
    s, m = out_dev((), gpu), out_dev((), gpu)
    run(compiled("vec_sum_max"), [to_dev(x.reshape(N), gpu), s, m])
    assert np.float32(host(m)).view(np.uint32) == wm.view(np.uint32)[0]
    assert_reduce_close(np.array([host(s)]), ws, np.array([np.sqrt((x.astype(np.float64) ** 2).sum())]), N,
                        "full sum")


def test_split_rows_repeated_shapes(gpu):
    """Split rows keep their partials in the program's workspace, laid out per
    launch from the row count: launches in a row with different row counts
    (and so different layouts, the workspace reused or regrown) all stay
    exact on the max and within tolerance on the sum."""
    prog = compiled("row_sum_max_dyn")
    for R, C in [(3, 100_000), (3, 100_000), (2, 300_000), (5, 50_000), (1, 200_004), (3, 100_000)]:
        x = inputs.normal((R, C), 1.0, R + C)
        ws, wm = oracle.row_sum_max(x)
        s, m = out_dev((R,), gpu), out_dev((R,), gpu)
        run(prog, [to_dev(x, gpu), s, m])
        assert np.array_equal(host(m).view(np.uint32), wm.view(np.uint32)), (R, C)
        assert_reduce_close(host(s), ws, np.sqrt((x.astype(np.float64) ** 2).sum(1)), C, "repeated split")


def test_split_integer_rows(gpu):
    """The split path on u32 monoids: exact."""
    from tcacomp_amd.compiler import TensorDesc
    import torch
    R, C = 2, 1_000_000
    x = np.random.default_rng(11).integers(0, 2**32, size=(R, C), dtype=np.uint64).astype(np.uint32)
    xt = torch.from_numpy(x.view(np.int32)).to(gpu)
    outs = [torch.zeros(R, dtype=torch.int32, device=gpu) for _ in range(3)]
    run(compiled("row_stats_u32_dyn"), [TensorDesc(xt.data_ptr(), (R, C), 4)] +
        [TensorDesc(o.data_ptr(), (R,), 4) for o in outs])
    got = [o.cpu().numpy().view(np.uint32) for o in outs]
    assert np.array_equal(got[0], (x.astype(np.uint64).sum(1) % (1 << 32)).astype(np.uint32))
    assert np.array_equal(got[1], np.bitwise_xor.reduce(x, axis=1))
    assert np.array_equal(got[2], x.max(1))


def test_stream_empty_grid(gpu):
    s, m = out_dev((0,), gpu), out_dev((0,), gpu)
    run(compiled("row_sum_max_dyn"), [to_dev(np.zeros((0, 5), np.float32), gpu), s, m])  # no workgroups launched


# Few long rows of a multi-pass nest: one grid of row chunks per pass (rows <=
# 255 in the streamed range, or up to 4095 rows of >= 16384 vectors), against
# the streamed kernel (256 rows of 8250 vectors) and the oracle; V 4, 2 and 1
# rows, chunk counts from 3 to 512.
MULTIPASS_SPLIT_SHAPES = [(1, 40000), (7, 32772), (3, 100003), (2, 1_000_002), (255, 33000), (256, 33000),
                          (1, 4_000_000), (300, 65540), (1000, 16385)]


@pytest.mark.parametrize("flags", [0, EMIT_NO_PASS_FUSION], ids=["online", "passes"])
@pytest.mark.parametrize("R,C", MULTIPASS_SPLIT_SHAPES)
def test_split_softmax(gpu, R, C, flags):
    """Both lowerings of split rows: the online normaliser (max and exp-sum
    in one read of each chunk) and one partial + merge per pass."""
    _say("split C3", R, C, flags)
    x = inputs.normal((R, C), 2.0, 0)
    want = oracle.softmax(x)
    y = out_dev((R, C), gpu)
    run(compiled("softmax_dyn", flags), [to_dev(x, gpu), y])
    got = host(y)
    assert canaries(got) == 0
    rel = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want.astype(np.float64)), 1e-30)
    assert rel.max() <= reduce_tol(C), "softmax relative error %g" % rel.max()
    assert np.abs(got.astype(np.float64).sum(1) - 1.0).max() <= reduce_tol(C)


# The most elements a tensor may hold: the u32 index domain less the
# kernels' index headroom (2^16).
TOP = 2 ** 32 - 2 ** 16 - 1


@pytest.mark.parametrize("C", [TOP, TOP - 3], ids=["V1", "V4"])
def test_split_rows_at_the_element_limit(gpu, C):
    """One row as long as a tensor may be (17 GB of f32), split over 512
    chunks, the vector indices within 2^16 of 2^32: zeros with marks 1, 2, 4
    at the first, the middle and the last element. Row sum + max must be
    exactly 7 and 4 (an index that wrapped or stopped short changes one);
    softmax must give a zero 1 / S and a mark e^m / S, S = (C - 3) + e + e^2
    + e^4 (one read: the online normaliser); layernorm (gamma 1, beta 0;
    one read: sum and centred sum of squares) must give (x - mean) / sqrt(var
    + eps) from the closed-form mean 7 / C and variance (21 - 49 / C) / C."""
    import torch
    _say("split rows at the element limit", C)
    x = torch.zeros((1, C), device=gpu)
    x[0, 0], x[0, C // 2], x[0, C - 1] = 1.0, 2.0, 4.0
    s, m = out_dev((1,), gpu), out_dev((1,), gpu)
    run(compiled("row_sum_max_dyn"), [x, s, m])
    assert host(s)[0] == 7.0 and host(m)[0] == 4.0, (host(s), host(m))
    at = [0, 1, C // 2, C - 2, C - 1]
    y = torch.full_like(x, CANARY)
    run(compiled("softmax_dyn"), [x, y])
    S = (C - 3) + np.e + np.e ** 2 + np.e ** 4
    got = y[0, at].double().cpu().numpy()
    want = np.array([np.e, 1.0, np.e ** 2, 1.0, np.e ** 4]) / S
    assert np.all(np.abs(got - want) <= 1e-4 * want), (got, want)
    assert abs(float(y.sum(dtype=torch.float64)) - 1.0) <= 1e-4
    assert int((y == CANARY).sum()) == 0
    g, b = torch.ones((C,), device=gpu), torch.zeros((C,), device=gpu)
    inv_n, eps = float(np.float32(1.0 / C)), 1e-5
    y.fill_(CANARY)
    run(compiled("layernorm_dyn"), [x, g, b, y], scalars=[inv_n, eps])
    mean, var = 7.0 / C, (21.0 - 49.0 / C) / C
    xa = np.array([1.0, 0.0, 2.0, 0.0, 4.0])
    want = (xa - mean) / np.sqrt(var + eps)
    got = y[0, at].double().cpu().numpy()
    assert np.all(np.abs(got - want) <= 1e-4 * np.abs(want) + 1e-6), (got, want)
    assert int((y == CANARY).sum()) == 0
    del x, y, g, b
    torch.cuda.empty_cache()


@pytest.mark.parametrize("flags", [0, EMIT_NO_PASS_FUSION], ids=["pairwise", "passes"])
@pytest.mark.parametrize("R,C", [(7, 40000), (3, 100_003), (5, 300_000), (2, 1_000_002), (300, 40000), (4100, 20001)])
def test_split_row_stats_shift(gpu, R, C, flags):
    """A mean whose piped map adds a per-row input (m = sum(x) inv_n +
    shift[r]) and a sum of squares about it whose piped map reads m (rs =
    rsqrtf(T inv_n + eps) + m / 2), both outputs, then y = (x - m) rs; split
    rows in both lowerings, V 4, 1 and 2, the 1x and 4x row-map chunks, and
    streamed rows (300 of 40000, 4100 of 20001: the pair in one read).
    m against the float64 sum (the reduction tolerance on ||x||_2, plus the
    piped map's two roundings); rs against float64 from the device's m
    (T = sum (x - m)^2 to the reduction tolerance on ||(x - m)^2||_2,
    carried through rsqrt to first order, plus 4 ulp); y against (x - m) rs
    from the device's m and rs (two roundings)."""
    _say("split row stats shift", R, C, flags)
    x = inputs.normal((R, C), 1.0, 7)
    shift = inputs.uniform((R,), -2.0, 2.0, 8)
    inv_n, eps = float(np.float32(1.0 / C)), 1e-5
    m, rs, y = out_dev((R,), gpu), out_dev((R,), gpu), out_dev((R, C), gpu)
    run(compiled("row_stats_shift_dyn", flags), [to_dev(x, gpu), to_dev(shift, gpu), m, rs, y], scalars=[inv_n, eps])
    gm, grs, gy = host(m).astype(np.float64), host(rs).astype(np.float64), host(y)
    assert canaries(gy) == 0 and canaries(host(m)) == 0 and canaries(host(rs)) == 0
    u, tol = 2.0 ** -24, reduce_tol(C)
    xd = x.astype(np.float64)
    s64 = xd.sum(1) * inv_n
    m64 = s64 + shift.astype(np.float64)
    bound_m = tol * np.sqrt((xd * xd).sum(1)) * inv_n + 2 * u * (np.abs(s64) + np.abs(m64))
    assert np.all(np.abs(gm - m64) <= bound_m), np.abs(gm - m64) / bound_m
    d = xd - gm[:, None]
    T = (d * d).sum(1)
    q = T * inv_n + eps
    r64 = 1.0 / np.sqrt(q)
    rs64 = r64 + 0.5 * gm
    e_q = tol * np.sqrt((d ** 4).sum(1)) * inv_n
    bound_rs = 0.5 * e_q / q * r64 + 4 * u * (r64 + np.abs(rs64))
    assert np.all(np.abs(grs - rs64) <= bound_rs), np.abs(grs - rs64) / bound_rs
    y64 = d * grs[:, None]
    assert np.all(np.abs(gy - y64) <= 2 * u * np.abs(d) * np.abs(grs)[:, None] + 2 * u * np.abs(y64))


@pytest.mark.parametrize("flags", [0, EMIT_NO_PASS_FUSION], ids=["pairwise", "passes"])
@pytest.mark.parametrize("C", [100_000, 300_000])
def test_split_layernorm_special_rows(gpu, C, flags):
    """Split layernorm rows that stress the one-read variance: a large
    offset (mean 1000, spread 1: the sum of squares about each chunk's own
    mean, not raw squares), a constant row (variance 0), a step between the
    row's halves (the chunks' means differ: the between-chunk terms carry
    the variance), and rows holding +inf or NaN, which are NaN throughout
    as the sequential definition gives them (the oracle). Both lowerings,
    the 1x and the 4x row-map chunks."""
    _say("split C4 special rows", C, flags)
    x = inputs.normal((6, C), 1.0, 6)
    x[0] += 1000.0
    x[1] = 3.0
    x[2, : C // 2] -= 5.0
    x[2, C // 2:] += 5.0
    x[3, C // 3] = np.inf
    x[4, C // 2] = np.nan
    x[5] *= 1e-3
    g, b = inputs.uniform((C,), 0.5, 1.5, 1), inputs.uniform((C,), -0.1, 0.1, 2)
    inv_n, eps = float(np.float32(1.0 / C)), 1e-5
    want = oracle.layernorm(x, g, b, inv_n, eps)
    y = out_dev((6, C), gpu)
    run(compiled("layernorm_dyn", flags), [to_dev(x, gpu), to_dev(g, gpu), to_dev(b, gpu), y], scalars=[inv_n, eps])
    got = host(y)
    assert canaries(got) == 0
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.isnan(got[3]).all() and np.isnan(got[4]).all()
    fin = [0, 1, 2, 5]
    xd = x[fin].astype(np.float64)
    mean = xd.sum(1, keepdims=True) * inv_n
    var = ((xd - mean) ** 2).sum(1, keepdims=True) * inv_n
    want64 = (xd - mean) / np.sqrt(var + eps) * g.astype(np.float64) + b.astype(np.float64)
    assert_layernorm_close(got[fin], want64, x[fin], g, b, eps, "split C4 special rows C=%d" % C)


@pytest.mark.parametrize("C", [40000, 1_000_002])
def test_split_softmax_special_values(gpu, C):
    """Split rows fold the max and the exp-sum in one read (the online
    normaliser); special values must come out as the sequential definition
    gives them (the oracle): -inf entries of a finite row are 0, a row of
    only -inf is NaN (expf(-inf - -inf)), a +inf entry makes its row NaN
    (expf(inf - inf)), a NaN entry makes its row NaN, and a row whose
    maximum is the first or the last element scales the others right."""
    _say("split C3 special values", C)
    x = inputs.normal((6, C), 2.0, 4)
    x[0, ::7] = -np.inf
    x[1, :] = -np.inf
    x[2, C // 3] = np.inf
    x[3, C // 2] = np.nan
    x[4, 0] = 40.0
    x[5, -1] = 40.0
    want = oracle.softmax(x)
    y = out_dev((6, C), gpu)
    run(compiled("softmax_dyn"), [to_dev(x, gpu), y])
    got = host(y)
    assert np.array_equal(np.isnan(got), np.isnan(want)), [int(np.isnan(got[i]).sum()) for i in range(6)]
    fin = ~np.isnan(want)
    rel = np.abs(got[fin].astype(np.float64) - want[fin]) / np.maximum(np.abs(want[fin].astype(np.float64)), 1e-30)
    assert rel.max() <= reduce_tol(C), "softmax relative error %g" % rel.max()
    assert np.all(got[0, ::7] == 0.0)
    assert np.isnan(got[1]).all() and np.isnan(got[2]).all() and np.isnan(got[3]).all()


@pytest.mark.parametrize("flags", [0, EMIT_NO_PASS_FUSION], ids=["pairwise", "passes"])
@pytest.mark.parametrize("R,C", MULTIPASS_SPLIT_SHAPES)
def test_split_layernorm(gpu, R, C, flags):
    """Both lowerings of split rows: the mean and the centred sum of squares
    in one read of each chunk (each chunk's sum and sum of squares about its
    own mean, merged pairwise), and one partial + merge per pass."""
    _say("split C4", R, C, flags)
    x = inputs.normal((R, C), 1.0, 0)
    g, b = inputs.uniform((C,), 0.5, 1.5, 1), inputs.uniform((C,), -0.1, 0.1, 2)
    inv_n, eps = float(np.float32(1.0 / C)), 1e-5
    want = oracle.layernorm(x, g, b, inv_n, eps)
    y = out_dev((R, C), gpu)
    run(compiled("layernorm_dyn", flags), [to_dev(x, gpu), to_dev(g, gpu), to_dev(b, gpu), y], scalars=[inv_n, eps])
    got = host(y)
    assert canaries(got) == 0
    # At a million terms the oracle's sequential fp32 sum of squares is itself
    # off by ~1e-3 in the output (20x the bound, measured against float64), so
    # the bound holds the GPU to the float64 evaluation of the same formula,
    # and the oracle to the reference's own end-to-end tolerance
    # (internal/e2e/e2e_test.go:20, reduceTol 2e-3).
    xd = x.astype(np.float64)
    mean = xd.sum(1, keepdims=True) * inv_n
    var = ((xd - mean) ** 2).sum(1, keepdims=True) * inv_n
    want64 = (xd - mean) / np.sqrt(var + eps) * g.astype(np.float64) + b.astype(np.float64)
    assert_layernorm_close(got, want64, x, g, b, eps, "split C4 R=%d C=%d vs float64" % (R, C))
    diff = float(np.abs(got.astype(np.float64) - want).max())
    print("split C4 R=%d C=%d: max |gpu - oracle| %.3g" % (R, C, diff))
    if C <= 1_100_000:  # at 4 M terms the sequential fold alone is off by ~1.2e-2
        assert diff <= 2e-3


# Streamed rows of a multi-pass nest (too long for the register cache, too
# many or too short to split): V 4, 2 and 1, 256 to 4100 rows, rows of 8193
# to 20001 vectors (every lane 8 to 20 vectors, a ragged last round).
STREAMED_PAIR_SHAPES = [(256, 40000), (300, 20002), (257, 12001), (4100, 20001), (4096, 32772)]


@pytest.mark.parametrize("flags", [0, EMIT_NO_PASS_FUSION], ids=["online", "passes"])
@pytest.mark.parametrize("R,C", STREAMED_PAIR_SHAPES)
def test_streamed_softmax(gpu, R, C, flags):
    """The streamed body folds the max and the exp-sum in one read of the
    row (each lane's online pair, merged over the row's lanes and waves);
    unfused, one read per pass. Against the oracle."""
    _say("streamed C3", R, C, flags)
    x = inputs.normal((R, C), 2.0, 5)
    want = oracle.softmax(x)
    y = out_dev((R, C), gpu)
    run(compiled("softmax_dyn", flags), [to_dev(x, gpu), y])
    got = host(y)
    assert canaries(got) == 0
    rel = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want.astype(np.float64)), 1e-30)
    assert rel.max() <= reduce_tol(C), "softmax relative error %g" % rel.max()
    assert np.abs(got.astype(np.float64).sum(1) - 1.0).max() <= reduce_tol(C)


@pytest.mark.parametrize("flags", [0, EMIT_NO_PASS_FUSION], ids=["pairwise", "passes"])
@pytest.mark.parametrize("R,C", STREAMED_PAIR_SHAPES)
def test_streamed_layernorm(gpu, R, C, flags):
    """The streamed body folds the sum and the centred sum of squares in one
    read of the row (each lane's pairwise triple, merged over the row's
    lanes and waves); unfused, one read per pass. Against the float64
    evaluation of the formula, and the oracle within the reference's own
    end-to-end tolerance."""
    _say("streamed C4", R, C, flags)
    x = inputs.normal((R, C), 1.0, 5)
    g, b = inputs.uniform((C,), 0.5, 1.5, 1), inputs.uniform((C,), -0.1, 0.1, 2)
    inv_n, eps = float(np.float32(1.0 / C)), 1e-5
    want = oracle.layernorm(x, g, b, inv_n, eps)
    y = out_dev((R, C), gpu)
    run(compiled("layernorm_dyn", flags), [to_dev(x, gpu), to_dev(g, gpu), to_dev(b, gpu), y], scalars=[inv_n, eps])
    got = host(y)
    assert canaries(got) == 0
    xd = x.astype(np.float64)
    mean = xd.sum(1, keepdims=True) * inv_n
    var = ((xd - mean) ** 2).sum(1, keepdims=True) * inv_n
    want64 = (xd - mean) / np.sqrt(var + eps) * g.astype(np.float64) + b.astype(np.float64)
    assert_layernorm_close(got, want64, x, g, b, eps, "streamed C4 R=%d C=%d vs float64" % (R, C))
    assert float(np.abs(got.astype(np.float64) - want).max()) <= 2e-3


@pytest.mark.parametrize("flags", [0, EMIT_NO_PASS_FUSION], ids=["fused", "passes"])
@pytest.mark.parametrize("R,C", [(256, 40000), (4100, 20001)])
def test_streamed_special_rows(gpu, R, C, flags):
    """Streamed softmax and layernorm rows holding special values, as the
    split tests hold them: softmax rows with -inf entries (0 out), only
    -inf (NaN), a +inf or a NaN entry (NaN), the maximum first or last;
    layernorm rows offset by 1000, constant (variance 0), a step between
    the halves, +inf, NaN, and a small spread. The other rows are normal."""
    _say("streamed special rows", R, C, flags)
    x = inputs.normal((R, C), 2.0, 4)
    x[0, ::7] = -np.inf
    x[1, :] = -np.inf
    x[2, C // 3] = np.inf
    x[3, C // 2] = np.nan
    x[4, 0] = 40.0
    x[5, -1] = 40.0
    want = oracle.softmax(x)
    y = out_dev((R, C), gpu)
    run(compiled("softmax_dyn", flags), [to_dev(x, gpu), y])
    got = host(y)
    assert np.array_equal(np.isnan(got), np.isnan(want)), [int(np.isnan(got[i]).sum()) for i in range(6)]
    fin = ~np.isnan(want)
    rel = np.abs(got[fin].astype(np.float64) - want[fin]) / np.maximum(np.abs(want[fin].astype(np.float64)), 1e-30)
    assert rel.max() <= reduce_tol(C), "softmax relative error %g" % rel.max()
    assert np.all(got[0, ::7] == 0.0)
    assert np.isnan(got[1]).all() and np.isnan(got[2]).all() and np.isnan(got[3]).all()

    x = inputs.normal((R, C), 1.0, 6)
    x[0] += 1000.0
    x[1] = 3.0
    x[2, : C // 2] -= 5.0
    x[2, C // 2:] += 5.0
    x[3, C // 3] = np.inf
    x[4, C // 2] = np.nan
    x[5] *= 1e-3
    g, b = inputs.uniform((C,), 0.5, 1.5, 1), inputs.uniform((C,), -0.1, 0.1, 2)
    inv_n, eps = float(np.float32(1.0 / C)), 1e-5
    want = oracle.layernorm(x, g, b, inv_n, eps)
    y = out_dev((R, C), gpu)
    run(compiled("layernorm_dyn", flags), [to_dev(x, gpu), to_dev(g, gpu), to_dev(b, gpu), y], scalars=[inv_n, eps])
    got = host(y)
    assert canaries(got) == 0
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.isnan(got[3]).all() and np.isnan(got[4]).all()
    fin = [i for i in range(R) if i not in (3, 4)]
    xd = x[fin].astype(np.float64)
    mean = xd.sum(1, keepdims=True) * inv_n
    var = ((xd - mean) ** 2).sum(1, keepdims=True) * inv_n
    want64 = (xd - mean) / np.sqrt(var + eps) * g.astype(np.float64) + b.astype(np.float64)
    assert_layernorm_close(got[fin], want64, x[fin], g, b, eps, "streamed C4 special rows R=%d C=%d" % (R, C))


# Register-cached (4- and 8-deep), streamed (4- and 1-wide) and split rows
# (1x and 4x row-map chunks).
AFFINE_SHAPES = [(37, 5000), (37, 20002), (300, 40000), (4100, 20001), (3, 100_003), (2, 1_000_002)]


@pytest.mark.parametrize("flags", [0, EMIT_NO_PASS_FUSION], ids=["online", "passes"])
@pytest.mark.parametrize("R,C", AFFINE_SHAPES)
def test_pair_affine_softmax(gpu, R, C, flags):
    """Softmax of E = x t + bias[c] with its max and exp-sum stored: the
    one-read pair's element expression reads a scalar and a column vector.
    Against float64 from the same float32 inputs: E's own rounding (the
    device may contract x t + bias into one fma) moves each exponent by
    <= u (|x t| + |E|), so the outputs get that on top of the reduction
    tolerance, and the max is within it."""
    _say("affine softmax", R, C, flags)
    x = inputs.normal((R, C), 2.0, 11)
    bias = inputs.uniform((C,), -1.0, 1.0, 12)
    t = 0.7
    mx, den, y = out_dev((R,), gpu), out_dev((R,), gpu), out_dev((R, C), gpu)
    run(compiled("softmax_affine_dyn", flags), [to_dev(x, gpu), to_dev(bias, gpu), mx, den, y], scalars=[t])
    gm, gd, gy = host(mx).astype(np.float64), host(den).astype(np.float64), host(y)
    assert canaries(gy) == 0 and canaries(host(mx)) == 0 and canaries(host(den)) == 0
    u = 2.0 ** -24
    P = x.astype(np.float64) * np.float64(np.float32(t))
    E = P + bias.astype(np.float64)
    e_round = u * (np.abs(P) + np.abs(E))  # E's rounding: an fma, or a product and a sum
    m64 = E.max(1)
    assert np.all(np.abs(gm - m64) <= e_round.max(1)), np.abs(gm - m64).max()
    # against the device's max: the terms and the sum carry E's rounding
    p = np.exp(E - gm[:, None])
    d64 = p.sum(1)
    e_tol = reduce_tol(C) + 2 * e_round.max() + 2 * u * np.abs(gm).max()
    assert np.all(np.abs(gd - d64) <= e_tol * d64), (np.abs(gd - d64) / d64).max()
    y64 = p / d64[:, None]
    rel = np.abs(gy.astype(np.float64) - y64) / np.maximum(y64, 1e-30)
    assert rel.max() <= 2 * e_tol, "affine softmax relative error %g" % rel.max()


@pytest.mark.parametrize("flags", [0, EMIT_NO_PASS_FUSION], ids=["pairwise", "passes"])
@pytest.mark.parametrize("R,C", AFFINE_SHAPES)
def test_pair_affine_moments(gpu, R, C, flags):
    """Mean and variance of E = x g[c] + r[row], both stored, then y = (E -
    m) rsqrtf(v + eps): the one-read pair's element expression reads a
    column and a row vector. Against float64 from the same float32 inputs,
    with E's own rounding (<= u (|x g| + |E|), an fma or a product and a
    sum) on top of the reduction tolerance; y from the device's m and v."""
    _say("affine moments", R, C, flags)
    x = inputs.normal((R, C), 1.0, 13)
    g = inputs.uniform((C,), 0.5, 1.5, 14)
    r = inputs.uniform((R,), -2.0, 2.0, 15)
    inv_n, eps = float(np.float32(1.0 / C)), 1e-5
    m, v, y = out_dev((R,), gpu), out_dev((R,), gpu), out_dev((R, C), gpu)
    run(compiled("row_moments_affine_dyn", flags), [to_dev(x, gpu), to_dev(g, gpu), to_dev(r, gpu), m, v, y],
        scalars=[inv_n, eps])
    gm, gv, gy = host(m).astype(np.float64), host(v).astype(np.float64), host(y).astype(np.float64)
    assert canaries(gy) == 0 and canaries(host(m)) == 0 and canaries(host(v)) == 0
    u, tol = 2.0 ** -24, reduce_tol(C)
    P = x.astype(np.float64) * g.astype(np.float64)
    E = P + r.astype(np.float64)[:, None]
    e_round = u * (np.abs(P) + np.abs(E))  # E's rounding: an fma, or a product and a sum
    s64 = E.sum(1) * inv_n
    bound_m = (tol * np.sqrt((E * E).sum(1)) + e_round.sum(1)) * inv_n + 2 * u * np.abs(s64)
    assert np.all(np.abs(gm - s64) <= bound_m), (np.abs(gm - s64) / bound_m).max()
    d = E - gm[:, None]
    v64 = (d * d).sum(1) * inv_n
    bound_v = (tol * np.sqrt((d ** 4).sum(1)) + 2 * (np.abs(d) * e_round).sum(1)) * inv_n + 2 * u * v64
    assert np.all(np.abs(gv - v64) <= bound_v), (np.abs(gv - v64) / bound_v).max()
    rs = 1.0 / np.sqrt(gv + eps)
    y64 = d * rs[:, None]
    # E - m rounded, rsqrtf (a few ulp) of v + eps rounded, the product rounded
    bound_y = (e_round + 2 * u * np.abs(d)) * rs[:, None] + 8 * u * np.abs(y64)
    assert np.all(np.abs(gy - y64) <= bound_y), (np.abs(gy - y64) / np.maximum(bound_y, 1e-300)).max()


@pytest.mark.parametrize("flags", [0, EMIT_NO_PASS_FUSION], ids=["online", "passes"])
@pytest.mark.parametrize("R,C", AFFINE_SHAPES)
def test_pair_softmax_bf16_rows(gpu, R, C, flags):
    """Softmax of bf16 rows computed in f32 (a Cast per element) into an f32
    output: the pair's loads are 8-byte bf16 vectors. Against the oracle fed
    the bf16 values widened to f32 (exact), so the arithmetic is the same."""
    _say("bf16 softmax", R, C, flags)
    xb = oracle.to_bf16_bits(inputs.normal((R, C), 2.0, 16))
    want = oracle.softmax(oracle.bf16_bits_to_f32(xb))
    import torch
    y = out_dev((R, C), gpu)
    run(compiled("softmax_bf16_dyn", flags), [to_dev(xb.view(np.int16), gpu).view(torch.bfloat16), y])
    got = host(y)
    assert canaries(got) == 0
    rel = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want.astype(np.float64)), 1e-30)
    assert rel.max() <= reduce_tol(C), "bf16 softmax relative error %g" % rel.max()
    assert np.abs(got.astype(np.float64).sum(1) - 1.0).max() <= reduce_tol(C)
