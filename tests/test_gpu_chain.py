"""Chained reductions in one chain (MidChain.Reduce then AfterReduce.Reduce,
pkg/chain.go:262 applied twice). The emitter splits such a chain into an
inner reduction into a local and an outer reduction of that local, so each
runs on the row/streaming families (and split rows); the fold keeps its
structure: the inner init once per element of the local, the outer init
once per output. Integer-valued inputs make every sum exact, so the device
matches the closed form exactly in any fold order, and matches the generic
lowering of the same program (one thread per output, sequential folds).

With at least 1024 segments (outputs of the outer reduction) the pair runs
as one segment kernel instead: a block per segment folds each row's inner
reduction and then the rows, the local never stored; the shapes with
B >= 1024 reach it (every vector width, rows longer than 4 vectors per
lane, no rows, empty rows)."""
import sys

import numpy as np
import pytest

from helpers import CANARY, compiled, host, out_dev, run, to_dev
from tcacomp_amd.pkg import EMIT_NO_FUSION, EMIT_NO_GEMM

pytestmark = pytest.mark.gpu
GENERIC = EMIT_NO_FUSION | EMIT_NO_GEMM


def _ints(shape, bound, seed):
    return np.random.default_rng(seed).integers(-bound, bound + 1, size=shape).astype(np.float32)


@pytest.mark.parametrize("B,R,C", [(1, 1, 1), (3, 5, 7), (2, 1000, 64), (4, 300, 5000), (1, 20000, 16),
                                   (2, 0, 4), (2, 3, 0), (3, 7, 70001),
                                   # segment kernel
                                   (1024, 1, 1), (1024, 40, 96), (1500, 3, 1000), (2048, 0, 8), (1030, 5, 0),
                                   (1100, 70, 3), (1024, 9, 4100), (1024, 300, 6), (1023, 40, 96)])
def test_chain_sum_max(gpu, B, R, C):
    print("chain_sum_max", B, R, C, flush=True)
    sys.stdout.flush()
    x = _ints((B, R, C), 8, B * 1000 + R + C)
    s = -0.5
    inner = x.astype(np.float64).sum(axis=2).astype(np.float32)  # exact: small integers
    want = (np.max(inner, axis=1, initial=-np.inf).astype(np.float32) * np.float32(s)).astype(np.float32)
    for flags in (0, GENERIC):
        if flags and R * C > 1 << 20:
            continue  # the generic lowering folds a whole output per thread
        o = out_dev((B,), gpu)
        run(compiled("chain_sum_max", flags), [to_dev(x, gpu), o], scalars=[s])
        np.testing.assert_array_equal(host(o), want, err_msg="flags %d" % flags)


@pytest.mark.parametrize("R,C", [(1, 1), (0, 5), (5, 0), (1000, 1000), (16, 1 << 19), (100000, 3), (3, 70001)])
def test_chain_total(gpu, R, C):
    print("chain_total", R, C, flush=True)
    sys.stdout.flush()
    x = _ints((R, C), 1, R + C)
    assert np.abs(x).sum() < 2 ** 24  # exact in any order
    want = np.float32(x.astype(np.float64).sum())
    for flags in (0, GENERIC):
        if flags and R * C > 1 << 20:
            continue  # the generic lowering folds the whole matrix in one thread
        t = out_dev((), gpu)
        run(compiled("chain_total", flags), [to_dev(x, gpu), t])
        assert host(t) == want, "flags %d: %r != %r" % (flags, host(t), want)


@pytest.mark.parametrize("B,R,C", [(1, 1, 1), (5, 3, 7), (3, 1000, 100), (2, 20, 70001), (300, 2, 3), (0, 4, 4),
                                   (4, 0, 4), (4, 4, 0), (1200, 3, 7), (2000, 17, 130)])
def test_chain3_max_total(gpu, B, R, C):
    """Three reduces in one chain: split twice (inner, middle, outer)."""
    print("chain3_max_total", B, R, C, flush=True)
    sys.stdout.flush()
    x = _ints((B, R, C), 4, B * 77 + R * 5 + C)
    want = np.float32(np.max(x.astype(np.float64).sum(axis=(1, 2)), initial=-np.inf))  # exact: small integers
    for flags in (0, GENERIC):
        if flags and B * R * C > 1 << 20:
            continue  # the generic lowering folds everything in one thread
        t = out_dev((), gpu)
        run(compiled("chain3_max_total", flags), [to_dev(x, gpu), t])
        assert host(t) == want, "flags %d: %r != %r" % (flags, host(t), want)


@pytest.mark.parametrize("R,C", [(1, 1), (0, 3), (3, 0), (7, 1000), (40, 70001), (1000, 16)])
def test_chain_halving(gpu, R, C):
    """A streamed inner sum feeding a generic outer fold that is not
    associative (acc / 2 + now), through the HBM local between them. The
    expected value repeats the fold in float32, one rounding per operation
    as on the device (no contraction)."""
    print("chain_halving", R, C, flush=True)
    sys.stdout.flush()
    x = _ints((R, C), 4, R * 3 + C)
    rows = x.astype(np.float64).sum(axis=1).astype(np.float32)  # exact: small integers
    acc = np.float32(0)
    for v in rows:
        acc = np.float32(np.float32(acc * np.float32(0.5)) + v)
    t = out_dev((), gpu)
    run(compiled("chain_halving"), [to_dev(x, gpu), t])
    assert host(t) == acc, "%r != %r" % (host(t), acc)
