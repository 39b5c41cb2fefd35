"""Prefix fusion: a per-row chain (iterating only the row axis) between the
reductions and the row map of a layernorm, fused into the same row / stream
kernel (one kernel, the per-row value in registers) and also stored as an
output. y against the oracle's layernorm (same arithmetic: (x - mean) *
rsqrtf(var + eps) * gamma + beta), each element within the reduction
tolerance 1e-5*sqrt(K) carried through the normalisation (helpers.layernorm_bound); rstd against a float64 evaluation of 1/sqrt(var + eps) within
the same bound (rsqrtf on the device is ocml's, the oracle's 1/sqrtf)."""
import numpy as np
import pytest

import oracle
from helpers import assert_layernorm_close, canaries, compiled, host, out_dev, reduce_tol, run, to_dev
from tcacomp_amd import inputs

pytestmark = pytest.mark.gpu


def _check(name, R, C, gpu):
    x = inputs.normal((R, C), 1.0, 0)
    g, b = inputs.uniform((C,), 0.5, 1.5, 1), inputs.uniform((C,), -0.1, 0.1, 2)
    inv_n, eps = float(np.float32(1.0 / C)), 1e-5
    want = oracle.layernorm(x, g, b, inv_n, eps)
    y, rstd = out_dev((R, C), gpu), out_dev((R,), gpu)
    run(compiled(name), [to_dev(x, gpu), to_dev(g, gpu), to_dev(b, gpu), y, rstd], scalars=[inv_n, eps])
    got, gr = host(y), host(rstd)
    assert canaries(got) == 0 and canaries(gr) == 0
    assert_layernorm_close(got, want, x, g, b, eps, "prefix %s R=%d C=%d" % (name, R, C))
    xd = x.astype(np.float64)
    var = ((xd - xd.mean(1, keepdims=True)) ** 2).mean(1)
    wr = 1.0 / np.sqrt(var + eps)
    rel = np.abs(gr - wr) / wr
    assert rel.max() <= reduce_tol(C), "rstd rel err %g" % rel.max()


@pytest.mark.parametrize("R", [1, 37, 4096])
def test_prefix_row_family(gpu, R):
    _check("layernorm_rstd_1024", R, 1024, gpu)


@pytest.mark.parametrize("C", [3, 1024, 5000, 20000])
@pytest.mark.parametrize("R", [1, 37])
def test_prefix_stream_family(gpu, R, C):
    _check("layernorm_rstd_dyn", R, C, gpu)


@pytest.mark.parametrize("R,C", [(300, 40000), (4100, 20001)])
def test_prefix_streamed_rows(gpu, R, C):
    """Streamed rows (beyond the register cache, too many to split): the
    mean and the centred sum of squares in one read, then the per-row rstd
    chain and the row map."""
    _check("layernorm_rstd_dyn", R, C, gpu)
