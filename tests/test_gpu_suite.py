"""The reference's 14-kernel suite (testing/kernels/**.tca at the dims of
testing/suite.toml), run through the HIP path and checked the way the
reference's runners check it (testing/runners/*.cu): inputs from the
elem(i) formula, the canary prefill, and maxdiff <= the suite tolerance
(testing/suite.toml:6-10). The stricter contract tolerances of this build
are asserted too.
"""
import sys

import numpy as np
import pytest

import oracle
from helpers import canaries, compiled, host, out_dev, reduce_tol, run, to_dev
from tcacomp_amd import programs

pytestmark = pytest.mark.gpu

SUITE_TOL = {"dup_expr": 1e-5, "dup_const": 1e-5, "axpy3": 1e-5, "mlp": 2e-3, "softmax": 2e-3, "mm_small": 2e-3,
             "mm_mid": 2e-3, "mm_splitk": 2e-3, "transpose": 1e-5, "row_sum": 2e-3, "scale_copy": 1e-5,
             "gemm": 2e-3, "qk_score": 2e-3, "layernorm": 1e-5}

RANK3 = {"dup_expr": False, "dup_const": False, "axpy3": False, "scale_copy": False, "transpose": False,
         "layernorm": False, "row_sum": True, "softmax": True}


@pytest.mark.parametrize("name", sorted(programs.SUITE))
def test_suite_kernel(gpu, name):
    print("suite", name, flush=True)
    sys.stdout.flush()
    _, dims, scalars = programs.SUITE[name]
    p = compiled(name)
    sc = list(scalars.values())
    if name in RANK3:
        middle = RANK3[name]
        if middle:
            R, K, C = dims
            shape = (R, K, C)
        else:
            R, C, K = dims
            shape = (R, C, K)
        n = R * C * K
        x = oracle.elem(n).reshape(shape)
        z = oracle.elem(n).reshape(shape)  # the runners fill both from elem(i)
        want = oracle.suite_rank3(name, x, z, middle, sc)
        out = out_dev((R, C), gpu)
        run(p, [to_dev(x, gpu), to_dev(z, gpu), out], scalars=sc)
        terms = K
    else:
        M, K, N = dims
        if name == "qk_score":
            H, D, Nn = dims  # q [H, D], kk [N, D] (testing/runners/qk_score.cu:10)
            a = oracle.elem(H * D).reshape(H, D)
            b = oracle.elem(Nn * D).reshape(Nn, D)
            want = oracle.gemm(a, b, b_nk=True, epi=oracle.EPI_SCALE, scale=scalars["scale"])
            out = out_dev((H, Nn), gpu)
            terms = D
        else:
            a = oracle.elem(M * K).reshape(M, K)
            b = oracle.elem(K * N).reshape(K, N)
            want = oracle.gemm(a, b, epi=oracle.EPI_GELU if name == "mlp" else oracle.EPI_NONE)
            out = out_dev((M, N), gpu)
            terms = K
        run(p, [to_dev(a, gpu), to_dev(b, gpu), out], scalars=sc)
    got = host(out)
    assert canaries(got) == 0, "unwritten outputs"
    maxdiff = float(np.abs(got.astype(np.float64) - want.astype(np.float64)).max())
    print("MAXDIFF", name, maxdiff, flush=True)
    assert maxdiff <= SUITE_TOL[name], "maxdiff %g exceeds the suite tolerance %g" % (maxdiff, SUITE_TOL[name])
    rel = maxdiff / max(1e-30, float(np.abs(want).max()))
    assert rel <= reduce_tol(terms) * 4, rel
