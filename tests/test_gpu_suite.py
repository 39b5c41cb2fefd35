"""The reference's 14-kernel suite (testing/kernels/**.tca at the dims of
testing/suite.toml), run through the HIP path and checked the way the
reference's runners and orchestrator check it: inputs from the elem(i)
formula, the canary prefill, the runner protocol printed
(testing/runners/common.cuh:50-90) and parsed back
(testing/orchestrator.py:140-164), and the pass rule canary == 0 and
maxdiff <= the suite tolerance (testing/suite.toml:6-10,
testing/orchestrator.py:319-345). The stricter contract tolerance of this
build is asserted too. BENCH_US is the runner's BenchReport: host wall time
of launch + synchronize per iteration.
"""
import sys
import time

import numpy as np
import pytest

import oracle
from helpers import canaries, compiled, host, out_dev, reduce_tol, to_dev
from tcacomp_amd import suite

pytestmark = pytest.mark.gpu


def _oracle(name, ins):
    sc = suite.scalars(name)
    if name in suite.RANK3_MIDDLE:
        return oracle.suite_rank3(name, ins[0], ins[1], suite.RANK3_MIDDLE[name], sc)
    if name == "qk_score":
        return oracle.gemm(ins[0], ins[1], b_nk=True, epi=oracle.EPI_SCALE, scale=sc[0])
    return oracle.gemm(ins[0], ins[1], epi=oracle.EPI_GELU if name == "mlp" else oracle.EPI_NONE)


@pytest.mark.parametrize("name", sorted(suite.REGISTRY))
def test_suite_kernel(gpu, name):
    import torch
    print("suite", name, flush=True)
    sys.stdout.flush()
    ins, out_shape = suite.host_inputs(name)
    want = _oracle(name, ins)
    p = compiled(name)
    out = out_dev(out_shape, gpu)
    args = [to_dev(a, gpu) for a in ins] + [out]
    p.launch(args, scalars=suite.scalars(name))
    torch.cuda.synchronize()
    got = host(out)
    bench = []
    for _ in range(20):
        t0 = time.perf_counter()
        p.launch(args, scalars=suite.scalars(name))
        torch.cuda.synchronize()
        bench.append((time.perf_counter() - t0) * 1e6)
    text = suite.protocol(got, want, canaries(got), bench)
    print(text, end="", flush=True)
    proto = suite.parse_protocol(text)
    assert not suite.verify(name, proto), (name, suite.verify(name, proto))
    assert proto["checksum"] == float(got.astype(np.float64).sum())
    dims = suite.REGISTRY[name][1]
    # the reduced extent: K of [R, C, K] rank-3 kernels, else the middle dim
    # ([R, K, C] middle-axis reductions, [M, K, N] contractions, [H, D, N] qk_score)
    terms = dims[2] if name in suite.RANK3_MIDDLE and not suite.RANK3_MIDDLE[name] else dims[1]
    rel = proto["maxdiff"] / max(1e-30, float(np.abs(want).max()))
    assert rel <= reduce_tol(terms) * 4, rel
