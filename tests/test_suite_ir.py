"""The CPU oracle's suite kernels against the suite programs themselves.

oracle.suite_rank3 and oracle.gemm's epilogues restate the 14 suite kernels
by hand (oracle/oracle.c). Here each is checked against an independent CPU
evaluation (tests/ir_eval.py) of the program's IR, which
tests/test_syntax.py pins to the reference's own testing/kernels/**.tca
sources: a term written wrongly in the oracle fails here even where the
GPU test, checking the device against that same oracle, would agree with
it. Inputs: the runners' elem(i) fill and two seeded random sets, at the
suite dims. Both sides fold every sum sequentially in ascending index in
float32, so sums agree bit for bit; builtins (tanhf, expf, rsqrtf) differ
by the last bit between libm and a float64 evaluation rounded once, so
the comparison is relative 1e-5 sqrt(K) (north_star's contraction bound),
with K the longest fold.
"""
import math

import numpy as np
import pytest

import ir_eval
import oracle
from tcacomp_amd import programs, suite


def _oracle(name, ins):
    sc = suite.scalars(name)
    if name in suite.RANK3_MIDDLE:
        return oracle.suite_rank3(name, ins[0], ins[1], suite.RANK3_MIDDLE[name], sc)
    if name == "qk_score":
        return oracle.gemm(ins[0], ins[1], b_nk=True, epi=oracle.EPI_SCALE, scale=sc[0])
    return oracle.gemm(ins[0], ins[1], epi=oracle.EPI_GELU if name == "mlp" else oracle.EPI_NONE)


def _ir(name, ins):
    prog = programs.SUITE[name][0]()
    p = ir_eval.parse(prog.IRFull())
    inputs = [t for t, (_, _) in p.tensors.items() if not any(s.store[0] == t for s in p.statements)]
    arrays = dict(zip(inputs, ins))
    dims = {}
    for t, a in arrays.items():
        for d, n in zip(p.tensors[t][1], a.shape):
            dims[d] = n
    sc = dict(zip(p.scalars, suite.scalars(name)))
    out = ir_eval.evaluate(p, arrays, sc, dims)
    stored = [s.store[0] for s in p.statements]
    return out[stored[-1]], max(n for n in dims.values())


@pytest.mark.parametrize("name", sorted(suite.REGISTRY))
@pytest.mark.parametrize("fill", ["elem", "rand0", "rand1"])
def test_oracle_suite_formula_matches_program(name, fill):
    ins, _ = suite.host_inputs(name)
    if fill != "elem":
        rng = np.random.default_rng(int(fill[-1]) * 1009 + len(name))
        ins = [rng.uniform(-1, 1, a.shape).astype(np.float32) for a in ins]
    want = _oracle(name, ins)
    got, k = _ir(name, ins)
    assert got.shape == want.shape
    # NaN where both sides take a root of a negative sum (layernorm on signed inputs)
    assert np.array_equal(np.isnan(got), np.isnan(want)), (name, fill)
    ok = ~np.isnan(want)
    tol = 1e-5 * math.sqrt(k)
    err = np.abs(got[ok].astype(np.float64) - want[ok].astype(np.float64))
    scale = np.maximum(np.abs(want[ok].astype(np.float64)), 1.0)
    assert np.all(err <= tol * scale), (name, fill, float((err / scale).max(initial=0)))


def test_interpreter_sees_a_planted_term():
    """A formula that differs from the program by one term fails the check
    above: the oracle's axpy3 with beta's term dropped."""
    ins, _ = suite.host_inputs("axpy3")
    got, _ = _ir("axpy3", ins)
    s = suite.scalars("axpy3")
    x, z = ins
    acc = (np.float32(s[0]) * x).sum(axis=2, dtype=np.float32)  # beta * z dropped
    wrong = acc + np.float32(s[2]) * np.tanh(acc)
    assert not np.allclose(got, wrong, rtol=1e-4)
    right = oracle.suite_rank3("axpy3", x, z, False, s)
    assert np.allclose(got, right, rtol=1e-5)
