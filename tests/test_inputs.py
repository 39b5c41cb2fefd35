"""The seeded synthetic-input generators (tcacomp_amd/inputs.py)."""
import numpy as np

from tcacomp_amd import inputs


def test_counter_based_and_deterministic():
    a = inputs.uniform((1000,), -1, 1, 3)
    assert np.array_equal(a, inputs.uniform((1000,), -1, 1, 3))
    # any slice regenerates independently (chunking does not change values)
    assert np.array_equal(inputs.uniform((1000,), -1, 1, 3, chunk=7), a)
    assert np.array_equal(inputs.normal((999,), 2.0, 1, chunk=10), inputs.normal((999,), 2.0, 1))
    # tensor ids and seeds decorrelate
    assert not np.array_equal(a, inputs.uniform((1000,), -1, 1, 4))
    assert not np.array_equal(a, inputs.uniform((1000,), -1, 1, 3, seed=1))


def test_distributions():
    u = inputs.uniform((1 << 20,), -1, 1, 0)
    assert u.min() >= -1 and u.max() < 1
    assert abs(float(u.mean())) < 5e-3 and abs(float(u.var()) - 1 / 3) < 5e-3
    n = inputs.normal((1 << 20,), 2.0, 0)
    assert abs(float(n.mean())) < 1e-2 and abs(float(n.std()) - 2.0) < 1e-2
    assert np.isfinite(n).all()


def test_elem_matches_the_oracle():
    """The product's elem(i) (the suite runners' input formula) equals the C
    oracle's restatement of testing/runners/common.cuh:19-21."""
    import oracle
    for n in (0, 1, 999, 1001, 1 << 20):
        assert np.array_equal(inputs.elem(n), oracle.elem(n)), n
