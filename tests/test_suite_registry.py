"""The suite registry (tcacomp_amd/suite.py) against the reference's
testing/suite.toml where the reference tree is mounted, and the runner
protocol's print/parse round trip and pass rule (host only)."""
import os

import numpy as np
import pytest

from tcacomp_amd import programs, suite

SUITE_TOML = "/root/reference/testing/suite.toml"


def test_registry_matches_suite_toml():
    if not os.path.exists(SUITE_TOML):
        pytest.skip("reference tree not mounted")
    tomli = pytest.importorskip("tomli")
    with open(SUITE_TOML, "rb") as f:
        data = tomli.load(f)
    tests = {t["name"]: t for t in data["test"]}
    assert set(tests) == set(suite.REGISTRY)
    for name, (cat, dims, tol, bench_bytes) in suite.REGISTRY.items():
        t = tests[name]
        assert (t["category"], tuple(t["dims"]), t["tolerance"], t["bench_bytes"]) == (cat, dims, tol, bench_bytes), name
        assert {k: float(v) for k, v in t["scalars"].items()} == programs.SUITE[name][2], name
        assert tuple(programs.SUITE[name][1]) == dims, name


def test_protocol_round_trip_and_pass_rule():
    got = np.array([1.0, 2.5, -0.125, 3.0], np.float32)
    want = np.array([1.0, 2.5, -0.125, 3.0005], np.float32)
    p = suite.parse_protocol(suite.protocol(got, want, 0, [10.0, 8.0, 12.0]))
    assert p["canary"] == 0 and p["checksum"] == 6.375 and p["bench"] == (10.0, 8.0, 12.0)
    assert abs(p["maxdiff"] - 0.0005) < 1e-6 and p["samples"][0] == float(1.0).hex()
    assert suite.verify("mm_mid", p) == []          # 2e-3 tolerance
    assert suite.verify("axpy3", p) != []           # 1e-5 tolerance
    assert suite.verify("mm_mid", suite.parse_protocol("CANARY 3\nMAXDIFF 0\n")) != []
    assert suite.verify("mm_mid", suite.parse_protocol("CHECKSUM 1\n")) == ["protocol lines missing"]
    assert "malformed" in suite.parse_protocol("CANARY x\n")
