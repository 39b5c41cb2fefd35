"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is chosen so a plausible restatement mistake fails it: a
dropped term, a wrong sign, a transposed operand, a wrong index, a wrong
init. Anchors: the reference's input formula and known values
(testing/runners/common.cuh:19-21), the reference's runtime unit layer built
from its own sources (oracle/_ref, runtime/tests/cpu_tests.cpp: 6166 checks),
exact arithmetic (small integers, dyadic rationals), closed forms and
invariants, and float64 re-evaluation.
"""
import math
import os
import subprocess

import numpy as np
import pytest

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))


def test_elem_formula_known_values():
    # v(i) = float((i * 2654435761u) % 1000u) / 1000.0f with u32 wraparound
    e = oracle.elem(4)
    assert e[0] == np.float32(0.0)
    assert e[1] == np.float32(761) / np.float32(1000)  # 2654435761 % 1000
    assert e[2] == np.float32(226) / np.float32(1000)  # 5308871522 mod 2^32 = 1013904226
    ref = np.array([np.float32(((i * 2654435761) % (1 << 32)) % 1000) / np.float32(1000) for i in range(5000)],
                   np.float32)
    assert np.array_equal(oracle.elem(5000), ref)


def test_bf16_rne_matches_c_and_known_values():
    L = oracle.lib()
    vals = np.array([0.0, -0.0, 1.0, 1.00390625, 1.005859375, 1.0078125, 3.1415926, -2.5e-3, 65504.0,
                     float("inf"), -float("inf"), 1e-40], np.float32)
    vec = oracle.to_bf16_bits(vals)
    for v, h in zip(vals, vec):
        assert L.oracle_f32_to_bf16(float(v)) == int(h)
    # ties to even: 1 + 2^-8 is exactly halfway between 1 and 1 + 2^-7 -> rounds to 1.0
    assert oracle.bf16_bits_to_f32(oracle.to_bf16_bits(np.array([1.00390625], np.float32)))[0] == 1.0
    # 1 + 3*2^-9 rounds up to 1 + 2^-7
    assert oracle.bf16_bits_to_f32(oracle.to_bf16_bits(np.array([1.005859375], np.float32)))[0] == 1.0078125
    rng = np.random.default_rng(0)
    x = rng.standard_normal(10000).astype(np.float32)
    back = oracle.bf16_bits_to_f32(oracle.to_bf16_bits(x))
    assert np.all(np.abs(back - x) <= np.abs(x) * 2.0 ** -8)


def test_scale_relu_closed_form():
    x = np.array([-1.0, -0.5, 0.0, 0.25, 1.0], np.float32)
    y = np.array([1.0, 0.5, -0.25, 0.125, -2.0], np.float32)
    z = oracle.scale_relu(x, y, 1.5)
    assert np.array_equal(z, np.array([0.0, 0.0, 0.0, 0.5, 0.0], np.float32))
    z = oracle.scale_relu(x, y, -2.0)
    assert np.array_equal(z, np.array([3.0, 1.5, 0.0, 0.0, 0.0], np.float32))


def test_row_sum_max_exact_dyadic():
    # dyadic values with small exponents: every partial sum is exact in fp32
    rng = np.random.default_rng(1)
    x = (rng.integers(-512, 512, (17, 300)) / 64.0).astype(np.float32)
    s, m = oracle.row_sum_max(x)
    assert np.array_equal(s, x.astype(np.float64).sum(1).astype(np.float32))
    assert np.array_equal(m, x.max(1))
    # init is -inf for max and +0 for sum: an empty row would return them;
    # a single-column row returns the element itself
    s1, m1 = oracle.row_sum_max(np.ascontiguousarray(x[:, :1]))
    assert np.array_equal(s1, x[:, 0]) and np.array_equal(m1, x[:, 0])


def test_row_sum_sequential_order():
    # 2^24 + 1 + 1 ... : sequential fp32 folding loses every +1 after 2^24
    x = np.array([[2.0 ** 24] + [1.0] * 8], np.float32)
    s, _ = oracle.row_sum_max(x)
    assert s[0] == np.float32(2.0 ** 24)
    x = np.array([[1.0] * 8 + [2.0 ** 24]], np.float32)
    s, _ = oracle.row_sum_max(x)
    assert s[0] == np.float32(2.0 ** 24 + 8)


def test_row_parallel_bitwise_equal():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((101, 257)).astype(np.float32)
    assert all(np.array_equal(a, b) for a, b in zip(oracle.row_sum_max(x, 1), oracle.row_sum_max(x, 7)))
    assert np.array_equal(oracle.softmax(x, 1), oracle.softmax(x, 5))


def test_softmax_invariants():
    rng = np.random.default_rng(3)
    x = (2.0 * rng.standard_normal((64, 500))).astype(np.float32)
    y = oracle.softmax(x)
    assert np.all(y > 0) and np.all(y <= 1)
    assert np.abs(y.astype(np.float64).sum(1) - 1).max() < 1e-5
    # float64 re-evaluation
    xd = x.astype(np.float64)
    e = np.exp(xd - xd.max(1, keepdims=True))
    ref = e / e.sum(1, keepdims=True)
    assert np.abs(y - ref).max() / ref.max() < 1e-5
    # shift by a power of two keeps the result (max subtraction is exact)
    y2 = oracle.softmax((x + np.float32(8.0)).astype(np.float32))
    assert np.abs(y2 - y).max() < 1e-6
    # argmax is preserved, a uniform row is uniform
    assert np.array_equal(y.argmax(1), x.argmax(1))
    assert np.allclose(oracle.softmax(np.zeros((2, 8), np.float32)), 0.125)


def test_layernorm_against_float64_and_special_cases():
    rng = np.random.default_rng(4)
    R, C = 50, 96
    x = rng.standard_normal((R, C)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, C).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, C).astype(np.float32)
    y = oracle.layernorm(x, g, b, 1.0 / C, 1e-5)
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    var = ((xd - mu) ** 2).mean(1, keepdims=True)
    ref = (xd - mu) / np.sqrt(var + 1e-5) * g + b
    assert np.abs(y - ref).max() < 1e-5
    # gamma = 1, beta = 0: rows have mean ~0 and variance ~1
    y1 = oracle.layernorm(x, np.ones(C, np.float32), np.zeros(C, np.float32), 1.0 / C, 0.0)
    assert np.abs(y1.mean(1)).max() < 1e-5 and np.abs(y1.var(1) - 1).max() < 1e-4
    # a constant row normalises to beta (x - mean == 0 exactly)
    yc = oracle.layernorm(np.full((1, C), 3.0, np.float32), g, b, 1.0 / C, 1e-5)
    assert np.array_equal(yc[0], b)


@pytest.mark.parametrize("C", [96, 1024])
def test_layernorm_bound_is_tight(C):
    """The per-element layernorm parity bound of the GPU tests
    (helpers.layernorm_bound): the oracle's fp32 evaluation is inside it
    against float64, and plausible mistakes are outside it: the mean off by
    1e-4, rstd off by 1e-4 relative, gamma applied reversed, beta dropped."""
    from helpers import layernorm_bound
    rng = np.random.default_rng(C)
    R = 64
    x = rng.standard_normal((R, C)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, C).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, C).astype(np.float32)
    eps = 1e-5
    bound = layernorm_bound(x, g, b, eps)
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    rs = 1.0 / np.sqrt(((xd - mu) ** 2).mean(1, keepdims=True) + eps)
    exact = (xd - mu) * rs * g + b
    y = oracle.layernorm(x, g, b, float(np.float32(1.0 / C)), eps)
    assert (np.abs(y - exact) / bound).max() < 0.5
    planted = {"mean + 1e-4": (xd - mu - 1e-4) * rs * g + b,
               "rstd * (1 + 1e-4)": (xd - mu) * rs * (1 + 1e-4) * g + b,
               "gamma reversed": (xd - mu) * rs * g[::-1] + b,
               "beta dropped": (xd - mu) * rs * g}
    for what, wrong in planted.items():
        assert (np.abs(wrong - exact) > bound).any(), what
    # An element at the row mean is held to about 1e-5 * |gamma|, not to a
    # fraction of the row's largest output.
    assert bound.min() < 2e-5 and bound.min() < 1e-3 * np.abs(exact).max()


def test_gemm_exact_small_integers_and_orientation():
    rng = np.random.default_rng(5)
    M, N, K = 13, 11, 29
    a = rng.integers(-8, 9, (M, K)).astype(np.float32)
    b = rng.integers(-8, 9, (K, N)).astype(np.float32)
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    assert np.array_equal(oracle.gemm(a, b), want)
    # [n][k] orientation of B gives the same product
    assert np.array_equal(oracle.gemm(a, np.ascontiguousarray(b.T), b_nk=True), want)
    # a transposed operand would not pass: the matrices are not symmetric
    assert not np.array_equal(oracle.gemm(np.ascontiguousarray(a[:, :N]), np.ascontiguousarray(b[:N, :])),
                              oracle.gemm(np.ascontiguousarray(b[:N, :].T), np.ascontiguousarray(a[:, :N].T)))
    # identity
    eye = np.eye(K, dtype=np.float32)
    assert np.array_equal(oracle.gemm(a, eye), a)
    # (AB)^T = B^T A^T
    bt = np.ascontiguousarray(b.T)
    at = np.ascontiguousarray(a.T)
    assert np.array_equal(oracle.gemm(bt, at), want.T)
    # K = 0: the empty reduction returns init (+0)
    z = oracle.gemm(np.zeros((3, 0), np.float32), np.zeros((0, 4), np.float32))
    assert np.array_equal(z, np.zeros((3, 4), np.float32))


def test_gemm_bf16_matches_f32_on_bf16_values():
    rng = np.random.default_rng(6)
    a = oracle.to_bf16_bits(rng.uniform(-1, 1, (9, 40)).astype(np.float32))
    b = oracle.to_bf16_bits(rng.uniform(-1, 1, (40, 7)).astype(np.float32))
    af, bf = oracle.bf16_bits_to_f32(a), oracle.bf16_bits_to_f32(b)
    assert np.array_equal(oracle.gemm(a, b), oracle.gemm(af, bf))


def test_gemm_epilogues_closed_form():
    a = np.ones((2, 4), np.float32)
    b = np.ones((4, 3), np.float32)
    assert np.array_equal(oracle.gemm(a, b, epi=oracle.EPI_SCALE, scale=0.125), np.full((2, 3), 0.5, np.float32))
    u = np.float32(4.0)
    gelu = np.float32(0.5) * u * (np.float32(1.0) + np.tanh(np.float32(0.79788456) * (u + np.float32(0.044715) * u * u * u)))
    got = oracle.gemm(a, b, epi=oracle.EPI_GELU)
    assert abs(float(got[0, 0]) - float(gelu)) < 1e-6


@pytest.mark.parametrize("kind,scalars", [("dup_expr", (1.5, 0.25)), ("dup_const", ()), ("axpy3", (2.0, 0.5, 0.75)),
                                          ("scale_copy", (1.25, -0.125)), ("transpose", ()),
                                          ("layernorm", (0.015625, 1e-5))])
def test_suite_rank3_closed_forms(kind, scalars):
    """Constant inputs x = v, z = w: every kernel collapses to K * f(v, w)."""
    R, C, K = 3, 5, 8
    v, w = 0.5, 0.25
    x = np.full((R, C, K), v, np.float32)
    z = np.full((R, C, K), w, np.float32)
    got = oracle.suite_rank3(kind, x, z, False, scalars)
    s = scalars
    if kind == "dup_expr":
        t = ((v * v + v * v) * s[0] + (v * v + v * v) * s[1]) * w
        want = K * t
    elif kind == "dup_const":
        t = (0.5 * (v + 0.5 * v * v) * (1 + 0.044715 * v) + math.tanh(0.79788456 * (v + 0.044715 * v) +
                                                                     0.79788456 * 0.5 * v) * 0.5) * w
        want = K * t
    elif kind == "axpy3":
        acc = K * (s[0] * v + s[1] * w)
        want = acc + s[2] * math.tanh(acc)
    elif kind == "scale_copy":
        want = K * (s[0] * v + s[1]) * w
    elif kind == "transpose":
        want = K * v * w
    else:
        acc = K * v * v * w
        want = acc / math.sqrt(acc * s[0] + s[1])
    assert np.allclose(got, want, rtol=2e-6, atol=0)


def test_suite_middle_axis_indexing():
    """row_sum/softmax reduce the MIDDLE axis of [R, K, C]: a one-hot x
    checks the reduced index is k, not j (a wrong index fails)."""
    R, K, C = 2, 4, 6
    x = np.zeros((R, K, C), np.float32)
    x[1, 2, 3] = 5.0
    z = np.ones((R, K, C), np.float32)
    out = oracle.suite_rank3("row_sum", x, z, True)
    want = np.zeros((R, C), np.float32)
    want[1, 3] = 5.0
    assert np.array_equal(out, want)
    out = oracle.suite_rank3("softmax", x, z, True)
    assert out[1, 3] == np.float32(3.0 + math.exp(5.0)) or abs(out[1, 3] - (3 + math.exp(5.0))) < 1e-4
    assert abs(out[0, 0] - 4.0) < 1e-6


def test_reference_runtime_unit_layer():
    """The reference's own CPU unit layer (runtime/tests/cpu_tests.cpp),
    compiled from its sources by oracle/Makefile: its reducer algebra
    (SeqReducer 1.5 + 2.25 = 3.75, init-once, empty-reduce-returns-init) is
    the fold the oracle restates."""
    if not os.path.isdir("/root/reference"):
        pytest.skip("reference tree not mounted")
    if not os.path.exists(oracle.REF_CPU_TESTS) and not oracle.build_ref():
        pytest.skip("reference CPU layer did not build")
    r = subprocess.run([oracle.REF_CPU_TESTS], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0
    assert "0 failures" in r.stdout
