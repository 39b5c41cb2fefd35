"""Shared helpers for the parity tests: compile-from-cache, run on the GPU,
and the stated tolerances."""
import math

import numpy as np

from tcacomp_amd import compiler, programs

CANARY = -12345.0  # testing/runners/softmax.cu:24: catches unwritten outputs

_cache = {}


def compiled(name, flags=0):
    """CompiledProgram for a registered program (tcacomp_amd.programs)."""
    key = (name, flags)
    if key not in _cache:
        if name in programs.CONFIG_PROGRAMS:
            factory = programs.CONFIG_PROGRAMS[name]
        else:
            factory = programs.SUITE[name][0]
        _cache[key] = compiler.compile_program(factory(), flags=flags)
    return _cache[key]


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def out_dev(shape, dev, dtype=None):
    import torch
    return torch.full(shape, CANARY, dtype=dtype or torch.float32, device=dev)


def run(prog, tensors, scalars=(), free_dims=()):
    import torch
    prog.launch(tensors, free_dims=free_dims, scalars=scalars)
    torch.cuda.synchronize()


def host(t):
    return t.cpu().numpy()


def canaries(a):
    return int(np.count_nonzero(a == np.float32(CANARY)))


def reduce_tol(K):
    """Reductions/contractions: |gpu - oracle| <= 1e-5 * sqrt(K) * ||terms||_2."""
    return 1e-5 * math.sqrt(max(K, 1))


def assert_reduce_close(got, want, term_l2, K, what=""):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = reduce_tol(K) * np.maximum(term_l2, np.finfo(np.float32).tiny)
    bad = err > bound
    assert not bad.any(), "%s: %d element(s) outside 1e-5*sqrt(K)*||terms||; worst err %g vs bound %g" % (
        what, int(bad.sum()), float(err.max()), float(bound.reshape(-1)[np.argmax(err.reshape(-1))]))


def layernorm_bound(x, gamma, beta, eps):
    """Per-element bound on |gpu - oracle| for y = (x - mean) * rsqrt(var + eps)
    * gamma + beta over the last axis: the reduction tolerance carried
    through the normalisation to first order, in float64.

      mean error   e_m = tol * ||x_row||_2 / C
      var error    e_v = tol * ||(x - mean)^2||_2 / C
      rstd error   relative 0.5 * e_v / (var + eps) + 4 * 2^-24 (rsqrt ulps, var + eps)
      y error      (e_m + |x - mean| * rstd_rel) * rstd * |gamma|
                   + 8 * 2^-24 * (|x - mean| * rstd * |gamma| + |beta|)  (the row map's roundings)
    with tol = 1e-5 * sqrt(C). An element at the row mean is held to about
    1e-5 * |gamma|, not to a fraction of the largest output."""
    x = x.astype(np.float64)
    C = x.shape[-1]
    tol = reduce_tol(C)
    mean = x.mean(-1, keepdims=True)
    d = x - mean
    var = (d * d).mean(-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    e_m = tol * np.sqrt((x * x).sum(-1, keepdims=True)) / C
    e_v = tol * np.sqrt((d ** 4).sum(-1, keepdims=True)) / C
    r_rel = 0.5 * e_v / (var + eps) + 4 * 2.0 ** -24
    g = np.abs(gamma.astype(np.float64))
    return (e_m + np.abs(d) * r_rel) * rstd * g + 8 * 2.0 ** -24 * (np.abs(d) * rstd * g + np.abs(beta))


def assert_layernorm_close(got, want, x, gamma, beta, eps, what="layernorm"):
    """Every element within layernorm_bound; returns the worst err / bound."""
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = layernorm_bound(x, gamma, beta, eps)
    ratio = err / bound
    worst = float(ratio.max()) if ratio.size else 0.0
    i = int(np.argmax(ratio)) if ratio.size else 0
    print("%s: max err %.3g, worst err/bound %.3g" % (what, float(err.max()) if err.size else 0.0, worst))
    assert worst <= 1.0, "%s: element %d err %g exceeds its bound %g" % (
        what, i, float(err.reshape(-1)[i]), float(bound.reshape(-1)[i]))
    return worst


def ulp_diff(a, b):
    """|a - b| in float32 ulps (sign-magnitude ordering)."""
    ai = a.astype(np.float32).view(np.int32).astype(np.int64)
    bi = b.astype(np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    return np.abs(ai - bi)


def fused_var_merge_depth(R):
    """Merges along any chain of the column family's one-read mean and
    variance, for every geometry: a thread's groups of rows (<= R / 16 + 2),
    row slots (<= 256), the chunks of a merge wave and the waves (<= 1024 /
    16 + 16)."""
    return -(-R // 16) + 2 + min(R, 256) + 64 + 16


def fused_var_bound(x, m, inv_n):
    """(exact, bound) for the one-read variance over axis -2 of x [..., R, C]
    given the device's mean m [..., C]: exact = inv_n * sum over R of
    (x - m)^2 in float64, and the bound 2 (D + 16) kappa u T (D the merge
    depth, kappa^2 = 1 + R mean^2 / sum (x - mean)^2; each merge adds
    non-negative terms with a few roundings each, and a merge's difference
    of means an absolute error of a few u times the mean) plus the sum's own
    rounding, gamma_R sum|x|, entering as (gamma_R sum|x|)^2 / R, plus the
    final multiply's rounding. Pinned against a float32 model of the kernels
    in tests/test_col_fused_model.py, where a dropped between-group term or
    a wrong pair weight leaves it."""
    u = 2.0 ** -24
    R = x.shape[-2]
    x64 = x.astype(np.float64)
    d = x64 - np.asarray(m, np.float64)[..., None, :]
    T = (d * d).sum(axis=-2)
    if R == 0:
        return T * float(inv_n), np.zeros_like(T)
    mu = x64.mean(axis=-2)
    c = x64 - mu[..., None, :]
    Tc = (c * c).sum(axis=-2)
    kappa = np.sqrt(1.0 + R * mu * mu / np.where(Tc > 0, Tc, 1.0))
    kappa = np.where(Tc > 0, kappa, 1.0)
    g = R * u / (1 - R * u)
    sum_err = (g * np.abs(x64).sum(axis=-2)) ** 2 / R
    b = (2 * (fused_var_merge_depth(R) + 16) * kappa * u + 2.0 ** -23) * T + sum_err
    return T * float(inv_n), b * float(inv_n)
