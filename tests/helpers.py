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


def ulp_diff(a, b):
    """|a - b| in float32 ulps (sign-magnitude ordering)."""
    ai = a.astype(np.float32).view(np.int32).astype(np.int64)
    bi = b.astype(np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    return np.abs(ai - bi)
