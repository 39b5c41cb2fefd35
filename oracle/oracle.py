"""TEST INFRASTRUCTURE ONLY: numpy face of the C oracle (oracle.c).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module. It restates the reference's CPU loops; it is the
checker, never the thing measured or shipped.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")
REF_CPU_TESTS = os.path.join(HERE, "_ref", "cpu_tests")

_lib = None
_F = ctypes.POINTER(ctypes.c_float)
_U16 = ctypes.POINTER(ctypes.c_uint16)

EPI_NONE, EPI_GELU, EPI_SCALE = 0, 1, 2
SUITE_KIND = {"dup_expr": 0, "dup_const": 1, "axpy3": 2, "scale_copy": 3, "row_sum": 4, "softmax": 5,
              "transpose": 6, "layernorm": 7}


def build():
    r = subprocess.run(["make", "-C", HERE, "-s"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + r.stdout + r.stderr)


def build_ref():
    """Builds the reference's runtime CPU layer from its own sources (only
    where /root/reference is mounted)."""
    r = subprocess.run(["make", "-C", HERE, "-s", "ref"], capture_output=True, text=True)
    return r.returncode == 0


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        l = ctypes.CDLL(LIB_PATH)
        l.oracle_elem.restype = ctypes.c_float
        l.oracle_elem.argtypes = [ctypes.c_uint32]
        l.oracle_fill_elem.argtypes = [_F, ctypes.c_uint64]
        l.oracle_f32_to_bf16.restype = ctypes.c_uint16
        l.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        l.oracle_bf16_to_f32.restype = ctypes.c_float
        l.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
        l.oracle_scale_relu.argtypes = [_F, _F, ctypes.c_float, _F, ctypes.c_uint64, ctypes.c_int]
        l.oracle_row_sum_max.argtypes = [_F, ctypes.c_uint32, ctypes.c_uint32, _F, _F, ctypes.c_int]
        l.oracle_softmax.argtypes = [_F, ctypes.c_uint32, ctypes.c_uint32, _F, ctypes.c_int]
        l.oracle_layernorm.argtypes = [_F, _F, _F, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float,
                                       ctypes.c_float, _F, ctypes.c_int]
        l.oracle_gemm.argtypes = [_F, _F, _U16, _U16, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                  ctypes.c_int, ctypes.c_int, ctypes.c_float, _F, ctypes.c_int]
        l.oracle_suite_rank3.argtypes = [ctypes.c_int, _F, _F, ctypes.c_uint32, ctypes.c_uint32,
                                         ctypes.c_uint32, ctypes.c_int, _F, _F]
        _lib = l
    return _lib


def _f(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def _u16(a):
    if a is None:
        return None
    assert a.dtype == np.uint16 and a.flags.c_contiguous
    return a.ctypes.data_as(_U16)


def elem(n):
    out = np.empty(n, np.float32)
    lib().oracle_fill_elem(_f(out), n)
    return out


def to_bf16_bits(x):
    """fp32 -> bf16 bit patterns (round to nearest even)."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    L = lib()
    flat, fo = x.reshape(-1), out.reshape(-1)
    # vectorised RNE (same rule as oracle_f32_to_bf16, cross-checked in tests)
    u = flat.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    fo[:] = r
    del L
    return out


def bf16_bits_to_f32(h):
    return (h.astype(np.uint32) << 16).view(np.float32)


def scale_relu(x, y, a, threads=1):
    z = np.empty_like(x)
    lib().oracle_scale_relu(_f(x), _f(y), a, _f(z), x.size, threads)
    return z


def row_sum_max(x, threads=1):
    R, C = x.shape
    s = np.empty(R, np.float32)
    m = np.empty(R, np.float32)
    lib().oracle_row_sum_max(_f(x), R, C, _f(s), _f(m), threads)
    return s, m


def softmax(x, threads=1):
    R, C = x.shape
    y = np.empty_like(x)
    lib().oracle_softmax(_f(x), R, C, _f(y), threads)
    return y


def layernorm(x, gamma, beta, inv_n, eps, threads=1):
    R, C = x.shape
    y = np.empty_like(x)
    lib().oracle_layernorm(_f(x), _f(gamma), _f(beta), R, C, inv_n, eps, _f(y), threads)
    return y


def gemm(a, b, b_nk=False, epi=EPI_NONE, scale=1.0, threads=1):
    """fp32 inputs (float32 arrays) or bf16 inputs (uint16 bit arrays)."""
    M, K = a.shape
    N = b.shape[0] if b_nk else b.shape[1]
    c = np.empty((M, N), np.float32)
    if a.dtype == np.uint16:
        lib().oracle_gemm(None, None, _u16(a), _u16(b), M, N, K, int(b_nk), epi, scale, _f(c), threads)
    else:
        lib().oracle_gemm(_f(a), _f(b), None, None, M, N, K, int(b_nk), epi, scale, _f(c), threads)
    return c


def suite_rank3(kind, x, z, middle, scalars=()):
    if middle:
        R, K, C = x.shape
    else:
        R, C, K = x.shape
    out = np.empty((R, C), np.float32)
    s = np.array(list(scalars) + [0.0] * (3 - len(scalars)), np.float32)
    lib().oracle_suite_rank3(SUITE_KIND[kind], _f(x), _f(z), R, C, K, int(middle), _f(s), _f(out))
    return out
