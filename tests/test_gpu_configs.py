"""GPU parity of the five benchmark configurations against the CPU oracle.

Tolerances (stated, per the reference's contract for this path):
  - elementwise maps: bit-identical (0 ulp; contraction off on both sides);
  - max reductions: bit-identical (order-independent);
  - sums / contractions: |gpu - oracle| <= 1e-5 * sqrt(K) * ||terms||_2;
  - softmax / layernorm outputs: relative 1e-5 * sqrt(K) (expf, rsqrt are
    ocml on the device and glibc / 1/sqrtf on the host);
  - the generic family folds sequentially from init exactly as the oracle
    does, so its sums and contractions are bit-identical.
Every launch goes through tca_program_launch (the C ABI).
"""
import math
import sys

import numpy as np
import pytest

import oracle
from helpers import (assert_layernorm_close, assert_reduce_close, canaries, compiled, host, out_dev, reduce_tol, run,
                     to_dev)
from tcacomp_amd import inputs
from tcacomp_amd.compiler import TensorDesc
from tcacomp_amd.pkg import EMIT_NO_FUSION, EMIT_NO_GEMM, EMIT_NO_GEMM_SPLIT

pytestmark = pytest.mark.gpu
GENERIC = EMIT_NO_FUSION | EMIT_NO_GEMM
# Contractions at these shapes take the small-tile K-split kernel (output
# planes of M*N <= 2^20); TILES holds the same programs to the oracle on the
# 128/256 tile kernels.
TILES = EMIT_NO_GEMM_SPLIT
SPLIT = pytest.mark.parametrize("flags", [0, TILES], ids=["small", "tiles"])


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


# ---------------------------------------------------------------- C1
@pytest.mark.parametrize("name,flags", [("scale_relu", 0), ("scale_relu_map", 0), ("scale_relu", GENERIC)])
@pytest.mark.parametrize("M,N", [(1, 1), (3, 5), (1000, 1003), (512, 4096), (4096, 4096)])
def test_c1_scale_relu_bitwise(gpu, name, flags, M, N):
    _say("C1", name, flags, M, N)
    x = inputs.uniform((M, N), -1, 1, 0)
    y = inputs.uniform((M, N), -1, 1, 1)
    a = 1.5
    want = oracle.scale_relu(x.reshape(-1), y.reshape(-1), a).reshape(M, N)
    p = compiled(name, flags)
    shape = (M, N) if name == "scale_relu_map" else (M, N, 1)
    z = out_dev((M, N), gpu)
    run(p, [to_dev(x.reshape(shape), gpu), to_dev(y.reshape(shape), gpu), z], scalars=[a])
    got = host(z)
    assert canaries(got) == 0
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "C1 is not bit-identical"


def test_c1_empty(gpu):
    p = compiled("scale_relu")
    x = to_dev(np.zeros((0, 7, 1), np.float32), gpu)
    z = out_dev((0, 7), gpu)
    run(p, [x, x, z], scalars=[1.5])  # grid of 0 workgroups: nothing launched


# ---------------------------------------------------------------- C2
@pytest.mark.parametrize("name,C", [("row_sum_max_8192", 8192), ("row_sum_max_1000", 1000), ("row_sum_max_64", 64)])
@pytest.mark.parametrize("R", [1, 7, 300])
def test_c2_row_sum_max(gpu, name, C, R):
    _say("C2", name, R)
    x = inputs.normal((R, C), 1.0, 0)
    ws, wm = oracle.row_sum_max(x)
    p = compiled(name)
    s, m = out_dev((R,), gpu), out_dev((R,), gpu)
    run(p, [to_dev(x, gpu), s, m])
    gs, gm = host(s), host(m)
    assert canaries(gs) == 0 and canaries(gm) == 0
    assert np.array_equal(gm, wm), "row max must be exact"
    assert_reduce_close(gs, ws, np.sqrt((x.astype(np.float64) ** 2).sum(1)), C, "row sum")


def test_c2_full_size(gpu):
    R, C = 8192, 8192
    _say("C2 full", R, C)
    x = inputs.normal((R, C), 1.0, 0)
    ws, wm = oracle.row_sum_max(x, threads=8)
    p = compiled("row_sum_max_8192")
    s, m = out_dev((R,), gpu), out_dev((R,), gpu)
    run(p, [to_dev(x, gpu), s, m])
    assert np.array_equal(host(m), wm)
    assert_reduce_close(host(s), ws, np.sqrt((x.astype(np.float64) ** 2).sum(1)), C, "row sum")


def test_c2_generic_is_sequential(gpu):
    """The generic family folds in the oracle's order: bit-identical sums."""
    R, C = 37, 1000
    x = inputs.normal((R, C), 1.0, 3)
    ws, wm = oracle.row_sum_max(x)
    p = compiled("row_sum_max_1000", GENERIC)
    s, m = out_dev((R,), gpu), out_dev((R,), gpu)
    run(p, [to_dev(x, gpu), s, m])
    assert np.array_equal(host(s), ws) and np.array_equal(host(m), wm)


def test_c2_special_values(gpu):
    """-inf init: an all -inf row has max -inf; +inf dominates; NaN-free."""
    C = 64
    x = np.zeros((3, C), np.float32)
    x[0, :] = -np.inf
    x[1, 5] = np.inf
    x[2, :] = np.arange(C, dtype=np.float32) - 40
    ws, wm = oracle.row_sum_max(x)
    p = compiled("row_sum_max_64")
    s, m = out_dev((3,), gpu), out_dev((3,), gpu)
    run(p, [to_dev(x, gpu), s, m])
    assert np.array_equal(host(m), wm)
    assert np.array_equal(host(s)[1:], ws[1:]) and host(s)[0] == -np.inf


# ---------------------------------------------------------------- C3
def _softmax_check(got, want, C):
    rel = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want.astype(np.float64)), 1e-30)
    assert rel.max() <= reduce_tol(C), "softmax relative error %g" % rel.max()
    rows = got.astype(np.float64).sum(1)
    assert np.abs(rows - 1.0).max() <= reduce_tol(C)


@pytest.mark.parametrize("name,C,flags", [("softmax_4096", 4096, 0), ("softmax_200", 200, 0),
                                          ("softmax_200", 200, GENERIC), ("softmax_16384", 16384, 0)])
@pytest.mark.parametrize("R", [1, 5, 257])
def test_c3_softmax(gpu, name, C, flags, R):
    _say("C3", name, flags, R)
    x = inputs.normal((R, C), 2.0, 0)
    want = oracle.softmax(x)
    p = compiled(name, flags)
    y = out_dev((R, C), gpu)
    run(p, [to_dev(x, gpu), y])
    got = host(y)
    assert canaries(got) == 0
    _softmax_check(got, want, C)


def test_c3_full_size(gpu):
    R, C = 16384, 4096
    _say("C3 full")
    x = inputs.normal((R, C), 2.0, 0)
    want = oracle.softmax(x, threads=8)
    p = compiled("softmax_4096")
    y = out_dev((R, C), gpu)
    run(p, [to_dev(x, gpu), y])
    _softmax_check(host(y), want, C)


# ---------------------------------------------------------------- C4
@pytest.mark.parametrize("name,C,flags", [("layernorm_1024", 1024, 0), ("layernorm_96", 96, 0),
                                          ("layernorm_96", 96, GENERIC)])
@pytest.mark.parametrize("R", [1, 9, 1000])
def test_c4_layernorm(gpu, name, C, flags, R):
    _say("C4", name, flags, R)
    x = inputs.normal((R, C), 1.0, 0)
    g = inputs.uniform((C,), 0.5, 1.5, 1)
    bta = inputs.uniform((C,), -0.1, 0.1, 2)
    inv_n, eps = np.float32(1.0 / C), np.float32(1e-5)
    want = oracle.layernorm(x, g, bta, float(inv_n), float(eps))
    p = compiled(name, flags)
    y = out_dev((R, C), gpu)
    run(p, [to_dev(x, gpu), to_dev(g, gpu), to_dev(bta, gpu), y], scalars=[float(inv_n), float(eps)])
    got = host(y)
    assert canaries(got) == 0
    assert_layernorm_close(got, want, x, g, bta, float(eps), "C4 %s R=%d" % (name, R))


def test_c4_full_size(gpu):
    R, C = 32768, 1024
    x = inputs.normal((R, C), 1.0, 0)
    g = inputs.uniform((C,), 0.5, 1.5, 1)
    bta = inputs.uniform((C,), -0.1, 0.1, 2)
    want = oracle.layernorm(x, g, bta, 1.0 / C, 1e-5, threads=8)
    p = compiled("layernorm_1024")
    y = out_dev((R, C), gpu)
    run(p, [to_dev(x, gpu), to_dev(g, gpu), to_dev(bta, gpu), y], scalars=[1.0 / C, 1e-5])
    got = host(y)
    assert canaries(got) == 0
    assert_layernorm_close(got, want, x, g, bta, 1e-5, "C4 full size")


# ---------------------------------------------------------------- C5
def _gemm_bound(a, b, K):
    an = np.sqrt((a.astype(np.float64) ** 2).sum(1))[:, None]
    bn = np.sqrt((b.astype(np.float64) ** 2).sum(0))[None, :]
    return an * bn


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (33, 65, 17), (128, 128, 128), (200, 136, 300), (512, 384, 1024),
                                   (64, 64, 0)])
@SPLIT
def test_c5_gemm_f32(gpu, M, N, K, flags):
    _say("C5 f32", M, N, K, flags)
    a = inputs.uniform((M, K), -1, 1, 0)
    b = inputs.uniform((K, N), -1, 1, 1)
    want = oracle.gemm(a, b)
    p = compiled("gemm_f32", flags)
    c = out_dev((M, N), gpu)
    run(p, [to_dev(a, gpu), to_dev(b, gpu), c])
    got = host(c)
    assert canaries(got) == 0
    assert_reduce_close(got, want, _gemm_bound(a, b, K), K, "gemm f32")


@pytest.mark.parametrize("M,N,K", [(1, 1, 8), (33, 65, 17), (128, 128, 128), (200, 136, 300), (512, 384, 1024)])
@SPLIT
def test_c5_gemm_bf16(gpu, M, N, K, flags):
    import torch
    _say("C5 bf16", M, N, K, flags)
    a = oracle.to_bf16_bits(inputs.uniform((M, K), -1, 1, 0))
    b = oracle.to_bf16_bits(inputs.uniform((K, N), -1, 1, 1))
    want = oracle.gemm(a, b)
    p = compiled("gemm_bf16", flags)
    c = out_dev((M, N), gpu)
    ta = to_dev(a.view(np.int16), gpu).view(torch.bfloat16)
    tb = to_dev(b.view(np.int16), gpu).view(torch.bfloat16)
    run(p, [ta, tb, c])
    got = host(c)
    assert canaries(got) == 0
    assert_reduce_close(got, want, _gemm_bound(oracle.bf16_bits_to_f32(a), oracle.bf16_bits_to_f32(b), K), K,
                        "gemm bf16")


@pytest.mark.parametrize("M,N,K", [(1, 1, 8), (33, 65, 17), (256, 256, 32), (512, 768, 512), (300, 520, 96)])
@SPLIT
def test_c5_gemm_bf16_nt(gpu, M, N, K, flags):
    """B given as [N][K]: shapes cover the direct-to-LDS interior path
    (256-multiples, K % 32 == 0) and the general edge path in one launch."""
    import torch
    _say("C5 bf16 NT", M, N, K, flags)
    a = oracle.to_bf16_bits(inputs.uniform((M, K), -1, 1, 0))
    b = oracle.to_bf16_bits(inputs.uniform((N, K), -1, 1, 1))
    want = oracle.gemm(a, b, b_nk=True)
    c = out_dev((M, N), gpu)
    run(compiled("gemm_bf16_nt", flags), [to_dev(a.view(np.int16), gpu).view(torch.bfloat16),
                                          to_dev(b.view(np.int16), gpu).view(torch.bfloat16), c])
    got = host(c)
    assert canaries(got) == 0
    bound = _gemm_bound(oracle.bf16_bits_to_f32(a), np.ascontiguousarray(oracle.bf16_bits_to_f32(b).T), K)
    assert_reduce_close(got, want, bound, K, "gemm bf16 nt")


@pytest.mark.parametrize("M,N,K", [(96, 160, 64), (256, 512, 96), (512, 512, 256), (512, 768, 320), (512, 256, 192),
                                   (768, 512, 512), (520, 512, 256)])
@SPLIT
def test_c5_gemm_exact_integers(gpu, M, N, K, flags):
    """Small-integer operands: every product and partial sum is exact in
    fp32, so any order gives the exact result (pins the MFMA lane layout,
    the LDS swizzles and the transposing B reads: a transposed, shifted or
    mis-swizzled fragment cannot pass). Whole 256x256 tiles take the bf16
    direct-to-LDS kernels: A in 64-deep slices for K % 64 == 0 and K >= 256
    (K = 256 and 320 are its shortest loops: 8 and 10 steps, the peeled
    tail only), 32-deep slices otherwise (K = 96, 192); the rest the
    general path, in the same launch when tiles of both kinds exist (with
    `tiles`; the default build runs them all on the small-tile kernel)."""
    import torch
    _say("C5 exact", M, N, K, flags)
    rng = np.random.default_rng(5)
    a = rng.integers(-4, 5, (M, K)).astype(np.float32)
    b = rng.integers(-4, 5, (K, N)).astype(np.float32)
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    c = out_dev((M, N), gpu)
    run(compiled("gemm_f32", flags), [to_dev(a, gpu), to_dev(b, gpu), c])
    assert np.array_equal(host(c), want)
    ab, bb = oracle.to_bf16_bits(a), oracle.to_bf16_bits(b)
    c = out_dev((M, N), gpu)
    run(compiled("gemm_bf16", flags), [to_dev(ab.view(np.int16), gpu).view(torch.bfloat16),
                                       to_dev(bb.view(np.int16), gpu).view(torch.bfloat16), c])
    assert np.array_equal(host(c), want)
    bt = np.ascontiguousarray(bb.T)
    c = out_dev((M, N), gpu)
    run(compiled("gemm_bf16_nt", flags), [to_dev(ab.view(np.int16), gpu).view(torch.bfloat16),
                                          to_dev(bt.view(np.int16), gpu).view(torch.bfloat16), c])
    assert np.array_equal(host(c), want)


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 64), (4100, 4104, 40), (4352, 4096, 16), (4097, 4096, 33),
                                   (4096, 4101, 48), (4095, 4096, 48), (2100, 3000, 40), (1000, 4224, 33),
                                   (4096, 4096, 128), (4352, 4608, 160), (4096, 4352, 224)])
@pytest.mark.parametrize("nt", [False, True])
def test_c5_gemm_f32_large_exact(gpu, M, N, K, nt):
    """fp32 contractions at C5's scale with ragged edges (M, N not multiples
    of the tile, K not a multiple of the 16-deep slice, unaligned rows), B as
    [K][N] and as [N][K], on all three kernels: from M, N >= 4096 on the
    4-wave direct-to-LDS kernel when every tile is whole (K % 32 == 0,
    K >= 128; here its shortest main loops) and 256x256 tiles with 16 waves
    otherwise, 128x128 tiles below. Small-integer operands make every result
    exact, so every tile, slice and edge must be exact."""
    _say("C5 f32 large", M, N, K, "nt" if nt else "")
    rng = np.random.default_rng(M + N + K)
    a = rng.integers(-4, 5, (M, K)).astype(np.float32)
    b = rng.integers(-4, 5, (K, N)).astype(np.float32)
    want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)  # exact: small integers
    name = "gemm_f32_nt" if nt else "gemm_f32"
    p = compiled(name)
    big = M >= 4096 and N >= 4096
    whole = big and M % 256 == 0 and N % 256 == 0 and K % 32 == 0 and K >= 128
    assert p.selected_symbols([TensorDesc(0x1000, (M, K), 0), TensorDesc(0x1000, (N, K) if nt else (K, N), 0),
                               TensorDesc(0x1000, (M, N), 0)]) == ["tca_%s_k0%s" % (name, "_w" if whole else "_v" if big else "")]
    c = out_dev((M, N), gpu)
    bd = np.ascontiguousarray(b.T) if nt else b
    run(p, [to_dev(a, gpu), to_dev(bd, gpu), c])
    assert np.array_equal(host(c), want)


def test_c5_full_size_f32(gpu):
    M = N = K = 4096
    a = inputs.uniform((M, K), -1, 1, 0)
    b = inputs.uniform((K, N), -1, 1, 1)
    c = out_dev((M, N), gpu)
    run(compiled("gemm_f32"), [to_dev(a, gpu), to_dev(b, gpu), c])
    got = host(c)
    rows = np.random.default_rng(2).choice(M, 16, replace=False)
    want = oracle.gemm(np.ascontiguousarray(a[rows]), b, threads=8)
    assert_reduce_close(got[rows], want, _gemm_bound(a[rows], b, K), K, "gemm f32 4096^3 sample")
    assert math.isfinite(float(got.sum()))


def test_c5_generic_is_sequential(gpu):
    M, N, K = 40, 24, 77
    a = inputs.uniform((M, K), -1, 1, 0)
    b = inputs.uniform((K, N), -1, 1, 1)
    c = out_dev((M, N), gpu)
    run(compiled("gemm_f32", GENERIC), [to_dev(a, gpu), to_dev(b, gpu), c])
    assert np.array_equal(host(c), oracle.gemm(a, b))


def test_c5_full_size_bf16(gpu):
    import torch
    M = N = K = 4096
    a = oracle.to_bf16_bits(inputs.uniform((M, K), -1, 1, 0))
    b = oracle.to_bf16_bits(inputs.uniform((K, N), -1, 1, 1))
    c = out_dev((M, N), gpu)
    run(compiled("gemm_bf16"), [to_dev(a.view(np.int16), gpu).view(torch.bfloat16),
                                to_dev(b.view(np.int16), gpu).view(torch.bfloat16), c])
    got = host(c)
    # Check a seeded sample of rows against the oracle (full oracle is minutes of CPU).
    rows = np.random.default_rng(1).choice(M, 16, replace=False)
    want = oracle.gemm(np.ascontiguousarray(a[rows]), b, threads=8)
    bound = _gemm_bound(oracle.bf16_bits_to_f32(a[rows]), oracle.bf16_bits_to_f32(b), K)
    assert_reduce_close(got[rows], want, bound, K, "gemm bf16 4096^3 sample")
    assert math.isfinite(float(got.sum()))


@pytest.mark.parametrize("name", ["gemm_f32", "gemm_f32_nt", "gemm_bf16", "gemm_bf16_nt"])
def test_c5_full_size_exact(gpu, name):
    """C5's full shape, 4096^3, on small-integer operands in [-4, 4]: exact
    in bf16 and fp32, every product exact and every partial sum an integer
    of magnitude <= 16 * 4096 < 2^24, so every one of the 16.8 M outputs
    (every tile, slice and MFMA lane) must equal the float64 product."""
    import torch
    M = N = K = 4096
    _say("C5 full exact", name)
    rng = np.random.default_rng(11)
    a = rng.integers(-4, 5, (M, K)).astype(np.float32)
    b = rng.integers(-4, 5, (K, N)).astype(np.float32)
    want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    if name == "gemm_f32":
        ta, tb = to_dev(a, gpu), to_dev(b, gpu)
    elif name == "gemm_f32_nt":
        ta, tb = to_dev(a, gpu), to_dev(np.ascontiguousarray(b.T), gpu)
    else:
        bb = oracle.to_bf16_bits(b)
        if name == "gemm_bf16_nt":
            bb = np.ascontiguousarray(bb.T)
        ta = to_dev(oracle.to_bf16_bits(a).view(np.int16), gpu).view(torch.bfloat16)
        tb = to_dev(bb.view(np.int16), gpu).view(torch.bfloat16)
    c = out_dev((M, N), gpu)
    run(compiled(name), [ta, tb, c])
    got = host(c)
    assert canaries(got) == 0
    bad = np.argwhere(got != want)
    assert bad.size == 0, "%s: %d of %d outputs differ; first at %s: %g vs %g" % (
        name, len(bad), M * N, tuple(bad[0]), got[tuple(bad[0])], want[tuple(bad[0])])
