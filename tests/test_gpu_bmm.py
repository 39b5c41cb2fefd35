"""Batched contractions: out[b][m][n] = sum_k lhs[b][m][k] * rhs[b][k][n]
(rhs [b][n][k] for the attention-scores orientation, or one rhs shared by
every batch), lowered on the MFMA contraction kernels with one grid of tiles
per batch. Every batch is checked against the oracle's sequential fp32
contraction of that batch, at shapes that take each kernel of the family
(edge tiles, the 8-wave and 4-wave direct-to-LDS 16-bit kernels, the 128 and
256 fp32 tiles), and the fp32 whole-tile kernel at full size on integers,
where every output must equal the float64 product exactly."""
import sys

import numpy as np
import pytest

import oracle
from helpers import assert_reduce_close, canaries, compiled, host, out_dev, run, to_dev
from tcacomp_amd import inputs
from tcacomp_amd.pkg import EMIT_NO_GEMM_SPLIT

pytestmark = pytest.mark.gpu
# Batches of small planes take the small-tile kernel by default; with
# EMIT_NO_GEMM_SPLIT the tile kernels the shapes were chosen for.
SPLIT = pytest.mark.parametrize("flags", [0, EMIT_NO_GEMM_SPLIT], ids=["small", "tiles"])


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _dev16(a, gpu):
    import torch
    if a.dtype == np.float16:
        return to_dev(a, gpu)
    return to_dev(a.view(np.int16), gpu).view(torch.bfloat16)


def _f32(a):
    return a.astype(np.float32) if a.dtype == np.float16 else (a if a.dtype == np.float32 else oracle.bf16_bits_to_f32(a))


def _check(got, a, b, nt, scale=1.0, what=""):
    """Each batch against the oracle (a or b 2-D: shared by every batch)."""
    for i in range(got.shape[0]):
        ai = _f32(a[i] if a.ndim == 3 else a)
        bi = _f32(b[i] if b.ndim == 3 else b)
        want = oracle.gemm(ai, bi, b_nk=nt)
        if scale != 1.0:
            want = (want * np.float32(scale)).astype(np.float32)
        b_kn = np.ascontiguousarray(bi.T) if nt else bi
        bound = np.sqrt((ai.astype(np.float64) ** 2).sum(1))[:, None] * np.sqrt((b_kn.astype(np.float64) ** 2).sum(0))[None, :]
        assert_reduce_close(got[i], want, abs(scale) * bound, ai.shape[1], "%s batch %d" % (what, i))


@pytest.mark.parametrize("B,M,N,K", [(3, 33, 65, 17), (2, 256, 256, 128), (2, 300, 130, 64)])
@SPLIT
def test_bmm_f32(gpu, B, M, N, K, flags):
    _say("bmm f32", B, M, N, K, flags)
    a = inputs.uniform((B, M, K), -1, 1, 0)
    b = inputs.uniform((B, K, N), -1, 1, 1)
    c = out_dev((B, M, N), gpu)
    run(compiled("bmm_f32", flags), [to_dev(a, gpu), to_dev(b, gpu), c])
    got = host(c)
    assert canaries(got) == 0
    _check(got, a, b, False, what="bmm f32")


def test_bmm_f32_whole_tiles_exact(gpu):
    """B = 2 of 4096 x 4096 x 128: the 4-wave direct-to-LDS fp32 kernel on
    integers in [-4, 4] (every partial sum exact in fp32)."""
    Bn, M, N, K = 2, 4096, 4096, 128
    _say("bmm f32 whole tiles", Bn, M, N, K)
    rng = np.random.default_rng(21)
    a = rng.integers(-4, 5, (Bn, M, K)).astype(np.float32)
    b = rng.integers(-4, 5, (Bn, K, N)).astype(np.float32)
    c = out_dev((Bn, M, N), gpu)
    run(compiled("bmm_f32"), [to_dev(a, gpu), to_dev(b, gpu), c])
    got = host(c)
    for i in range(Bn):
        want = (a[i].astype(np.float64) @ b[i].astype(np.float64)).astype(np.float32)
        assert np.array_equal(got[i], want), "batch %d" % i


# Edge kernel only, the 8-wave kernel (K % 64 != 0), the 4-wave kernel
# (K % 64 == 0, K >= 256), and whole tiles beside edge tiles.
BF16_SHAPES = [(3, 33, 65, 40), (4, 256, 512, 96), (2, 512, 256, 256), (3, 300, 264, 256)]


@pytest.mark.parametrize("B,M,N,K", BF16_SHAPES)
@SPLIT
def test_bmm_bf16_nt(gpu, B, M, N, K, flags):
    _say("bmm bf16 nt", B, M, N, K, flags)
    a = oracle.to_bf16_bits(inputs.uniform((B, M, K), -1, 1, 2))
    b = oracle.to_bf16_bits(inputs.uniform((B, N, K), -1, 1, 3))
    c = out_dev((B, M, N), gpu)
    run(compiled("bmm_bf16_nt", flags), [_dev16(a, gpu), _dev16(b, gpu), c])
    got = host(c)
    assert canaries(got) == 0
    _check(got, a, b, True, what="bmm bf16 nt")


@pytest.mark.parametrize("B,M,N,K", [(3, 300, 520, 256), (2, 256, 256, 96), (1, 17, 9, 8)])
@SPLIT
def test_bmm_f16_shared_rhs_scale(gpu, B, M, N, K, flags):
    _say("bmm f16 shared", B, M, N, K, flags)
    a = inputs.uniform((B, M, K), -1, 1, 4).astype(np.float16)
    b = inputs.uniform((K, N), -1, 1, 5).astype(np.float16)
    c = out_dev((B, M, N), gpu)
    run(compiled("bmm_f16_shared_scale", flags), [to_dev(a, gpu), to_dev(b, gpu), c], scalars=[0.5])
    got = host(c)
    assert canaries(got) == 0
    _check(got, a, b, False, scale=0.5, what="bmm f16 shared")


def test_bmm_empty_batch(gpu):
    """B = 0: nothing to compute, no launch, no error."""
    a = np.zeros((0, 64, 32), np.float32)
    b = np.zeros((0, 32, 64), np.float32)
    c = out_dev((0, 64, 64), gpu)
    run(compiled("bmm_f32"), [to_dev(a, gpu), to_dev(b, gpu), c])
