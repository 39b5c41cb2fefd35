"""The contraction over f16 inputs (fp32 accumulate): C[m][n] = sum_k
f32(A[m][k]) * f32(B[k][n]) with A, B f16 (the DSL's Cast from f16, pkg
types TF16, internal/ir/types.go:13), lowered on the bf16 kernels with the
_f16 MFMAs. The oracle takes the f16 values widened to f32, which is the
program's own Cast, and folds k in order; random operands in [-1, 1] carry
10-bit mantissas, so an operand read as bf16 could not pass."""
import sys

import numpy as np
import pytest

import oracle
from helpers import assert_reduce_close, canaries, compiled, host, out_dev, run, to_dev
from tcacomp_amd import inputs
from tcacomp_amd.pkg import EMIT_NO_GEMM_SPLIT

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _bound(a, b_kn, K):
    return np.sqrt((a.astype(np.float64) ** 2).sum(1))[:, None] * np.sqrt((b_kn.astype(np.float64) ** 2).sum(0))[None, :]


# Edge kernel only (ragged), the 8-wave direct-to-LDS kernel (K % 64 != 0),
# the 4-wave kernel (K % 64 == 0, K >= 256) with edge tiles beside it.
SHAPES = [(1, 1, 8), (33, 65, 17), (256, 256, 32), (256, 512, 96), (512, 384, 1024), (300, 520, 256)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("nt", [False, True])
@pytest.mark.parametrize("flags", [0, EMIT_NO_GEMM_SPLIT], ids=["small", "tiles"])
def test_gemm_f16(gpu, M, N, K, nt, flags):
    """These output planes take the small-tile kernel by default and the
    tile kernels named above with EMIT_NO_GEMM_SPLIT."""
    _say("C5 f16", M, N, K, "nt" if nt else "nn", flags)
    a = inputs.uniform((M, K), -1, 1, 0).astype(np.float16)
    b = inputs.uniform((N, K) if nt else (K, N), -1, 1, 1).astype(np.float16)
    want = oracle.gemm(a.astype(np.float32), b.astype(np.float32), b_nk=nt)
    c = out_dev((M, N), gpu)
    run(compiled("gemm_f16_nt" if nt else "gemm_f16", flags), [to_dev(a, gpu), to_dev(b, gpu), c])
    got = host(c)
    assert canaries(got) == 0
    b_kn = np.ascontiguousarray(b.T) if nt else b
    assert_reduce_close(got, want, _bound(a, b_kn, K), K, "gemm f16")


@pytest.mark.parametrize("name", ["gemm_f16", "gemm_f16_nt"])
def test_gemm_f16_full_size_exact(gpu, name):
    """4096^3 on integers in [-4, 4] (exact in f16, every partial sum an
    integer below 2^24): every output, so every tile, slice and lane, must
    equal the float64 product."""
    M = N = K = 4096
    _say("C5 f16 full exact", name)
    rng = np.random.default_rng(13)
    a = rng.integers(-4, 5, (M, K)).astype(np.float16)
    b = rng.integers(-4, 5, (K, N)).astype(np.float16)
    want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    bb = np.ascontiguousarray(b.T) if name == "gemm_f16_nt" else b
    c = out_dev((M, N), gpu)
    run(compiled(name), [to_dev(a, gpu), to_dev(bb, gpu), c])
    got = host(c)
    assert canaries(got) == 0
    bad = np.argwhere(got != want)
    assert bad.size == 0, "%s: %d of %d outputs differ; first at %s" % (name, len(bad), M * N, tuple(bad[0]))
