"""The reference's own numerical end-to-end tests (internal/e2e), restated
on the device: the same programs (tcacomp_amd.programs.E2E, built through the
pkg rungs or from .tca text), the same shapes, the same inputs (elem(i) =
((i * 2654435761) mod 2^32 mod 1000) / 1000, testing/runners/common.cuh:
19-21, internal/e2e/e2e_test.go:192-200), the canary pre-fill, and the same
acceptance: canary count 0 and max |gpu - reference| <= reduceTol = 2e-3
(internal/e2e/e2e_test.go:20) against the reference's sequential fp32 CPU
loops, here the C oracle's. Each reduction is also held to this build's own
bound, 1e-5 * sqrt(K) * ||terms||_2. The runner protocol lines (KERNEL,
CANARY, CHECKSUM, REF_CHECKSUM, MAXDIFF, SAMPLES) are printed as the
reference's runners print them (e2e_test.go:113-123)."""
import sys

import numpy as np
import pytest

import oracle
from helpers import assert_reduce_close, canaries, host, out_dev, run, to_dev
from tcacomp_amd import compiler, programs, suite

pytestmark = pytest.mark.gpu
REDUCE_TOL = 2e-3  # internal/e2e/e2e_test.go:20
_progs = {}


def e2e(name):
    if name not in _progs:
        _progs[name] = compiler.compile_program(programs.E2E[name]())
    return _progs[name]


def _say(*a, **kw):
    print(*a, flush=True, **kw)
    sys.stdout.flush()


def _report(kernel, got, want, n_canary):
    _say("KERNEL %s" % kernel)
    _say(suite.protocol(got, want, n_canary), end="")
    maxdiff = float(np.abs(got.astype(np.float64) - want.astype(np.float64)).max()) if got.size else 0.0
    assert n_canary == 0, "%s: %d unwritten outputs" % (kernel, n_canary)
    assert maxdiff <= REDUCE_TOL, "%s: max abs diff %g > %g" % (kernel, maxdiff, REDUCE_TOL)


@pytest.mark.parametrize("kernel", ["Redwarp", "ReduceT1"])
def test_e2e_row_sum_1024x512(gpu, kernel):
    # TestReduceWarpE2E (e2e_test.go:300-330) and TestReduceT1E2E
    # (reduce3_test.go:344-376): two schedules of one graph in the reference,
    # one kernel family here; both compare with reduceReference (:227-240).
    R, C = 1024, 512
    _say("e2e", kernel, R, C)
    lhs = oracle.elem(R * C).reshape(R, C)
    want, _ = oracle.row_sum_max(lhs)
    out = out_dev((R,), gpu)
    run(e2e("redwarp"), [to_dev(lhs, gpu), out])
    got = host(out)
    _report(kernel, got, want, canaries(got))
    assert_reduce_close(got, want, np.sqrt((lhs.astype(np.float64) ** 2).sum(1)), C, kernel)


def test_e2e_reduce3(gpu):
    # TestReduce3E2E (reduce3_test.go:308-342): out[i][j] = sum_k lhs[i][j][k]
    # over [64, 32, 512], reduce3Reference (:288-300).
    d0, d1, d2 = 64, 32, 512
    _say("e2e Reduce3", d0, d1, d2)
    lhs = oracle.elem(d0 * d1 * d2).reshape(d0, d1, d2)
    want, _ = oracle.row_sum_max(lhs.reshape(d0 * d1, d2))
    want = want.reshape(d0, d1)
    out = out_dev((d0, d1), gpu)
    run(e2e("red3"), [to_dev(lhs, gpu), out])
    got = host(out)
    _report("Reduce3", got, want, canaries(got))
    assert_reduce_close(got, want, np.sqrt((lhs.astype(np.float64) ** 2).sum(2)), d2, "Reduce3")


@pytest.mark.parametrize("name", ["matmul_scale_written", "matmul_scale_omitted", "matmul_scale_pkg"])
def test_e2e_frontend_matmul_scale(gpu, name):
    # TestFrontendMatmulScale (frontend_test.go:340-396): both .tca forms at
    # M = 64, N = 128, Q = 64, scale 1.5, against frontendMatmulScaleReference
    # (:194-208: a sequential fp32 sum of products, then times scale); the
    # pkg-built oracle program (pkg/oracle_test.go:17-53) on the same run.
    M, N, Q, scale = 64, 128, 64, 1.5
    _say("e2e", name, M, N, Q)
    lhs = oracle.elem(M * N).reshape(M, N)
    rhs = oracle.elem(N * Q).reshape(N, Q)
    acc = oracle.gemm(lhs, rhs)
    want = (acc * np.float32(scale)).astype(np.float32)
    out = out_dev((M, Q), gpu)
    run(e2e(name), [to_dev(lhs, gpu), to_dev(rhs, gpu), out], scalars=[scale])
    got = host(out)
    _report("FrontendMatmulScale", got, want, canaries(got))
    terms = np.sqrt((lhs.astype(np.float64) ** 2).sum(1))[:, None] * np.sqrt((rhs.astype(np.float64) ** 2).sum(0))[None, :]
    assert_reduce_close(got, want, scale * terms, N, name)


def test_e2e_matmul_store_1024(gpu):
    # The matmul_store golden's program (MmLaunch, e2e_test.go:69-124):
    # out[m][n][k] = lhs[m][k] * rhs[n][k] at d0 = d1 = d2 = 1024 (4 GiB of
    # output). Every output is one fp32 product, so the reference checks it
    # exactly (checksum and first 8 values, matmulReference :202-225; the
    # reference's own run of this fixture is skipped there,
    # matmulGoldenDesignGapSkip). Here: the first 8 values and 4096 seeded
    # samples exactly against the oracle's inputs multiplied on the host, and
    # every element bit for bit against the same IEEE product formed on the
    # device.
    import torch
    d = 1024
    _say("e2e Mm", d, d, d)
    lhs = oracle.elem(d * d).reshape(d, d)
    rhs = oracle.elem(d * d).reshape(d, d)
    tl, tr = to_dev(lhs, gpu), to_dev(rhs, gpu)
    out = out_dev((d, d, d), gpu)
    run(e2e("mm"), [tl, tr, out])
    first8 = host(out.view(-1)[:8])
    want8 = (lhs[0, :8] * rhs[0, :8]).astype(np.float32)
    rng = np.random.default_rng(0x7CA0C0DE)
    idx = rng.integers(0, d, size=(4096, 3))
    flat = torch.from_numpy((idx[:, 0] * d * d + idx[:, 1] * d + idx[:, 2]).astype(np.int64)).to(gpu)
    got_s = host(out.view(-1)[flat])
    want_s = (lhs[idx[:, 0], idx[:, 2]] * rhs[idx[:, 1], idx[:, 2]]).astype(np.float32)
    n_canary = int((out == -12345.0).sum().item())
    _say("KERNEL Mm")
    _say("CANARY %d" % n_canary)
    _say("SAMPLES" + "".join(" " + float(v).hex() for v in first8))
    assert n_canary == 0
    assert np.array_equal(first8.view(np.uint32), want8.view(np.uint32))
    assert np.array_equal(got_s.view(np.uint32), want_s.view(np.uint32))
    for m0 in range(0, d, 128):  # slabs of 512 MiB: the expected product stays small
        want = tl[m0:m0 + 128, None, :] * tr[None, :, :]
        assert torch.equal(out[m0:m0 + 128].view(torch.int32), want.view(torch.int32)), "Mm slab at m = %d" % m0
    del out
