"""Contractions with small output planes (M*N <= 2^20) on the small-tile
kernel: 32x32 tiles of C, the k steps of a chunk dealt over the 16 waves of
a workgroup and summed in wave order, and, when the tiles are fewer than the
split target, P chunks of K merged in chunk order by a second kernel
(the split-k schedule class of testing/kernels/tiling/mm_splitk.tca:1-2,
testing/suite.toml:86-93).

Bars: on small-integer operands every partial sum is an integer below 2^24,
so any summation order gives the exact product and every output must equal
it (pins tile coordinates, the MFMA lane layout, the wave and chunk
partition, edges and the merge); on random operands the outputs are held to
the oracle's sequential fp32 fold within 1e-5*sqrt(K)*||terms||_2 (a sample
of rows at the large shapes). The sweep shapes with M*N > 2^20 run on the
tile kernels; they are checked the same way.
"""
import sys

import numpy as np
import pytest

import oracle
from helpers import assert_reduce_close, canaries, compiled, host, out_dev, run, to_dev
from tcacomp_amd import inputs
from tcacomp_amd.compiler import TensorDesc

pytestmark = pytest.mark.gpu

SMALL_MAX = 1 << 20
SWEEP = [(M, N, K) for M in (64, 256, 1024, 2048) for N in (64, 256, 1024, 2048) for K in (64, 4096)]


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _chunks(K, tiles, kc_min):
    """P of the split record (and of gemm_split_chunks): 512 workgroups."""
    if K == 0 or tiles == 0:
        return 1
    return max(1, min((K + kc_min - 1) // kc_min, 512 // tiles))


def _dev(a, gpu, bf16):
    import torch
    if not bf16:
        return to_dev(a, gpu)
    return to_dev(oracle.to_bf16_bits(a).view(np.int16), gpu).view(torch.bfloat16)


def _expect_kernels(p, name, shapes, M, N, K, batch=1):
    """The kernels a launch runs: the small-tile kernel (and its merge when
    the split has P > 1 chunks) for planes of M*N <= 2^20, tile kernels above."""
    dt = 2 if "bf16" in name else 1 if "f16" in name else 0  # input dtype codes; C is f32
    got = p.selected_symbols([TensorDesc(0x1000, s, dt if i < 2 else 0) for i, s in enumerate(shapes)])
    if M * N <= SMALL_MAX:
        tiles = batch * ((M + 31) // 32) * ((N + 31) // 32)
        P = _chunks(K, tiles, 1024 if "bf16" in name or "f16" in name else 512)
        want = ["tca_%s_k0_s" % name] + (["tca_%s_k0_sm" % name] if P > 1 else [])
        assert got == want, (got, want)
    else:
        assert all(not s.endswith("_s") and not s.endswith("_sm") for s in got), got
    return got


@pytest.mark.parametrize("M,N,K", SWEEP)
def test_sweep_exact(gpu, M, N, K):
    """Every output exact on integers in [-4, 4], f32 and bf16, B as [K][N]
    and [N][K]."""
    rng = np.random.default_rng(7 * M + 3 * N + K)
    a = rng.integers(-4, 5, (M, K)).astype(np.float32)
    b = rng.integers(-4, 5, (K, N)).astype(np.float32)
    want = a @ b  # exact in fp32: |partial sums| <= 16 K < 2^24
    bt = np.ascontiguousarray(b.T)
    for name in ("gemm_f32", "gemm_f32_nt", "gemm_bf16", "gemm_bf16_nt"):
        nt, bf = name.endswith("_nt"), "bf16" in name
        _say("small sweep exact", name, M, N, K)
        p = compiled(name)
        _expect_kernels(p, name, [(M, K), (N, K) if nt else (K, N), (M, N)], M, N, K)
        c = out_dev((M, N), gpu)
        run(p, [_dev(a, gpu, bf), _dev(bt if nt else b, gpu, bf), c])
        got = host(c)
        bad = np.argwhere(got != want)
        assert bad.size == 0, "%s %s: %d outputs differ, first at %s: %g vs %g" % (
            name, (M, N, K), len(bad), tuple(bad[0]), got[tuple(bad[0])], want[tuple(bad[0])])


@pytest.mark.parametrize("M,N,K", SWEEP)
def test_sweep_random(gpu, M, N, K):
    """Random U(-1, 1) operands against the oracle (every row up to 256 rows,
    a seeded sample of 16 rows beyond), f32 and bf16, both orientations."""
    a = inputs.uniform((M, K), -1, 1, 0)
    b = inputs.uniform((K, N), -1, 1, 1)
    rows = np.arange(M) if M <= 256 else np.sort(np.random.default_rng(M + N + K).choice(M, 16, replace=False))
    for name in ("gemm_f32", "gemm_f32_nt", "gemm_bf16", "gemm_bf16_nt"):
        nt, bf = name.endswith("_nt"), "bf16" in name
        _say("small sweep random", name, M, N, K)
        aa, bb = (oracle.to_bf16_bits(a), oracle.to_bf16_bits(b)) if bf else (a, b)
        af = oracle.bf16_bits_to_f32(aa) if bf else aa
        bf32 = oracle.bf16_bits_to_f32(bb) if bf else bb
        c = out_dev((M, N), gpu)
        run(compiled(name), [_dev(a, gpu, bf), _dev(np.ascontiguousarray(b.T) if nt else b, gpu, bf), c])
        got = host(c)
        assert canaries(got) == 0
        want = oracle.gemm(np.ascontiguousarray(aa[rows]), bb, threads=8)
        bound = np.sqrt((af[rows].astype(np.float64) ** 2).sum(1))[:, None] * \
            np.sqrt((bf32.astype(np.float64) ** 2).sum(0))[None, :]
        assert_reduce_close(got[rows], want, bound, K, "%s %s" % (name, (M, N, K)))


# Edges of the small kernel: ragged tiles (M, N not multiples of 32), K not
# a multiple of the 8- or 16-deep step and of the 4- or 8-element vector
# (unaligned rows: guarded scalar loads), one step, chunks P > 1 with a
# short last chunk, the largest plane it takes (2^20 outputs), and interior
# tiles whose last step of K is short while the rows stay vector-aligned
# (K % 8 == 4 for f32, K % 16 == 8 for 16-bit: the unguarded loop hands that
# step to the guarded one, in one chunk or the last of several).
EDGE = [(1, 1, 1), (31, 33, 7), (32, 32, 8), (65, 97, 4099), (7, 1000, 1025), (96, 64, 12345), (1024, 1024, 33),
        (512, 2048, 40), (33, 30, 20000), (64, 64, 0), (96, 64, 700), (64, 96, 4104), (128, 32, 1000),
        (32, 64, 12), (64, 64, 24)]


@pytest.mark.parametrize("M,N,K", EDGE)
@pytest.mark.parametrize("name", ["gemm_f32", "gemm_f32_nt", "gemm_bf16", "gemm_bf16_nt", "gemm_f16", "gemm_f16_nt"])
def test_small_edges_exact(gpu, M, N, K, name):
    _say("small edge exact", name, M, N, K)
    nt, half = name.endswith("_nt"), "f16" in name and "bf16" not in name
    rng = np.random.default_rng(M * 31 + N * 17 + K)
    a = rng.integers(-4, 5, (M, K)).astype(np.float32)
    b = rng.integers(-4, 5, (K, N)).astype(np.float32)
    want = a @ b
    bd = np.ascontiguousarray(b.T) if nt else b
    p = compiled(name)
    _expect_kernels(p, name, [(M, K), bd.shape, (M, N)], M, N, K)
    if half:
        ta, tb = to_dev(a.astype(np.float16), gpu), to_dev(bd.astype(np.float16), gpu)
    else:
        bf = "bf16" in name
        ta, tb = _dev(a, gpu, bf), _dev(bd, gpu, bf)
    c = out_dev((M, N), gpu)
    run(p, [ta, tb, c])
    got = host(c)
    bad = np.argwhere(got != want)
    assert bad.size == 0, "%s %s: %d outputs differ, first at %s" % (name, (M, N, K), len(bad), tuple(bad[0]))


def test_small_twice_smaller_second(gpu):
    """The partial scratch is reused: a split launch (P = 8) and then a
    smaller one (P = 2) on the same program must both be exact."""
    p = compiled("gemm_f32")
    for (M, N, K) in [(64, 64, 4096), (96, 64, 700)]:
        rng = np.random.default_rng(K)
        a = rng.integers(-4, 5, (M, K)).astype(np.float32)
        b = rng.integers(-4, 5, (K, N)).astype(np.float32)
        _expect_kernels(p, "gemm_f32", [(M, K), (K, N), (M, N)], M, N, K)
        c = out_dev((M, N), gpu)
        run(p, [to_dev(a, gpu), to_dev(b, gpu), c])
        assert np.array_equal(host(c), a @ b), (M, N, K)


# Batched small planes: one 32x32 tile grid per batch, the chunks over all
# batches' tiles; per-batch and shared operands in both B orientations.
BATCHED = [("bmm_f32", 3, 33, 65, 17), ("bmm_f32", 2, 64, 64, 4096), ("bmm_f32_nt_shared_a", 3, 40, 72, 2000),
           ("bmm_f32_nt_shared_a", 2, 256, 256, 96), ("bmm_bf16", 2, 64, 96, 3000), ("bmm_bf16", 4, 100, 30, 40),
           ("bmm_bf16_nt", 2, 64, 64, 4096)]


@pytest.mark.parametrize("name,B,M,N,K", BATCHED)
def test_small_batched_exact(gpu, name, B, M, N, K):
    _say("small batched exact", name, B, M, N, K)
    nt = name.endswith("_nt") or "_nt_" in name
    shared_a = name.endswith("shared_a")
    rng = np.random.default_rng(B + M + N + K)
    a = rng.integers(-4, 5, (M, K) if shared_a else (B, M, K)).astype(np.float32)
    b = rng.integers(-4, 5, (B, K, N)).astype(np.float32)
    want = np.stack([(a if shared_a else a[i]) @ b[i] for i in range(B)])
    bd = np.ascontiguousarray(b.transpose(0, 2, 1)) if nt else b
    p = compiled(name)
    _expect_kernels(p, name, [a.shape, bd.shape, (B, M, N)], M, N, K, batch=B)
    bf = "bf16" in name
    c = out_dev((B, M, N), gpu)
    run(p, [_dev(a, gpu, bf), _dev(bd, gpu, bf), c])
    got = host(c)
    for i in range(B):
        assert np.array_equal(got[i], want[i]), "batch %d" % i


@pytest.mark.parametrize("name", ["bmm_f32_nt_shared_a", "bmm_bf16"])
def test_batched_tile_kernels_exact(gpu, name):
    """The same operand layouts on the tile kernels (planes above 2^20):
    f32 [N][K] B with a shared A on the 16-wave 256x256 kernel (M = 4100 is
    not a whole number of tiles), bf16 [K][N] B per batch on the direct-to-
    LDS 4-wave kernel and the edge kernel."""
    B, M, N, K = (2, 4100, 4096, 32) if name == "bmm_f32_nt_shared_a" else (2, 1024, 1544, 320)
    _say("batched tiles exact", name, B, M, N, K)
    nt, shared_a = name.endswith("shared_a"), name.endswith("shared_a")
    rng = np.random.default_rng(B * M + N + K)
    a = rng.integers(-4, 5, (M, K) if shared_a else (B, M, K)).astype(np.float32)
    b = rng.integers(-4, 5, (B, K, N)).astype(np.float32)
    bd = np.ascontiguousarray(b.transpose(0, 2, 1)) if nt else b
    p = compiled(name)
    syms = _expect_kernels(p, name, [a.shape, bd.shape, (B, M, N)], M, N, K, batch=B)
    if name == "bmm_f32_nt_shared_a":
        assert syms == ["tca_bmm_f32_nt_shared_a_k0_v"], syms
    bf = "bf16" in name
    c = out_dev((B, M, N), gpu)
    run(p, [_dev(a, gpu, bf), _dev(bd, gpu, bf), c])
    got = host(c)
    for i in range(B):
        want = ((a if shared_a else a[i]) @ b[i])
        assert np.array_equal(got[i], want), "batch %d" % i
