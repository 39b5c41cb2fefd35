"""Host-only checks of the contractions' launch plans: which kernels a
launch selects by the size of the output plane (the small-tile K-split
kernel for M*N <= 2^20, the 128/256 tile kernels above), the chunk count P
of the K split and the grids it implies, and that a plan printed back by the
library (tca_program_plan_text) parses to the same plan: same text again,
same selection at every shape, product guards and pow2 flags included.
tests/test_gpu_gemm_small.py runs the kernels."""
import ctypes
import struct

import pytest

from tcacomp_amd import _lib, compiler, programs
from tcacomp_amd.compiler import TensorDesc
from tcacomp_amd.pkg import EMIT_NO_GEMM_SPLIT

SMALL_MAX = 1 << 20


def _parse(text):
    h = ctypes.c_void_p()
    rc = _lib.lib().tca_program_parse(text.encode(), ctypes.byref(h))
    assert rc == 0, _lib.last_error()
    return h


def _selected(h, shapes, n, dt=0):
    """Kernels a launch runs; `dt` is the dtype code of every tensor but the
    last (f32 0, f16 1, bf16 2), the last one (the output) f32."""
    arr = compiler._descriptors([TensorDesc(0x1000, s, dt if i + 1 < len(shapes) else 0) for i, s in enumerate(shapes)])
    sel = (ctypes.c_uint8 * n)()
    grids = (ctypes.c_uint64 * n)()
    blocks = (ctypes.c_uint32 * n)()
    rc = _lib.lib().tca_program_selected(h, arr, len(shapes), None, 0, sel, grids, blocks, n)
    assert rc == 0, _lib.last_error()
    # what a launch runs: guards hold and the grid is not empty (a merge
    # whose split leaves one chunk has grid 0 and is not launched)
    return [(i, grids[i], blocks[i]) for i in range(n) if sel[i] and grids[i]]


def _chunks(K, tiles, kc_min):
    if K == 0 or tiles == 0:
        return 1
    return max(1, min((K + kc_min - 1) // kc_min, 512 // tiles))


@pytest.mark.parametrize("name", ["gemm_f32", "gemm_f32_nt", "gemm_bf16", "gemm_bf16_nt", "gemm_f16"])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (64, 64, 64), (64, 64, 4096), (256, 256, 4096), (128, 96, 128),
                                   (1024, 1024, 4096), (512, 2048, 40), (1025, 1024, 64), (2048, 2048, 4096),
                                   (64, 64, 0), (0, 64, 64), (33, 30, 20000)])
def test_small_plane_selection(name, M, N, K):
    e = programs.CONFIG_PROGRAMS[name]().emit()
    syms = e.kernel_symbols()
    h = _parse(e.plan)
    nt = name.endswith("_nt")
    dt = 2 if "bf16" in name else 1 if "f16" in name else 0
    sel = _selected(h, [(M, K), (N, K) if nt else (K, N), (M, N)], len(syms), dt)
    names = [syms[i][len("tca_" + name + "_k0"):] for i, _, _ in sel]
    kc_min = 512 if name.startswith("gemm_f32") else 1024
    if M * N == 0:
        assert names == [], names
    elif M * N <= SMALL_MAX:
        tiles = ((M + 31) // 32) * ((N + 31) // 32)
        P = _chunks(K, tiles, kc_min)
        assert names == (["_s", "_sm"] if P > 1 else ["_s"]), names
        grids = {syms[i][-3:]: g for i, g, _ in sel}
        assert grids[syms[sel[0][0]][-3:]] == tiles * P
        if P > 1:
            assert grids["_sm"] == tiles
        assert all(b == 1024 for _, _, b in sel)
        # the partial scratch holds P chunks of every tile: never past its 512 tiles
        assert tiles * P <= 512 or P == 1
    else:
        assert names and not any(n in ("_s", "_sm") for n in names), names
    _lib.lib().tca_program_unload(h)


def test_tile_only_build_has_no_small_kernel():
    e = programs.CONFIG_PROGRAMS["gemm_bf16"]().emit(flags=EMIT_NO_GEMM_SPLIT)
    assert "_k0_s " not in e.plan and "__gemmpart" not in e.plan and "M*N" not in e.plan


@pytest.mark.parametrize("name", ["gemm", "mlp", "mm_mid", "mm_small", "mm_splitk", "qk_score"])
def test_suite_contractions_take_one_small_kernel(name):
    """The reference suite's contractions (testing/suite.toml dims) run on the
    small-tile kernel alone: K <= 256 is one chunk, so no merge launch."""
    from tcacomp_amd import suite
    e = programs.SUITE[name][0]().emit()
    syms = e.kernel_symbols()
    h = _parse(e.plan)
    ins, oshape = suite.host_inputs(name)
    sel = _selected(h, [a.shape for a in ins] + [oshape], len(syms))
    assert [syms[i] for i, _, _ in sel] == ["tca_%s_k0_s" % name]
    _lib.lib().tca_program_unload(h)


def test_small_kernel_source_and_scratch():
    e = programs.CONFIG_PROGRAMS["bmm_f32_nt_shared_a"]().emit()
    # one plan-only scratch of 512 tiles x 1024 floats, passed to both kernels
    assert "dim __gemmdim0 524288" in e.plan and "tensor __gemmpart0 f32 local 1 __gemmdim0" in e.plan
    assert e.plan.count("arg ptr __gemmpart0") == 2
    assert "split K 512 512 0 3 B/1 M/32 N/32" in e.plan and "split K 512 512 1 3 B/1 M/32 N/32" in e.plan
    # the shared A is not offset by the batch, B ([b][n][k]) and C are
    assert "gemm_small<false, true, decltype(epi)>(t0, (t1 + (size_t)bb * K * N), (t2 + (size_t)bb * M * N)" in e.source


PLANS = [("gemm_bf16", programs.CONFIG_PROGRAMS["gemm_bf16"]), ("bmm_f32", programs.CONFIG_PROGRAMS["bmm_f32"]),
         ("layernorm_dyn", programs.CONFIG_PROGRAMS["layernorm_dyn"]),
         ("softmax_dyn", programs.CONFIG_PROGRAMS["softmax_dyn"]),
         ("col_mean_var_dyn", programs.CONFIG_PROGRAMS["col_mean_var_dyn"])]


@pytest.mark.parametrize("name,factory", PLANS)
def test_plan_text_round_trip(name, factory):
    """Parse -> print -> parse: the printed plan prints the same again and
    selects the same kernels with the same grids and blocks at every probed
    shape (the streaming plans' exact-fit guards carry `pow2`, the
    contractions' product guards M*N)."""
    e = factory().emit()
    h1 = _parse(e.plan)
    t1 = _lib.lib().tca_program_plan_text(h1).decode()
    h2 = _parse(t1)
    t2 = _lib.lib().tca_program_plan_text(h2).decode()
    assert t1 == t2
    if name.endswith("_dyn") and name != "col_mean_var_dyn":
        assert " pow2" in t1
    if name.startswith(("gemm", "bmm")):
        assert "M*N 0 1048576 1 0" in t1
    n = len(e.kernel_symbols())
    if name == "gemm_bf16":
        probes = [[(M, K), (K, N), (M, N)] for M, N, K in [(64, 64, 4096), (4096, 4096, 4096), (300, 520, 96),
                                                            (2048, 2048, 64), (4096, 4104, 40)]]
    elif name == "bmm_f32":
        probes = [[(B, M, K), (B, K, N), (B, M, N)] for B, M, N, K in [(2, 64, 64, 4096), (3, 33, 65, 17),
                                                                      (2, 4096, 4096, 128), (1, 2048, 1024, 64)]]
    elif name == "col_mean_var_dyn":
        probes = [[(1, R, C), (1, C), (1, C)] for R, C in [(8192, 8192), (64, 1 << 20), (7, 9)]]
    else:
        probes = [[(R, C)] + ([(C,), (C,)] if name == "layernorm_dyn" else []) + [(R, C)]
                  for R, C in [(3, 16384), (3, 16388), (8192, 8192), (255, 32772), (1, 1 << 20), (7, 8193)]]
    dt = 2 if name == "gemm_bf16" else 0
    for shapes in probes:
        assert _selected(h1, shapes, n, dt) == _selected(h2, shapes, n, dt), shapes
    _lib.lib().tca_program_unload(h1)
    _lib.lib().tca_program_unload(h2)


@pytest.mark.parametrize("guard,M,N,ok", [("M*N 0 100 1 0", 10, 10, True), ("M*N 0 100 1 0", 10, 11, False),
                                          ("M*N*M 1000 1000 1 0", 10, 10, True), ("M*N 0 18446744073709551615 7 0", 7, 3, True),
                                          ("M*N 0 18446744073709551615 7 0", 5, 3, False)])
def test_product_guard(guard, M, N, ok):
    plan = ("tca-plan 1\nprogram g\ndim M 0\ndim N 0\ntensor x f32 in 2 M N\nkernel k 64 0 1 M/1\narg ptr x\n"
            "when %s\nend\n" % guard)
    h = _parse(plan)
    assert bool(_selected(h, [(M, N)], 1)) == ok
    _lib.lib().tca_program_unload(h)


@pytest.mark.parametrize("bad", ["when Q*N 0 1 1 0", "when M* 0 1 1 0", "when *M 0 1 1 0"])
def test_product_guard_names_known_dims(bad):
    plan = "tca-plan 1\nprogram g\ndim M 0\ndim N 0\ntensor x f32 in 2 M N\nkernel k 64 0 1 M/1\narg ptr x\n%s\nend\n" % bad
    h = ctypes.c_void_p()
    assert _lib.lib().tca_program_parse(plan.encode(), ctypes.byref(h)) != 0
    assert "unknown dim" in _lib.last_error()


# Findings of the plan fuzzer (tests/c/fuzz.cpp under AddressSanitizer and
# UBSan, tests/sanitize.py), kept as regression cases: each input must be
# refused with the stated error.
FUZZ_FINDINGS = [
    # no program record: the plan parsed with an empty name, and its printed
    # form ("program " alone) did not parse again
    ("tca-plan 1\ndim R 0\ntensor x f32 in 1 R\nkernel k 64 0 1 R/64\narg ptr x\nend\n", "no program record"),
    ("tca-plan 1\nprogram a\nprogram b\ndim R 0\ntensor x f32 in 1 R\nkernel k 64 0 1 R/64\narg ptr x\nend\n",
     "duplicate program record"),
]


@pytest.mark.parametrize("text,msg", FUZZ_FINDINGS)
def test_plan_fuzz_findings(text, msg):
    h = ctypes.c_void_p()
    assert _lib.lib().tca_program_parse(text.encode(), ctypes.byref(h)) != 0
    assert msg in _lib.last_error(), _lib.last_error()


def test_workspace_overflow_is_an_error():
    """A local whose bytes at the bound dims do not fit in size_t (free dims
    chosen by the caller) fails the launch contract instead of wrapping the
    workspace size (a fuzz finding: the layout of tca_program_kernel_args and
    of a launch overflowed, and the query added the wrapped offset to a null
    workspace base)."""
    text = ("tca-plan 1\nprogram ovf\ndim A 0\ndim Bd 0\ndim Cd 0\ntensor x f32 in 1 A\n"
            "tensor w f32 local 3 A Bd Cd\nkernel k 64 0 1 A/64\narg ptr x\narg ptr w\nend\n")
    h = _parse(text)
    arr = compiler._descriptors([compiler.TensorDesc(0x1000, (1024,), 0)])
    buf = (ctypes.c_ubyte * 64)()
    size = ctypes.c_size_t()
    for fd, ok in (((1 << 31, 1 << 31), False), ((1 << 20, 1 << 12), True)):
        free = (ctypes.c_uint32 * 2)(*fd)
        rc = _lib.lib().tca_program_kernel_args(h, arr, 1, free, 2, None, 0, 0, buf, 64, ctypes.byref(size))
        if ok:
            assert rc == 0, _lib.last_error()
            assert struct.unpack_from("<Q", bytes(buf), 8)[0] == 0  # the only local, at workspace offset 0
        else:
            assert rc != 0 and "exceeds the address space" in _lib.last_error(), _lib.last_error()
    _lib.lib().tca_program_unload(h)
