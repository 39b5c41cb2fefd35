"""Host-only checks of the C ABI: every declared symbol is exported, the
launch plan parses, the shape contract of the reference launcher
(internal/cg/cxx/launch.go:98-130) and the wave64 launch grammar
(replacing runtime/tca/launch.h:37-58) hold — no GPU needed."""
import ctypes
import os
import re

import pytest

from tcacomp_amd import _lib, build, compiler, programs
from tcacomp_amd.compiler import TensorDesc
from tcacomp_amd.pkg import EMIT_NO_FUSION, EMIT_NO_GEMM, EMIT_NO_PASS_FUSION

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in sorted(os.listdir(os.path.join(REPO, "include"))):
        text = open(os.path.join(REPO, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(tca_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_functions()
    assert len(names) >= 50
    for n in sorted(names):
        assert hasattr(L, n), "libtcacomp.so does not export %s" % n
    bound = {s[0] for s in _lib.SIGNATURES}
    assert names == bound, "ctypes bindings and headers disagree: %s" % (names ^ bound)


def test_validate_launch_grammar():
    L = _lib.lib()
    assert L.tca_rt_validate_launch(1, 256, 0) == 0
    assert L.tca_rt_validate_launch(1, 1024, 160 * 1024) == 0
    assert L.tca_rt_validate_launch(0, 256, 0) == _lib.TCA_ERR_LAUNCH
    assert L.tca_rt_validate_launch(1, 96, 0) == _lib.TCA_ERR_LAUNCH  # not a multiple of 64
    assert "64-lane" in _lib.last_error()
    assert L.tca_rt_validate_launch(1, 32, 0) == _lib.TCA_ERR_LAUNCH  # a 32-lane warp is not a wave
    assert L.tca_rt_validate_launch(1, 2048, 0) == _lib.TCA_ERR_LAUNCH
    assert L.tca_rt_validate_launch(1, 256, 160 * 1024 + 1) == _lib.TCA_ERR_LAUNCH


def test_grid_term_cap():
    rc, h = parse(PLAN.replace("M*N/1024", "M*N/1024:7"))
    assert rc == 0, _lib.last_error()
    rc, h2 = parse(PLAN.replace("M*N/1024", "M*N/1024:0"))
    assert rc == _lib.TCA_ERR_INVALID and "bad cap" in _lib.last_error()


def test_launch_guards():
    """`when` records: parsed, validated, and the variant selection they make."""
    guarded = PLAN.replace("arg scalar a\n", "arg scalar a\nwhen N 0 16 4 0\nwhen M 2 9 1 0\n")
    rc, h = parse(guarded)
    assert rc == 0, _lib.last_error()
    P = 0x1000

    def selected(m, n):
        ts = [TensorDesc(P, (m, n, 4), 0), TensorDesc(P, (n,), 0), TensorDesc(P, (m, n), 0)]
        arr = compiler._descriptors(ts)
        fd = (ctypes.c_uint32 * 1)(3)
        out = (ctypes.c_uint8 * 1)()
        assert _lib.lib().tca_program_selected(h, arr, 3, fd, 1, out, None, None, 1) == 0, _lib.last_error()
        return out[0]
    assert selected(5, 8) == 1
    assert selected(5, 6) == 0  # N % 4 != 0
    assert selected(5, 20) == 0  # N > 16
    assert selected(1, 8) == 0  # M < 2
    assert selected(9, 0) == 1  # bounds inclusive; 0 % 4 == 0
    for bad, msg in [("when N 0 16 0 0", "bad guard"), ("when N 0 16 4 4", "bad guard"),
                     ("when N 9 8 1 0", "bad guard"), ("when Q 0 16 4 0", "unknown dim"),
                     ("when N 0 16", "when <dim>")]:
        rc, _ = parse(PLAN.replace("arg scalar a\n", "arg scalar a\n%s\n" % bad))
        assert rc == _lib.TCA_ERR_INVALID and msg in _lib.last_error(), (bad, _lib.last_error())
    rc, _ = parse(PLAN.replace("kernel k0", "when N 0 1 1 0\nkernel k0"))
    assert rc == _lib.TCA_ERR_INVALID and "before any kernel" in _lib.last_error()


@pytest.mark.parametrize("R,C,variants", [
    # rows of exactly 4 * 2^k vectors take the exact-fit kernel (c4e)
    (3, 0, ["c4"]), (3, 64, ["c4e"]), (3, 4096, ["c4e"]), (3, 4100, ["c4"]), (3, 16384, ["c4e"]), (3, 16380, ["c4"]),
    (300, 16388, ["s4"]), (3, 6, ["c2"]), (3, 2046, ["c2"]), (3, 8190, ["c2"]), (300, 8194, ["s2"]),
    (3, 1, ["c1"]), (3, 1023, ["c1"]), (3, 4095, ["c1"]), (300, 4097, ["s1"]),
    # few long rows: the split pair (partial folds, then the merge), in launch order
    (3, 16388, ["p4", "m4"]), (255, 8194, ["p2", "m2"]), (1, 4097, ["p1", "m1"]), (256, 16388, ["s4"])])
def test_stream_variant_selection(R, C, variants):
    """The guards of the streaming row family partition (rows, row length):
    one kernel per (vector width, cached | streamed), or for <= 255 long rows
    a split pair, and exactly that runs."""
    e = programs.CONFIG_PROGRAMS["row_sum_max_dyn"]().emit()
    rc, h = parse(e.plan)
    assert rc == 0, _lib.last_error()
    P = 0x1000
    arr = compiler._descriptors([TensorDesc(P, (R, C), 0), TensorDesc(P, (R,), 0), TensorDesc(P, (R,), 0)])
    syms = e.kernel_symbols()
    out = (ctypes.c_uint8 * len(syms))()
    grids = (ctypes.c_uint64 * len(syms))()
    assert _lib.lib().tca_program_selected(h, arr, 3, None, 0, out, grids, None, len(syms)) == 0, _lib.last_error()
    chosen = [s for s, f in zip(syms, out) if f]
    assert chosen == ["tca_row_sum_max_dyn_k0_" + v for v in variants]
    assert [g for g, f in zip(grids, out) if not f] == [0] * (len(syms) - len(variants))


@pytest.mark.parametrize("prog,dtype,R,C,variants", [
    # bf16 rows summed into f32: 8-element (16-byte) vectors, halved by the row length's residue
    ("row_sum_bf16_dyn", 2, 3, 1000, ["c8"]), ("row_sum_bf16_dyn", 2, 3, 32768, ["c8e"]),
    ("row_sum_bf16_dyn", 2, 300, 32776, ["s8"]), ("row_sum_bf16_dyn", 2, 3, 32776, ["p8", "m8"]),
    ("row_sum_bf16_dyn", 2, 3, 12, ["c4"]), ("row_sum_bf16_dyn", 2, 300, 16388, ["s4"]),
    ("row_sum_bf16_dyn", 2, 3, 6, ["c2"]), ("row_sum_bf16_dyn", 2, 3, 5, ["c1"]),
    # u8 rows: 16-element vectors
    ("row_sum_u8_dyn", 7, 3, 4096, ["c16e"]), ("row_sum_u8_dyn", 7, 300, 65552, ["s16"]),
    ("row_sum_u8_dyn", 7, 1, 65552, ["p16", "m16"]), ("row_sum_u8_dyn", 7, 3, 1000, ["c8"]),
    ("row_sum_u8_dyn", 7, 3, 20, ["c4"]), ("row_sum_u8_dyn", 7, 3, 6, ["c2"]), ("row_sum_u8_dyn", 7, 3, 0, ["c16"]),
    ("row_sum_u8_dyn", 7, 300, 4097, ["s1"])])
def test_narrow_stream_variant_selection(prog, dtype, R, C, variants):
    """Narrow element types: the widest width moves 16 bytes of the row's
    element type per load (8 bf16, 16 u8); the guards still partition the
    row lengths, one kernel (or one split pair) per launch."""
    e = programs.CONFIG_PROGRAMS[prog]().emit()
    rc, h = parse(e.plan)
    assert rc == 0, _lib.last_error()
    P = 0x1000
    nout = 2 if prog.startswith("row_sum_bf16") else 1
    arr = compiler._descriptors([TensorDesc(P if R * C else 0, (R, C), dtype)] +
                                [TensorDesc(P, (R,), 0)] * nout)
    syms = e.kernel_symbols()
    out = (ctypes.c_uint8 * len(syms))()
    assert _lib.lib().tca_program_selected(h, arr, 1 + nout, None, 0, out, None, None, len(syms)) == 0, \
        _lib.last_error()
    assert [s for s, f in zip(syms, out) if f] == ["tca_%s_k0_%s" % (prog, v) for v in variants]


@pytest.mark.parametrize("R,C,variant,part_grid,merge_grid", [
    (8192, 8192, 4, 64 * 16, 128),     # 64 column blocks (32 vectors each) x P = min(128, 1024 / 64) row chunks
    (65536, 1024, 4, 8 * 128, 16),     # P = min(1024, 128); the merge takes 64 outputs per block
    (1024, 65536, 4, 512 * 2, 1024),   # P = min(16, 2)
    (16, 4 << 20, 4, 32768, 0),        # the column blocks alone exceed 1024: P = 1, no merge
    (100, 3, 1, 2, 1),                 # odd columns: 1-element vectors; P = min(2, 1024)
    (64, 1022, 2, 16, 0),              # C % 4 == 2: 511 vectors, 16 column blocks; P = min(1, 64) = 1
    (0, 100, 4, 1, 0),                 # no rows: one chunk, init stored
    (100, 0, 4, 0, 0)])                # no columns: nothing runs
def test_col_split_geometry(R, C, variant, part_grid, merge_grid):
    """Column family: P row chunks per column block (>= 64 rows each, at most
    1024 blocks in all), the merge launched only when P > 1."""
    e = programs.CONFIG_PROGRAMS["col_sum_max_dyn"]().emit()
    assert set(e.families()) == {"col"}
    rc, h = parse(e.plan)
    assert rc == 0, _lib.last_error()
    P = 0x1000
    arr = compiler._descriptors([TensorDesc(P if R * C else 0, (R, C), 0), TensorDesc(P if C else 0, (C,), 0),
                                 TensorDesc(P if C else 0, (C,), 0)])
    syms = e.kernel_symbols()
    out = (ctypes.c_uint8 * len(syms))()
    grids = (ctypes.c_uint64 * len(syms))()
    assert _lib.lib().tca_program_selected(h, arr, 3, None, 0, out, grids, None, len(syms)) == 0, _lib.last_error()
    sel = {s: g for s, f, g in zip(syms, out, grids) if f}
    base = "tca_col_sum_max_dyn_k0_"
    assert sel == {base + "p%d" % variant: part_grid, base + "m%d" % variant: merge_grid}, sel


@pytest.mark.parametrize("fused", [True, False], ids=["one_read", "passes"])
@pytest.mark.parametrize("B,R,C,want,want_passes", [
    # 8 column blocks, P = min(16, 128) = 16 > 1: one fused partial + merge, or a pair per pass
    (1, 1000, 1000, {"p4": 8 * 16, "m4": 16}, {"p4_1": 8 * 16, "m4_1": 16, "p4_2": 8 * 16, "m4_2": 16}),
    # <= 64 rows: P = 1, one kernel (the fused partial finishing, or the whole-column kernel over both passes)
    (3, 64, 1000, {"p4": 3 * 8}, {"w4": 3 * 8}),
    (1, 0, 1000, {"p4": 8}, {"w4": 8}),
    # 1094 column blocks leave room for one chunk: P = 1 over 100 rows
    (1, 100, 140000, {"p4": 1094}, {"w4": 1094}),
    # odd columns: 1-element vectors, 3 column blocks, P = min(16, 170) = 16
    (2, 1000, 65, {"p1": 2 * 3 * 16, "m1": 3}, {"p1_1": 2 * 3 * 16, "m1_1": 3, "p1_2": 2 * 3 * 16, "m1_2": 3}),
    (1, 100, 0, {}, {})])
def test_col_passes_geometry(B, R, C, want, want_passes, fused):
    """A column nest of two passes (a variance reading its mean). Fused (the
    default): a partial keeping the sum and the centred sum of squares, read
    once, finishing itself with one row chunk (split mode 0) and followed by
    a merge with more (mode 1). With EMIT_NO_PASS_FUSION: with one row chunk
    the whole-column kernel (split mode 2) runs both passes, with more each
    pass is a partial (mode 3) and merge (mode 1) pair."""
    from tcacomp_amd.pkg import EMIT_NO_PASS_FUSION
    e = programs.CONFIG_PROGRAMS["col_mean_var_dyn"]().emit(flags=0 if fused else EMIT_NO_PASS_FUSION)
    assert set(e.families()) == {"col"}
    rc, h = parse(e.plan)
    assert rc == 0, _lib.last_error()
    P = 0x1000
    n = B * R * C
    arr = compiler._descriptors([TensorDesc(P if n else 0, (B, R, C), 0), TensorDesc(P if B * C else 0, (B, C), 0),
                                 TensorDesc(P if B * C else 0, (B, C), 0)])
    syms = e.kernel_symbols()
    out = (ctypes.c_uint8 * len(syms))()
    grids = (ctypes.c_uint64 * len(syms))()
    assert _lib.lib().tca_program_selected(h, arr, 3, None, 0, out, grids, None, len(syms)) == 0, _lib.last_error()
    sel = {s[len("tca_col_mean_var_dyn_k0_"):]: g for s, f, g in zip(syms, out, grids) if f and g}
    assert sel == (want if fused else want_passes), sel
    order = [s for s, f, g in zip(syms, out, grids) if f and g]
    assert order == sorted(order, key=syms.index)  # launch order: partials before their merges, pass 1 first


@pytest.mark.parametrize("B,C,want", [
    (1024, 96, ["g4"]), (5000, 6, ["g2"]), (1024, 7, ["g1"]),
    # fewer than 1024 segments: the two nests' own kernels (row sums into the local, then their max)
    (1023, 96, ["c4", "k1_c4"]), (3, 7, ["c1", "k1_c4"])])
def test_chain_segment_selection(B, C, want):
    """A chained reduction folds in one segment kernel from 1024 segments
    on (one block each); below that the inner and outer nests keep their
    own kernels, which spread a segment over many blocks."""
    e = programs.CONFIG_PROGRAMS["chain_sum_max"]().emit()
    assert "seg" in e.families()
    rc, h = parse(e.plan)
    assert rc == 0, _lib.last_error()
    R = 40
    arr = compiler._descriptors([TensorDesc(0x1000, (B, R, C), 0), TensorDesc(0x1000, (B,), 0)])
    syms = e.kernel_symbols()
    out = (ctypes.c_uint8 * len(syms))()
    grids = (ctypes.c_uint64 * len(syms))()
    assert _lib.lib().tca_program_selected(h, arr, 2, None, 0, out, grids, None, len(syms)) == 0, _lib.last_error()
    sel = [s[len("tca_chain_sum_max_k0_"):] if s.startswith("tca_chain_sum_max_k0_") else s[len("tca_chain_sum_max_"):]
           for s, f, g in zip(syms, out, grids) if f and g]
    assert sel == want, sel
    if want[0].startswith("g"):
        assert [g for s, f, g in zip(syms, out, grids) if f and g] == [B]


def test_chain_segment_static_drops_the_local():
    """With the segment count known at compile time (>= 1024), the segment
    kernel is the only one and the local between the reductions is not in
    the plan at all (no workspace)."""
    from tcacomp_amd.pkg import TF32, At, Call, NewBuilder
    b = NewBuilder("chain_static_seg")
    B, R, C = b.Dim("B", 2048), b.Dim("R", 0), b.Dim("C", 64)
    x = b.Tensor("x", TF32, B, R, C)
    o = b.Tensor("o", TF32, B)
    (b.Stmt().Iter(B, R, C).Map([At(x, B, R, C)], lambda v: v).As(B, R, C)
     .Reduce(b.Float32(0), lambda a, v: b.Add(a, v)).Reduce(b.Float32(0), lambda a, v: Call("fmaxf", a, v)).Store(o, B))
    e = b.Build().emit()
    assert e.families() == ["seg"], e.report
    assert "__chain" not in e.plan
    b2 = NewBuilder("chain_static_few")
    B, R, C = b2.Dim("B", 1000), b2.Dim("R", 0), b2.Dim("C", 64)
    x = b2.Tensor("x", TF32, B, R, C)
    o = b2.Tensor("o", TF32, B)
    (b2.Stmt().Iter(B, R, C).Map([At(x, B, R, C)], lambda v: v).As(B, R, C)
     .Reduce(b2.Float32(0), lambda a, v: b2.Add(a, v)).Reduce(b2.Float32(0), lambda a, v: Call("fmaxf", a, v))
     .Store(o, B))
    e2 = b2.Build().emit()
    assert "seg" not in e2.families() and "__chain" in e2.plan


@pytest.mark.parametrize("M,N,K,want", [
    (4096, 4096, 4096, ["_w"]),      # every tile whole, K % 64 == 0, K >= 256: the 64-deep-A kernel alone
    (4096, 4096, 4128, ["_v"]),      # K % 64 == 32: the 32-deep kernel alone
    (4096, 4096, 192, ["_v"]),       # K % 64 == 0 but K < 256
    (4096, 4096, 256, ["_w"]),
    (4100, 4096, 4096, ["_w", ""]),  # a partial bottom row of tiles: both, each skipping the other's tiles
    (4096, 4104, 4096, ["_w", ""]),
    (4100, 4096, 4128, ["_v", ""]),
    (4096, 4096, 4100, [""]),        # K % 32 != 0: no tile takes the direct-to-LDS path
    (4096, 4100, 4096, [""]),        # N % 8 != 0: [K][N] rows not 16-byte aligned, no direct-to-LDS tile
    (257, 4096, 4096, ["_w", ""]), (1025, 1025, 16, [""]),
    # output planes of at most 2^20 elements: the small-tile K-split kernel
    (255, 4096, 4096, ["_s"]), (512, 512, 0, ["_s"]), (512, 512, 16, ["_s"]), (64, 64, 4096, ["_s", "_sm"])])
def test_bf16_gemm_kernel_selection(M, N, K, want):
    """The bf16 contraction's three tile kernels: an 8-wave direct-to-LDS kernel
    runs when a whole tile can take it (A in 64-deep slices when K % 64 == 0
    and K >= 256, else in 32-deep slices), the register-staged one unless
    every tile does (plan `when` / `unless` guards); output planes of
    M*N <= 2^20 take the small-tile kernel instead (and its merge when K is
    split over workgroups)."""
    e = programs.CONFIG_PROGRAMS["gemm_bf16"]().emit()
    rc, h = parse(e.plan)
    assert rc == 0, _lib.last_error()
    arr = compiler._descriptors([TensorDesc(0x1000, (M, K), 2), TensorDesc(0x1000, (K, N), 2),
                                 TensorDesc(0x1000, (M, N), 0)])
    syms = e.kernel_symbols()
    out = (ctypes.c_uint8 * len(syms))()
    grids = (ctypes.c_uint64 * len(syms))()
    assert _lib.lib().tca_program_selected(h, arr, 3, None, 0, out, grids, None, len(syms)) == 0, _lib.last_error()
    sel = [s[len("tca_gemm_bf16_k0"):] for s, f, g in zip(syms, out, grids) if f and g]
    assert sel == want, (M, N, K, sel)


@pytest.mark.parametrize("M,N,K,want", [
    (4096, 4096, 4096, ["_w"]),      # whole tiles, K % 32 == 0, K >= 128: the 4-wave direct-to-LDS kernel
    (4096, 4096, 128, ["_w"]),
    (4352, 4608, 160, ["_w"]),
    (4096, 4096, 96, ["_v"]),        # K < 128: the 16-wave 256x256 kernel
    (4096, 4096, 4112, ["_v"]),      # K % 32 == 16
    (4100, 4096, 4096, ["_v"]),      # a partial row of tiles
    (4096, 4100, 4096, ["_v"]),
    (4095, 4096, 4096, [""]),        # below 4096: 128x128 tiles
    (1024, 8192, 4096, [""]), (1025, 1024, 64, [""]),
    (1024, 1024, 4096, ["_s"]), (512, 512, 0, ["_s"]), (32, 32, 4096, ["_s", "_sm"])])
def test_f32_gemm_kernel_selection(M, N, K, want):
    """The fp32 contraction's three kernels, exactly one launched: the 4-wave
    direct-to-LDS kernel when M, N >= 4096 and every tile is whole (M, N
    multiples of 256, K % 32 == 0, K >= 128), the 16-wave 256x256 kernel for
    the other shapes from M, N >= 4096 on, 128x128 tiles below."""
    e = programs.CONFIG_PROGRAMS["gemm_f32"]().emit()
    rc, h = parse(e.plan)
    assert rc == 0, _lib.last_error()
    arr = compiler._descriptors([TensorDesc(0x1000, (M, K), 0), TensorDesc(0x1000, (K, N), 0),
                                 TensorDesc(0x1000, (M, N), 0)])
    syms = e.kernel_symbols()
    out = (ctypes.c_uint8 * len(syms))()
    grids = (ctypes.c_uint64 * len(syms))()
    assert _lib.lib().tca_program_selected(h, arr, 3, None, 0, out, grids, None, len(syms)) == 0, _lib.last_error()
    sel = [s[len("tca_gemm_f32_k0"):] for s, f, g in zip(syms, out, grids) if f and g]
    assert sel == want, (M, N, K, sel)


def test_pow2_guard():
    """`when`/`unless` ... pow2: dim % mod == 0 and dim / mod a power of two
    (the streaming family's exact-fit kernels)."""
    plan = ("tca-plan 1\nprogram p\ndim C 0\ntensor x f32 in 1 C\n"
            "kernel ke 256 0 1 C/256\narg ptr x\nwhen C 0 4294967295 16 0 pow2\n"
            "kernel kg 256 0 1 C/256\narg ptr x\nunless C 0 4294967295 16 0 pow2\nend\n")
    rc, h = parse(plan)
    assert rc == 0, _lib.last_error()
    for C, want in ((0, "kg"), (16, "ke"), (32, "ke"), (48, "kg"), (64, "ke"), (16 << 20, "ke"), (17, "kg"),
                    (16 * 1023, "kg")):
        arr = compiler._descriptors([TensorDesc(0x1000 if C else 0, (C,), 0)])
        out = (ctypes.c_uint8 * 2)()
        assert _lib.lib().tca_program_selected(h, arr, 1, None, 0, out, None, None, 2) == 0, _lib.last_error()
        assert [k for k, f in zip(("ke", "kg"), out) if f] == [want], C
    _lib.lib().tca_program_unload(h)
    rc, _ = parse(plan.replace("16 0 pow2", "16 1 pow2", 1))
    assert rc == _lib.TCA_ERR_INVALID and "bad guard" in _lib.last_error()
    rc, _ = parse(plan.replace(" pow2\n", " pow3\n", 1))
    assert rc == _lib.TCA_ERR_INVALID and "[pow2]" in _lib.last_error()


def test_unless_guard_parse():
    for rec, ok in [("unless M 0 16 4 0", True), ("unless M 0 16 0 0", False), ("unless Q 0 16 4 0", False),
                    ("unless M 0 16", False)]:
        rc, _ = parse(PLAN.replace("arg scalar a\n", "arg scalar a\n%s\n" % rec))
        assert (rc == 0) == ok, (rec, _lib.last_error())
    # skipped only when every unless guard holds
    rc, h = parse(PLAN.replace("arg scalar a\n", "arg scalar a\nunless M 0 16 1 0\nunless N 0 8 4 0\n"))
    assert rc == 0, _lib.last_error()

    def selected(m, n):
        ts = [TensorDesc(0x1000, (m, n, 4), 0), TensorDesc(0x1000, (n,), 0), TensorDesc(0x1000, (m, n), 0)]
        arr = compiler._descriptors(ts)
        fd = (ctypes.c_uint32 * 1)(3)
        o = (ctypes.c_uint8 * 1)()
        assert _lib.lib().tca_program_selected(h, arr, 3, fd, 1, o, None, None, 1) == 0, _lib.last_error()
        return o[0]
    assert selected(5, 8) == 0  # both hold: skipped
    assert selected(5, 6) == 1  # N % 4 != 0
    assert selected(20, 8) == 1  # M > 16
    assert selected(20, 6) == 1


def test_split_record_parse():
    for rec, ok in [("split M 64 2048 0 1 N/256", True), ("split M 64 2048 1 2 1/1 N/4", True),
                    ("split Q 64 2048 0 1 N/256", False), ("split M 0 2048 0 1 N/256", False),
                    ("split M 64 0 0 1 N/256", False), ("split M 64 2048 2 1 N/256", True),
                    ("split M 64 2048 3 1 N/256", True), ("split M 64 2048 4 1 N/256", False),
                    ("split M 64 2048 0 2 N/256", False), ("split M 64 2048 0 1 N/pack", False),
                    ("split M 64 2048 0 1 Q/4", False)]:
        rc, _ = parse(PLAN.replace("arg scalar a\n", "arg scalar a\n%s\n" % rec))
        assert (rc == 0) == ok, (rec, _lib.last_error())


@pytest.mark.parametrize("M,P", [(1, 1), (64, 1), (65, 2), (10**6, 512)])
def test_split_modes_grid(M, P):
    """The grid each split mode gives. The test plan's kernel grid is
    ceil(M * N / 1024) * F = 3M at N = 1024, F = 3; its split has N/256 = 4
    column blocks, so P = min(ceil(M / 64), 2048 / 4). Mode 0 multiplies the
    grid by P, mode 1 launches only when P > 1, mode 2 only when P == 1,
    mode 3 multiplies by P but only when P > 1."""
    base = 3 * M
    want = {0: base * P, 1: base if P > 1 else 0, 2: base if P == 1 else 0, 3: base * P if P > 1 else 0}
    for mode, grid in want.items():
        rc, h = parse(PLAN.replace("arg scalar a\n", "arg scalar a\nsplit M 64 2048 %d 1 N/256\n" % mode))
        assert rc == 0, _lib.last_error()
        ts = [TensorDesc(0x1000, (M, 1024, 4), 0), TensorDesc(0x1000, (1024,), 0), TensorDesc(0x1000, (M, 1024), 0)]
        arr = compiler._descriptors(ts)
        fd = (ctypes.c_uint32 * 1)(3)
        sel = (ctypes.c_uint8 * 1)()
        grids = (ctypes.c_uint64 * 1)()
        assert _lib.lib().tca_program_selected(h, arr, 3, fd, 1, sel, grids, None, 1) == 0, _lib.last_error()
        assert sel[0] == 1 and grids[0] == grid, (M, mode, grids[0], grid)


@pytest.mark.parametrize("R,C,part_grid,merge_grid", [(1, 16388, 2, 1), (3, 10**6, 3 * 62, 1),
                                                      (255, 8 * 10**6, 255 * 489, 64), (1, 4 * 10**8, 512, 1)])
def test_split_geometry(R, C, part_grid, merge_grid):
    """Split rows: P = min(512, ceil(C / (4096 V))) chunks per row, one
    1024-lane block per chunk; the merge takes one wave per row, 4 per block."""
    e = programs.CONFIG_PROGRAMS["row_sum_max_dyn"]().emit()
    _, h = parse(e.plan)
    P = 0x1000
    arr = compiler._descriptors([TensorDesc(P, (R, C), 0), TensorDesc(P, (R,), 0), TensorDesc(P, (R,), 0)])
    syms = e.kernel_symbols()
    out = (ctypes.c_uint8 * len(syms))()
    grids = (ctypes.c_uint64 * len(syms))()
    blocks = (ctypes.c_uint32 * len(syms))()
    assert _lib.lib().tca_program_selected(h, arr, 3, None, 0, out, grids, blocks, len(syms)) == 0, _lib.last_error()
    sel = [(s, g, b) for s, f, g, b in zip(syms, out, grids, blocks) if f]
    assert [g for _, g, _ in sel] == [part_grid, merge_grid] and [b for _, _, b in sel] == [1024, 256], sel


@pytest.mark.parametrize("R,C,grid,block", [
    (1000, 0, 4, 256),         # 1 lane per row, 256 rows per 256-lane block
    (1000, 16, 4, 256),        # 4 vectors: still 1 lane
    (1000, 68, 32, 256),       # 17 vectors: 8 lanes, 32 rows per block
    (1000, 1024, 250, 256),    # 256 vectors: 64 lanes, 4 rows per block
    (1000, 4096, 1000, 256),   # 1024 vectors: 256 lanes, one row per block
    (1000, 4100, 1000, 512),   # 1025 vectors: 512 lanes, the block grows to the row
    (1000, 16384, 1000, 1024),  # 4096 vectors: 1024 lanes
    (1000, 80000, 1000, 1024),  # streamed: 1024 lanes
    (5, 3, 1, 256),            # odd length: 1-element vectors, 1 lane
    (1000, 2047, 1000, 512),   # 2047 one-element vectors: 512 lanes
    (0, 64, 0, 256)])          # no rows: no launch
def test_pack_record(R, C, grid, block):
    """pack <C> <epl> <min block>: S lanes per row as the kernel chooses them
    (smallest power of two with S * epl >= C, at most the kernel's block),
    max(min block, S) lanes per block, one block per group of rows."""
    e = programs.CONFIG_PROGRAMS["row_sum_max_dyn"]().emit()
    _, h = parse(e.plan)
    P = 0x1000
    arr = compiler._descriptors([TensorDesc(P if R * C else 0, (R, C), 0), TensorDesc(P if R else 0, (R,), 0),
                                 TensorDesc(P if R else 0, (R,), 0)])
    syms = e.kernel_symbols()
    out = (ctypes.c_uint8 * len(syms))()
    grids = (ctypes.c_uint64 * len(syms))()
    blocks = (ctypes.c_uint32 * len(syms))()
    assert _lib.lib().tca_program_selected(h, arr, 3, None, 0, out, grids, blocks, len(syms)) == 0, _lib.last_error()
    assert (sum(grids), sum(blocks)) == (grid, block), (list(grids), list(blocks))


def test_pack_record_parse():
    for rec, term, ok in [("pack N 16 256", "M/pack", True), ("pack N 16 256", "M/pack:9", True),
                          ("", "M/pack", False), ("pack Q 16 256", "M/pack", False),
                          ("pack N 0 256", "M/pack", False), ("pack N 16 96", "M/pack", False),
                          ("pack N 16 512", "M/pack", False), ("pack N 16", "M/pack", False)]:
        text = PLAN.replace("M*N/1024", term).replace("arg scalar a\n", "arg scalar a\n%s\n" % rec if rec else
                                                        "arg scalar a\n")
        rc, _ = parse(text)
        assert (rc == 0) == ok, (rec, term, _lib.last_error())


PLAN = """tca-plan 1
program p
dim M 0
dim N 0
dim e4 4
dim F 0
tensor x f32 in 3 M N e4
tensor w f32 in 1 N
tensor y f32 out 2 M N
tensor tmp f32 local 1 M
scalar a f32
kernel k0 256 0 2 M*N/1024 F/1
arg ptr x
arg ptr y
arg dim M
arg scalar a
end
"""


def parse(text):
    h = ctypes.c_void_p()
    rc = _lib.lib().tca_program_parse(text.encode(), ctypes.byref(h))
    return rc, h


def test_plan_parse_and_signature():
    rc, h = parse(PLAN)
    assert rc == 0, _lib.last_error()
    n = [ctypes.c_uint32() for _ in range(4)]
    assert _lib.lib().tca_program_signature(h, *[ctypes.byref(x) for x in n]) == 0
    assert [x.value for x in n] == [3, 1, 1, 1]  # x, w, y; free dim F; scalar a; one kernel
    assert _lib.lib().tca_program_kernel_name(h, 0) == b"k0"
    assert _lib.lib().tca_program_kernel_name(h, 1) is None
    _lib.lib().tca_program_unload(h)


@pytest.mark.parametrize("bad,msg", [
    ("", "empty plan"),
    ("tca-plan 2\nend\n", "tca-plan 1"),
    (PLAN.replace("end\n", ""), "missing 'end'"),
    (PLAN.replace("tensor w f32 in 1 N", "tensor w f99 in 1 N"), "unknown dtype"),
    (PLAN.replace("M*N/1024", "M*Q/1024"), "unknown dim"),
    (PLAN.replace("M*N/1024", "M*N/0"), "bad divisor"),
    (PLAN.replace("arg dim M", "arg dim Z"), "unknown"),
    (PLAN.replace("dim N 0", "dim M 0"), "duplicate dim"),
])
def test_plan_parse_errors(bad, msg):
    rc, h = parse(bad)
    assert rc == _lib.TCA_ERR_INVALID
    assert msg in _lib.last_error()


def _check(h, tensors, free=()):
    arr = compiler._descriptors(tensors)
    fd = (ctypes.c_uint32 * max(1, len(free)))(*free)
    rc = _lib.lib().tca_program_check(h, arr, len(tensors), fd, len(free))
    return rc, _lib.last_error()


def test_shape_contract():
    _, h = parse(PLAN)
    P = 0x1000  # never dereferenced by the host-only check
    ok = [TensorDesc(P, (5, 7, 4), 0), TensorDesc(P, (7,), 0), TensorDesc(P, (5, 7), 0)]
    assert _check(h, ok, (3,)) == (0, _check(h, ok, (3,))[1])
    rc, msg = _check(h, ok[:2], (3,))
    assert rc == _lib.TCA_ERR_INVALID and "takes 3 tensor" in msg
    rc, msg = _check(h, ok, ())
    assert rc == _lib.TCA_ERR_INVALID and "free dim" in msg
    rc, msg = _check(h, [TensorDesc(P, (5, 7, 4), 0), TensorDesc(P, (8,), 0), TensorDesc(P, (5, 7), 0)], (3,))
    assert rc == _lib.TCA_ERR_SHAPE and "w.Dim(0)" in msg and "N = 7" in msg
    rc, msg = _check(h, [TensorDesc(P, (5, 7, 3), 0), ok[1], ok[2]], (3,))
    assert rc == _lib.TCA_ERR_SHAPE and "const extent" in msg
    rc, msg = _check(h, [TensorDesc(P, (5, 7), 0), ok[1], ok[2]], (3,))
    assert rc == _lib.TCA_ERR_SHAPE and "rank" in msg
    rc, msg = _check(h, [ok[0], TensorDesc(P, (7,), 2), ok[2]], (3,))
    assert rc == _lib.TCA_ERR_SHAPE and "dtype" in msg
    rc, msg = _check(h, [TensorDesc(0, (5, 7, 4), 0), ok[1], ok[2]], (3,))
    assert rc == _lib.TCA_ERR_INVALID and "null" in msg
    rc, msg = _check(h, [TensorDesc(P + 4, (5, 7, 4), 0), ok[1], ok[2]], (3,))
    assert rc == _lib.TCA_ERR_INVALID and "aligned" in msg
    # empty tensors may carry a null pointer
    assert _check(h, [TensorDesc(0, (0, 7, 4), 0), ok[1], TensorDesc(0, (0, 7), 0)], (3,))[0] == 0
    # the u32 element-index domain (design/rt.md:392-399)
    rc, msg = _check(h, [TensorDesc(P, (70000, 70000, 4), 0), TensorDesc(P, (70000,), 0),
                         TensorDesc(P, (70000, 70000), 0)], (3,))
    assert rc == _lib.TCA_ERR_SHAPE and "2^32" in msg
    _lib.lib().tca_program_unload(h)


def test_program_launch_without_module_is_refused():
    _, h = parse(PLAN)
    arr = compiler._descriptors([TensorDesc(0x1000, (5, 7, 4), 0), TensorDesc(0x1000, (7,), 0),
                                 TensorDesc(0x1000, (5, 7), 0)])
    fd = (ctypes.c_uint32 * 1)(3)
    sc = (ctypes.c_double * 1)(1.0)
    rc = _lib.lib().tca_program_launch(h, arr, 3, fd, 1, sc, 1, None)
    assert rc == _lib.TCA_ERR_INVALID and "parsed, not loaded" in _lib.last_error()
    _lib.lib().tca_program_unload(h)


EXPECTED_FAMILIES = {
    # contractions: the small-tile kernel and its merge, then three tile kernels
    "scale_relu": ["elementwise"], "scale_relu_map": ["elementwise"], "row_sum_max_8192": ["row"], "gemm_bf16_nt": ["gemm"] * 5,
    "softmax_4096": ["row"], "layernorm_1024": ["row"], "gemm_f32": ["gemm"] * 5, "gemm_bf16": ["gemm"] * 5,
    # softmax's max and exp-sum passes share one partial when split (online normaliser), and the row
    # map computes their merge itself
    "copy_f32": ["elementwise"], "row_sum_max_dyn": ["stream"] * 13, "softmax_dyn": ["stream"] * 16,
    "layernorm_dyn": ["stream"] * 19, "layernorm_rstd_1024": ["row"], "layernorm_rstd_dyn": ["stream"] * 10,
    # narrow rows: one more width per halving of the element size (8 bf16, 16 u8 elements per vector)
    "row_sum_bf16_dyn": ["stream"] * 17, "row_sum_u8_dyn": ["stream"] * 21, "row_stats_u32_dyn": ["stream"] * 13,
    # column reductions: a (partial, merge) pair per vector width
    "col_sum_max_dyn": ["col"] * 6, "col_mean_bf16": ["col"] * 8, "col_sum_u8": ["col"] * 10,
    # chained reductions split into an inner reduce into a local and an outer reduce of it; with a
    # segment dim (B) the pair also has a segment kernel per vector width, chosen from 1024 segments on
    "chain_sum_max": ["seg"] * 3 + ["stream"] * 20, "chain_total": ["stream"] * 23,
    "chain3_max_total": ["seg"] * 3 + ["stream"] * 30,
}


def test_prefix_chain_fuses_into_the_row_kernel():
    """A per-row chain (iterating only the row axis) fuses with the row nest
    around it; its value stays in registers when it is a local and is stored
    once per row when it is an output."""
    e = programs.CONFIG_PROGRAMS["layernorm_rstd_1024"]().emit()
    assert e.families() == ["row"]
    assert "per-row map into rstd" in e.source
    assert "tensor rstd f32 out 1 R" in e.plan and "local" not in e.plan


@pytest.mark.parametrize("name", sorted(EXPECTED_FAMILIES))
def test_config_classification(name):
    e = programs.CONFIG_PROGRAMS[name]().emit()
    assert e.families() == EXPECTED_FAMILIES[name], e.report


def test_split_chain_keeps_the_combiner_rules():
    """A chained reduction is split into one chain per reduce, and each is
    classified on its own: the inner sum streams, while an outer fold that
    is not associative-commutative (acc / 2 + now) keeps the generic
    family's sequential order."""
    fams = programs.CONFIG_PROGRAMS["chain_halving"]().emit().families()
    assert fams[-1] == "generic" and set(fams[:-1]) == {"stream"}, fams


def test_fusion_disabled_lowers_every_chain_generically():
    e = programs.CONFIG_PROGRAMS["softmax_4096"]().emit(flags=EMIT_NO_FUSION | EMIT_NO_GEMM)
    assert e.families() == ["generic"] * 3
    assert "tensor mx f32 local 1 R" in e.plan  # locals move to the HBM workspace


def test_fused_locals_stay_in_registers():
    e = programs.CONFIG_PROGRAMS["layernorm_1024"]().emit()
    assert "local" not in e.plan  # mean/var never touch HBM
    assert e.source.count("__syncthreads") == 0  # one wave per row: no cross-wave exchange


def test_nonfinite_literals_are_valid_hip():
    # The reference formats -inf as the invalid token "-Inff" (internal/cg/cxx/naming.go:103-109).
    src = programs.CONFIG_PROGRAMS["row_sum_max_8192"]().emit().source
    assert "(-(__builtin_inff()))" in src and "Inff" not in src


def test_device_flags():
    e = programs.CONFIG_PROGRAMS["scale_relu"]().emit()
    assert "-ffp-contract=off" in e.hipcc and "--offload-arch=gfx950" in e.hipcc
    assert "-packed-fp32-ops" in e.hipcc and "-fno-gpu-flush-denormals-to-zero" in e.hipcc


def test_target_other_than_gfx950_is_refused():
    from tcacomp_amd.pkg import BuildError
    with pytest.raises(BuildError, match="unsupported target"):
        programs.CONFIG_PROGRAMS["scale_relu"]().emit(target="sm_86")


def test_every_registered_program_is_prebuilt():
    """build() must have produced every code object the GPU tests and the
    bench launch (a GPU box never compiles)."""
    missing = []
    for name, factory, flags in programs.all_builds():
        e = factory().emit(flags=flags)
        key = compiler.cache_key(e.source, e.hipcc)
        p = os.path.join(compiler.KCACHE, "%s-%s.hsaco" % (factory().name, key))
        if not os.path.exists(p):
            missing.append(name)
    assert not missing, "not prebuilt (run __graft_entry__.build()): %s" % missing


def test_cache_key_follows_included_headers(tmp_path, monkeypatch):
    """A code object's key covers the headers its source includes, followed
    transitively, and no others: editing the contraction header leaves the
    keys of row kernels (whose traffic figures are profiled per key) alone,
    and editing a header a kernel includes changes its key."""
    row = programs.CONFIG_PROGRAMS["row_sum_max_8192"]().emit()
    gemm = programs.CONFIG_PROGRAMS["gemm_bf16"]().emit()
    assert '#include "tca/hip/gemm.h"' in gemm.source and "gemm.h" not in row.source
    inc = tmp_path / "include"
    import shutil
    shutil.copytree(compiler.INCLUDE_DIR, inc)
    monkeypatch.setattr(compiler, "INCLUDE_DIR", str(inc))
    k_row, k_gemm = compiler.cache_key(row.source, row.hipcc), compiler.cache_key(gemm.source, gemm.hipcc)
    with open(inc / "tca" / "hip" / "gemm.h", "a") as f:
        f.write("// edited\n")
    assert compiler.cache_key(row.source, row.hipcc) == k_row
    assert compiler.cache_key(gemm.source, gemm.hipcc) != k_gemm
    with open(inc / "tca" / "hip" / "device.h", "a") as f:
        f.write("// edited\n")
    assert compiler.cache_key(row.source, row.hipcc) != k_row


def test_every_registered_plan_parses():
    """The runtime's plan parser (the one tca_program_load runs) accepts the
    plan of every program the tests and the bench launch: no duplicate or
    unknown dims, well-formed guards and split records; checked on the CPU
    so a malformed plan never reaches a GPU run."""
    bad = []
    for name, factory, flags in programs.all_builds():
        rc, h = parse(factory().emit(flags=flags).plan)
        if rc != 0:
            bad.append("%s: %s" % (name, _lib.last_error()))
        else:
            _lib.lib().tca_program_unload(h)
    assert not bad, bad


def test_build_sources_listed():
    for s in build.SOURCES:
        assert os.path.exists(os.path.join(build.CSRC, s))


def test_runtime_null_arguments_are_refused_before_hip():
    """Host-side validation of the memory and launch entry points: a null
    pointer with a non-zero size is TCA_ERR_INVALID with a message, no HIP
    call is made (so this runs without a GPU)."""
    L = _lib.lib()
    assert L.tca_rt_memcpy_h2d(None, None, 16) == _lib.TCA_ERR_INVALID and "null" in _lib.last_error()
    assert L.tca_rt_memcpy_d2h(None, None, 16) == _lib.TCA_ERR_INVALID
    assert L.tca_rt_memset(None, 0, 16) == _lib.TCA_ERR_INVALID
    assert L.tca_rt_memcpy_h2d(None, None, 0) == 0  # nothing to copy
    assert L.tca_rt_free(None) == 0
    assert L.tca_rt_launch(None, b"k", 1, 64, 0, None, 0, None) == _lib.TCA_ERR_INVALID


def _gemm_asm(name, tmp_path):
    """The program's emitted source compiled to gfx950 assembly (host-only)."""
    import subprocess
    e = programs.CONFIG_PROGRAMS[name]().emit()
    src = tmp_path / "k.hip"
    src.write_text(e.source)
    asm = tmp_path / "k.s"
    flags = [f for f in e.hipcc if f != "--genco"]  # assembly, not a code object
    r = subprocess.run([os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")] + flags +
                       ["--cuda-device-only", "-S", "-o", str(asm), "-I", os.path.join(REPO, "tcacomp_amd", "csrc", "include"),
                        str(src)], capture_output=True, text=True)
    if r.returncode != 0 and "No such file" in (r.stderr or ""):
        pytest.skip("hipcc not available")
    assert r.returncode == 0, r.stderr[-2000:]
    return asm.read_text().split("\n")


@pytest.mark.parametrize("name", ["gemm_bf16", "gemm_bf16_nt", "gemm_f16", "gemm_f16_nt", "gemm_f32", "gemm_f32_nt"])
def test_dma_gemm_reloads_nothing_from_scratch(name, tmp_path):
    """The contractions' direct-to-LDS main loops wait on hand-counted vmcnt
    values for their loads; a register spill reloaded from scratch while
    they are in flight would share that counter (an fp32 port that spilled
    computed wrong results). From the first direct-to-LDS load to the end of
    that path (its s_endpgm) nothing may be reloaded from scratch; the
    register-staged edge path after it may. Host-only: compiles to gfx950
    assembly."""
    lines = _gemm_asm(name, tmp_path)
    dma = [i for i, l in enumerate(lines) if "global_load_lds_dwordx4" in l]
    assert dma
    end = next(i for i in range(dma[-1], len(lines)) if "s_endpgm" in lines[i])
    reloads = [lines[i].strip() for i in range(dma[0], end) if "scratch_load" in lines[i]]
    assert not reloads, reloads[:4]


def _regs(op):
    """VGPR or AGPR numbers named by one assembly operand (v5, v[4:7], a[0:3])."""
    m = re.fullmatch(r"([va])(?:(\d+)|\[(\d+):(\d+)\])", op.strip())
    if not m:
        return m, set()
    lo = int(m.group(2) if m.group(2) is not None else m.group(3))
    hi = int(m.group(2) if m.group(2) is not None else m.group(4))
    return m.group(1), set(range(lo, hi + 1))


def _vgpr_writes(line):
    """VGPRs an instruction writes: its first operand when that is a VGPR,
    for every instruction that has a destination (not stores, LDS writes,
    direct-to-LDS loads or scalar instructions)."""
    parts = line.strip().split(None, 1)
    if len(parts) < 2 or parts[0].startswith(("s_", ";", ".")):
        return set()
    mn = parts[0]
    if "store" in mn or mn.startswith(("ds_write", "ds_store")) or "load_lds" in mn:
        return set()
    kind, regs = _regs(parts[1].split(",")[0])
    return regs if kind == "v" else set()


@pytest.mark.parametrize("name", ["gemm_bf16", "gemm_bf16_nt", "gemm_f16", "gemm_f16_nt", "gemm_f32", "gemm_f32_nt"])
def test_asm_mfma_kernel_hazards_covered(name, tmp_path):
    """The 4-wave contractions issue their MFMAs as inline asm, which the
    compiler's hazard recogniser does not model. Checked on its gfx950
    assembly: every MFMA accumulates in place in AGPRs (dst == SrcC); every
    MFMA A/B operand register reaches the MFMA from a ds_read only (along
    the straight line and around the main loop's back edge), never from a
    VALU write; the AGPR zero-init is followed by two s_nop 7 before the
    first MFMA; three s_nop 7 separate the last MFMA from the first
    instruction that reads an AGPR outside an MFMA (an 8-pass bf16 MFMA
    needs 11 wait states there, a 16-pass fp32 one 19)."""
    lines = _gemm_asm(name, tmp_path)
    sym = "tca_%s_k0_w:" % name
    start = next(i for i, l in enumerate(lines) if l.startswith(sym))
    end = next(i for i in range(start, len(lines)) if lines[i].startswith(".Lfunc_end"))
    body = lines[start:end]
    mf = [i for i, l in enumerate(body) if l.strip().startswith("v_mfma")]
    assert len(mf) > 64
    heads = [i for i, l in enumerate(body) if "Loop Header" in l]
    assert len(heads) == 1, heads
    head = heads[0]
    label = body[head].split(":")[0]
    tail = max(i for i, l in enumerate(body) if l.strip().startswith("s_cbranch") and l.strip().endswith(label))

    def writers(idx, reg):
        """Instructions whose write of reg can reach body[idx]."""
        found, i, wrapped = [], idx - 1, False
        while i >= 0:
            if i == head and head < idx <= tail and not wrapped:
                # around the back edge first, then on into the preheader
                for j in range(tail, idx, -1):
                    if reg in _vgpr_writes(body[j]):
                        found.append(j)
                        break
                wrapped = True
            if reg in _vgpr_writes(body[i]):
                found.append(i)
                return found
            i -= 1
        return found

    bad = []
    for i in mf:
        ops = [o.strip() for o in body[i].strip().split(None, 1)[1].split(",")]
        assert ops[0] == ops[3] and ops[0].startswith("a["), body[i]
        for op in ops[1:3]:
            kind, regs = _regs(op)
            assert kind == "v", body[i]
            for r in regs:
                for w in writers(i, r):
                    if not body[w].strip().startswith("ds_read"):
                        bad.append((body[i].strip(), body[w].strip()))
    assert not bad, bad[:4]
    nop7 = [i for i, l in enumerate(body) if l.strip() == "s_nop 7"]
    inits = [i for i, l in enumerate(body) if l.strip().startswith("v_accvgpr_write")]
    assert inits and max(inits) < mf[0]
    assert len([i for i in nop7 if max(inits) < i < mf[0]]) >= 2
    readers = [i for i, l in enumerate(body) if i > mf[-1] and re.search(r"\ba\[?\d", l)
               and not l.strip().startswith(("v_mfma", ";"))]
    assert readers
    assert len([i for i in nop7 if mf[-1] < i < readers[0]]) >= 3
    assert not [l for l in body if re.search(r"\ba\[?\d", l) and l.strip().startswith("v_accvgpr_read")
                and mf[0] < body.index(l) < mf[-1]]


@pytest.fixture(scope="module")
def device_helpers(tmp_path_factory):
    """tests/c/device_edge.hip built for the host: the __host__ __device__
    chunk helpers of tca/hip/device.h, the very code the kernels run."""
    import subprocess
    out = tmp_path_factory.mktemp("edge") / "device_edge"
    hipcc = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    r = subprocess.run([hipcc, "--offload-arch=gfx950", "-O1", "-I", os.path.join(REPO, "tcacomp_amd", "csrc", "include"),
                        os.path.join(REPO, "tests", "c", "device_edge.hip"), "-o", str(out)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]

    def run(lines):
        p = subprocess.run([str(out)], input="\n".join(lines) + "\n", capture_output=True, text=True, timeout=60)
        assert p.returncode == 0, p.stderr
        return [int(v) for v in p.stdout.split()]
    return run


U32 = 2 ** 32 - 1


def test_device_ceil_div_at_the_u32_edge(device_helpers):
    cases = [(0, 1), (0, 4096), (1, 4096), (4096, 4096), (4097, 4096), (U32, 1), (U32, 64), (U32, 4096),
             (U32 - 63, 64), (U32 - 4095, 4096), (U32, 512), (2 ** 31, 3), (U32, U32)]
    got = device_helpers(["ceil_div %d %d" % c for c in cases])
    assert got == [-(-a // b) for a, b in cases]


def _constants(source, names):
    vals = {}
    for n in names:
        m = re.search(r"\b%s = (\d+)u" % n, source)
        assert m, n
        vals[n] = int(m.group(1))
    return vals


# The most elements a tensor may hold (the u32 domain less the kernels'
# index headroom); larger tensors are refused (test_element_limit_keeps_index_headroom).
TOP = 2 ** 32 - 2 ** 16 - 1


@pytest.mark.parametrize("R,C", [(TOP, 1), (2 ** 31, 1), (TOP // 4, 4), (TOP // 3, 3), (TOP // 64, 64),
                                 (64 * 1024 + 1, 2), (1, TOP)])
def test_column_split_device_matches_plan_at_the_u32_edge(device_helpers, R, C):
    """Column family: the partial kernel's grid is column blocks x P with P
    from the plan's 64-bit split record; each block recomputes P with the
    device's col_split. They must agree for every R x C the plan accepts (with a
    32-bit round-up that wraps, blocks with p >= 1 took the one-chunk store
    path and the merge read partials nobody wrote)."""
    p = compiler.CompiledProgram("col_sum_max_dyn", programs.CONFIG_PROGRAMS["col_sum_max_dyn"]().emit(), "")
    k = _constants(p.source, ["RMIN", "BLOCKS", "SPAN"])
    ts = [TensorDesc(0x1000, (R, C), 0), TensorDesc(0x1000, (C,), 0), TensorDesc(0x1000, (C,), 0)]
    syms = p.kernel_symbols()
    arr = compiler._descriptors(ts)
    sel = (ctypes.c_uint8 * len(syms))()
    grids = (ctypes.c_uint64 * len(syms))()
    blocks = (ctypes.c_uint32 * len(syms))()
    assert _lib.lib().tca_program_selected(p.parsed(), arr, 3, None, 0, sel, grids, blocks, len(syms)) == 0, \
        _lib.last_error()
    part = [i for i, s in enumerate(syms) if sel[i] and re.search(r"_p\d+$", s)]
    assert len(part) == 1, [s for i, s in enumerate(syms) if sel[i]]
    v = int(syms[part[0]].rsplit("_p", 1)[1])
    cb, = device_helpers(["ceil_div %d %d" % (C // v, k["SPAN"])])
    P, = device_helpers(["col_split %d %d %d %d" % (R, cb, k["RMIN"], k["BLOCKS"])])
    assert grids[part[0]] == cb * P, (syms[part[0]], grids[part[0]], cb, P)
    merge = [i for i, s in enumerate(syms) if sel[i] and re.search(r"_m\d+$", s)]
    assert (grids[merge[0]] > 0) == (P > 1)


@pytest.mark.parametrize("R,C", [(1, TOP), (1, TOP - 1), (3, TOP // 3 - 2), (255, TOP // 255 - 4), (1, 16388)])
def test_split_rows_device_matches_plan_at_the_u32_edge(device_helpers, R, C):
    """Split rows: the grid is rows x P from the plan (64-bit, capped at
    PMAX); the device recomputes P = min(PMAX, ceil_div(VECS, CV)) and the
    chunk length L = ceil_div(VECS, P). They must agree, and chunks
    [p*L, p*L + min(L, VECS - p*L)) must tile [0, VECS) exactly."""
    prog = programs.CONFIG_PROGRAMS["row_sum_max_dyn"]()
    p = compiler.CompiledProgram("row_sum_max_dyn", prog.emit(), "")
    src = p.source
    assert "min(PMAX, tca::hip::ceil_div(VECS, CV))" in src and "tca::hip::ceil_div(VECS, P)" in src
    assert "hi = lo + min(L, VECS - lo)" in src
    k = _constants(src, ["CV", "PMAX"])
    ts = [TensorDesc(0x1000, (R, C), 0), TensorDesc(0x1000, (R,), 0), TensorDesc(0x1000, (R,), 0)]
    syms = p.kernel_symbols()
    arr = compiler._descriptors(ts)
    sel = (ctypes.c_uint8 * len(syms))()
    grids = (ctypes.c_uint64 * len(syms))()
    assert _lib.lib().tca_program_selected(p.parsed(), arr, 3, None, 0, sel, grids, None, len(syms)) == 0, \
        _lib.last_error()
    part = [i for i, s in enumerate(syms) if sel[i] and re.search(r"_p\d+$", s)]
    assert len(part) == 1, [s for i, s in enumerate(syms) if sel[i]]
    v = int(syms[part[0]].rsplit("_p", 1)[1])
    vecs = C // v
    cdiv, = device_helpers(["ceil_div %d %d" % (vecs, k["CV"])])
    P = min(k["PMAX"], cdiv)
    assert grids[part[0]] == R * P
    L, = device_helpers(["ceil_div %d %d" % (vecs, P)])
    covered = 0
    for q in range(P):
        lo = q * L
        assert lo < vecs
        hi = lo + min(L, vecs - lo)
        assert hi <= U32 and lo == covered and hi - lo > 1024
        covered = hi
    assert covered == vecs


def _bias_program(transposed=True):
    """y[r][c] = x[r][c] * g[c] + b[r] (+ z[c][r], read transposed)."""
    from tcacomp_amd.pkg import TF32, At, NewBuilder
    bld = NewBuilder("ew_bcast" if transposed else "ew_bias")
    R, C = bld.Dim("R", 0), bld.Dim("C", 0)
    x = bld.Tensor("x", TF32, R, C)
    z = bld.Tensor("z", TF32, C, R) if transposed else None
    g, b = bld.Tensor("g", TF32, C), bld.Tensor("b", TF32, R)
    y = bld.Tensor("y", TF32, R, C)
    ops = [At(x, R, C), At(g, C), At(b, R)] + ([At(z, C, R)] if transposed else [])
    if transposed:
        body = lambda v, w, u, t: bld.Add(bld.Add(bld.Mul(v, w), u), t)  # noqa: E731
    else:
        body = lambda v, w, u: bld.Add(bld.Mul(v, w), u)  # noqa: E731
    bld.Stmt().Iter(R, C).Map(ops, body).As(R, C).Store(y, R, C)
    return bld.Build()


def test_elementwise_broadcast_operands_take_the_row_vector_path():
    # With the innermost extent a multiple of the vector width (tested at run
    # time), coordinates are decomposed once per vector: g[c] is one vector
    # load, b[r] one scalar load; x is aligned with the store and keeps its
    # streamed vector load.
    src = _bias_program(False).emit().source
    # tensors in declaration order: x t0, g t1, b t2, y t3
    assert "if (d1 % 4u == 0u) {" in src
    assert "const auto ra1 = tca::hip::load_vec<float, 4>(t1 + c1_v);" in src
    assert "const float ra2 = t2[c0_v];" in src
    assert "a0[u] = tca::hip::load_vec_nt<float, 4>(t0 + base + u * 1024u);" in src
    # An elementwise map whose operands all align with the store is unchanged.
    assert "% 4u == 0u" not in programs.CONFIG_PROGRAMS["scale_relu_map"]().emit().source


def test_elementwise_transposed_operand_takes_the_lds_tile_kernel():
    # z[c][r] under y[r][c]: with at most two transposed operands, 128x128
    # tiles for 1024 threads, z staged through LDS rows of 129 words, read
    # back transposed; the grid is (outer) x ceil(R/128) x ceil(C/128).
    e = _bias_program(True).emit()
    src = e.source
    # tensors in declaration order: x t0, z t1, g t2, b t3, y t4
    assert "__shared__ uint32_t tr_lds[1][16512];" in src
    assert "__launch_bounds__(1024)" in src
    assert "tca::hip::load_vec_nt<float, 4>(t1 + (l) * d0 + p)" in src
    assert "tr_lds[0][(4u * tc + q) * 129u + pr]" in src
    assert "tca::hip::store_vec_nt<float, 4>(t4 + (p) * d1 + lb, out);" in src
    assert "kernel tca_ew_bcast_k0 1024 0 3 1/1 R/128 C/128" in e.plan
    ptr = 0x1000
    for R, C, grid in ((1000, 1000, 8 * 8), (64, 4100, 1 * 33), (0, 5, 0), (5, 70001, 1 * 547), (128, 256, 2)):
        prog = compiler.CompiledProgram("ew_bcast", e, "")
        ts = [TensorDesc(ptr if R * C else 0, (R, C), 0), TensorDesc(ptr if R * C else 0, (C, R), 0),
              TensorDesc(ptr if C else 0, (C,), 0), TensorDesc(ptr if R else 0, (R,), 0),
              TensorDesc(ptr if R * C else 0, (R, C), 0)]
        arr = compiler._descriptors(ts)
        sel = (ctypes.c_uint8 * 1)()
        grids = (ctypes.c_uint64 * 1)()
        _lib.check(_lib.lib().tca_program_selected(prog.parsed(), arr, 5, None, 0, sel, grids, None, 1))
        assert grids[0] == grid, (R, C, grids[0])


def test_elementwise_three_transposed_operands_keep_64_tiles():
    # Three transposed operands would need 198 KiB of LDS at 128x128: 64x64
    # tiles for 256 threads (LDS rows of 65 words, 3 x 16.6 KiB).
    from tcacomp_amd.pkg import TF32, At, NewBuilder
    bld = NewBuilder("ew_tr3")
    R, C = bld.Dim("R", 0), bld.Dim("C", 0)
    zs = [bld.Tensor("z%d" % i, TF32, C, R) for i in range(3)]
    y = bld.Tensor("y", TF32, R, C)
    bld.Stmt().Iter(R, C).Map([At(z, C, R) for z in zs],
                              lambda a, b, c: bld.Add(bld.Add(a, b), c)).As(R, C).Store(y, R, C)
    e = bld.Build().emit()
    assert "__shared__ uint32_t tr_lds[3][4160];" in e.source and "__launch_bounds__(256)" in e.source
    assert "tr_lds[2][(4u * tc + q) * 65u + pr]" in e.source
    assert "kernel tca_ew_tr3_k0 256 0 3 1/1 R/64 C/64" in e.plan


@pytest.mark.parametrize("name,deep", [("softmax_dyn", True), ("layernorm_dyn", True), ("layernorm_rstd_dyn", True),
                                       ("row_stats_shift_dyn", True), ("softmax_bf16_dyn", True),
                                       ("softmax_affine_dyn", False), ("row_moments_affine_dyn", False)])
def test_stream_row_caches_fit_registers(name, deep, tmp_path):
    """Nests of several passes keep rows of up to 8192 vectors in registers
    (a variant with 8 vectors per lane of a 1024-lane block, taken above the
    4-vector cache's 4096): every kernel of the program compiles without
    scratch. A nest whose passes read a column vector in more than one pass
    (the affine programs: the vector's loads stay live across the passes)
    keeps the 4-deep cache only and streams longer rows. Host-only: compiles
    to gfx950 assembly."""
    lines = _gemm_asm(name, tmp_path)
    text = "\n".join(lines)
    names = re.findall(r"^\s+\.name:\s+(tca_\S+)", text, re.M)
    priv = [int(v) for v in re.findall(r"\.private_segment_fixed_size: (\d+)", text)]
    assert any(n.endswith("_c4x8") for n in names) == deep, names
    assert len(names) == len(priv)
    assert all(p == 0 for p in priv), [(n, p) for n, p in zip(names, priv) if p]
    plan = programs.CONFIG_PROGRAMS[name]().emit().plan
    if deep:  # f32 rows of 4 * 4096 < C <= 4 * 8192 take the 8-deep cache; longer rows stream
        assert "when C 16388 32768 4 0" in plan and "when C 32772 4294967295 4 0" in plan
    else:
        assert "when C 16388 4294967295 4 0" in plan


def test_single_pass_stream_nest_keeps_one_cache_depth():
    plan = programs.CONFIG_PROGRAMS["row_sum_max_dyn"]().emit().plan
    assert "_c4x8" not in plan and "when C 16388 4294967295 4 0" in plan


@pytest.mark.parametrize("R,C,variants", [
    # rows of <= 8192 vectors stay in registers whatever the row count
    (3, 32768, ["c4x8"]), (3, 16384, ["c4e"]),
    # longer rows: streamed from 256 rows on, split into passes below
    (256, 32772, ["s4"]), (255, 32772, ["p4_1", "w4_3"]),
    (1, 1 << 20, ["p4_1", "w4_3"]), (2, 16386, ["p2_1", "w2_3"]),
    (7, 8193, ["p1_1", "w1_3"]), (300, 8193, ["s1"]),
    # more rows split too when each holds >= 16384 vectors, up to 4095 rows
    (256, 65536, ["p4_1", "w4_3"]), (256, 65532, ["s4"]), (4095, 65536, ["p4_1", "w4_3"]),
    (4096, 65536, ["s4"]), (1000, 16385, ["p1_1", "w1_3"]), (1000, 16383, ["s1"]), (300, 32770, ["p2_1", "w2_3"])])
def test_multipass_split_selection(R, C, variants):
    """Few long rows of a nest of several passes (softmax: max, sum, map):
    each pass over its own grid of row chunks, in pass order; the max and
    the exp-sum share one read (pass 1's partial, the online normaliser), so
    pass 2 has no kernels, and the row map (pass 3) merges their partials
    itself, so no merge kernel runs either. Up to 4095 rows of at least
    16384 vectors split as well; shorter rows and more rows stream."""
    e = programs.CONFIG_PROGRAMS["softmax_dyn"]().emit()
    rc, h = parse(e.plan)
    assert rc == 0, _lib.last_error()
    arr = compiler._descriptors([TensorDesc(0x1000, (R, C), 0), TensorDesc(0x1000, (R, C), 0)])
    syms = e.kernel_symbols()
    out = (ctypes.c_uint8 * len(syms))()
    assert _lib.lib().tca_program_selected(h, arr, 2, None, 0, out, None, None, len(syms)) == 0, _lib.last_error()
    assert [s for s, f in zip(syms, out) if f] == ["tca_softmax_dyn_k0_" + v for v in variants]
    _lib.lib().tca_program_unload(h)


@pytest.mark.parametrize("name,pair", [("softmax_dyn", "tca::hip::online_expsum_add(om, os, ev);"),
                                       ("layernorm_dyn", "tca::hip::chan_add(cs, cm, cn, ev);"),
                                       ("softmax_affine_dyn", "tca::hip::online_expsum_add(om, os, ev);"),
                                       ("row_moments_affine_dyn", "tca::hip::chan_add(cs, cm, cn, ev);")])
def test_streamed_pair_shares_one_read(name, pair):
    """The streamed body (more rows than split, or rows too long for the
    register cache) folds the softmax's max and exp-sum, or layernorm's sum
    and centred sum of squares, in one read of the row; the register-cached
    bodies keep the two passes (both under one template, the branch on NV);
    without pass fusion the streamed body reads the row once per pass."""
    def rows_body(src):  # the row body: up to the next function template
        at = src.index("_rows(")
        return src[at:src.index("\ntemplate <", at)]

    body = rows_body(programs.CONFIG_PROGRAMS[name]().emit().source)
    assert "in one read of a streamed row" in body and "    if constexpr (NV > 0u) {" in body
    assert body.count(pair) == 3  # the lane's first vector, the unrolled loop, the tail
    body = rows_body(programs.CONFIG_PROGRAMS[name]().emit(flags=EMIT_NO_PASS_FUSION).source)
    assert "in one read of a streamed row" not in body and pair not in body


@pytest.mark.parametrize("flags,C,variants", [
    (0, 1 << 20, ["p4_1", "wl4_3"]), (0, 262140, ["p4_1", "w4_3"]), (0, 262142, ["p2_1", "wl2_3"]),
    (EMIT_NO_PASS_FUSION, 1 << 20, ["p4_1", "m4_1", "p4_2", "m4_2", "w4_3"])])
def test_split_layernorm_selection(flags, C, variants):
    """Layernorm's mean and centred sum of squares share one read of each
    chunk (pass 1's partial holds each chunk's sum and its sum of squares
    about its own mean), merged by the row map, whose chunks are 4x longer
    from 65536 vectors a row on; unfused, each pass has a partial and a
    merge."""
    e = programs.CONFIG_PROGRAMS["layernorm_dyn"]().emit(flags=flags)
    rc, h = parse(e.plan)
    assert rc == 0, _lib.last_error()
    R = 3
    arr = compiler._descriptors([TensorDesc(0x1000, (R, C), 0), TensorDesc(0x1000, (C,), 0),
                                 TensorDesc(0x1000, (C,), 0), TensorDesc(0x1000, (R, C), 0)])
    syms = e.kernel_symbols()
    out = (ctypes.c_uint8 * len(syms))()
    assert _lib.lib().tca_program_selected(h, arr, 4, None, 0, out, None, None, len(syms)) == 0, _lib.last_error()
    assert [s for s, f in zip(syms, out) if f] == ["tca_layernorm_dyn_k0_" + v for v in variants]
    _lib.lib().tca_program_unload(h)
    if flags == 0:
        assert "tca::hip::chan_add(cs, cm, cn, ev);" in e.source
        assert "ptotal += c < PF ? mv[k] + nc * dc * dc : 0.0f;" in e.source


def test_split_pair_finish_binds_row_values():
    """The fused pair's finish in the row map: the mean's piped map loads
    its per-row operand (shift, tensor 1) at the row, and the sum of
    squares' piped map reads the mean the map computed (aval), not memory."""
    e = programs.CONFIG_PROGRAMS["row_stats_shift_dyn"]().emit()
    assert "const float ars1 = t1[c0];" in e.source
    assert "(aval * 0x1p-1f)" in e.source
    assert "_wl4_3" in e.plan and "_m4_1" not in e.plan


def _select(name, descs):
    """(status, last error) of selecting `name`'s kernels for tensors shaped `descs`."""
    e = programs.CONFIG_PROGRAMS[name]().emit()
    rc, h = parse(e.plan)
    assert rc == 0, _lib.last_error()
    syms = e.kernel_symbols()
    out = (ctypes.c_uint8 * len(syms))()
    arr = compiler._descriptors([TensorDesc(0x1000, s, 0) for s in descs])
    st = _lib.lib().tca_program_selected(h, arr, len(descs), None, 0, out, None, None, len(syms))
    err = _lib.last_error()
    _lib.lib().tca_program_unload(h)
    return st, err


def test_element_limit_keeps_index_headroom():
    """A tensor holds at most 2^32 - 2^16 - 1 elements: the split kernels
    step a u32 vector index up to 5120 past the row's vectors before
    comparing (a row of 2^32 - 1 odd elements would wrap it). The largest
    row selects the split pair; one element more is refused before any
    launch, and so is a shape whose 64-bit element product wraps to 0
    (2^31 x 2^31 x 4: counted as empty, it skipped every check before); an
    extent of 0 beside huge ones is an empty tensor."""
    top = (1 << 32) - (1 << 16) - 1
    st, err = _select("row_sum_max_dyn", [(1, top), (1,), (1,)])
    assert st == 0, err
    st, err = _select("row_sum_max_dyn", [(1, top + 1), (1,), (1,)])
    assert st == _lib.TCA_ERR_SHAPE and "2^32-2^16-1" in err, err
    big = (1 << 32) - 1
    st, err = _select("col_mean_var_dyn", [(1 << 31, 1 << 31, 4), (1 << 31, 4), (1 << 31, 4)])
    assert st == _lib.TCA_ERR_SHAPE and "2^32-2^16-1" in err, err
    st, err = _select("col_mean_var_dyn", [(0, big, big), (0, big), (0, big)])
    assert st == 0, err
