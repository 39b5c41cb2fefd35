"""Host-only checks of the random row programs and of their CPU evaluator
(oracle/dsl_eval.py): every program builds and emits; the vectorized
evaluator agrees with a brute-force element loop in the reference's
sequential fold order (runtime/tca/reducer.h:36-57) on tiny shapes, with
hand-computed answers, and with the C oracle's row sum and max."""
import re

import numpy as np
import pytest

import oracle
from dsl_eval import evaluate, evaluate_grid, evaluate_grid_scalar, evaluate_scalar
import randprog
from randprog import Spec

SPECS = [s for s in randprog.specs() if getattr(s, "kind", "row") == "row"]
GRIDS = [s for s in randprog.specs() if getattr(s, "kind", "row") == "grid"]


def test_programs_are_deterministic_and_distinct():
    first, again = randprog.specs(), randprog.specs()
    assert sorted(s.name for s in SPECS + GRIDS) == sorted(s.name for s in first)
    assert [s.name for s in first] == [s.name for s in again]
    assert [repr(s.stmts) for s in first] == [repr(s.stmts) for s in again]
    shape = lambda s: repr(sorted((k, v) for k, v in vars(s).items() if k != "name"))  # noqa: E731
    assert len({shape(s) for s in SPECS + GRIDS}) == len(again)


@pytest.mark.parametrize("spec", [s for s in SPECS if s.name.startswith("rand_")], ids=lambda s: s.name)
def test_program_emits_one_fused_nest(spec):
    e = randprog.build(spec).emit()
    fams = set(e.families())
    assert fams == ({"stream"} if spec.c == 0 or spec.c == 70000 else {"row"}), e.report


def _tiny_inputs(spec, shape, seed):
    rng = np.random.default_rng(seed)
    rows, C = shape[:-1], shape[-1]
    if spec.elem == "f32":
        tiles = {t: rng.integers(-4, 5, size=shape).astype(np.float32) for t, _ in spec.tiles}
        col = rng.integers(-2, 3, size=(C,)).astype(np.float32) if spec.col else None
        row = rng.integers(-4, 5, size=rows).astype(np.float32) if spec.row else None
    else:
        tiles = {t: rng.integers(0, 1 << 32, size=shape, dtype=np.uint64).astype(np.uint32) for t, _ in spec.tiles}
        col = rng.integers(0, 1 << 32, size=(C,), dtype=np.uint64).astype(np.uint32) if spec.col else None
        row = rng.integers(0, 1 << 32, size=rows, dtype=np.uint64).astype(np.uint32) if spec.row else None
    return tiles, col, row


@pytest.mark.parametrize("spec", SPECS, ids=lambda s: s.name)
def test_evaluator_matches_brute_force(spec):
    rows = (3,) if spec.outer == 1 else (2, 2)
    for C in (0, 1, 5):
        tiles, col, row = _tiny_inputs(spec, rows + (C,), C)
        fast, exact = evaluate(spec, tiles, col, row, dict(spec.scalars))
        assert exact
        slow = evaluate_scalar(spec, tiles, col, row, dict(spec.scalars))
        assert sorted(fast) == sorted(slow) == sorted(spec.outputs())
        for k in fast:
            np.testing.assert_array_equal(fast[k], slow[k], err_msg="%s C=%d %s" % (spec.name, C, k))


def _spec(stmts, elem="f32", tiles=(("x0", "f32"),), col=False, row=False, scalars=()):
    return Spec("hand", elem, 0, 1, list(tiles), col, row, list(scalars), stmts)


X0 = ("leaf", "x0")


def test_known_answers_f32():
    spec = _spec([
        {"kind": "reduce", "expr": X0, "comb": "sum", "piped": None, "out": "o0", "local": False},
        {"kind": "reduce", "expr": X0, "comb": "max", "piped": None, "out": "l1", "local": True},
        # piped: v * s0 + r
        {"kind": "reduce", "expr": ("mul", X0, ("leaf", "g")), "comb": "min",
         "piped": ("add", ("mul", ("leaf", "v"), ("leaf", "s0")), ("leaf", "r")), "out": "o2", "local": False},
        {"kind": "rowmap", "expr": ("sub", ("leaf", "l1"), ("const", 1.0)), "out": "o3", "local": False},
        {"kind": "map", "expr": ("sub", X0, ("leaf", "l1")), "out": "y4", "local": False},
    ], col=True, row=True, scalars=[("s0", 2.0)])
    x = np.array([[1, 2, 3], [4, -5, 6]], np.float32)
    g = np.array([1, -1, 2], np.float32)
    r = np.array([10, 20], np.float32)
    out, exact = evaluate(spec, {"x0": x}, g, r, {"s0": 2.0})
    assert exact
    np.testing.assert_array_equal(out["o0"], [6, 5])
    np.testing.assert_array_equal(out["o2"], [2 * -2 + 10, 2 * 4 + 20])  # min(x*g): rows [1,-2,6], [4,5,12]
    np.testing.assert_array_equal(out["o3"], [2, 5])
    np.testing.assert_array_equal(out["y4"], [[-2, -1, 0], [-2, -11, 0]])


def test_known_answers_empty_rows_and_u32():
    spec = _spec([
        {"kind": "reduce", "expr": X0, "comb": c, "piped": None, "out": "o%d" % i, "local": False}
        for i, c in enumerate(["sum", "max", "min"])])
    out, _ = evaluate(spec, {"x0": np.zeros((2, 0), np.float32)}, None, None, {})
    np.testing.assert_array_equal(out["o0"], [0, 0])
    np.testing.assert_array_equal(out["o1"], [-np.inf, -np.inf])
    np.testing.assert_array_equal(out["o2"], [np.inf, np.inf])
    spec = _spec([
        {"kind": "reduce", "expr": X0, "comb": c, "piped": None, "out": "o%d" % i, "local": False}
        for i, c in enumerate(["sum", "xor", "max", "min"])], elem="u32", tiles=(("x0", "u32"),))
    x = np.array([[0xFFFFFFFF, 2, 5]], np.uint32)
    out, _ = evaluate(spec, {"x0": x}, None, None, {})
    assert [int(out[k][0]) for k in ("o0", "o1", "o2", "o3")] == [6, 0xFFFFFFFF ^ 2 ^ 5, 0xFFFFFFFF, 2]
    out, _ = evaluate(spec, {"x0": np.zeros((1, 0), np.uint32)}, None, None, {})
    assert [int(out[k][0]) for k in ("o0", "o1", "o2", "o3")] == [0, 0, 0, 0xFFFFFFFF]


def test_evaluator_matches_c_oracle_row_sum_max():
    """The reference's row_sum runner restated in C (oracle.c), on exact data."""
    spec = _spec([
        {"kind": "reduce", "expr": X0, "comb": "sum", "piped": None, "out": "o0", "local": False},
        {"kind": "reduce", "expr": X0, "comb": "max", "piped": None, "out": "o1", "local": False}])
    x = np.random.default_rng(5).integers(-100, 101, size=(64, 777)).astype(np.float32)
    out, exact = evaluate(spec, {"x0": x}, None, None, {})
    s, m = oracle.row_sum_max(x)
    assert exact
    np.testing.assert_array_equal(out["o0"], s)
    np.testing.assert_array_equal(out["o1"], m)


def test_inexact_sums_are_reported():
    spec = _spec([{"kind": "reduce", "expr": X0, "comb": "sum", "piped": None, "out": "o0", "local": False}])
    _, exact = evaluate(spec, {"x0": np.full((1, 4), 0.5, np.float32)}, None, None, {})
    assert not exact  # non-integer terms
    _, exact = evaluate(spec, {"x0": np.full((1, 3), 2.0 ** 23, np.float32)}, None, None, {})
    assert not exact  # partial sums past 2^24
    # infinities fix a sum in any order: -inf, NaN (both signs), and small integers beside them
    x = np.array([[-np.inf, 1, 2], [np.inf, -np.inf, 3], [np.nan, 1, 1]], np.float32)
    out, exact = evaluate(spec, {"x0": x}, None, None, {})
    assert exact
    np.testing.assert_array_equal(out["o0"], [-np.inf, np.nan, np.nan])


def _grid_inputs(spec, R, C, seed, B=2):
    rng = np.random.default_rng(seed)
    if spec.elem == "f32":
        gen = lambda *shape: rng.integers(-4, 5, size=shape).astype(np.float32)  # noqa: E731
    else:
        gen = lambda *shape: rng.integers(0, 1 << 32, size=shape, dtype=np.uint64).astype(np.uint32)  # noqa: E731
    lead = (B,) if spec.batch else ()
    return (gen(*lead, R, C), gen(*lead, C, R) if spec.trans else None, gen(C) if spec.col else None,
            gen(R) if spec.row else None)


@pytest.mark.parametrize("spec", GRIDS, ids=lambda s: s.name)
def test_grid_evaluator_matches_brute_force(spec):
    for R, C in ((3, 4), (1, 1), (0, 3), (4, 0)):
        x0, xt, g, r = _grid_inputs(spec, R, C, R * 10 + C)
        fast, exact = evaluate_grid(spec, x0, xt, g, r, dict(spec.scalars))
        assert exact
        slow = evaluate_grid_scalar(spec, x0, xt, g, r, dict(spec.scalars))
        assert sorted(fast) == sorted(slow) == sorted(spec.outputs())
        for k in fast:
            np.testing.assert_array_equal(fast[k], slow[k], err_msg="%s %dx%d %s" % (spec.name, R, C, k))


COLCHAINS = [s for s in GRIDS if s.name.startswith("gridc")]


def test_colchain_programs_fuse_dependent_reductions():
    """A dependent column program whose first two reductions read no
    transposed tile emits them as one column nest of several passes: a
    whole-column kernel per vector width, and a partial + merge pair per
    pass. (A transposed tile xt [C, R] is contiguous along R: those nests
    lower as row reductions of the stream family.)"""
    fused = 0
    for spec in COLCHAINS:
        if any("xt" in randprog.leaves(st["expr"]) for st in spec.stmts[:2]):
            continue
        e = randprog.build(spec).emit()
        k0 = [line.split() for line in e.report.splitlines() if "_k0_" in line.split()[0]]
        assert {f for _, f, *_ in k0} == {"col"}, e.report
        syms = [sym for sym, *_ in k0]
        assert any(re.search(r"_k0_w\d+$", x) for x in syms), syms
        passes = {int(m.group(1)) for m in (re.search(r"_k0_p\d+_(\d+)$", x) for x in syms) if m}
        assert len(passes) >= 2 and passes == {int(m.group(1)) for m in
                                               (re.search(r"_k0_m\d+_(\d+)$", x) for x in syms) if m}
        fused += 1
    assert fused >= 10, fused


def test_colchain_generator_reads_earlier_results():
    """Every dependent column program has a reduction that reads the result
    of an earlier one, and some of those results are locals."""
    for spec in COLCHAINS:
        outs = [st["out"] for st in spec.stmts if st["kind"] == "colreduce"]
        assert any(set(randprog.leaves(st["expr"])) & set(outs[:k])
                   for k, st in enumerate(s for s in spec.stmts if s["kind"] == "colreduce")), spec.name
    assert any(st["local"] for spec in COLCHAINS for st in spec.stmts)


def test_grid_known_answers():
    from randprog import GridSpec
    spec = GridSpec("hand", "f32", 0, [("x0", "f32")], True, True, False, [], [
        {"kind": "map", "expr": ("sub", X0, ("leaf", "xt")), "comb": None, "piped": None, "out": "m0"},
        {"kind": "tmap", "expr": X0, "comb": None, "piped": None, "out": "t1"},
        {"kind": "colreduce", "expr": X0, "comb": "sum", "piped": ("mul", ("leaf", "v"), ("leaf", "g")),
         "out": "c2"}])
    x = np.array([[1, 2], [3, 4]], np.float32)
    xt = np.array([[10, 20], [30, 40]], np.float32)  # xt[c, r]
    out, _ = evaluate_grid(spec, x, xt, np.array([1, -1], np.float32), None, {})
    np.testing.assert_array_equal(out["m0"], [[1 - 10, 2 - 30], [3 - 20, 4 - 40]])
    np.testing.assert_array_equal(out["t1"], [[1, 3], [2, 4]])
    np.testing.assert_array_equal(out["c2"], [4, -6])


def test_grid_dependent_known_answers():
    """A reduction reading an earlier one at its own column, by hand: c0 =
    column sums (a local), c1 = max over rows of x - c0, piped + c0."""
    from randprog import GridSpec
    spec = GridSpec("hand", "f32", 0, [("x0", "f32")], False, False, False, [], [
        {"kind": "colreduce", "expr": X0, "comb": "sum", "piped": None, "out": "c0", "local": True},
        {"kind": "colreduce", "expr": ("sub", X0, ("leaf", "c0")), "comb": "max",
         "piped": ("add", ("leaf", "v"), ("leaf", "c0")), "out": "c1", "local": False},
        {"kind": "map", "expr": ("mul", X0, ("leaf", "c0")), "comb": None, "piped": None, "out": "m2",
         "local": False}])
    x = np.array([[1, 2], [3, 5]], np.float32)
    out, exact = evaluate_grid(spec, x, None, None, None, {})
    assert exact and sorted(out) == ["c1", "m2"]
    np.testing.assert_array_equal(out["c1"], [max(1 - 4, 3 - 4) + 4, max(2 - 7, 5 - 7) + 7])
    np.testing.assert_array_equal(out["m2"], [[4, 14], [12, 35]])
    slow = evaluate_grid_scalar(spec, x, None, None, None, {})
    for k in out:
        np.testing.assert_array_equal(out[k], slow[k])


ROWCHAINS = [s for s in SPECS if s.name.startswith("rowc")]


def test_rowchain_programs_fold_in_segment_kernels():
    """Every chained reduction over rows [B, R] of the random programs (a
    chain with two Reduce rungs, or a reduce into a local and a rowreduce
    of it) emits a segment kernel beside the two nests' own kernels,
    guarded on B: one kernel per vector width, over B blocks."""
    seen = 0
    for spec in ROWCHAINS:
        if spec.outer != 2:
            continue
        e = randprog.build(spec).emit()
        pairs = sum(1 for st in spec.stmts if st["kind"] in ("chain", "rowreduce"))
        seg_nests = {line.split()[0].rsplit("_", 1)[0] for line in e.report.splitlines() if line.split()[1] == "seg"}
        assert len(seg_nests) == pairs, (spec.name, e.report)
        for line in e.plan.split("kernel ")[1:]:
            if "_g" in line.split()[0] and line.split()[0].rsplit("_", 1)[1].startswith("g"):
                assert "when B 1024 4294967295 1 0" in line, line
        seen += pairs
    assert seen >= 12, seen


def test_rowchain_known_answers():
    """chain and rowreduce by hand over x [2, 3, 2] (B, R, C)."""
    spec = Spec("hand", "f32", 0, 2, [("x0", "f32")], False, False, [], [
        {"kind": "chain", "expr": X0, "comb": "sum", "comb2": "max", "piped": ("mul", ("leaf", "v"),
                                                                                 ("const", 2.0)),
         "out": "o0", "local": False},
        {"kind": "reduce", "expr": X0, "comb": "max", "piped": None, "out": "l1", "local": True},
        {"kind": "rowreduce", "expr": ("sub", ("leaf", "l1"), ("const", 1.0)), "comb": "sum", "piped": None,
         "out": "o2", "local": False}])
    x = np.array([[[1, 2], [3, -4], [0, 5]], [[-1, -1], [2, 2], [7, -9]]], np.float32)
    out, exact = evaluate(spec, {"x0": x}, None, None, {})
    assert exact and sorted(out) == ["o0", "o2"]
    np.testing.assert_array_equal(out["o0"], [max(3, -1, 5) * 2, max(-2, 4, -2) * 2])
    np.testing.assert_array_equal(out["o2"], [(2 - 1) + (3 - 1) + (5 - 1), (-1 - 1) + (2 - 1) + (7 - 1)])
    slow = evaluate_scalar(spec, {"x0": x}, None, None, {})
    for k in out:
        np.testing.assert_array_equal(out[k], slow[k])
