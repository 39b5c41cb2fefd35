"""The DSL builder through the C ABI (tca_cg.h) — the reference's pkg tests
restated: eager checks (pkg/builder_test.go:21-160), typestate
(pkg/builder_test.go:162), determinism (pkg/determinism_test.go:19-46)."""
import os

import pytest

from tcacomp_amd.pkg import (TBF16, TF32, TI32, TU32, At, BuildError, Call, Cast, NewBuilder, Select)


def dims(b):
    return b.Dim("m", 0), b.Dim("k", 0), b.Dim("n", 0)


def test_wrong_map_arity():
    b = NewBuilder("arity")
    m, k, n = dims(b)
    lhs, rhs = b.Tensor("lhs", TF32, m, n), b.Tensor("rhs", TF32, n, k)
    with pytest.raises(BuildError, match="arity"):
        b.Stmt().Iter(m, k, n).Map([At(lhs, m, n), At(rhs, n, k)], lambda l: l)


def test_wrong_piped_map_arity():
    b = NewBuilder("arity-piped")
    m, k, n = dims(b)
    lhs = b.Tensor("lhs", TF32, m, n)
    ar = b.Stmt().Iter(m, k, n).Map([At(lhs, m, n)], lambda v: v).As(m, k, n).Reduce(
        b.Float32(0), lambda acc, v: b.Add(acc, v))
    with pytest.raises(BuildError, match="arity"):
        ar.Map([], lambda a, c: a)


def test_duplicate_axis_in_as_surfaces_at_next_rung():
    b = NewBuilder("dup-as")
    m, k, n = dims(b)
    lhs, rhs = b.Tensor("lhs", TF32, m, n), b.Tensor("rhs", TF32, n, k)
    mid = b.Stmt().Iter(m, k, n).Map([At(lhs, m, n), At(rhs, n, k)], lambda l, r: b.Mul(l, r)).As(m, k, k)
    with pytest.raises(BuildError, match="@n"):
        mid.Reduce(b.Float32(0), lambda acc, v: b.Add(acc, v))


def test_omit_live_axis_in_as():
    b = NewBuilder("omit-as")
    m, k, n = dims(b)
    lhs = b.Tensor("lhs", TF32, m, n)
    mid = b.Stmt().Iter(m, k, n).Map([At(lhs, m, n)], lambda l: l).As(m)
    with pytest.raises(BuildError):
        mid.Reduce(b.Float32(0), lambda acc, v: b.Add(acc, v))


def test_heterogeneous_reducer():
    b = NewBuilder("hetero")
    m, k, n = dims(b)
    lhs = b.Tensor("lhs", TF32, m, n)
    mid = b.Stmt().Iter(m, k, n).Map([At(lhs, m, n)], lambda l: l).As(m, k, n)
    with pytest.raises(BuildError, match="homogeneous"):
        mid.Reduce(b.Int32(0), lambda acc, v: b.Add(acc, v))


def test_combiner_type_must_match():
    b = NewBuilder("hetero2")
    m, n = b.Dim("m", 0), b.Dim("n", 0)
    x = b.Tensor("x", TF32, m, n)
    mid = b.Stmt().Iter(m, n).Map([At(x, m, n)], lambda v: v).As(m, n)
    with pytest.raises(BuildError, match="homogeneous"):
        mid.Reduce(b.Float32(0), lambda acc, v: b.Lt(acc, v))


def test_wrong_subscript_count():
    b = NewBuilder("subscripts")
    m, k, n = dims(b)
    lhs, rhs = b.Tensor("lhs", TF32, m, n), b.Tensor("rhs", TF32, n, k)
    with pytest.raises(BuildError, match="rank"):
        b.Stmt().Iter(m, k, n).Map([At(lhs, m), At(rhs, n, k)], lambda l, r: b.Mul(l, r))


def test_undeclared_dim():
    b = NewBuilder("undeclared")
    m, k, n = dims(b)
    lhs, rhs = b.Tensor("lhs", TF32, m, n), b.Tensor("rhs", TF32, n, k)
    foreign = NewBuilder("other").Dim("z", 0)
    with pytest.raises(BuildError, match="declared"):
        b.Stmt().Iter(m, k, n).Map([At(lhs, m, foreign), At(rhs, n, k)], lambda l, r: b.Mul(l, r))


def test_unknown_builtin():
    b = NewBuilder("builtin")
    with pytest.raises(BuildError, match="not a registered pure scalar builtin"):
        Call("threadIdx_x", b.Float32(1))


def test_builtin_arity_and_type():
    b = NewBuilder("builtin2")
    with pytest.raises(BuildError, match="expects 1"):
        Call("expf", b.Float32(1), b.Float32(2))
    with pytest.raises(BuildError, match="must be f32"):
        Call("expf", b.Int32(1))
    assert Call("umin", b.UInt32(1), b.UInt32(2)).Type() == TU32


def test_bad_operand_axis():
    b = NewBuilder("operand-axis")
    m, k, n = dims(b)
    lhs = b.Tensor("lhs", TF32, m, n)
    with pytest.raises(BuildError, match="dim"):
        b.Stmt().Iter(m, k, n).Map([At(lhs, m, k)], lambda l: l)


def test_operand_axis_must_be_live():
    b = NewBuilder("live")
    m, n = b.Dim("m", 0), b.Dim("n", 0)
    x = b.Tensor("x", TF32, m, n)
    with pytest.raises(BuildError, match="not a live axis"):
        b.Stmt().Iter(m).Map([At(x, m, n)], lambda v: v)


def test_implicit_promotion_rejected():
    b = NewBuilder("promo")
    e = b.Add(b.Float32(1), b.Int32(1))
    assert "implicit promotions are not supported" in e.Err()
    m = b.Dim("m", 0)
    x = b.Tensor("x", TF32, m)
    y = b.Tensor("y", TF32, m)
    mid = b.Stmt().Iter(m).Map([At(x, m)], lambda v: v).As(m)
    with pytest.raises(BuildError, match="implicit promotions"):
        mid.Reduce(b.Float32(0), lambda acc, v: b.Add(acc, b.Int32(1)))
    del y


def test_select_and_cast_rules():
    b = NewBuilder("sel")
    assert "condition must be bool" in Select(b.Float32(1), b.Float32(1), b.Float32(2)).Err()
    assert "identical types" in Select(b.Bool(True), b.Float32(1), b.Int32(2)).Err()
    assert Select(b.Lt(b.Float32(1), b.Float32(2)), b.Float32(1), b.Float32(2)).Err() is None
    assert "redundant cast" in Cast(b.Float32(1), TF32).Err()
    assert "cast registry" in Cast(b.Bool(True), TF32).Err()
    assert Cast(b.Float32(1), TBF16).Type() == TBF16


def test_operator_classes():
    b = NewBuilder("ops")
    assert "integer type" in b.Mod(b.Float32(1), b.Float32(2)).Err()
    assert "must be bool" in b.And(b.Int32(1), b.Int32(2)).Err()
    assert b.Eq(b.Int32(1), b.Int32(1)).Type() == 9  # bool
    assert b.BitXor(b.UInt32(1), b.UInt32(3)).Type() == TU32


def test_duplicate_declarations_deferred_to_build():
    b = NewBuilder("dups")
    m = b.Dim("m", 0)
    b.Dim("m", 4)  # recorded, not raised
    x = b.Tensor("x", TF32, m)
    y = b.Tensor("y", TF32, m)
    with pytest.raises(BuildError, match="already declared"):
        b.Stmt().Iter(m).Map([At(x, m)], lambda v: v).As(m).Store(y, m)


def test_negative_extent():
    b = NewBuilder("neg")
    b.Dim("m", -3)
    with pytest.raises(BuildError, match="extent must be >= 0"):
        b.Build()


def test_unstored_chain_rejected_at_build():
    b = NewBuilder("open")
    m = b.Dim("m", 0)
    x = b.Tensor("x", TF32, m)
    b.Stmt().Iter(m).Map([At(x, m)], lambda v: v).As(m)
    with pytest.raises(BuildError, match="never stored"):
        b.Build()


def test_store_checks():
    b = NewBuilder("store")
    m, n = b.Dim("m", 0), b.Dim("n", 0)
    x = b.Tensor("x", TF32, m, n)
    out_mn = b.Tensor("o", TF32, m, n)
    out_m = b.Tensor("om", TF32, m)
    ar = b.Stmt().Iter(m, n).Map([At(x, m, n)], lambda v: v).As(m, n).Reduce(b.Float32(0), lambda a, v: b.Add(a, v))
    with pytest.raises(BuildError, match="not a live axis"):
        ar.Store(out_mn, m, n)
    b2 = NewBuilder("store2")
    m2, n2 = b2.Dim("m", 0), b2.Dim("n", 0)
    x2 = b2.Tensor("x", TF32, m2, n2)
    o2 = b2.Tensor("o", TF32, m2)
    mid = b2.Stmt().Iter(m2, n2).Map([At(x2, m2, n2)], lambda v: v).As(m2, n2)
    with pytest.raises(BuildError, match="single-owner"):
        mid.Store(o2, m2)
    del out_m


def test_store_type_must_match():
    b = NewBuilder("store-type")
    m = b.Dim("m", 0)
    x = b.Tensor("x", TF32, m)
    o = b.Tensor("o", TI32, m)
    with pytest.raises(BuildError, match="cannot be stored"):
        b.Stmt().Iter(m).Map([At(x, m)], lambda v: v).As(m).Store(o, m)


def test_piped_as_must_be_live_order():
    b = NewBuilder("piped-as")
    m, n, k = b.Dim("m", 0), b.Dim("n", 0), b.Dim("k", 0)
    x = b.Tensor("x", TF32, m, n, k)
    o = b.Tensor("o", TF32, m, n)
    t = (b.Stmt().Iter(m, n, k).Map([At(x, m, n, k)], lambda v: v).As(m, n, k)
         .Reduce(b.Float32(0), lambda a, v: b.Add(a, v)).Map([], lambda v: v).As(n, m))
    with pytest.raises(BuildError, match="incoming axis order"):
        t.Store(o, m, n)


def test_local_read_before_store():
    b = NewBuilder("local-order")
    r, c = b.Dim("r", 0), b.Dim("c", 8)
    x = b.Tensor("x", TF32, r, c)
    loc = b.Local("loc", TF32, r)
    y = b.Tensor("y", TF32, r, c)
    with pytest.raises(BuildError, match="read before any statement stores it"):
        b.Stmt().Iter(r, c).Map([At(x, r, c), At(loc, r)], lambda l, s: b.Add(l, s))
    del y


def test_chained_reductions_and_full_typestate():
    b = NewBuilder("chain")
    i, j, k = b.Dim("i", 0), b.Dim("j", 0), b.Dim("k", 4)
    x = b.Tensor("x", TF32, i, j, k)
    o = b.Tensor("o", TF32, i)
    s = b.ScalarParam("s", TF32)
    (b.Stmt().Iter(i, j, k).Map([At(x, i, j, k)], lambda v: v).As(i, j, k)
     .Reduce(b.Float32(0), lambda a, v: b.Add(a, v))
     .Reduce(b.Float32(float("-inf")), lambda a, v: Call("fmaxf", a, v))
     .Map([], lambda v: b.Mul(v, s)).As(i).Store(o, i))
    p = b.Build()
    ir = p.IRFull()
    assert "reduce init=0:f32 over @k" in ir and "reduce init=-inf:f32 over @j" in ir
    assert "store o[@i]" in ir


def _oracle_program(name):
    # The doc-pinned matmul_scale shape (pkg/oracle_test.go:60-63).
    b = NewBuilder(name)
    m, k, n = dims(b)
    lhs, rhs = b.Tensor("lhs", TF32, m, n), b.Tensor("rhs", TF32, n, k)
    out = b.Tensor("out", TF32, m, k)
    scale = b.ScalarParam("scale", TF32)
    (b.Stmt().Iter(m, k, n).Map([At(lhs, m, n), At(rhs, n, k)], lambda l, r: b.Mul(l, r)).As(m, k, n)
     .Reduce(b.Float32(0), lambda a, v: b.Add(a, v)).Map([], lambda v: b.Mul(v, scale)).As(m, k).Store(out, m, k))
    return b.Build()


def test_determinism_print_and_emit():
    p1, p2 = _oracle_program("matmul_scale"), _oracle_program("matmul_scale")
    assert p1.IR() == p2.IR() and p1.IRFull() == p2.IRFull()
    e1, e2 = p1.emit(), p2.emit()
    assert e1.source == e2.source and e1.plan == e2.plan


def test_ir_full_dump_shape():
    ir = _oracle_program("matmul_scale").IRFull()
    assert ir.splitlines()[0] == "program matmul_scale"
    assert "map on(lhs[@m][@n], rhs[@n][@k]) (l: f32, r: f32) { %0 = mul l r; -> %0: f32 } as(@m, @k, @n)" in ir
    assert "reduce init=0:f32 over @n (acc: f32, now: f32) { %0 = add acc now; -> %0: f32 }" in ir
    assert "map pipe+on() (v: f32) { %0 = mul v $scale; -> %0: f32 } as(@m, @k)" in ir


def test_gvn_hash_consing_folds_duplicates():
    """dup_expr's repeated v*v + v*v: identical subexpressions are one node
    (the reference's HIR GVN, testing/kernels/dedup/dup_expr.tca:1-5)."""
    b = NewBuilder("gvn")
    m = b.Dim("m", 0)
    x = b.Tensor("x", TF32, m)
    o = b.Tensor("o", TF32, m)
    seen = {}

    def body(v):
        a = b.Add(b.Mul(v, v), b.Mul(v, v))
        c = b.Add(b.Mul(v, v), b.Mul(v, v))
        seen["same"] = a.idx == c.idx
        return b.Mul(a, c)
    b.Stmt().Iter(m).Map([At(x, m)], body).As(m).Store(o, m)
    assert seen["same"]
    ir = b.Build().IRFull()
    assert ir.count(" mul ") == 2 and ir.count(" add ") == 1


def test_build_freezes():
    b = NewBuilder("frozen")
    m = b.Dim("m", 0)
    x = b.Tensor("x", TF32, m)
    o = b.Tensor("o", TF32, m)
    b.Stmt().Iter(m).Map([At(x, m)], lambda v: v).As(m).Store(o, m)
    b.Build()
    b.Dim("late", 0)
    b2 = NewBuilder("fresh")
    assert b2.Build().IRFull().startswith("program fresh")


def _matmul_scale_reference_order():
    """pkg/oracle_test.go:16-56, call for call: the builder calls (and so the
    graph IDs they take) in the reference's order."""
    b = NewBuilder("matmul_scale")
    m, k, n = b.Dim("m", 0), b.Dim("k", 0), b.Dim("n", 0)
    lhs = b.Tensor("lhs", TF32, m, n)
    rhs = b.Tensor("rhs", TF32, n, k)
    out = b.Tensor("output", TF32, m, k)
    scale = b.ScalarParam("scale", TF32)
    (b.Stmt().Iter(m, k, n).Map([At(lhs, m, n), At(rhs, n, k)], lambda l, r: b.Mul(l, r)).As(m, k, n)
     .Reduce(b.Float32(0.0), lambda acc, v: b.Add(acc, v)).Map([], lambda v: b.Mul(v, scale)).As(m, k)
     .Store(out, m, k))
    return b.Build()


def test_ir_print_matches_reference_golden():
    """tca_builder_ir is the reference's ir.Print: byte-identical to its
    doc-pinned golden (pkg/testdata/matmul_scale.ir, copied verbatim into
    tests/golden/; pkg/oracle_test.go:58-63 asserts the same bytes)."""
    golden = open(os.path.join(os.path.dirname(__file__), "golden", "matmul_scale.ir")).read()
    assert _matmul_scale_reference_order().IR() == golden


def test_ir_print_notation():
    """Stages the golden does not reach, in the printer's rules
    (internal/ir/print.go): chained reductions, a local (a MemNew in the
    reference: no name, `?`), select / cast / call / unary rendering,
    precedence parentheses (binPrec: right operand parenthesized at equal
    precedence), typed constants, and one end node over every output in
    first-store order, numbered with the first output chain's reserved ID.
    Statement IDs beyond the first chain follow the reference's allocation
    counts; the reference holds no golden for them (parity unpinned)."""
    b = NewBuilder("notation")
    r, c = b.Dim("r", 0), b.Dim("c", 8)
    x = b.Tensor("x", TF32, r, c)
    s = b.Tensor("s", TF32, r)
    q = b.Tensor("q", TF32, r)
    t = b.Local("t", TF32, r)
    a = b.ScalarParam("a", TF32)
    (b.Stmt().Iter(r, c).Map([At(x, r, c)], lambda v: b.Sub(v, b.Sub(a, b.Float32(1.5)))).As(r, c)
     .Reduce(b.Neg(b.Float32(float("inf"))), lambda acc, v: Call("fmaxf", acc, v)).Store(t, r))
    (b.Stmt().Iter(r, c).Map([At(x, r, c), At(t, r)], lambda l, m: Select(b.Gt(l, m), Cast(b.Int32(3), TF32), b.Mul(l, b.Add(m, b.Float32(1e-5))))).As(r, c)
     .Reduce(b.Float32(0), lambda acc, v: b.Add(acc, v)).Store(s, r))
    (b.Stmt().Iter(r).Map([At(t, r)], lambda v: b.Div(v, b.Float32(1e6))).As(r).Store(q, r))
    ir = b.Build().IR()
    # params r, c, x, s, q (1-5), the local (6-7), a (8): the first chain reserves 9 and 10
    assert ir.startswith("statement #9:\n  iter(@r, @c) -> map(x[@r][@c], lambda(v): v - (a - 1.5)) as (@r, @c) |\n"
                         "  reduce(init=-+Inf.0, %0, lambda(acc, now): fmaxf(acc, now)) |\n  memstore(%?[@r], %0)\n"), ir
    assert ("map(x[@r][@c], ?, lambda(l, r): l > r ? cast<f32>(3) : l * (r + 1e-05)) as (@r, @c) |\n"
            "  reduce(init=0.0, %0, lambda(acc, now): acc + now) |\n  memstore(%s[@r], %0)\n") in ir
    assert "iter(@r) -> map(?, lambda(v): v / 1e+06) as (@r) |\n  memstore(%q[@r], %0)\n" in ir
    ids = [int(l.split("#")[1].rstrip(":")) for l in ir.splitlines() if l.startswith("statement #")]
    assert ids[:3] == sorted(ids[:3]) and len(set(ids)) == 4
    # the end node: the reserved end ID of chain 2, the first to store an output
    assert ir.endswith("statement #%d:\n  return %%s, %%q\n" % (ids[1] + 1))


@pytest.mark.parametrize("value,text", [
    (0.0, "0.0"), (-0.0, "-0.0"), (0.1, "0.1"), (0.3, "0.3"), (2.5, "2.5"), (-0.75, "-0.75"),
    (100000.0, "100000.0"), (123456.7, "123456.7"), (1e6, "1e+06"), (16777216.0, "1.6777216e+07"),
    (0.0001, "0.0001"), (0.00001, "1e-05"), (3.4028234663852886e38, "3.4028235e+38"),
    (1.401298464324817e-45, "1e-45"), (1.1754943508222875e-38, "1.1754944e-38"),
    (float("inf"), "+Inf.0"), (float("nan"), "NaN.0")])
def test_ir_print_float_constants(value, text):
    """Float constants as the reference spells them (internal/ir/print.go
    FormatConst): Go's strconv.FormatFloat(v, 'g', -1, 32), then ".0" when
    the result has no '.', 'e' or 'E'."""
    b = NewBuilder("k")
    m = b.Dim("m", 0)
    x, o = b.Tensor("x", TF32, m), b.Tensor("o", TF32, m)
    b.Stmt().Iter(m).Map([At(x, m)], lambda v: b.Mul(v, b.Float32(value))).As(m).Store(o, m)
    assert "lambda(v): v * %s)" % text in b.Build().IR()
