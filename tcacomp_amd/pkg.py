"""Python face of the DSL builder — the reference's Go ``pkg`` API.

Same names, argument meaning and checks as pkg/builder.go:122-370,
pkg/chain.go:360-552 and pkg/expr.go:140-341; every call forwards to the
C++ builder behind include/tca_cg.h. Where Go returns ``(rung, error)``
this raises ``BuildError`` carrying the same message. Declaration-time
violations are deferred exactly as in Go: they surface at the next
error-returning rung (Map, Reduce, Store) or at Build.

    b = NewBuilder("gemm")
    M, N, K = b.Dim("M", 0), b.Dim("N", 0), b.Dim("K", 0)
    lhs = b.Tensor("lhs", TF32, M, K)
    rhs = b.Tensor("rhs", TF32, K, N)
    out = b.Tensor("out", TF32, M, N)
    (b.Stmt().Iter(M, N, K)
        .Map([At(lhs, M, K), At(rhs, K, N)], lambda l, r: b.Mul(l, r))
        .As(M, N, K)
        .Reduce(b.Float32(0), lambda acc, v: b.Add(acc, v))
        .Store(out, M, N))
    prog = b.Build()
"""
import ctypes
import inspect

from . import _lib
from ._lib import tca_operand

# Element types (internal/ir/types.go; numbering shared with the C ABI).
TF32, TF16, TBF16, TI32, TU32, TI8, TI16, TU8, TU16, TBool = range(10)
ELEM_NAMES = ["f32", "f16", "bf16", "i32", "u32", "i8", "i16", "u8", "u16", "bool"]

# Binary / unary operator codes (tca_cg.h).
(_ADD, _SUB, _MUL, _DIV, _MOD, _EQ, _NE, _LT, _LE, _GT, _GE, _LAND, _LOR, _AND, _OR, _XOR, _SHL,
 _SHR) = range(18)
_NEG, _POS, _LNOT, _NOT = range(4)

EMIT_NO_FUSION = 1
EMIT_NO_GEMM = 2
EMIT_NO_GEMM_SPLIT = 4  # no small-tile K-split contraction kernels (the tile kernels only)
EMIT_NO_PASS_FUSION = 8  # every pass of a multi-pass nest reads its input (no one-read fusions)


class BuildError(Exception):
    """A rung, Build or Emit rejected the program (the Go `error` value)."""


def _ints(seq):
    arr = (ctypes.c_int32 * max(1, len(seq)))()
    for i, v in enumerate(seq):
        arr[i] = v
    return arr


class Dim:
    """Handle of a declared shape dimension; extent 0 = dynamic."""

    def __init__(self, b, idx, name, extent):
        self.b, self.idx, self._name, self._extent = b, idx, name, extent

    def Name(self):
        return self._name

    def Extent(self):
        return self._extent

    def __repr__(self):
        return "Dim(@%s, %d)" % (self._name, self._extent)


class Tensor:
    """Handle of a declared tensor parameter or local."""

    def __init__(self, b, idx, name, elem, dims, local=False):
        self.b, self.idx, self._name, self._elem, self.dims, self.local = b, idx, name, elem, list(dims), local

    def Name(self):
        return self._name

    def Elem(self):
        return self._elem

    def Rank(self):
        return len(self.dims)


class Operand:
    def __init__(self, t, axes):
        self.t, self.axes = t, list(axes)

    def Tensor(self):
        return self.t

    def Axes(self):
        return list(self.axes)


def At(t, *axes):
    """One structural access t[axes...] (pkg/builder.go:112-118)."""
    return Operand(t, axes)


class Expr:
    """A typed scalar expression (pkg/expr.go:34-60). Operators forward to
    the builder's typed constructors; plain Python numbers become literals
    of the other operand's type."""

    def __init__(self, b, idx):
        self.b, self.idx = b, idx

    def Type(self):
        return _lib.lib().tca_expr_dtype(self.b._h, self.idx)

    def Err(self):
        m = _lib.lib().tca_expr_error(self.b._h, self.idx)
        return m.decode() if m else None

    def _lit(self, v):
        if isinstance(v, Expr):
            return v
        t = self.Type()
        return self.b._const(t if t >= 0 else TF32, v)

    def __add__(self, o): return self.b.Add(self, self._lit(o))
    def __radd__(self, o): return self.b.Add(self._lit(o), self)
    def __sub__(self, o): return self.b.Sub(self, self._lit(o))
    def __rsub__(self, o): return self.b.Sub(self._lit(o), self)
    def __mul__(self, o): return self.b.Mul(self, self._lit(o))
    def __rmul__(self, o): return self.b.Mul(self._lit(o), self)
    def __truediv__(self, o): return self.b.Div(self, self._lit(o))
    def __rtruediv__(self, o): return self.b.Div(self._lit(o), self)
    def __neg__(self): return self.b.Neg(self)


class Program:
    """A built (verified, frozen) program."""

    def __init__(self, b):
        self.b = b
        self.name = b.name

    def IR(self):
        """The reference's canonical print (internal/ir/print.go:34)."""
        s = _lib.lib().tca_builder_ir(self.b._h)
        return s.decode() if s else ""

    def IRFull(self):
        """This build's structural dump: equal dumps, same program."""
        s = _lib.lib().tca_builder_ir_full(self.b._h)
        return s.decode() if s else ""

    def emit(self, kernel_name=None, target=None, flags=0):
        """Runs the HIP emitter (the cxx.Emit seam) and returns EmitResult."""
        L = _lib.lib()
        out = ctypes.c_void_p()
        rc = L.tca_emit(self.b._h, kernel_name.encode() if kernel_name else None,
                        target.encode() if target else None, flags, ctypes.byref(out))
        if rc != 0:
            raise BuildError(L.tca_builder_error(self.b._h).decode())
        try:
            n = L.tca_emit_hipcc_argc(out)
            return EmitResult(
                source=L.tca_emit_source(out).decode(),
                plan=L.tca_emit_plan(out).decode(),
                report=L.tca_emit_report(out).decode(),
                hipcc=[L.tca_emit_hipcc_arg(out, i).decode() for i in range(n)],
            )
        finally:
            L.tca_emit_free(out)


class EmitResult:
    def __init__(self, source, plan, report, hipcc):
        self.source, self.plan, self.report, self.hipcc = source, plan, report, hipcc

    def families(self):
        return [line.split()[1] for line in self.report.splitlines() if line.strip()]

    def kernel_symbols(self):
        return [line.split()[0] for line in self.report.splitlines() if line.strip()]


class Builder:
    """The public builder root (pkg/builder.go:35-45)."""

    def __init__(self, name):
        self.name = name
        self._h = _lib.lib().tca_builder_new(name.encode())
        if not self._h:
            raise MemoryError("tca_builder_new failed")

    @classmethod
    def _adopt(cls, name, handle):
        """Wraps a builder handle made elsewhere (the .tca frontend)."""
        b = cls.__new__(cls)
        b.name = name
        b._h = handle
        return b

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.lib().tca_builder_free(h)
            except Exception:
                pass
            self._h = None

    def _err(self):
        return _lib.lib().tca_builder_error(self._h).decode()

    # ---- declarations (pkg/builder.go:163-295)
    def Dim(self, name, extent):
        idx = _lib.lib().tca_builder_dim(self._h, name.encode(), int(extent))
        return Dim(self, idx, name, int(extent))

    def _decl(self, fn, name, elem, dims, local):
        for d in dims:
            if not isinstance(d, Dim) or d.b is not self:
                ids = [-1]
                break
        else:
            ids = [d.idx for d in dims]
        idx = fn(self._h, name.encode(), elem, len(dims), _ints(ids))
        return Tensor(self, idx, name, elem, dims, local)

    def Tensor(self, name, elem, *dims):
        return self._decl(_lib.lib().tca_builder_tensor, name, elem, dims, False)

    def Local(self, name, elem, *dims):
        """A `let` local. The reference takes an ir.Type; here its element
        type and dims. Any rank is accepted (the v0 rank>=2-dynamic wall is
        lifted: locals live in registers or an HBM workspace)."""
        return self._decl(_lib.lib().tca_builder_local, name, elem, dims, True)

    def ScalarParam(self, name, elem):
        return Expr(self, _lib.lib().tca_builder_scalar(self._h, name.encode(), elem))

    # ---- literals (pkg/expr.go:242-264)
    def _const(self, elem, v):
        return Expr(self, _lib.lib().tca_expr_const(self._h, elem, float(v)))

    def Float32(self, v): return self._const(TF32, v)
    def Int32(self, v): return self._const(TI32, v)
    def UInt32(self, v): return self._const(TU32, v)
    def Bool(self, v): return self._const(TBool, 1.0 if v else 0.0)

    # ---- operators (pkg/expr.go:179-240)
    def _bin(self, op, x, y):
        if not isinstance(x, Expr) or not isinstance(y, Expr):
            raise TypeError("operands must be Expr")
        return Expr(self, _lib.lib().tca_expr_binop(self._h, op, x.idx, y.idx))

    def _un(self, op, x):
        return Expr(self, _lib.lib().tca_expr_unop(self._h, op, x.idx))

    def Add(self, x, y): return self._bin(_ADD, x, y)
    def Sub(self, x, y): return self._bin(_SUB, x, y)
    def Mul(self, x, y): return self._bin(_MUL, x, y)
    def Div(self, x, y): return self._bin(_DIV, x, y)
    def Mod(self, x, y): return self._bin(_MOD, x, y)
    def Eq(self, x, y): return self._bin(_EQ, x, y)
    def Ne(self, x, y): return self._bin(_NE, x, y)
    def Lt(self, x, y): return self._bin(_LT, x, y)
    def Le(self, x, y): return self._bin(_LE, x, y)
    def Gt(self, x, y): return self._bin(_GT, x, y)
    def Ge(self, x, y): return self._bin(_GE, x, y)
    def And(self, x, y): return self._bin(_LAND, x, y)
    def Or(self, x, y): return self._bin(_LOR, x, y)
    def BitAnd(self, x, y): return self._bin(_AND, x, y)
    def BitOr(self, x, y): return self._bin(_OR, x, y)
    def BitXor(self, x, y): return self._bin(_XOR, x, y)
    def Shl(self, x, y): return self._bin(_SHL, x, y)
    def Shr(self, x, y): return self._bin(_SHR, x, y)
    def Neg(self, x): return self._un(_NEG, x)
    def Pos(self, x): return self._un(_POS, x)
    def Not(self, x): return self._un(_LNOT, x)
    def BitsNot(self, x): return self._un(_NOT, x)

    def Call(self, name, *args):
        return Call(name, *args)

    # ---- chains (pkg/builder.go:310-322)
    def Stmt(self):
        return StmtIter(self, _lib.lib().tca_stmt(self._h))

    def Build(self):
        if _lib.lib().tca_builder_build(self._h) != 0:
            raise BuildError(self._err())
        return Program(self)


def Select(cond, a, b):
    """pkg/expr.go:271-286."""
    bl = a.b
    return Expr(bl, _lib.lib().tca_expr_select(bl._h, cond.idx, a.idx, b.idx))


def Cast(e, t):
    """pkg/expr.go:293-306."""
    return Expr(e.b, _lib.lib().tca_expr_cast(e.b._h, e.idx, t))


def Call(name, *args):
    """pkg/expr.go:316-341: a registered pure scalar builtin. Raises where
    Go returns an error."""
    if not args:
        raise BuildError("function %s: no arguments" % name)
    b = args[0].b
    e = Expr(b, _lib.lib().tca_expr_call(b._h, name.encode(), len(args), _ints([a.idx for a in args])))
    err = e.Err()
    if err:
        raise BuildError(err)
    return e


# ---- typestate rungs (pkg/chain.go:16-26) ---------------------------------

def _arity(fn):
    try:
        sig = inspect.signature(fn)
    except (TypeError, ValueError):
        return None
    n = 0
    for p in sig.parameters.values():
        if p.kind == p.VAR_POSITIONAL:
            return None
        if p.kind in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD):
            n += 1
    return n


class _Rung:
    def __init__(self, b, chain):
        self.b, self.chain = b, chain

    def _fail(self):
        raise BuildError(self.b._err())

    def _map(self, ops, fn, piped):
        L = _lib.lib()
        want = len(ops) + (1 if piped else 0)
        got = _arity(fn)
        if got is not None and got != want:
            raise BuildError(
                "map: lambda arity mismatch: lambda takes %d argument(s), the map passes %d "
                "(piped value first, then operands)" % (got, want))
        arr = (tca_operand * max(1, len(ops)))()
        for i, o in enumerate(ops):
            if not isinstance(o, Operand):
                raise TypeError("map operands must be pkg.At(...) accesses")
            arr[i].tensor = o.t.idx if o.t.b is self.b else -1
            arr[i].rank = len(o.axes)
            for a, ax in enumerate(o.axes[:8]):
                arr[i].axes[a] = ax.idx if ax.b is self.b else -1
        params = (ctypes.c_int32 * (len(ops) + 1))()
        n = ctypes.c_uint32()
        if L.tca_chain_map_begin(self.b._h, self.chain, len(ops), arr, params, ctypes.byref(n)) != 0:
            self._fail()
        args = [Expr(self.b, params[i]) for i in range(n.value)]
        body = fn(*args)
        if not isinstance(body, Expr):
            raise BuildError("map: lambda must return a pkg.Expr")
        if L.tca_chain_map_end(self.b._h, self.chain, body.idx) != 0:
            self._fail()

    def _as(self, dims):
        ids = [d.idx if isinstance(d, Dim) and d.b is self.b else -1 for d in dims]
        _lib.lib().tca_chain_as(self.b._h, self.chain, len(ids), _ints(ids))

    def _reduce(self, init, fn):
        L = _lib.lib()
        if fn is None:
            raise BuildError("reduce: nil combiner")
        acc, now = ctypes.c_int32(), ctypes.c_int32()
        if L.tca_chain_reduce_begin(self.b._h, self.chain, init.idx, ctypes.byref(acc), ctypes.byref(now)) != 0:
            self._fail()
        body = fn(Expr(self.b, acc.value), Expr(self.b, now.value))
        if not isinstance(body, Expr):
            raise BuildError("reduce: combiner must return a pkg.Expr")
        if L.tca_chain_reduce_end(self.b._h, self.chain, body.idx) != 0:
            self._fail()

    def _store(self, t, axes):
        ids = [a.idx if isinstance(a, Dim) and a.b is self.b else -1 for a in axes]
        tid = t.idx if isinstance(t, Tensor) and t.b is self.b else -1
        if _lib.lib().tca_chain_store(self.b._h, self.chain, tid, len(ids), _ints(ids)) != 0:
            self._fail()
        return Stored(self.b, self.chain)


class StmtIter(_Rung):
    def Iter(self, *dims):
        ids = [d.idx if isinstance(d, Dim) and d.b is self.b else -1 for d in dims]
        _lib.lib().tca_chain_iter(self.b._h, self.chain, len(ids), _ints(ids))
        return RootMap(self.b, self.chain)


class RootMap(_Rung):
    def Map(self, ops, fn):
        self._map(ops, fn, piped=False)
        return RootAs(self.b, self.chain)


class RootAs(_Rung):
    def As(self, *dims):
        self._as(dims)
        return MidChain(self.b, self.chain)


class MidChain(_Rung):
    def Reduce(self, init, fn):
        self._reduce(init, fn)
        return AfterReduce(self.b, self.chain)

    def Store(self, t, *axes):
        """Elementwise store straight after the root map (extension over
        the reference v0 rungs, whose wall W1 forbids it)."""
        return self._store(t, axes)


class AfterReduce(_Rung):
    def Reduce(self, init, fn):
        self._reduce(init, fn)
        return AfterReduce(self.b, self.chain)

    def Map(self, ops, fn):
        self._map(ops, fn, piped=True)
        return AfterMap(self.b, self.chain)

    def Store(self, t, *axes):
        return self._store(t, axes)


class AfterMap(_Rung):
    def As(self, *dims):
        self._as(dims)
        return Tail(self.b, self.chain)


class Tail(_Rung):
    def Store(self, t, *axes):
        return self._store(t, axes)


class Stored(_Rung):
    pass


def NewBuilder(name):
    """pkg/builder.go:122."""
    return Builder(name)
