"""TEST INFRASTRUCTURE: seeded random row programs of the DSL, the emitter's
families exercised on programs nobody wrote by hand.

A program is a *spec* (plain Python data) and is built into a pkg.Program by
build(spec); tests evaluate the same spec on the CPU. Each program iterates
rows (one or two row axes, dynamic) and a column axis C (static or dynamic)
through a random sequence of statements in the shapes the reference's DSL
expresses with its chain rungs (pkg/chain.go:360-552):

- reduce : out[rows] = fold over C of map(expr), from init (sum / max / min,
           or wrapping sum / xor / umax / umin on u32), optionally followed
           by a piped map of the reduced value and row scalars
           (pkg/chain.go:301-316);
- rowmap : out[rows] = expr over row scalars: a per-row chain one level
           shallower than the row nest (internal/opt/gvn/gvn_test.go:458-518);
- map    : y[rows, C] = expr over row tiles, column vectors, row scalars.

Operands: row tiles x<k> [rows, C] (f32, bf16 cast to f32, u32, u8 cast to
u32), a column vector g [C], a row vector r [rows], scalar parameters s<k>,
literals, and the results of earlier reduce / rowmap statements (locals or
outputs). Expressions use + - * min max select(a < b) and, on f32, negation,
fabsf and a / (|b| + 1); on u32, xor, and, or. The value ranges the tests
feed keep every f32 sum exact (integer-valued terms, partial sums below
2^24), so any fold order gives the one correctly rounded result.
"""
import os
import random

from tcacomp_amd.pkg import EMIT_NO_FUSION, EMIT_NO_GEMM, TBF16, TF32, TU8, TU32, At, Call, Cast, NewBuilder, Select

F32_OPS = ["add", "sub", "mul", "max", "min", "sel", "neg", "abs", "div1"]
U32_OPS = ["add", "sub", "mul", "max", "min", "sel", "xor", "and", "or"]
F32_COMBS = ["sum", "max", "min"]
U32_COMBS = ["sum", "xor", "max", "min"]
F32_CONSTS = [-3.0, -2.0, -1.0, 1.0, 2.0, 3.0]
U32_CONSTS = [1, 3, 255, 0x9E3779B9]
# Static row lengths: register rows of every vector width, a row longer than
# the registers hold (streamed with a compile-time extent).
STATIC_C = [1, 3, 6, 64, 100, 1000, 1024, 4100, 20000, 70000]


class Spec:
    """One random program. `elem` is "f32" or "u32"; `c` the static row
    length (0: dynamic); `outer` the number of row axes (1 or 2); `tiles`
    [(name, storage elem)], `col`/`row` whether g [C] / r [rows] exist;
    `scalars` [(name, value)]; `stmts` in program order."""

    def __init__(self, name, elem, c, outer, tiles, col, row, scalars, stmts):
        self.name, self.elem, self.c, self.outer = name, elem, c, outer
        self.tiles, self.col, self.row, self.scalars, self.stmts = tiles, col, row, scalars, stmts

    def outputs(self):
        return [s["out"] for s in self.stmts if not s["local"]]


def leaves(e, out=None):
    """Operand names an expression reads, in first-use order."""
    out = [] if out is None else out
    if e[0] == "leaf":
        if e[1] not in out:
            out.append(e[1])
    elif e[0] != "const":
        for a in e[1:]:
            leaves(a, out)
    return out


def _expr(rng, elem, pool, depth, allow_div, max_mul):
    """A random tree over `pool` (operand names) of at most `depth` levels
    with at most `max_mul` multiplications."""
    consts = F32_CONSTS if elem == "f32" else U32_CONSTS
    if depth == 0 or rng.random() < 0.25:
        if pool and rng.random() < 0.85:
            return ("leaf", rng.choice(pool))
        return ("const", rng.choice(consts))
    ops = list(F32_OPS if elem == "f32" else U32_OPS)
    if not allow_div and "div1" in ops:
        ops.remove("div1")
    if max_mul <= 0:
        ops.remove("mul")
    op = rng.choice(ops)
    if op in ("neg", "abs"):
        return (op, _expr(rng, elem, pool, depth - 1, allow_div, max_mul))
    used = 1 if op == "mul" else 0
    n = 4 if op == "sel" else 2
    budget = max_mul - used
    args = []
    for _ in range(n):
        a = _expr(rng, elem, pool, depth - 1, allow_div, budget)
        budget -= count_mul(a)
        args.append(a)
    return (op,) + tuple(args)


def count_mul(e):
    if e[0] in ("leaf", "const"):
        return 0
    return (1 if e[0] == "mul" else 0) + sum(count_mul(a) for a in e[1:])


def _has_leaf(e):
    return bool(leaves(e))


def generate(seed, elem, dynamic):
    """The spec of random program `seed` (deterministic)."""
    rng = random.Random(0x7CA0C0DE ^ (seed * 0x9E3779B1))
    outer = 2 if rng.random() < 0.3 else 1
    c = 0 if dynamic else rng.choice(STATIC_C)
    ntiles = rng.choice([1, 1, 2])
    if elem == "f32":
        tiles = [("x0", rng.choice(["f32", "f32", "bf16"]))] + [("x%d" % k, "f32") for k in range(1, ntiles)]
        scalars = [("s%d" % k, rng.choice([-1.0, 2.0, 3.0])) for k in range(rng.choice([0, 1, 2]))]
    else:
        tiles = [("x0", rng.choice(["u32", "u32", "u8"]))] + [("x%d" % k, "u32") for k in range(1, ntiles)]
        scalars = [("s%d" % k, rng.choice([3, 0x01000193, 0xFFFFFFFF])) for k in range(rng.choice([0, 1]))]
    col = rng.random() < 0.5
    row = rng.random() < 0.4
    tile_pool = [t for t, _ in tiles] + (["g"] if col else [])
    sc_pool = [s for s, _ in scalars]
    bounded = ["r"] if row else []  # row scalars whose magnitude the inputs bound (f32 exactness)
    any_rows = list(bounded)
    stmts = []
    nred = rng.choice([1, 1, 2, 2, 3])
    plan = ["reduce"] * nred
    if rng.random() < 0.4:
        plan.append("rowmap")
    nmap = rng.choice([0, 1, 1, 2])
    for _ in range(nmap):
        plan.insert(rng.randrange(1, len(plan) + 1), "map")
    # A map before any reduction still needs a reduction after it: keep the first statement a reduce.
    combs = F32_COMBS if elem == "f32" else U32_COMBS
    for i, kind in enumerate(plan):
        if kind == "reduce":
            pool = tile_pool + (bounded if elem == "f32" else any_rows) + sc_pool
            e = _expr(rng, elem, pool, 2, False, 1)
            if not any(l in tile_pool for l in leaves(e)):
                e = ("add", ("leaf", rng.choice([t for t, _ in tiles])), e)
            comb = rng.choice(combs)
            piped = None
            if rng.random() < 0.4:
                ppool = ["v"] + any_rows + sc_pool
                piped = _expr(rng, elem, ppool, 2, elem == "f32", 2)
                if "v" not in leaves(piped):
                    piped = ("add", ("leaf", "v"), piped)
            st = {"kind": "reduce", "expr": e, "comb": comb, "piped": piped, "out": "l%d" % i,
                  "local": rng.random() < 0.6}
            if not st["local"]:
                st["out"] = "o%d" % i
            stmts.append(st)
            any_rows.append(st["out"])
            if comb in ("max", "min") and piped is None:
                bounded.append(st["out"])
        elif kind == "rowmap":
            pool = any_rows + sc_pool
            if not pool:
                continue
            e = _expr(rng, elem, pool, 2, elem == "f32", 2)
            if not _has_leaf(e):
                e = ("add", ("leaf", rng.choice(any_rows or pool)), e)
            if not any(l in any_rows for l in leaves(e)):
                if not any_rows:
                    continue
                e = ("add", ("leaf", rng.choice(any_rows)), e)
            local = rng.random() < 0.5
            st = {"kind": "rowmap", "expr": e, "out": ("l%d" if local else "o%d") % i, "local": local}
            stmts.append(st)
            any_rows.append(st["out"])
        else:
            pool = tile_pool + any_rows + sc_pool
            e = _expr(rng, elem, pool, 3, elem == "f32", 2)
            if not any(l in tile_pool for l in leaves(e)):
                e = ("add", ("leaf", rng.choice([t for t, _ in tiles])), e)
            stmts.append({"kind": "map", "expr": e, "out": "y%d" % i, "local": False})
    # Every local is read by a later statement; otherwise it becomes an output.
    for i, st in enumerate(stmts):
        if not st["local"]:
            continue
        later = set()
        for s2 in stmts[i + 1:]:
            later.update(leaves(s2["expr"]))
            if s2.get("piped") is not None:
                later.update(leaves(s2["piped"]))
        if st["out"] not in later:
            st["local"] = False
            new = "o" + st["out"][1:]
            for s2 in stmts[i + 1:]:
                s2["expr"] = _rename(s2["expr"], st["out"], new)
                if s2.get("piped") is not None:
                    s2["piped"] = _rename(s2["piped"], st["out"], new)
            st["out"] = new
    name = "rand_%s_%s_%d" % (elem, "dyn" if dynamic else "c%d" % c, seed)
    return Spec(name, elem, c, outer, tiles, col, row, scalars, stmts)


def generate_rowchain(seed, elem, dynamic):
    """A random program of chained reductions over rows [B, R] (one in ten
    over [R]): a `chain` statement (Reduce over C, then Reduce over R, in
    one chain: pkg/chain.go:262 twice) or a `reduce` into a local followed
    by a `rowreduce` of it over R (the same pattern written as two chains),
    with an optional piped map over the result; then possibly a second
    such statement or a plain row reduction. Both store one value per
    segment B (a scalar over [R])."""
    rng = random.Random(0x3C6EF372 ^ (seed * 0x9E3779B1))
    outer = 1 if rng.random() < 0.1 else 2
    c = 0 if dynamic else rng.choice(STATIC_C[:8])
    if elem == "f32":
        tiles = [("x0", rng.choice(["f32", "f32", "bf16"]))]
        scalars = [("s%d" % k, rng.choice([-1.0, 2.0, 3.0])) for k in range(rng.choice([0, 1]))]
    else:
        tiles = [("x0", rng.choice(["u32", "u32", "u8"]))]
        scalars = [("s%d" % k, rng.choice([3, 0xFFFFFFFF])) for k in range(rng.choice([0, 1]))]
    col = rng.random() < 0.5
    row = rng.random() < 0.3
    pool = ["x0"] + (["g"] if col else []) + (["r"] if row else [])
    sc_pool = [n for n, _ in scalars]
    combs = F32_COMBS if elem == "f32" else U32_COMBS
    stmts = []
    for i in range(rng.choice([1, 1, 2])):
        e = _expr(rng, elem, pool + sc_pool, 2, False, 1)
        if "x0" not in leaves(e):
            e = ("add", ("leaf", "x0"), e)
        piped = None
        if rng.random() < 0.4:
            piped = _expr(rng, elem, ["v"] + sc_pool, 2, False, 1)
            if "v" not in leaves(piped):
                piped = ("add", ("leaf", "v"), piped)
        if rng.random() < 0.6:
            stmts.append({"kind": "chain", "expr": e, "comb": rng.choice(combs), "comb2": rng.choice(combs),
                          "piped": piped, "out": "o%d" % i, "local": False})
        else:
            loc = "l%d" % i
            stmts.append({"kind": "reduce", "expr": e, "comb": rng.choice(combs), "piped": None, "out": loc,
                          "local": True})
            e2 = _expr(rng, elem, [loc] + sc_pool, 2, False, 1)
            if loc not in leaves(e2):
                e2 = ("add", ("leaf", loc), e2)
            stmts.append({"kind": "rowreduce", "expr": e2, "comb": rng.choice(combs), "piped": piped,
                          "out": "o%d" % i, "local": False})
    if rng.random() < 0.3:
        e = _expr(rng, elem, pool + sc_pool, 2, False, 1)
        if "x0" not in leaves(e):
            e = ("add", ("leaf", "x0"), e)
        stmts.append({"kind": "reduce", "expr": e, "comb": rng.choice(combs), "piped": None, "out": "o9",
                      "local": False})
    name = "rowc_%s_%s_%d" % (elem, "dyn" if dynamic else "c%d" % c, seed)
    return Spec(name, elem, c, outer, tiles, col, row, scalars, stmts)


def _rename(e, old, new):
    if e[0] == "leaf":
        return ("leaf", new) if e[1] == old else e
    if e[0] == "const":
        return e
    return (e[0],) + tuple(_rename(a, old, new) for a in e[1:])


_ELEM = {"f32": TF32, "bf16": TBF16, "u32": TU32, "u8": TU8}


def _lower(b, elem, e, env):
    """Builder expression of tree `e`; `env` maps operand names to Exprs."""
    k = e[0]
    if k == "leaf":
        return env[e[1]]
    if k == "const":
        return b.Float32(e[1]) if elem == "f32" else b.UInt32(e[1])
    a = [_lower(b, elem, x, env) for x in e[1:]]
    if k == "add":
        return b.Add(a[0], a[1])
    if k == "sub":
        return b.Sub(a[0], a[1])
    if k == "mul":
        return b.Mul(a[0], a[1])
    if k == "max":
        return Call("fmaxf" if elem == "f32" else "umax", a[0], a[1])
    if k == "min":
        return Call("fminf" if elem == "f32" else "umin", a[0], a[1])
    if k == "sel":
        return Select(b.Lt(a[0], a[1]), a[2], a[3])
    if k == "neg":
        return b.Neg(a[0])
    if k == "abs":
        return Call("fabsf", a[0])
    if k == "div1":
        return b.Div(a[0], b.Add(Call("fabsf", a[1]), b.Float32(1.0)))
    if k == "xor":
        return b.BitXor(a[0], a[1])
    if k == "and":
        return b.BitAnd(a[0], a[1])
    if k == "or":
        return b.BitOr(a[0], a[1])
    raise ValueError(k)


def build(spec):
    """The pkg.Program of a spec."""
    if getattr(spec, "kind", "row") == "grid":
        return _build_grid(spec)
    b = NewBuilder(spec.name)
    rows = [b.Dim("B", 0), b.Dim("R", 0)] if spec.outer == 2 else [b.Dim("R", 0)]
    C = b.Dim("C", 0) if spec.c == 0 else b.Dim("e%d" % spec.c, spec.c)
    full = rows + [C]
    work = TF32 if spec.elem == "f32" else TU32
    ops = {}  # operand name -> (tensor, axes, needs a cast to the work type)
    for t, st in spec.tiles:
        ops[t] = (b.Tensor(t, _ELEM[st], *full), full, st != spec.elem)
    if spec.col:
        ops["g"] = (b.Tensor("g", work, C), [C], False)
    if spec.row:
        ops["r"] = (b.Tensor("r", work, *rows), rows, False)
    scal = {n: b.ScalarParam(n, work) for n, _ in spec.scalars}
    for st in spec.stmts:
        if st["kind"] == "map":
            ops[st["out"]] = (b.Tensor(st["out"], work, *full), full, False)
        elif st["kind"] in ("chain", "rowreduce"):  # one value per segment rows[:-1]
            ops[st["out"]] = (b.Tensor(st["out"], work, *rows[:-1]), rows[:-1], False)
        elif st["local"]:
            ops[st["out"]] = (b.Local(st["out"], work, *rows), rows, False)
        else:
            ops[st["out"]] = (b.Tensor(st["out"], work, *rows), rows, False)

    def operands(e, extra=()):
        names = [n for n in leaves(e) if n not in scal and n not in extra]
        return names, [At(ops[n][0], *ops[n][1]) for n in names]

    def fn_for(e, names, pre=()):
        def f(*params):
            env = dict(zip(list(pre) + names, params))
            for n in names:
                if ops[n][2]:
                    env[n] = Cast(env[n], work)
            env.update(scal)
            return _lower(b, spec.elem, e, env)
        return f

    for st in spec.stmts:
        out_t = ops[st["out"]][0]
        if st["kind"] == "reduce":
            names, operand_list = operands(st["expr"])
            chain = b.Stmt().Iter(*full).Map(operand_list, fn_for(st["expr"], names)).As(*full)
            init, comb = _init_comb(b, spec.elem, st["comb"])
            chain = chain.Reduce(init, comb)
            if st["piped"] is not None:
                pnames, plist = operands(st["piped"], extra=("v",))
                chain = chain.Map(plist, fn_for(st["piped"], pnames, pre=("v",))).As(*rows)
            chain.Store(out_t, *rows)
        elif st["kind"] == "rowmap":
            names, operand_list = operands(st["expr"])
            b.Stmt().Iter(*rows).Map(operand_list, fn_for(st["expr"], names)).As(*rows).Store(out_t, *rows)
        elif st["kind"] in ("chain", "rowreduce"):
            names, operand_list = operands(st["expr"])
            it = full if st["kind"] == "chain" else rows
            chain = b.Stmt().Iter(*it).Map(operand_list, fn_for(st["expr"], names)).As(*it)
            init, comb = _init_comb(b, spec.elem, st["comb"])
            chain = chain.Reduce(init, comb)
            if st["kind"] == "chain":  # a second reduction in the same chain: over the last row axis
                init2, comb2 = _init_comb(b, spec.elem, st["comb2"])
                chain = chain.Reduce(init2, comb2)
            if st["piped"] is not None:
                pnames, plist = operands(st["piped"], extra=("v",))
                chain = chain.Map(plist, fn_for(st["piped"], pnames, pre=("v",))).As(*rows[:-1])
            chain.Store(out_t, *rows[:-1])
        else:
            names, operand_list = operands(st["expr"])
            b.Stmt().Iter(*full).Map(operand_list, fn_for(st["expr"], names)).As(*full).Store(out_t, *full)
    return b.Build()


def _init_comb(b, elem, comb):
    if elem == "f32":
        if comb == "sum":
            return b.Float32(0.0), lambda acc, v: b.Add(acc, v)
        if comb == "max":
            return b.Neg(b.Float32(float("inf"))), lambda acc, v: Call("fmaxf", acc, v)
        return b.Float32(float("inf")), lambda acc, v: Call("fminf", acc, v)
    if comb == "sum":
        return b.UInt32(0), lambda acc, v: b.Add(acc, v)
    if comb == "xor":
        return b.UInt32(0), lambda acc, v: b.BitXor(acc, v)
    if comb == "max":
        return b.UInt32(0), lambda acc, v: Call("umax", acc, v)
    return b.UInt32(0xFFFFFFFF), lambda acc, v: Call("umin", acc, v)


class GridSpec:
    """One random grid program over [R, C]: elementwise maps (`map` stores
    y [R, C], `tmap` stores the transposed z [C, R]) and reductions over the
    leading axis (`colreduce`: out [C] = fold over R, the iteration order
    written As(C, R) so the reduce drops R). Operands: row tiles x<k> [R, C],
    a transposed tile xt [C, R] read at (c, r), g [C], r [R], scalars, and
    (chain programs) the results of earlier colreduce statements, read at
    their own column — a later reduction reading an earlier one is a
    dependent column nest (a variance reading its mean). A statement with
    "local": True stores a local that only later statements read."""

    kind = "grid"

    def __init__(self, name, elem, c, tiles, trans, col, row, scalars, stmts, batch=False):
        self.name, self.elem, self.c, self.tiles, self.trans = name, elem, c, tiles, trans
        self.col, self.row, self.scalars, self.stmts = col, row, scalars, stmts
        self.batch = batch  # a leading batch axis B: x0 [B, R, C], xt [B, C, R], outputs per batch

    def outputs(self):
        return [s["out"] for s in self.stmts if not s.get("local")]


def generate_grid(seed, elem, dynamic, batch=False):
    """The spec of random grid program `seed` (deterministic); `batch` adds a
    leading batch axis to every tile and output (g and r stay [C] and [R])."""
    rng = random.Random(0x6A09E667 ^ (seed * 0x9E3779B1))
    c = 0 if dynamic else rng.choice(STATIC_C[:8])
    if elem == "f32":
        tiles = [("x0", rng.choice(["f32", "f32", "bf16"]))]
        scalars = [("s%d" % k, rng.choice([-1.0, 2.0, 3.0])) for k in range(rng.choice([0, 1]))]
    else:
        tiles = [("x0", rng.choice(["u32", "u8"]))]
        scalars = [("s%d" % k, rng.choice([3, 0xFFFFFFFF])) for k in range(rng.choice([0, 1]))]
    trans = rng.random() < 0.6
    col = rng.random() < 0.5
    row = rng.random() < 0.5
    pool = ["x0"] + (["xt"] if trans else []) + (["g"] if col else []) + (["r"] if row else [])
    sc_pool = [n for n, _ in scalars]
    stmts = []
    for i in range(rng.choice([1, 2, 3])):
        kind = rng.choice(["map", "map", "tmap", "colreduce"])
        if kind == "colreduce":
            e = _expr(rng, elem, pool + sc_pool, 2, False, 1)
            comb = rng.choice(F32_COMBS if elem == "f32" else U32_COMBS)
            piped = None
            if rng.random() < 0.4:
                piped = _expr(rng, elem, ["v"] + (["g"] if col else []) + sc_pool, 2, elem == "f32", 2)
                if "v" not in leaves(piped):
                    piped = ("add", ("leaf", "v"), piped)
        else:
            e = _expr(rng, elem, pool + sc_pool, 3, elem == "f32", 2)
            comb = piped = None
        if not any(l in ("x0", "xt") for l in leaves(e)):
            e = ("add", ("leaf", rng.choice(["x0", "xt"] if trans else ["x0"])), e)
        stmts.append({"kind": kind, "expr": e, "comb": comb, "piped": piped, "out": "%s%d" % (kind[0], i)})
    name = "grid%s_%s_%s_%d" % ("3" if batch else "", elem, "dyn" if dynamic else "c%d" % c, seed)
    return GridSpec(name, elem, c, tiles, trans, col, row, scalars, stmts, batch)


def generate_colchain(seed, elem, dynamic, batch=False):
    """A random grid program of dependent column reductions: a first
    colreduce over the tiles, then colreduces (at least one), maps and
    piped maps that read earlier colreduce results at their own column.
    Combining with an earlier result is mostly + and -, with no division,
    so f32 values stay integers and the tests' input ranges keep every sum
    exact. Each result a later statement reads is a local half the time."""
    rng = random.Random(0xBB67AE85 ^ (seed * 0x9E3779B1))
    c = 0 if dynamic else rng.choice(STATIC_C[:8])
    if elem == "f32":
        tiles = [("x0", rng.choice(["f32", "f32", "bf16"]))]
        scalars = [("s%d" % k, rng.choice([-1.0, 2.0, 3.0])) for k in range(rng.choice([0, 1]))]
    else:
        tiles = [("x0", rng.choice(["u32", "u8"]))]
        scalars = [("s%d" % k, rng.choice([3, 0xFFFFFFFF])) for k in range(rng.choice([0, 1]))]
    trans = rng.random() < 0.4
    col = rng.random() < 0.5
    row = rng.random() < 0.4
    pool = ["x0"] + (["xt"] if trans else []) + (["g"] if col else []) + (["r"] if row else [])
    sc_pool = [n for n, _ in scalars]
    stmts, prev = [], []
    n = rng.choice([2, 3, 4])
    for i in range(n):
        kind = "colreduce" if i < 2 else rng.choice(["colreduce", "colreduce", "map"])
        e = _expr(rng, elem, pool + sc_pool, 2, False, 1)
        if not any(l in ("x0", "xt") for l in leaves(e)):
            e = ("add", ("leaf", rng.choice(["x0", "xt"] if trans else ["x0"])), e)
        if prev and (i == 1 or rng.random() < 0.7):
            op = rng.choice(["add", "sub", "add", "sub"] + (["mul"] if count_mul(e) == 0 else []))
            e = (op, e, ("leaf", rng.choice(prev)))
        comb = piped = None
        if kind == "colreduce":
            comb = rng.choice(F32_COMBS if elem == "f32" else U32_COMBS)
            if rng.random() < 0.4:
                piped = _expr(rng, elem, ["v"] + (["g"] if col else []) + sc_pool + prev, 2, False, 1)
                if "v" not in leaves(piped):
                    piped = ("add", ("leaf", "v"), piped)
        stmts.append({"kind": kind, "expr": e, "comb": comb, "piped": piped, "out": "%s%d" % (kind[0], i),
                      "local": False})
        if kind == "colreduce":
            prev.append("c%d" % i)
    read = set()
    for st in stmts:
        read.update(leaves(st["expr"]))
        if st["piped"] is not None:
            read.update(leaves(st["piped"]))
    for st in stmts:
        if st["out"] in read and rng.random() < 0.5:
            st["local"] = True
    name = "gridc%s_%s_%s_%d" % ("3" if batch else "", elem, "dyn" if dynamic else "c%d" % c, seed)
    return GridSpec(name, elem, c, tiles, trans, col, row, scalars, stmts, batch)


def _build_grid(spec):
    b = NewBuilder(spec.name)
    B = [b.Dim("B", 0)] if spec.batch else []
    R = b.Dim("R", 0)
    C = b.Dim("C", 0) if spec.c == 0 else b.Dim("e%d" % spec.c, spec.c)
    work = TF32 if spec.elem == "f32" else TU32
    ops = {}  # operand name -> (tensor, subscript axes, cast to the work type)
    x0_storage = spec.tiles[0][1]
    ops["x0"] = (b.Tensor("x0", _ELEM[x0_storage], *(B + [R, C])), B + [R, C], x0_storage != spec.elem)
    if spec.trans:
        ops["xt"] = (b.Tensor("xt", work, *(B + [C, R])), B + [C, R], False)
    if spec.col:
        ops["g"] = (b.Tensor("g", work, C), [C], False)
    if spec.row:
        ops["r"] = (b.Tensor("r", work, R), [R], False)
    scal = {n: b.ScalarParam(n, work) for n, _ in spec.scalars}
    outs = {}
    for st in spec.stmts:
        dims = {"map": B + [R, C], "tmap": B + [C, R], "colreduce": B + [C]}[st["kind"]]
        outs[st["out"]] = (b.Local if st.get("local") else b.Tensor)(st["out"], work, *dims)
        if st["kind"] == "colreduce":  # later statements read it at (batch, column)
            ops[st["out"]] = (outs[st["out"]], B + [C], False)

    def fn_for(e, names, pre=()):
        def f(*params):
            env = dict(zip(list(pre) + names, params))
            for n in names:
                if ops[n][2]:
                    env[n] = Cast(env[n], work)
            env.update(scal)
            return _lower(b, spec.elem, e, env)
        return f

    for st in spec.stmts:
        names = [n for n in leaves(st["expr"]) if n not in scal]
        operand_list = [At(ops[n][0], *ops[n][1]) for n in names]
        chain = b.Stmt().Iter(*(B + [R, C])).Map(operand_list, fn_for(st["expr"], names))
        if st["kind"] == "map":
            chain.As(*(B + [R, C])).Store(outs[st["out"]], *(B + [R, C]))
        elif st["kind"] == "tmap":
            chain.As(*(B + [R, C])).Store(outs[st["out"]], *(B + [C, R]))
        else:
            init, comb = _init_comb(b, spec.elem, st["comb"])
            chain = chain.As(*(B + [C, R])).Reduce(init, comb)
            if st["piped"] is not None:
                pnames = [n for n in leaves(st["piped"]) if n not in scal and n != "v"]
                chain = chain.Map([At(ops[n][0], *ops[n][1]) for n in pnames],
                                  fn_for(st["piped"], pnames, pre=("v",))).As(*(B + [C]))
            chain.Store(outs[st["out"]], *(B + [C]))
    return b.Build()


# The registered random programs: (elem, dynamic row length, seed).
PROGRAMS = ([("f32", True, s) for s in range(10)] + [("f32", False, s) for s in range(10, 20)] +
            [("u32", True, s) for s in range(20, 25)] + [("u32", False, s) for s in range(25, 30)])


# Random programs also built with fusion off (the generic family), so the
# same program and data check both lowerings.
GENERIC_TOO = {"rand_f32_dyn_0", "rand_f32_dyn_1", "rand_f32_c3_12", "rand_f32_c1000_15", "rand_u32_dyn_21",
               "rand_u32_c1000_26"}


# Random grid programs: (elem, dynamic row length, seed).
GRID_PROGRAMS = ([("f32", True, s) for s in range(40, 46)] + [("f32", False, s) for s in range(46, 50)] +
                 [("u32", True, s) for s in range(50, 53)] + [("u32", False, s) for s in range(53, 55)])


# Random grid programs with a leading batch axis: (elem, dynamic row length, seed).
GRID3_PROGRAMS = ([("f32", True, s) for s in range(60, 66)] + [("f32", False, s) for s in range(66, 68)] +
                  [("u32", True, s) for s in range(68, 70)])


# Random dependent column programs: (elem, dynamic row length, batch axis, seed).
COLCHAIN_PROGRAMS = ([("f32", True, False, s) for s in range(80, 86)] + [("f32", False, False, s) for s in (86, 87)] +
                     [("u32", True, False, s) for s in (88, 89)] + [("u32", False, False, 90)] +
                     [("f32", True, True, s) for s in (91, 92)] + [("u32", True, True, 93)])


# Random chained-reduction programs over rows: (elem, dynamic row length, seed).
ROWCHAIN_PROGRAMS = ([("f32", True, s) for s in range(100, 106)] + [("f32", False, s) for s in (106, 107)] +
                     [("u32", True, s) for s in (108, 109, 110)] + [("u32", False, 111)])


# Further seeds of every generator for a longer search, included when
# TCA_RANDPROG_EXTENDED=1 at build time (build() prebuilds them) and at test
# time (tests/test_gpu_random.py runs them): 277 programs.
EXTENDED = {
    "row": ([("f32", True, s) for s in range(1000, 1060)] + [("f32", False, s) for s in range(1100, 1140)] +
            [("u32", True, s) for s in range(1200, 1230)] + [("u32", False, s) for s in range(1300, 1320)]),
    "grid": ([("f32", True, s) for s in range(2000, 2030)] + [("f32", False, s) for s in range(2030, 2040)] +
             [("u32", True, s) for s in range(2040, 2050)]),
    "grid3": [("f32", True, s) for s in range(2100, 2110)] + [("u32", True, s) for s in range(2110, 2115)],
    "colchain": ([("f32", True, False, s) for s in range(3000, 3020)] +
                 [("u32", True, False, s) for s in range(3020, 3026)] + [("f32", True, True, s) for s in range(3030, 3036)]),
    "rowchain": [("f32", True, s) for s in range(4000, 4020)] + [("u32", True, s) for s in range(4020, 4030)],
}


def specs():
    rows, grids, grid3s, colchains, rowchains = (PROGRAMS, GRID_PROGRAMS, GRID3_PROGRAMS, COLCHAIN_PROGRAMS,
                                                 ROWCHAIN_PROGRAMS)
    if os.environ.get("TCA_RANDPROG_EXTENDED") == "1":
        rows, grids, grid3s = rows + EXTENDED["row"], grids + EXTENDED["grid"], grid3s + EXTENDED["grid3"]
        colchains, rowchains = colchains + EXTENDED["colchain"], rowchains + EXTENDED["rowchain"]
    return ([generate(seed, elem, dyn) for elem, dyn, seed in rows] +
            [generate_grid(seed, elem, dyn) for elem, dyn, seed in grids] +
            [generate_grid(seed, elem, dyn, True) for elem, dyn, seed in grid3s] +
            [generate_colchain(seed, elem, dyn, batch) for elem, dyn, batch, seed in colchains] +
            [generate_rowchain(seed, elem, dyn) for elem, dyn, seed in rowchains])


def all_builds():
    """(name, program factory, emit flags) of every code object the random
    programs need: build() prebuilds them beside the product's programs so a
    GPU run never compiles."""
    out = []
    for spec in specs():
        out.append((spec.name, (lambda s=spec: build(s)), 0))
        if spec.name in GENERIC_TOO:
            out.append((spec.name + "_generic", (lambda s=spec: build(s)), EMIT_NO_FUSION | EMIT_NO_GEMM))
    return out
