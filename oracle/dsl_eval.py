"""TEST INFRASTRUCTURE ONLY: CPU evaluation of the random row and grid
programs of tests/randprog.py (the checker of tests/test_gpu_random.py,
never the thing measured or shipped; only tests/ may import it).

The DSL semantics restated here, per statement:
- a chain's root map is evaluated per element of its iteration space
  (pkg/chain.go:360-420), operands bound by subscript (pkg/chain.go:153-176);
- Reduce drops the last live axis (pkg/chain.go:262) and folds
  acc = fn(acc, v) starting from init, once per output; an empty reduce
  yields init (runtime/tca/reducer.h:36-57; design/tca.md:299, :711);
- a second Reduce in the same chain (pkg/chain.go:262 applied again)
  drops the next live axis, folding the first one's results from its own
  init, once per remaining output;
- the piped map after a reduce sees the reduced value first, then its own
  operands, over the remaining axes (pkg/chain.go:301-316);
- stores write the chain's result at its store subscripts
  (pkg/chain.go:326-350); locals are read back by later chains.
Scalar arithmetic is IEEE float32 (numpy's float32 ufuncs are correctly
rounded, as the device's basic operations are under -ffp-contract=off) or
wrapping uint32.

The fold order of a float sum is not reproduced: evaluate() reports
whether every sum is exact (integer-valued finite terms, sum of their
magnitudes below 2^24 per output; infinities and NaNs fix the result in
any order), in which case every order gives the same float32 and the
device must match it exactly. evaluate_scalar() is a brute-force element
loop in the reference's sequential fold order, used to pin evaluate() on
tiny inputs.
"""
import numpy as np

EXACT_LIMIT = float(1 << 24)


def _f32(v):
    return np.float32(v)


def _binop(op, elem, a, b):
    if op == "add":
        return a + b
    if op == "sub":
        return a - b
    if op == "mul":
        return a * b
    if op == "max":
        return np.fmax(a, b) if elem == "f32" else np.maximum(a, b)
    if op == "min":
        return np.fmin(a, b) if elem == "f32" else np.minimum(a, b)
    if op == "div1":
        return a / (np.abs(b) + _f32(1.0))
    if op == "xor":
        return a ^ b
    if op == "and":
        return a & b
    if op == "or":
        return a | b
    raise ValueError(op)


def _eval(e, env, elem):
    k = e[0]
    if k == "leaf":
        return env[e[1]]
    if k == "const":
        return _f32(e[1]) if elem == "f32" else np.uint32(e[1])
    a = [_eval(x, env, elem) for x in e[1:]]
    if k == "sel":
        return np.where(a[0] < a[1], a[2], a[3])
    if k == "neg":
        return -a[0]
    if k == "abs":
        return np.abs(a[0])
    return _binop(k, elem, a[0], a[1])


def _init(elem, comb):
    if elem == "f32":
        return {"sum": _f32(0.0), "max": _f32(-np.inf), "min": _f32(np.inf)}[comb]
    return np.uint32({"sum": 0, "xor": 0, "max": 0, "min": 0xFFFFFFFF}[comb])


def _reduce(elem, comb, terms):
    """Reduced values of `terms` over the last axis, and whether a float sum
    is exact (order-independent)."""
    init = _init(elem, comb)
    if elem == "f32":
        if comb == "sum":
            # Non-finite terms fix the sum (an infinity, or NaN) in any
            # order; the finite ones must be integers summing below 2^24.
            t = terms.astype(np.float64)
            tf = np.where(np.isfinite(t), t, 0.0)
            exact = bool(np.all(np.floor(tf) == tf) and np.all(np.abs(tf).sum(axis=-1) < EXACT_LIMIT))
            return (init + t.sum(axis=-1)).astype(np.float32), exact
        f = np.fmax if comb == "max" else np.fmin
        if terms.shape[-1] == 0:
            return np.full(terms.shape[:-1], init, np.float32), True
        return f(init, f.reduce(terms, axis=-1)).astype(np.float32), True
    if comb == "sum":
        return (terms.astype(np.uint64).sum(axis=-1) % (1 << 32)).astype(np.uint32), True
    if comb == "xor":
        return np.bitwise_xor.reduce(terms, axis=-1).astype(np.uint32), True
    if terms.shape[-1] == 0:
        return np.full(terms.shape[:-1], init, np.uint32), True
    f = np.maximum if comb == "max" else np.minimum
    return f(init, f.reduce(terms, axis=-1)).astype(np.uint32), True


def evaluate(spec, tiles, col, row, scalars):
    """Expected outputs of `spec`. tiles: {name: array [rows..., C]} already
    in the work type (f32 or u32: bf16 and u8 storage widens exactly); col:
    g [C] or None; row: r [rows...] or None; scalars: {name: value}.
    Returns ({output name: array}, every float sum exact)."""
    elem = spec.elem
    dt = np.float32 if elem == "f32" else np.uint32
    first = next(iter(tiles.values()))
    full = first.shape
    rows = full[:-1]
    rowvals = {}
    if row is not None:
        rowvals["r"] = row.astype(dt)
    scal = {n: (_f32(v) if elem == "f32" else np.uint32(v)) for n, v in scalars.items()}
    outs, exact = {}, True
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        for st in spec.stmts:
            if st["kind"] in ("chain", "rowreduce"):
                # chain: fold over C, then over the last row axis (pkg/chain.go:262 twice);
                # rowreduce: fold row values over the last row axis. Both store [rows[:-1]].
                if st["kind"] == "chain":
                    env = {n: a.astype(dt) for n, a in tiles.items()}
                    if col is not None:
                        env["g"] = col.astype(dt)
                    env.update({n: v[..., None] for n, v in rowvals.items()})
                    env.update(scal)
                    val = np.broadcast_to(np.asarray(_eval(st["expr"], env, elem), dt), full)
                    inner, ok = _reduce(elem, st["comb"], val)
                    red, ok2 = _reduce(elem, st["comb2"], inner)
                else:
                    env = dict(rowvals)
                    env.update(scal)
                    val = np.broadcast_to(np.asarray(_eval(st["expr"], env, elem), dt), rows)
                    red, ok = _reduce(elem, st["comb"], np.array(val, dt))
                    ok2 = True
                exact = exact and ok and ok2
                if st["piped"] is not None:
                    penv = dict(scal)
                    penv["v"] = red
                    red = np.broadcast_to(np.asarray(_eval(st["piped"], penv, elem), dt), rows[:-1])
                outs[st["out"]] = np.array(red, dt)
                continue
            if st["kind"] in ("reduce", "map"):
                env = {n: a.astype(dt) for n, a in tiles.items()}
                if col is not None:
                    env["g"] = col.astype(dt)
                env.update({n: v[..., None] for n, v in rowvals.items()})
                env.update(scal)
                val = np.broadcast_to(np.asarray(_eval(st["expr"], env, elem), dt), full)
                if st["kind"] == "map":
                    outs[st["out"]] = np.array(val, dt)
                    continue
                red, ok = _reduce(elem, st["comb"], val)
                exact = exact and ok
                if st["piped"] is not None:
                    penv = dict(rowvals)
                    penv.update(scal)
                    penv["v"] = red
                    red = np.broadcast_to(np.asarray(_eval(st["piped"], penv, elem), dt), rows)
                res = np.array(red, dt)
            else:
                env = dict(rowvals)
                env.update(scal)
                res = np.array(np.broadcast_to(np.asarray(_eval(st["expr"], env, elem), dt), rows), dt)
            rowvals[st["out"]] = res
            if not st["local"]:
                outs[st["out"]] = res
    return outs, exact


def evaluate_scalar(spec, tiles, col, row, scalars):
    """Brute force: every output element computed alone, every reduce folded
    sequentially from init in ascending index order (runtime/tca/reducer.h:
    36-57), with float32 / uint32 scalars. For tiny shapes only."""
    elem = spec.elem
    cast = _f32 if elem == "f32" else np.uint32
    first = next(iter(tiles.values()))
    full = first.shape
    rows = full[:-1]
    C = full[-1]
    rowvals = {}
    if row is not None:
        rowvals["r"] = {idx: cast(row[idx]) for idx in np.ndindex(*rows)}
    scal = {n: cast(v) for n, v in scalars.items()}
    outs = {}
    combs = {"sum": lambda a, b: a + b, "xor": lambda a, b: a ^ b,
             "max": (lambda a, b: np.fmax(a, b)) if elem == "f32" else (lambda a, b: max(a, b)),
             "min": (lambda a, b: np.fmin(a, b)) if elem == "f32" else (lambda a, b: min(a, b))}
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        for st in spec.stmts:
            if st["kind"] in ("chain", "rowreduce"):
                out = np.zeros(rows[:-1], np.float32 if elem == "f32" else np.uint32)
                outer = st["comb2"] if st["kind"] == "chain" else st["comb"]
                for sidx in np.ndindex(*rows[:-1]):
                    acc2 = _init(elem, outer)
                    for r in range(rows[-1]):
                        ridx = sidx + (r,)
                        renv = {n: v[ridx] for n, v in rowvals.items()}
                        renv.update(scal)
                        if st["kind"] == "chain":
                            acc = _init(elem, st["comb"])
                            for c in range(C):
                                env = {n: cast(a[ridx + (c,)]) for n, a in tiles.items()}
                                if col is not None:
                                    env["g"] = cast(col[c])
                                env.update(renv)
                                acc = cast(combs[st["comb"]](acc, cast(_eval(st["expr"], env, elem))))
                            v = acc
                        else:
                            v = cast(_eval(st["expr"], renv, elem))
                        acc2 = cast(combs[outer](acc2, v))
                    if st["piped"] is not None:
                        env = dict(scal)
                        env["v"] = acc2
                        acc2 = cast(_eval(st["piped"], env, elem))
                    out[sidx] = acc2
                outs[st["out"]] = out
                continue
            if st["kind"] == "map":
                out = np.zeros(full, np.float32 if elem == "f32" else np.uint32)
                for idx in np.ndindex(*full):
                    env = {n: cast(a[idx]) for n, a in tiles.items()}
                    if col is not None:
                        env["g"] = cast(col[idx[-1]])
                    env.update({n: v[idx[:-1]] for n, v in rowvals.items()})
                    env.update(scal)
                    out[idx] = _eval(st["expr"], env, elem)
                outs[st["out"]] = out
                continue
            res = {}
            for ridx in np.ndindex(*rows):
                if st["kind"] == "reduce":
                    acc = _init(elem, st["comb"])
                    for c in range(C):
                        idx = ridx + (c,)
                        env = {n: cast(a[idx]) for n, a in tiles.items()}
                        if col is not None:
                            env["g"] = cast(col[c])
                        env.update({n: v[ridx] for n, v in rowvals.items()})
                        env.update(scal)
                        acc = cast(combs[st["comb"]](acc, cast(_eval(st["expr"], env, elem))))
                    if st["piped"] is not None:
                        env = {n: v[ridx] for n, v in rowvals.items()}
                        env.update(scal)
                        env["v"] = acc
                        acc = cast(_eval(st["piped"], env, elem))
                    res[ridx] = acc
                else:
                    env = {n: v[ridx] for n, v in rowvals.items()}
                    env.update(scal)
                    res[ridx] = cast(_eval(st["expr"], env, elem))
            rowvals[st["out"]] = res
            if not st["local"]:
                arr = np.zeros(rows, np.float32 if elem == "f32" else np.uint32)
                for ridx, v in res.items():
                    arr[ridx] = v
                outs[st["out"]] = arr
    return outs


def evaluate_grid(spec, x0, xt, col, row, scalars):
    """Expected outputs of a grid spec (randprog.GridSpec): x0 [(B,) R, C] in
    the work type, xt [(B,) C, R] (read at (c, r)), g [C], r [R] or None.
    `map` stores y [(B,) R, C], `tmap` its transpose [(B,) C, R],
    `colreduce` folds over R (the reduce drops the last live axis of
    As((B,) C, R)) into [(B,) C]; later statements read a colreduce result
    at (batch, column). Returns ({output: array} without the locals, every
    float sum exact)."""
    elem = spec.elem
    dt = np.float32 if elem == "f32" else np.uint32
    batch = getattr(spec, "batch", False)
    if not batch:  # one batch index, dropped from the outputs
        x0 = x0[None]
        xt = None if xt is None else xt[None]
    Bn, R, C = x0.shape
    env = {"x0": x0.astype(dt)}
    if xt is not None:
        env["xt"] = np.swapaxes(xt.astype(dt), 1, 2)
    if col is not None:
        env["g"] = col.astype(dt)[None, None, :]
    if row is not None:
        env["r"] = row.astype(dt)[None, :, None]
    scal = {n: (_f32(v) if elem == "f32" else np.uint32(v)) for n, v in scalars.items()}
    env.update(scal)
    outs, exact = {}, True
    colres = {}  # colreduce results [Bn, C], read by later statements at their own column
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        for st in spec.stmts:
            val = np.array(np.broadcast_to(np.asarray(_eval(st["expr"], env, elem), dt), (Bn, R, C)), dt)
            if st["kind"] == "map":
                out = val
            elif st["kind"] == "tmap":
                out = np.ascontiguousarray(np.swapaxes(val, 1, 2))
            else:
                red, ok = _reduce(elem, st["comb"], np.ascontiguousarray(np.swapaxes(val, 1, 2)))
                exact = exact and ok
                if st["piped"] is not None:
                    penv = dict(scal)
                    penv.update(colres)
                    penv["v"] = red
                    if col is not None:
                        penv["g"] = col.astype(dt)[None, :]
                    red = np.broadcast_to(np.asarray(_eval(st["piped"], penv, elem), dt), (Bn, C))
                out = np.array(red, dt)
                colres[st["out"]] = out
                env[st["out"]] = out[:, None, :]
            if not st.get("local"):
                outs[st["out"]] = out if batch else out[0]
    return outs, exact


def evaluate_grid_scalar(spec, x0, xt, col, row, scalars):
    """Brute force of evaluate_grid: one element at a time, folds in
    ascending r from init (runtime/tca/reducer.h:36-57). Tiny shapes only."""
    elem = spec.elem
    cast = _f32 if elem == "f32" else np.uint32
    dt = np.float32 if elem == "f32" else np.uint32
    batch = getattr(spec, "batch", False)
    if not batch:
        x0 = x0[None]
        xt = None if xt is None else xt[None]
    Bn, R, C = x0.shape
    scal = {n: cast(v) for n, v in scalars.items()}
    combs = {"sum": lambda a, b: a + b, "xor": lambda a, b: a ^ b,
             "max": (lambda a, b: np.fmax(a, b)) if elem == "f32" else (lambda a, b: max(a, b)),
             "min": (lambda a, b: np.fmin(a, b)) if elem == "f32" else (lambda a, b: min(a, b))}

    colres = {}  # colreduce results [Bn, C]

    def env_at(bb, r, c):
        env = {"x0": cast(x0[bb, r, c])}
        if xt is not None:
            env["xt"] = cast(xt[bb, c, r])
        if col is not None:
            env["g"] = cast(col[c])
        if row is not None:
            env["r"] = cast(row[r])
        env.update(scal)
        for name, res in colres.items():
            env[name] = cast(res[bb, c])
        return env

    outs = {}
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        for st in spec.stmts:
            if st["kind"] in ("map", "tmap"):
                out = np.zeros((Bn, R, C) if st["kind"] == "map" else (Bn, C, R), dt)
                for bb in range(Bn):
                    for r in range(R):
                        for c in range(C):
                            v = cast(_eval(st["expr"], env_at(bb, r, c), elem))
                            if st["kind"] == "map":
                                out[bb, r, c] = v
                            else:
                                out[bb, c, r] = v
            else:
                out = np.zeros((Bn, C), dt)
                for bb in range(Bn):
                    for c in range(C):
                        acc = _init(elem, st["comb"])
                        for r in range(R):
                            acc = cast(combs[st["comb"]](acc, cast(_eval(st["expr"], env_at(bb, r, c), elem))))
                        if st["piped"] is not None:
                            penv = dict(scal)
                            for name, res in colres.items():
                                penv[name] = cast(res[bb, c])
                            penv["v"] = acc
                            if col is not None:
                                penv["g"] = cast(col[c])
                            acc = cast(_eval(st["piped"], penv, elem))
                        out[bb, c] = acc
                colres[st["out"]] = out
            if not st.get("local"):
                outs[st["out"]] = out if batch else out[0]
    return outs
