"""TEST INFRASTRUCTURE: a CPU interpreter of the builder's structural IR
print (tca_builder_ir_full / Program.IRFull()), used to check the CPU
oracle's restatements of the suite kernels against the programs
themselves. The suite programs' IR is pinned to the reference's own
testing/kernels/**.tca sources (tests/test_syntax.py compiles that corpus
to identical IR), so evaluating that IR here checks each oracle formula
against the reference's program text rather than against a second
transcription of the formula.

Semantics (pkg/chain.go:360-552): a statement's root map is evaluated at
every point of its `as` axes, operands read at their subscripts; each
reduce folds the last live axis sequentially in ascending index from its
init (runtime/tca/reducer.h:36-57); a piped map sees the reduced value
first; the store writes the live axes at the store's subscripts. f32
arithmetic is numpy float32 (correctly rounded); builtins are evaluated in
float64 and rounded once to float32; integers wrap.
"""
import math
import re

import numpy as np

_DT = {"f32": np.float32, "i32": np.int32, "u32": np.uint32, "u8": np.uint8, "i8": np.int8, "i16": np.int16,
       "u16": np.uint16, "bool": np.bool_, "bf16": np.float32, "f16": np.float16}

_CALLS = {
    "expf": np.exp, "logf": np.log, "sqrtf": np.sqrt, "rsqrtf": lambda x: 1.0 / np.sqrt(x), "tanhf": np.tanh,
    "sinf": np.sin, "cosf": np.cos, "fabsf": np.abs, "exp2f": np.exp2, "log2f": np.log2,
    "fmaxf": np.fmax, "fminf": np.fmin, "powf": np.power,
}


class Stage:
    def __init__(self, kind, ops=(), params=(), body=(), result=None, rtype="f32", axes=(), init=None, over=None):
        self.kind, self.ops, self.params, self.body, self.result = kind, list(ops), list(params), list(body), result
        self.rtype, self.axes, self.init, self.over = rtype, list(axes), init, over


class Statement:
    def __init__(self, iters):
        self.iters, self.stages, self.store = iters, [], None


class Program:
    def __init__(self):
        self.dims, self.tensors, self.scalars, self.statements = {}, {}, {}, []


def _lambda(text):
    """'(l: f32, r: f32) { %0 = mul l r; -> %0: f32 }' -> params, body, result, type."""
    m = re.match(r"\((.*?)\) \{(.*) -> (\S+): (\w+) \}$", text.strip())
    params = [p.split(":")[0].strip() for p in m.group(1).split(",") if p.strip()]
    body = []
    for ins in m.group(2).split(";"):
        ins = ins.strip()
        if not ins:
            continue
        dst, rhs = ins.split(" = ")
        parts = rhs.split()
        body.append((dst, parts[0], parts[1:]))
    return params, body, m.group(3), m.group(4)


def _operands(text):
    inner = re.match(r"on\((.*)\)$", text).group(1)
    out = []
    for o in re.findall(r"(\w+)((?:\[@\w+\])*)", inner):
        out.append((o[0], re.findall(r"\[@(\w+)\]", o[1])))
    return out


def parse(text):
    p = Program()
    st = None
    for line in text.splitlines():
        s = line.strip()
        if s.startswith("dim @"):
            name, ext = s[5:].split()
            p.dims[name] = None if ext == "dynamic" else int(ext)
        elif s.startswith(("tensor ", "local ")):
            m = re.match(r"(?:tensor|local) (\w+): (\w+)\[(.*)\]$", s)
            p.tensors[m.group(1)] = (m.group(2), [d.strip()[1:] for d in m.group(3).split(",") if d.strip()])
        elif s.startswith("scalar "):
            m = re.match(r"scalar (\w+): (\w+)$", s)
            p.scalars[m.group(1)] = m.group(2)
        elif s.startswith("statement #"):
            m = re.match(r"statement #\d+ iter\((.*)\)$", s)
            st = Statement([a.strip()[1:] for a in m.group(1).split(",") if a.strip()])
            p.statements.append(st)
        elif s.startswith("map "):
            m = re.match(r"map (pipe\+)?(on\(.*?\)) (\(.*\}) as\((.*)\)$", s)
            params, body, result, rtype = _lambda(m.group(3))
            axes = [a.strip()[1:] for a in m.group(4).split(",") if a.strip()]
            st.stages.append(Stage("pipe" if m.group(1) else "map", _operands(m.group(2)), params, body, result,
                                   rtype, axes))
        elif s.startswith("reduce "):
            m = re.match(r"reduce init=(\S+) over @(\w+) (\(.*\})$", s)
            params, body, result, rtype = _lambda(m.group(3))
            st.stages.append(Stage("reduce", (), params, body, result, rtype, init=m.group(1), over=m.group(2)))
        elif s.startswith("store "):
            m = re.match(r"store (\w+)((?:\[@\w+\])*)$", s)
            st.store = (m.group(1), re.findall(r"\[@(\w+)\]", m.group(2)))
    return p


def _const(tok, rtype):
    dt = _DT[rtype]
    if ":" in tok:
        tok, t = tok.split(":")
        dt = _DT[t]
    if tok in ("true", "false"):
        return np.bool_(tok == "true")
    if dt in (np.float32, np.float16):
        return dt(float(tok.replace("inf", "inf")))
    return dt(int(float(tok)))


def _run(body, env, rtype):
    vals = dict(env)

    def arg(t):
        if t in vals:
            return vals[t]
        return _const(t, rtype)

    for dst, op, args in body:
        a = [arg(x) for x in args]
        with np.errstate(all="ignore"):
            if op in ("add", "sub", "mul", "div", "mod"):
                x, y = np.asarray(a[0]), np.asarray(a[1])
                if x.dtype.kind == "f":
                    y = y.astype(x.dtype)
                elif y.dtype.kind == "f":
                    x = x.astype(y.dtype)
                else:
                    y = y.astype(x.dtype)
                if op == "add":
                    r = x + y
                elif op == "sub":
                    r = x - y
                elif op == "mul":
                    r = x * y
                elif op == "div":
                    r = x / y if x.dtype.kind == "f" else np.where(y == 0, 0, x // np.where(y == 0, 1, y))
                else:
                    r = np.fmod(x, y) if x.dtype.kind == "f" else x % np.where(y == 0, 1, y)
            elif op in ("eq", "ne", "lt", "le", "gt", "ge"):
                r = {"eq": np.equal, "ne": np.not_equal, "lt": np.less, "le": np.less_equal, "gt": np.greater,
                     "ge": np.greater_equal}[op](a[0], a[1])
            elif op in ("land", "lor"):
                r = np.logical_and(a[0], a[1]) if op == "land" else np.logical_or(a[0], a[1])
            elif op in ("and", "or", "xor"):
                r = {"and": np.bitwise_and, "or": np.bitwise_or, "xor": np.bitwise_xor}[op](a[0], a[1])
            elif op in ("shl", "shr"):
                r = np.left_shift(a[0], a[1]) if op == "shl" else np.right_shift(a[0], a[1])
            elif op == "neg":
                r = -np.asarray(a[0])
            elif op == "pos":
                r = a[0]
            elif op == "lnot":
                r = np.logical_not(a[0])
            elif op == "not":
                r = np.invert(a[0])
            elif op == "select":
                r = np.where(a[0], a[1], a[2])
            elif op.startswith("cast."):
                t = _DT[op[5:]]
                r = np.asarray(a[0])
                r = np.trunc(r).astype(t) if r.dtype.kind == "f" and t not in (np.float32, np.float16) else r.astype(t)
            elif op in _CALLS:
                r = np.asarray(_CALLS[op](*[np.asarray(v, np.float64) for v in a]), np.float64).astype(np.float32)
            else:
                raise NotImplementedError(op)
        vals[dst] = r
    return vals


def _gather(prog, arrays, tensor, subs, live, ext):
    """tensor[subs] at every point of the live axes (in their order)."""
    shape = [ext[a] for a in live]
    idx = []
    for a in subs:
        k = live.index(a)
        s = [1] * len(live)
        s[k] = ext[a]
        idx.append(np.arange(ext[a]).reshape(s))
    src = arrays[tensor]
    v = src[tuple(idx)] if idx else src[()]
    return np.broadcast_to(v, shape)


def evaluate(prog, arrays, scalars, dims):
    """Runs every statement. arrays: {tensor: np.ndarray} for the inputs (in
    the work type); scalars: {name: value}; dims: {name: extent} for the
    dynamic dims. Returns {tensor: array} with every stored tensor."""
    ext = {n: (e if e is not None else dims[n]) for n, e in prog.dims.items()}
    arrays = dict(arrays)
    sc = {"$" + n: _DT[t](v) for n, v in ((n, scalars[n]) for n in prog.scalars) for t in [prog.scalars[n]]}
    for st in prog.statements:
        live, val = None, None
        for sg in st.stages:
            if sg.kind in ("map", "pipe"):
                env = dict(sc)
                params = list(sg.params)
                if sg.kind == "pipe":
                    env[params.pop(0)] = val
                src_live = sg.axes if sg.kind == "map" else live
                for (t, subs), name in zip(sg.ops, params):
                    env[name] = _gather(prog, arrays, t, subs, src_live, ext)
                out = _run(sg.body, env, sg.rtype)
                res = np.asarray(out[sg.result] if sg.result in out else _const(sg.result, sg.rtype))
                res = np.broadcast_to(res, [ext[a] for a in src_live]).astype(_DT[sg.rtype])
                if sg.kind == "pipe" and sg.axes != live:
                    res = np.transpose(res, [live.index(a) for a in sg.axes])
                live, val = list(sg.axes), np.array(res)
            else:  # reduce over the last live axis
                assert live[-1] == sg.over, (live, sg.over)
                n = ext[sg.over]
                acc = np.broadcast_to(np.asarray(_const(sg.init, sg.rtype)), val.shape[:-1]).astype(_DT[sg.rtype])
                for i in range(n):
                    out = _run(sg.body, {sg.params[0]: acc, sg.params[1]: val[..., i], **sc}, sg.rtype)
                    acc = np.asarray(out[sg.result]).astype(_DT[sg.rtype])
                live, val = live[:-1], acc
        t, subs = st.store
        perm = [live.index(a) for a in subs]
        arrays[t] = np.ascontiguousarray(np.transpose(val, perm) if perm else val)
    return arrays
