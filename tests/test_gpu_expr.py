"""The expression layer on the device: every operator, builtin and cast of
the DSL (pkg/expr.go:140-341, internal/ir/builtins.go:25-33), one output per
expression, over operands that include the IEEE special values.

Expected values are closed forms, not the oracle library: IEEE basic
operations (+ - * /, negation, fabs, comparisons and selects, fminf/fmaxf)
are correctly rounded on both sides, so the device must match numpy's
float32 results bit for bit (NaN compared as NaN-ness; fminf/fmaxf of
+0/-0 compared by value, C leaves the sign of the result open there);
fmaf is checked against the exactly rounded a*b+c (rational arithmetic,
round-to-nearest-even); sqrtf within 1 ulp of the float64 value; the
transcendentals within the ulp bounds stated in TRANSCENDENTAL_ULP of the
float64 value (the device uses ocml, the reference's GPU side NVIDIA's
library: bitwise parity is unpinned, as for every transcendental). Integer
operations follow C semantics on operands that avoid undefined behaviour
(no signed overflow, no division by zero, shift counts masked below the
width). Casts: f32 -> bf16 and f16 round to nearest even, f32 -> i32
truncates, i32 -> u8 keeps the low byte."""
from fractions import Fraction

import numpy as np
import pytest

import oracle
from helpers import compiled, run
from tcacomp_amd.compiler import TensorDesc

pytestmark = pytest.mark.gpu

U32 = 4
TRANSCENDENTAL_ULP = {"exp": 2, "log": 2, "rsqrt": 2, "sin": 4, "cos": 4, "tanh": 4}
N_RANDOM = 10000


def _f32_specials():
    v = [0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 0.5, 2.0, 3.0, 1e-40, -1e-40, 1e-45, -1e-45,
         3.4028235e38, -3.4028235e38, 1.1754944e-38, 88.7, -103.9, 1e10, -1e10, 6.2831855, 1e-7]
    return np.array(v, np.float32)


def _f32_operands(seed):
    rng = np.random.default_rng(seed)
    s = _f32_specials()
    wide = (rng.choice([-1.0, 1.0], N_RANDOM) * np.exp2(rng.uniform(-40, 40, N_RANDOM))).astype(np.float32)
    x = np.concatenate([np.repeat(s, len(s)), wide])
    y = np.concatenate([np.tile(s, len(s)), rng.permutation(wide)])
    return np.ascontiguousarray(x), np.ascontiguousarray(y)


def _launch(name, inputs, outs_spec, gpu):
    """inputs: numpy arrays; outs_spec: [(torch dtype, tca code or None)]."""
    import torch
    n = inputs[0].size
    dev_in, descs = [], []
    for a in inputs:
        if a.dtype == np.uint32:
            t = torch.from_numpy(a.view(np.int32)).to(gpu)
            descs.append(TensorDesc(t.data_ptr(), a.shape, U32))
        else:
            t = torch.from_numpy(a).to(gpu)
            descs.append(t)
        dev_in.append(t)
    outs = []
    for dt, code in outs_spec:
        t = torch.zeros(n, dtype=dt, device=gpu)
        outs.append(t)
        descs.append(TensorDesc(t.data_ptr(), (n,), code) if code is not None else t)
    run(compiled(name), descs)
    host = [(o.view(torch.int16) if o.dtype == torch.bfloat16 else o).cpu().numpy() for o in outs]
    return host, dev_in


def _same_bits(got, want, what):
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), "%s: NaN positions differ" % what
    g, w = got[~gn], want[~wn]
    bad = g.view(np.uint32) != w.view(np.uint32)
    assert not bad.any(), "%s: %d mismatch(es), e.g. got %r want %r" % (what, int(bad.sum()), g[bad][:3], w[bad][:3])


def _ulps(got, ref64):
    """|got - ref| in float32 ulps at ref (specials, and results past the
    float32 range, compared exactly with the reference rounded to float32)."""
    with np.errstate(over="ignore"):
        ref32 = ref64.astype(np.float32)
    ref64 = np.where(np.isfinite(ref32), ref64, ref32.astype(np.float64))
    out = np.zeros(got.shape)
    fin = np.isfinite(ref64) & np.isfinite(got)
    sp = np.spacing(np.abs(ref32[fin])).astype(np.float64)
    sp = np.maximum(sp, np.float64(np.float32(1e-45)))
    out[fin] = np.abs(got[fin].astype(np.float64) - ref64[fin]) / sp
    nf = ~fin
    same = (np.isnan(got[nf]) & np.isnan(ref64[nf])) | (got[nf].astype(np.float64) == ref64[nf])
    out[np.flatnonzero(nf)[~same]] = np.inf
    return out


def _fma_exact(a, b, c):
    """round-to-nearest-even float32 of the exact a*b+c (finite operands)."""
    out = np.empty(a.shape, np.float32)
    for i, (x, y, z) in enumerate(zip(a.tolist(), b.tolist(), c.tolist())):
        exact = Fraction(x) * Fraction(y) + Fraction(z)
        if exact == 0:  # the sign of a zero follows IEEE: float64 forms x*y and the sum exactly
            out[i] = np.float32(np.float64(x) * np.float64(y) + np.float64(z))
            continue
        r0 = np.float32(float(exact))
        if not np.isfinite(r0):
            out[i] = r0
            continue
        cands = [c_ for c_ in (np.nextafter(r0, np.float32(-np.inf)), r0, np.nextafter(r0, np.float32(np.inf)))
                 if np.isfinite(c_)]
        best = min(cands, key=lambda c_: (abs(Fraction(float(c_)) - exact), int(np.float32(c_).view(np.uint32)) & 1))
        out[i] = best
    return out


def test_expr_f32(gpu):
    import torch
    from tcacomp_amd import programs
    x, y = _f32_operands(1)
    names = [n for n, _ in programs.EXPR_F32]
    got, _ = _launch("expr_f32", [x, y], [(torch.float32, None)] * len(names), gpu)
    g = dict(zip(names, got))
    with np.errstate(all="ignore"):
        _same_bits(g["add"], x + y, "add")
        _same_bits(g["sub"], x - y, "sub")
        _same_bits(g["mul"], x * y, "mul")
        _same_bits(g["div"], x / y, "div")
        _same_bits(g["neg"], -x, "neg")
        _same_bits(g["sel"], np.where(x < y, x, y), "select(x < y)")
        _same_bits(g["fabs"], np.abs(x), "fabsf")
        for nm, f in (("fmin", np.fmin), ("fmax", np.fmax)):
            want = f(x, y)
            assert np.array_equal(np.isnan(g[nm]), np.isnan(want)), nm
            ok = ~np.isnan(want)
            assert np.array_equal(g[nm][ok], want[ok]), nm  # by value: +0 == -0
        fin = np.isfinite(x) & np.isfinite(y) & np.isfinite(x.astype(np.float64) * y + x)
        _same_bits(g["fma"][fin], _fma_exact(x[fin], y[fin], x[fin]), "fmaf")
        assert (_ulps(g["sqrt"], np.sqrt(x.astype(np.float64))) <= 1).all(), "sqrtf"
        x64 = x.astype(np.float64)
        refs = {"exp": np.exp(x64), "log": np.log(x64), "rsqrt": 1.0 / np.sqrt(x64), "sin": np.sin(x64),
                "cos": np.cos(x64), "tanh": np.tanh(x64)}
    for nm, ref in refs.items():
        u = _ulps(g[nm], ref)
        print("%s: max %.3f ulp" % (nm, u.max()))
        assert u.max() <= TRANSCENDENTAL_ULP[nm], "%s: %g ulp at x=%r" % (nm, u.max(), x[np.argmax(u)])


def test_expr_i32(gpu):
    import torch
    from tcacomp_amd import programs
    rng = np.random.default_rng(2)
    x = rng.integers(-2**15, 2**15, N_RANDOM, dtype=np.int64).astype(np.int32)
    y = rng.integers(-2**15, 2**15, N_RANDOM, dtype=np.int64).astype(np.int32)
    x[:8] = [0, 1, -1, 7, -7, 32767, -32768, 5]
    y[:8] = [1, -1, 7, -7, 3, -2, 7, 7]
    y[y == 0] = 3
    names = [n for n, _ in programs.EXPR_I32]
    got, _ = _launch("expr_i32", [x, y], [(torch.int32, None)] * len(names), gpu)
    g = dict(zip(names, got))
    X, Y = x.astype(np.int64), y.astype(np.int64)
    q = (np.abs(X) // np.abs(Y)) * np.sign(X) * np.sign(Y)  # C division truncates toward zero
    want = {"add": X + Y, "sub": X - Y, "mul": X * Y, "div": q, "mod": X - q * Y, "and": X & Y, "or": X | Y,
            "xor": X ^ Y, "shl": (X & 0xFFFF) << (Y & 15), "shr": X >> (Y & 31), "neg": -X, "not": ~X,
            "cmp": np.where((X < Y) & (X != 0), 1, np.where((X >= Y) | (Y == 7), 2, 3))}
    for nm in names:
        assert np.array_equal(g[nm].astype(np.int64), want[nm]), nm


def test_expr_u32(gpu):
    import torch
    from tcacomp_amd import programs
    rng = np.random.default_rng(3)
    x = rng.integers(0, 2**32, N_RANDOM, dtype=np.uint64).astype(np.uint32)
    y = rng.integers(0, 2**32, N_RANDOM, dtype=np.uint64).astype(np.uint32)
    x[:4] = [0, 0xFFFFFFFF, 1, 12345]
    y[:4] = [1, 1, 0xFFFFFFFF, 12345]
    y[y == 0] = 1
    y[4:1000] = y[4:1000] % 1000 + 1  # small divisors too
    names = [n for n, _ in programs.EXPR_U32]
    got, _ = _launch("expr_u32", [x, y], [(torch.int32, U32)] * len(names), gpu)
    g = {n: a.view(np.uint32).astype(np.uint64) for n, a in zip(names, got)}
    X, Y, M = x.astype(np.uint64), y.astype(np.uint64), np.uint64(0xFFFFFFFF)
    want = {"add": (X + Y) & M, "sub": (X - Y) & M, "mul": (X * Y) & M, "div": X // Y, "mod": X % Y,
            "shr": X >> (Y & np.uint64(31)), "umin": np.minimum(X, Y), "umax": np.maximum(X, Y),
            "not": (~X) & M, "le": np.where(X <= Y, X, Y)}
    for nm in names:
        assert np.array_equal(g[nm], want[nm]), nm


def test_expr_casts(gpu):
    import torch
    rng = np.random.default_rng(4)
    x = np.concatenate([np.array([0.0, -0.0, 1.0, -1.0, 0.5, 1.5, 2.5, -2.5, 65504.0, -65504.0, 6e-8, 1e-40,
                                  1.00390625, 1.01171875, 255.9, -255.9], np.float32),
                        (rng.standard_normal(N_RANDOM) * np.exp2(rng.uniform(-20, 15, N_RANDOM))).astype(np.float32)])
    x = np.ascontiguousarray(np.clip(x, -65504.0, 65504.0).astype(np.float32))
    k = rng.integers(-2**31, 2**31, x.size, dtype=np.int64).astype(np.int32)
    k[:6] = [0, 255, 256, -1, 2**24 + 1, -(2**31)]
    spec = [(torch.bfloat16, None), (torch.float16, None), (torch.int32, None), (torch.float32, None),
            (torch.uint8, None), (torch.int32, U32), (torch.float32, None)]
    got, _ = _launch("expr_casts", [x, k], spec, gpu)
    bf16, f16, trunc, tof32, tou8, tou32, bf16f32 = got
    assert np.array_equal(bf16.view(np.uint16), oracle.to_bf16_bits(x)), "f32 -> bf16 (RNE)"
    assert np.array_equal(f16.view(np.uint16), x.astype(np.float16).view(np.uint16)), "f32 -> f16 (RNE)"
    assert np.array_equal(trunc, x.astype(np.int32)), "f32 -> i32 (truncation)"
    assert np.array_equal(tof32.view(np.uint32), k.astype(np.float32).view(np.uint32)), "i32 -> f32 (RNE)"
    assert np.array_equal(tou8, (k.astype(np.int64) & 0xFF).astype(np.uint8)), "i32 -> u8 (low byte)"
    assert np.array_equal(tou32.view(np.uint32), k.view(np.uint32)), "i32 -> u32 (bits)"
    _same_bits(bf16f32, oracle.bf16_bits_to_f32(oracle.to_bf16_bits(x)), "f32 -> bf16 -> f32")
