"""DSL programs: the benchmark configurations and the reference's suite.

Each builder here is written against the pkg API exactly as a user of the
reference would write it (pkg/chain.go rung order). Dims that the reference
declares dynamic stay dynamic, so one code object serves every test size;
the row length of the fused row configurations is a compile-time constant
(as the reference's `8u`-style const dims are), which is what lets the row
live in registers.

Configurations:
  scale_relu      C1  z = max(a*x + y, 0)            (degenerate-reduce encoding,
                                                      testing/kernels/runtime/scale_copy.tca:3-10)
  scale_relu_map  C1  same, elementwise Store rung   (wall W1 lifted)
  row_sum_max     C2  row sum and row max             (two chains, one fused kernel)
  softmax         C3  row softmax via two locals
  layernorm       C4  mean/variance locals, then normalise with gamma/beta
  gemm_f32        C5  C = A.B fp32                    (testing/kernels/llm/gemm.tca:7-22)
  gemm_bf16       C5  C = cast(A).cast(B), bf16 inputs, fp32 accumulate

Reference suite (testing/kernels/**.tca, shapes in testing/suite.toml): see
SUITE below.
"""
import os

from .pkg import (TBF16, TF16, TF32, TI32, TU8, TU32, At, Call, Cast, NewBuilder, Select)


def _sum(b):
    return lambda acc, v: b.Add(acc, v)


def _static(b, name, extent):
    """A dim handle: dynamic under its name, or a compile-time extent under the
    e<extent> name the .tca frontend gives unnamed static dims."""
    return b.Dim(name, 0) if extent == 0 else b.Dim("e%d" % extent, extent)


def _neg_inf(b):
    """-inf as the .tca source spells it (-inf_f32: a negated literal)."""
    return b.Neg(b.Float32(float("inf")))


def scale_relu(cols=0):
    """C1 in the reference-legal encoding: x, y carry a trailing extent-1
    axis that a degenerate reduce drops."""
    b = NewBuilder("scale_relu")
    M, N, U = b.Dim("M", 0), _static(b, "N", cols), b.Dim("e1", 1)
    x = b.Tensor("x", TF32, M, N, U)
    y = b.Tensor("y", TF32, M, N, U)
    z = b.Tensor("z", TF32, M, N)
    a = b.ScalarParam("a", TF32)
    (b.Stmt().Iter(M, N, U)
     .Map([At(x, M, N, U), At(y, M, N, U)], lambda l, r: Call("fmaxf", b.Add(b.Mul(a, l), r), b.Float32(0)))
     .As(M, N, U)
     .Reduce(b.Float32(0), _sum(b))
     .Store(z, M, N))
    return b.Build()


def scale_relu_map():
    """C1 written directly as an elementwise chain (Store after the root as)."""
    b = NewBuilder("scale_relu_map")
    M, N = b.Dim("M", 0), b.Dim("N", 0)
    x = b.Tensor("x", TF32, M, N)
    y = b.Tensor("y", TF32, M, N)
    z = b.Tensor("z", TF32, M, N)
    a = b.ScalarParam("a", TF32)
    (b.Stmt().Iter(M, N)
     .Map([At(x, M, N), At(y, M, N)], lambda l, r: Call("fmaxf", b.Add(b.Mul(a, l), r), b.Float32(0)))
     .As(M, N)
     .Store(z, M, N))
    return b.Build()


def row_sum_max(cols=8192):
    """C2: two chains over the same nest; GVN-style fusion makes them one
    kernel reading x once."""
    b = NewBuilder("row_sum_max_%s" % (cols or "dyn"))
    R, C = b.Dim("R", 0), _static(b, "C", cols)
    x = b.Tensor("x", TF32, R, C)
    s = b.Tensor("sum", TF32, R)
    m = b.Tensor("max", TF32, R)
    (b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: v).As(R, C)
     .Reduce(b.Float32(0), _sum(b)).Store(s, R))
    (b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: v).As(R, C)
     .Reduce(_neg_inf(b), lambda acc, v: Call("fmaxf", acc, v)).Store(m, R))
    return b.Build()


def softmax(cols=4096):
    """C3: y = exp(x - rowmax) / rowsum(exp(x - rowmax))."""
    b = NewBuilder("softmax_%s" % (cols or "dyn"))
    R, C = b.Dim("R", 0), _static(b, "C", cols)
    x = b.Tensor("x", TF32, R, C)
    y = b.Tensor("y", TF32, R, C)
    mx = b.Local("mx", TF32, R)
    den = b.Local("den", TF32, R)
    (b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: v).As(R, C)
     .Reduce(_neg_inf(b), lambda acc, v: Call("fmaxf", acc, v)).Store(mx, R))
    (b.Stmt().Iter(R, C).Map([At(x, R, C), At(mx, R)], lambda l, r: Call("expf", b.Sub(l, r))).As(R, C)
     .Reduce(b.Float32(0), _sum(b)).Store(den, R))
    (b.Stmt().Iter(R, C)
     .Map([At(x, R, C), At(mx, R), At(den, R)], lambda l, r, s: b.Div(Call("expf", b.Sub(l, r)), s))
     .As(R, C).Store(y, R, C))
    return b.Build()


def layernorm(cols=1024):
    """C4: mean and (centred) variance over the row, then
    (x - mean) * rsqrtf(var + eps) * gamma + beta."""
    b = NewBuilder("layernorm_%s" % (cols or "dyn"))
    R, C = b.Dim("R", 0), _static(b, "C", cols)
    x = b.Tensor("x", TF32, R, C)
    gamma = b.Tensor("gamma", TF32, C)
    beta = b.Tensor("beta", TF32, C)
    y = b.Tensor("y", TF32, R, C)
    mean = b.Local("mean", TF32, R)
    var = b.Local("var", TF32, R)
    inv_n = b.ScalarParam("inv_n", TF32)
    eps = b.ScalarParam("eps", TF32)
    (b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: v).As(R, C)
     .Reduce(b.Float32(0), _sum(b))
     .Map([], lambda v: b.Mul(v, inv_n)).As(R).Store(mean, R))
    (b.Stmt().Iter(R, C)
     .Map([At(x, R, C), At(mean, R)], lambda l, r: b.Mul(b.Sub(l, r), b.Sub(l, r))).As(R, C)
     .Reduce(b.Float32(0), _sum(b))
     .Map([], lambda v: b.Mul(v, inv_n)).As(R).Store(var, R))
    (b.Stmt().Iter(R, C)
     .Map([At(x, R, C), At(mean, R), At(var, R), At(gamma, C), At(beta, C)],
          lambda l, r, s, t, u: b.Add(b.Mul(b.Mul(b.Sub(l, r), Call("rsqrtf", b.Add(s, eps))), t), u))
     .As(R, C).Store(y, R, C))
    return b.Build()


def row_stats_shift(cols=0):
    """A mean and a centred sum of squares whose piped maps read row values:
    m = sum(x) * inv_n + shift[r] (the sum's piped map reads a per-row
    input), rs = rsqrtf(sum((x - m)^2) * inv_n + eps) + 0.5 * m (the sum of
    squares' piped map reads m), then y = (x - m) * rs; m and rs are
    outputs. Exercises the one-read pair's finish beyond layernorm's."""
    b = NewBuilder("row_stats_shift_%s" % (cols or "dyn"))
    R, C = b.Dim("R", 0), _static(b, "C", cols)
    x = b.Tensor("x", TF32, R, C)
    shift = b.Tensor("shift", TF32, R)
    m = b.Tensor("m", TF32, R)
    rs = b.Tensor("rs", TF32, R)
    y = b.Tensor("y", TF32, R, C)
    inv_n = b.ScalarParam("inv_n", TF32)
    eps = b.ScalarParam("eps", TF32)
    (b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: v).As(R, C)
     .Reduce(b.Float32(0), _sum(b))
     .Map([At(shift, R)], lambda v, s: b.Add(b.Mul(v, inv_n), s)).As(R).Store(m, R))
    (b.Stmt().Iter(R, C)
     .Map([At(x, R, C), At(m, R)], lambda l, r: b.Mul(b.Sub(l, r), b.Sub(l, r))).As(R, C)
     .Reduce(b.Float32(0), _sum(b))
     .Map([At(m, R)], lambda v, a: b.Add(Call("rsqrtf", b.Add(b.Mul(v, inv_n), eps)), b.Mul(a, b.Float32(0.5))))
     .As(R).Store(rs, R))
    (b.Stmt().Iter(R, C)
     .Map([At(x, R, C), At(m, R), At(rs, R)], lambda l, a, s: b.Mul(b.Sub(l, a), s))
     .As(R, C).Store(y, R, C))
    return b.Build()


def softmax_affine(cols=0):
    """Softmax of E = x * t + bias[c] (t a scalar parameter, bias a column
    vector), its max and exp-sum also stored: mx = max E, den = sum expf(E -
    mx), y = expf(E - mx) / den. The one-read pair's element expression then
    reads a scalar and a column vector besides the row."""
    b = NewBuilder("softmax_affine_%s" % (cols or "dyn"))
    R, C = b.Dim("R", 0), _static(b, "C", cols)
    x = b.Tensor("x", TF32, R, C)
    bias = b.Tensor("bias", TF32, C)
    mx = b.Tensor("mx", TF32, R)
    den = b.Tensor("den", TF32, R)
    y = b.Tensor("y", TF32, R, C)
    t = b.ScalarParam("t", TF32)

    def e(v, c):
        return b.Add(b.Mul(v, t), c)

    (b.Stmt().Iter(R, C).Map([At(x, R, C), At(bias, C)], e).As(R, C)
     .Reduce(_neg_inf(b), lambda acc, v: Call("fmaxf", acc, v)).Store(mx, R))
    (b.Stmt().Iter(R, C).Map([At(x, R, C), At(bias, C), At(mx, R)], lambda v, c, m: Call("expf", b.Sub(e(v, c), m)))
     .As(R, C).Reduce(b.Float32(0), _sum(b)).Store(den, R))
    (b.Stmt().Iter(R, C)
     .Map([At(x, R, C), At(bias, C), At(mx, R), At(den, R)], lambda v, c, m, s: b.Div(Call("expf", b.Sub(e(v, c), m)), s))
     .As(R, C).Store(y, R, C))
    return b.Build()


def row_moments_affine(cols=0):
    """The mean and variance of E = x * g[c] + r[row] (a column and a row
    vector), both stored: m = sum(E) * inv_n, v = sum((E - m)^2) * inv_n,
    then y = (E - m) * rsqrtf(v + eps). The one-read pair's element
    expression then reads a column and a row vector besides the row."""
    b = NewBuilder("row_moments_affine_%s" % (cols or "dyn"))
    R, C = b.Dim("R", 0), _static(b, "C", cols)
    x = b.Tensor("x", TF32, R, C)
    g = b.Tensor("g", TF32, C)
    r = b.Tensor("r", TF32, R)
    m = b.Tensor("m", TF32, R)
    var = b.Tensor("v", TF32, R)
    y = b.Tensor("y", TF32, R, C)
    inv_n = b.ScalarParam("inv_n", TF32)
    eps = b.ScalarParam("eps", TF32)

    def e(v, c, w):
        return b.Add(b.Mul(v, c), w)

    (b.Stmt().Iter(R, C).Map([At(x, R, C), At(g, C), At(r, R)], e).As(R, C)
     .Reduce(b.Float32(0), _sum(b)).Map([], lambda s: b.Mul(s, inv_n)).As(R).Store(m, R))
    (b.Stmt().Iter(R, C)
     .Map([At(x, R, C), At(g, C), At(r, R), At(m, R)], lambda v, c, w, a: b.Mul(b.Sub(e(v, c, w), a), b.Sub(e(v, c, w), a)))
     .As(R, C).Reduce(b.Float32(0), _sum(b)).Map([], lambda s: b.Mul(s, inv_n)).As(R).Store(var, R))
    (b.Stmt().Iter(R, C)
     .Map([At(x, R, C), At(g, C), At(r, R), At(m, R), At(var, R)],
          lambda v, c, w, a, q: b.Mul(b.Sub(e(v, c, w), a), Call("rsqrtf", b.Add(q, eps))))
     .As(R, C).Store(y, R, C))
    return b.Build()


def softmax_bf16(cols=0):
    """Softmax of bf16 rows computed in f32 (Cast per element) into an f32
    output: the one-read pair over 8-byte bf16 vectors."""
    b = NewBuilder("softmax_bf16_%s" % (cols or "dyn"))
    R, C = b.Dim("R", 0), _static(b, "C", cols)
    x = b.Tensor("x", TBF16, R, C)
    y = b.Tensor("y", TF32, R, C)
    mx = b.Local("mx", TF32, R)
    den = b.Local("den", TF32, R)
    (b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: Cast(v, TF32)).As(R, C)
     .Reduce(_neg_inf(b), lambda acc, v: Call("fmaxf", acc, v)).Store(mx, R))
    (b.Stmt().Iter(R, C).Map([At(x, R, C), At(mx, R)], lambda l, r: Call("expf", b.Sub(Cast(l, TF32), r)))
     .As(R, C).Reduce(b.Float32(0), _sum(b)).Store(den, R))
    (b.Stmt().Iter(R, C)
     .Map([At(x, R, C), At(mx, R), At(den, R)], lambda l, r, s: b.Div(Call("expf", b.Sub(Cast(l, TF32), r)), s))
     .As(R, C).Store(y, R, C))
    return b.Build()


def layernorm_rstd(cols=1024):
    """C4 with the reciprocal standard deviation as its own per-row chain
    (iterating only the row axis, one level shallower than the others) and
    also stored as an output: mean, var -> rstd = rsqrtf(var + eps) ->
    y = (x - mean) * rstd * gamma + beta. Same arithmetic as layernorm()."""
    b = NewBuilder("layernorm_rstd_%s" % (cols or "dyn"))
    R, C = b.Dim("R", 0), _static(b, "C", cols)
    x = b.Tensor("x", TF32, R, C)
    gamma = b.Tensor("gamma", TF32, C)
    beta = b.Tensor("beta", TF32, C)
    y = b.Tensor("y", TF32, R, C)
    rstd = b.Tensor("rstd", TF32, R)
    mean = b.Local("mean", TF32, R)
    var = b.Local("var", TF32, R)
    inv_n = b.ScalarParam("inv_n", TF32)
    eps = b.ScalarParam("eps", TF32)
    (b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: v).As(R, C)
     .Reduce(b.Float32(0), _sum(b))
     .Map([], lambda v: b.Mul(v, inv_n)).As(R).Store(mean, R))
    (b.Stmt().Iter(R, C)
     .Map([At(x, R, C), At(mean, R)], lambda l, r: b.Mul(b.Sub(l, r), b.Sub(l, r))).As(R, C)
     .Reduce(b.Float32(0), _sum(b))
     .Map([], lambda v: b.Mul(v, inv_n)).As(R).Store(var, R))
    b.Stmt().Iter(R).Map([At(var, R)], lambda v: Call("rsqrtf", b.Add(v, eps))).As(R).Store(rstd, R)
    (b.Stmt().Iter(R, C)
     .Map([At(x, R, C), At(mean, R), At(rstd, R), At(gamma, C), At(beta, C)],
          lambda l, r, s, t, u: b.Add(b.Mul(b.Mul(b.Sub(l, r), s), t), u))
     .As(R, C).Store(y, R, C))
    return b.Build()


def vec_sum_max():
    """Full reductions: sum and max of a vector x [N] into two rank-0
    outputs (no row axis: the streaming family's split rows over the whole
    GPU)."""
    b = NewBuilder("vec_sum_max")
    N = b.Dim("N", 0)
    x = b.Tensor("x", TF32, N)
    s = b.Tensor("sum", TF32)
    m = b.Tensor("max", TF32)
    b.Stmt().Iter(N).Map([At(x, N)], lambda v: v).As(N).Reduce(b.Float32(0), _sum(b)).Store(s)
    b.Stmt().Iter(N).Map([At(x, N)], lambda v: v).As(N).Reduce(_neg_inf(b), lambda acc, v: Call("fmaxf", acc, v)).Store(m)
    return b.Build()


def row_stats_u32(cols=1000):
    """Integer row reductions over u32 [R, C]: wrapping sum, xor and umax
    (the monoid combiners of the row families on a 32-bit integer type)."""
    b = NewBuilder("row_stats_u32_%s" % (cols or "dyn"))
    R, C = b.Dim("R", 0), _static(b, "C", cols)
    x = b.Tensor("x", TU32, R, C)
    outs = [b.Tensor(n, TU32, R) for n in ("sum", "xor", "max")]
    inits = [b.UInt32(0), b.UInt32(0), b.UInt32(0)]
    fns = [lambda acc, v: b.Add(acc, v), lambda acc, v: b.BitXor(acc, v), lambda acc, v: Call("umax", acc, v)]
    for o, i, f in zip(outs, inits, fns):
        b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: v).As(R, C).Reduce(i, f).Store(o, R)
    return b.Build()


def row_sum_bf16(cols=1000):
    """Row sum and max of bf16 [R, C] accumulated in f32 (Cast per element)."""
    b = NewBuilder("row_sum_bf16_%s" % (cols or "dyn"))
    R, C = b.Dim("R", 0), _static(b, "C", cols)
    x = b.Tensor("x", TBF16, R, C)
    s = b.Tensor("sum", TF32, R)
    m = b.Tensor("max", TF32, R)
    (b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: Cast(v, TF32)).As(R, C)
     .Reduce(b.Float32(0), _sum(b)).Store(s, R))
    (b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: Cast(v, TF32)).As(R, C)
     .Reduce(_neg_inf(b), lambda acc, v: Call("fmaxf", acc, v)).Store(m, R))
    return b.Build()


def row_sum_u8(cols=1000):
    """Byte rows summed into u32 (Cast per element), then scaled to f32 by a
    piped map: out = f32(sum) * scale."""
    b = NewBuilder("row_sum_u8_%s" % (cols or "dyn"))
    R, C = b.Dim("R", 0), _static(b, "C", cols)
    x = b.Tensor("x", TU8, R, C)
    out = b.Tensor("out", TF32, R)
    scale = b.ScalarParam("scale", TF32)
    (b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: Cast(v, TU32)).As(R, C)
     .Reduce(b.UInt32(0), lambda acc, v: b.Add(acc, v))
     .Map([], lambda v: b.Mul(Cast(v, TF32), scale)).As(R).Store(out, R))
    return b.Build()


def col_sum_max():
    """Column sum and max of f32 x [R, C] (both dims run-time): reductions
    over the non-contiguous axis, written As(C, R) so the reduce drops R (the
    reference's middle-axis form, testing/kernels/runtime/row_sum.tca)."""
    b = NewBuilder("col_sum_max_dyn")
    R, C = b.Dim("R", 0), b.Dim("C", 0)
    x = b.Tensor("x", TF32, R, C)
    s = b.Tensor("sum", TF32, C)
    m = b.Tensor("max", TF32, C)
    b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: v).As(C, R).Reduce(b.Float32(0), _sum(b)).Store(s, C)
    (b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: v).As(C, R)
     .Reduce(_neg_inf(b), lambda acc, v: Call("fmaxf", acc, v)).Store(m, C))
    return b.Build()


def col_mean_var(local_mean=False):
    """Per-column mean and centred variance of f32 x [B, R, C] over R (the
    statistics of a batch norm over the leading axes): mean = sum_r x * inv_n,
    var = sum_r (x - mean)^2 * inv_n. The variance reads the mean at its own
    column, so one column nest runs two passes; with `local_mean` the mean is
    a local only the variance reads."""
    b = NewBuilder("col_mean_var%s_dyn" % ("_l" if local_mean else ""))
    B, R, C = b.Dim("B", 0), b.Dim("R", 0), b.Dim("C", 0)
    x = b.Tensor("x", TF32, B, R, C)
    mean = b.Local("mean", TF32, B, C) if local_mean else b.Tensor("mean", TF32, B, C)
    var = b.Tensor("var", TF32, B, C)
    inv_n = b.ScalarParam("inv_n", TF32)
    (b.Stmt().Iter(B, R, C).Map([At(x, B, R, C)], lambda v: v).As(B, C, R)
     .Reduce(b.Float32(0), _sum(b))
     .Map([], lambda v: b.Mul(v, inv_n)).As(B, C).Store(mean, B, C))
    (b.Stmt().Iter(B, R, C)
     .Map([At(x, B, R, C), At(mean, B, C)], lambda l, m: b.Mul(b.Sub(l, m), b.Sub(l, m))).As(B, C, R)
     .Reduce(b.Float32(0), _sum(b))
     .Map([], lambda v: b.Mul(v, inv_n)).As(B, C).Store(var, B, C))
    return b.Build()


def col_mean_bf16():
    """Per (batch, column) scaled sum of bf16 x [B, R, C] over R, plus a
    column offset: out[b, c] = sum_r f32(x[b, r, c]) * scale + g[c]."""
    b = NewBuilder("col_mean_bf16")
    B, R, C = b.Dim("B", 0), b.Dim("R", 0), b.Dim("C", 0)
    x = b.Tensor("x", TBF16, B, R, C)
    g = b.Tensor("g", TF32, C)
    out = b.Tensor("out", TF32, B, C)
    scale = b.ScalarParam("scale", TF32)
    (b.Stmt().Iter(B, R, C).Map([At(x, B, R, C)], lambda v: Cast(v, TF32)).As(B, C, R)
     .Reduce(b.Float32(0), _sum(b))
     .Map([At(g, C)], lambda v, gg: b.Add(b.Mul(v, scale), gg)).As(B, C).Store(out, B, C))
    return b.Build()


def col_mean_var_bf16():
    """Per-column mean and centred variance of bf16 x [B, R, C] over R, in
    f32: mean = sum_r f32(x) * inv_n, var = sum_r (f32(x) - mean)^2 *
    inv_n (16-byte vectors of 8 bf16 columns; the one-read column lowering
    with a cast in the mean's body)."""
    b = NewBuilder("col_mean_var_bf16")
    B, R, C = b.Dim("B", 0), b.Dim("R", 0), b.Dim("C", 0)
    x = b.Tensor("x", TBF16, B, R, C)
    mean = b.Tensor("mean", TF32, B, C)
    var = b.Tensor("var", TF32, B, C)
    inv_n = b.ScalarParam("inv_n", TF32)
    (b.Stmt().Iter(B, R, C).Map([At(x, B, R, C)], lambda v: Cast(v, TF32)).As(B, C, R)
     .Reduce(b.Float32(0), _sum(b))
     .Map([], lambda v: b.Mul(v, inv_n)).As(B, C).Store(mean, B, C))
    (b.Stmt().Iter(B, R, C)
     .Map([At(x, B, R, C), At(mean, B, C)],
          lambda l, m: b.Mul(b.Sub(Cast(l, TF32), m), b.Sub(Cast(l, TF32), m))).As(B, C, R)
     .Reduce(b.Float32(0), _sum(b))
     .Map([], lambda v: b.Mul(v, inv_n)).As(B, C).Store(var, B, C))
    return b.Build()


def col_sum_u8():
    """Column sums of bytes u8 x [R, C] into u32 (16-element vectors)."""
    b = NewBuilder("col_sum_u8")
    R, C = b.Dim("R", 0), b.Dim("C", 0)
    x = b.Tensor("x", TU8, R, C)
    s = b.Tensor("sum", TU32, C)
    (b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: Cast(v, TU32)).As(C, R)
     .Reduce(b.UInt32(0), lambda acc, v: b.Add(acc, v)).Store(s, C))
    return b.Build()


def chain_sum_max():
    """Chained reductions in one chain (pkg/chain.go:262 twice): o[b] =
    s * max over r of (sum over c of x[b, r, c])."""
    b = NewBuilder("chain_sum_max")
    B, R, C = b.Dim("B", 0), b.Dim("R", 0), b.Dim("C", 0)
    x = b.Tensor("x", TF32, B, R, C)
    o = b.Tensor("o", TF32, B)
    s = b.ScalarParam("s", TF32)
    (b.Stmt().Iter(B, R, C).Map([At(x, B, R, C)], lambda v: v).As(B, R, C)
     .Reduce(b.Float32(0), _sum(b))
     .Reduce(_neg_inf(b), lambda acc, v: Call("fmaxf", acc, v))
     .Map([], lambda v: b.Mul(v, s)).As(B).Store(o, B))
    return b.Build()


def chain_total():
    """A whole-matrix sum written as two chained sums: t = sum_r sum_c x[r, c]."""
    b = NewBuilder("chain_total")
    R, C = b.Dim("R", 0), b.Dim("C", 0)
    x = b.Tensor("x", TF32, R, C)
    t = b.Tensor("t", TF32)
    (b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: v).As(R, C)
     .Reduce(b.Float32(0), _sum(b)).Reduce(b.Float32(0), _sum(b)).Store(t))
    return b.Build()


def chain3_max_total():
    """Three chained reductions (pkg/chain.go:262 three times): t = max over b
    of (sum over r of (sum over c of x[b, r, c]))."""
    b = NewBuilder("chain3_max_total")
    B, R, C = b.Dim("B", 0), b.Dim("R", 0), b.Dim("C", 0)
    x = b.Tensor("x", TF32, B, R, C)
    t = b.Tensor("t", TF32)
    (b.Stmt().Iter(B, R, C).Map([At(x, B, R, C)], lambda v: v).As(B, R, C)
     .Reduce(b.Float32(0), _sum(b)).Reduce(b.Float32(0), _sum(b))
     .Reduce(_neg_inf(b), lambda acc, v: Call("fmaxf", acc, v)).Store(t))
    return b.Build()


def chain_halving():
    """A chained reduction whose outer fold is not associative: t = fold over
    r of (acc / 2 + sum over c of x[r, c]) from 0, in ascending r."""
    b = NewBuilder("chain_halving")
    R, C = b.Dim("R", 0), b.Dim("C", 0)
    x = b.Tensor("x", TF32, R, C)
    t = b.Tensor("t", TF32)
    (b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: v).As(R, C)
     .Reduce(b.Float32(0), _sum(b))
     .Reduce(b.Float32(0), lambda acc, v: b.Add(b.Mul(acc, b.Float32(0.5)), v)).Store(t))
    return b.Build()


# Expression-layer parity programs: one output per expression over [N]
# operands, so every operator, builtin and cast of the DSL (pkg/expr.go:
# 140-341, internal/ir/builtins.go:25-33) runs on the device.
EXPR_F32 = [
    ("add", lambda b, l, r: b.Add(l, r)), ("sub", lambda b, l, r: b.Sub(l, r)),
    ("mul", lambda b, l, r: b.Mul(l, r)), ("div", lambda b, l, r: b.Div(l, r)),
    ("neg", lambda b, l, r: b.Neg(l)), ("sel", lambda b, l, r: Select(b.Lt(l, r), l, r)),
    ("fmin", lambda b, l, r: Call("fminf", l, r)), ("fmax", lambda b, l, r: Call("fmaxf", l, r)),
    ("fma", lambda b, l, r: Call("fmaf", l, r, l)), ("fabs", lambda b, l, r: Call("fabsf", l)),
    ("sqrt", lambda b, l, r: Call("sqrtf", l)), ("exp", lambda b, l, r: Call("expf", l)),
    ("log", lambda b, l, r: Call("logf", l)), ("rsqrt", lambda b, l, r: Call("rsqrtf", l)),
    ("sin", lambda b, l, r: Call("sinf", l)), ("cos", lambda b, l, r: Call("cosf", l)),
    ("tanh", lambda b, l, r: Call("tanhf", l)),
]
EXPR_I32 = [
    ("add", lambda b, l, r: b.Add(l, r)), ("sub", lambda b, l, r: b.Sub(l, r)),
    ("mul", lambda b, l, r: b.Mul(l, r)), ("div", lambda b, l, r: b.Div(l, r)),
    ("mod", lambda b, l, r: b.Mod(l, r)), ("and", lambda b, l, r: b.BitAnd(l, r)),
    ("or", lambda b, l, r: b.BitOr(l, r)), ("xor", lambda b, l, r: b.BitXor(l, r)),
    ("shl", lambda b, l, r: b.Shl(b.BitAnd(l, b.Int32(0xFFFF)), b.BitAnd(r, b.Int32(15)))),
    ("shr", lambda b, l, r: b.Shr(l, b.BitAnd(r, b.Int32(31)))),
    ("neg", lambda b, l, r: b.Neg(l)), ("not", lambda b, l, r: b.BitsNot(l)),
    ("cmp", lambda b, l, r: Select(b.And(b.Lt(l, r), b.Ne(l, b.Int32(0))), b.Int32(1),
                                   Select(b.Or(b.Ge(l, r), b.Eq(r, b.Int32(7))), b.Int32(2), b.Int32(3)))),
]
EXPR_U32 = [
    ("add", lambda b, l, r: b.Add(l, r)), ("sub", lambda b, l, r: b.Sub(l, r)),
    ("mul", lambda b, l, r: b.Mul(l, r)), ("div", lambda b, l, r: b.Div(l, r)),
    ("mod", lambda b, l, r: b.Mod(l, r)), ("shr", lambda b, l, r: b.Shr(l, b.BitAnd(r, b.UInt32(31)))),
    ("umin", lambda b, l, r: Call("umin", l, r)), ("umax", lambda b, l, r: Call("umax", l, r)),
    ("not", lambda b, l, r: b.BitsNot(l)), ("le", lambda b, l, r: Select(b.Le(l, r), l, r)),
]


def _expr_program(name, elem, table):
    b = NewBuilder(name)
    N = b.Dim("N", 0)
    x, y = b.Tensor("x", elem, N), b.Tensor("y", elem, N)
    def bound(f):
        return lambda l, r: f(b, l, r)
    for out_name, f in table:
        out = b.Tensor(out_name, elem, N)
        b.Stmt().Iter(N).Map([At(x, N), At(y, N)], bound(f)).As(N).Store(out, N)
    return b.Build()


def expr_casts():
    """The casts between element types, from f32 x and i32 k over [N]."""
    b = NewBuilder("expr_casts")
    N = b.Dim("N", 0)
    x, k = b.Tensor("x", TF32, N), b.Tensor("k", TI32, N)
    outs = [("bf16", TBF16, lambda l, r: Cast(l, TBF16)), ("f16", TF16, lambda l, r: Cast(l, TF16)),
            ("trunc", TI32, lambda l, r: Cast(l, TI32)), ("tof32", TF32, lambda l, r: Cast(r, TF32)),
            ("tou8", TU8, lambda l, r: Cast(r, TU8)), ("tou32", TU32, lambda l, r: Cast(r, TU32)),
            ("bf16f32", TF32, lambda l, r: Cast(Cast(l, TBF16), TF32))]
    for out_name, elem, f in outs:
        out = b.Tensor(out_name, elem, N)
        b.Stmt().Iter(N).Map([At(x, N), At(k, N)], f).As(N).Store(out, N)
    return b.Build()


def copy_f32():
    """y = x over [R, C]: the plain copy whose counter readings calibrate
    FETCH_SIZE / WRITE_SIZE (known bytes in, known bytes out)."""
    b = NewBuilder("copy_f32")
    R, C = b.Dim("R", 0), b.Dim("C", 0)
    x = b.Tensor("x", TF32, R, C)
    y = b.Tensor("y", TF32, R, C)
    b.Stmt().Iter(R, C).Map([At(x, R, C)], lambda v: v).As(R, C).Store(y, R, C)
    return b.Build()


def _matmul(name, elem, b_nk=False, epilogue=None, scalars=(), names=None):
    """names = (M, K, N, lhs, rhs) spellings. Dims are declared in
    first-appearance order (M, K, N), as the .tca frontend declares them."""
    nm = names or ("M", "K", "N", "lhs", "rhs")
    b = NewBuilder(name)
    M, K, N = b.Dim(nm[0], 0), b.Dim(nm[1], 0), b.Dim(nm[2], 0)
    lhs = b.Tensor(nm[3], elem, M, K)
    rhs = b.Tensor(nm[4], elem, N, K) if b_nk else b.Tensor(nm[4], elem, K, N)
    out = b.Tensor("out", TF32, M, N)
    sc = [b.ScalarParam(s, TF32) for s in scalars]
    if elem == TF32:
        body = lambda l, r: b.Mul(l, r)  # noqa: E731
    else:
        body = lambda l, r: b.Mul(Cast(l, TF32), Cast(r, TF32))  # noqa: E731
    rb = At(rhs, N, K) if b_nk else At(rhs, K, N)
    ar = (b.Stmt().Iter(M, N, K).Map([At(lhs, M, K), rb], body).As(M, N, K)
          .Reduce(b.Float32(0), _sum(b)))
    if epilogue is not None:
        ar.Map([], lambda v: epilogue(b, v, *sc)).As(M, N).Store(out, M, N)
    else:
        ar.Store(out, M, N)
    return b.Build()


def gemm_f32():
    """C5 fp32."""
    return _matmul("gemm_f32", TF32)


def gemm_bf16():
    """C5 bf16 inputs, fp32 accumulate."""
    return _matmul("gemm_bf16", TBF16)


def gemm_f16():
    """C5's contraction with f16 inputs, fp32 accumulate (the bf16 kernels
    with the f16 MFMAs)."""
    return _matmul("gemm_f16", TF16)


def gemm_f16_nt():
    """f16 inputs with B given as [N][K]."""
    return _matmul("gemm_f16_nt", TF16, b_nk=True)


def gemm_bf16_nt():
    """C5 with B given as [N][K] (the qk_score orientation), bf16 inputs."""
    return _matmul("gemm_bf16_nt", TBF16, b_nk=True)


def gemm_f32_nt():
    """C5 fp32 with B given as [N][K]."""
    return _matmul("gemm_f32_nt", TF32, b_nk=True)


def _bmatmul(name, elem, b_nk=False, a_batched=True, b_batched=True, epilogue=None, scalars=()):
    """out[b][m][n] = sum_k lhs[b][m][k] * rhs[b][k][n] (rhs [b][n][k] when
    b_nk); an operand built without the batch axis is shared by every batch."""
    b = NewBuilder(name)
    B, M, K, N = b.Dim("B", 0), b.Dim("M", 0), b.Dim("K", 0), b.Dim("N", 0)
    lhs = b.Tensor("lhs", elem, *((B, M, K) if a_batched else (M, K)))
    rdims = (N, K) if b_nk else (K, N)
    rhs = b.Tensor("rhs", elem, *(((B,) + rdims) if b_batched else rdims))
    out = b.Tensor("out", TF32, B, M, N)
    sc = [b.ScalarParam(s, TF32) for s in scalars]
    if elem == TF32:
        body = lambda l, r: b.Mul(l, r)  # noqa: E731
    else:
        body = lambda l, r: b.Mul(Cast(l, TF32), Cast(r, TF32))  # noqa: E731
    la = At(lhs, B, M, K) if a_batched else At(lhs, M, K)
    rb = At(rhs, *(((B,) if b_batched else ()) + ((N, K) if b_nk else (K, N))))
    ar = (b.Stmt().Iter(B, M, N, K).Map([la, rb], body).As(B, M, N, K)
          .Reduce(b.Float32(0), _sum(b)))
    if epilogue is not None:
        ar.Map([], lambda v: epilogue(b, v, *sc)).As(B, M, N).Store(out, B, M, N)
    else:
        ar.Store(out, B, M, N)
    return b.Build()


def bmm_f32():
    """A batch of fp32 contractions, both operands per batch."""
    return _bmatmul("bmm_f32", TF32)


def bmm_bf16_nt():
    """A batch of bf16 contractions with B given as [b][N][K]: the per-head
    scores Q @ K^T of attention."""
    return _bmatmul("bmm_bf16_nt", TBF16, b_nk=True)


def bmm_f32_nt_shared_a():
    """fp32 contractions with one A [M][K] shared by every batch and B given
    as [b][N][K]."""
    return _bmatmul("bmm_f32_nt_shared_a", TF32, b_nk=True, a_batched=False)


def bmm_bf16():
    """A batch of bf16 contractions, B given as [b][K][N]."""
    return _bmatmul("bmm_bf16", TBF16)


def bmm_f16_shared_scale():
    """A batch of f16 contractions against one shared B, times a scale."""
    return _bmatmul("bmm_f16_shared_scale", TF16, b_batched=False,
                    epilogue=lambda b, v, s: b.Mul(v, s), scalars=("scale",))


# ---- the reference suite (testing/kernels/**.tca) ------------------------

def _rank3_reduce(name, k_extent, body, scalars=(), piped=None, piped_scalars=(), middle=False):
    """out[i][j] = sum_k f(x, z) over x, z [R, C, K] (or [R, K, C] when the
    reduced axis is the middle one, as row_sum.tca and softmax.tca)."""
    b = NewBuilder(name)
    kname = "K" if k_extent == 0 else "e%d" % k_extent
    if middle:  # dims in first-appearance order of x's shape, as the .tca frontend declares them
        R, K, C = b.Dim("R", 0), b.Dim(kname, k_extent), b.Dim("C", 0)
    else:
        R, C, K = b.Dim("R", 0), b.Dim("C", 0), b.Dim(kname, k_extent)
    shape = (R, K, C) if middle else (R, C, K)
    x = b.Tensor("x", TF32, *shape)
    z = b.Tensor("z", TF32, *shape)
    out = b.Tensor("out", TF32, R, C)
    sc = [b.ScalarParam(s, TF32) for s in scalars]
    psc = [b.ScalarParam(s, TF32) for s in piped_scalars]
    # the reduced axis iterates last (the frontend's relocation)
    ar = (b.Stmt().Iter(R, C, K)
          .Map([At(x, *shape), At(z, *shape)], lambda v, w: body(b, v, w, *sc))
          .As(R, C, K)
          .Reduce(b.Float32(0), _sum(b)))
    if piped is not None:
        ar.Map([], lambda v: piped(b, v, *psc)).As(R, C).Store(out, R, C)
    else:
        ar.Store(out, R, C)
    return b.Build()


def suite_dup_expr():
    # testing/kernels/dedup/dup_expr.tca:23-37
    return _rank3_reduce(
        "dup_expr", 8,
        lambda b, v, w, gain, bias: b.Mul(b.Add(b.Mul(b.Add(b.Mul(v, v), b.Mul(v, v)), gain),
                                                b.Mul(b.Add(b.Mul(v, v), b.Mul(v, v)), bias)), w),
        scalars=("gain", "bias"))


def suite_dup_const():
    # testing/kernels/dedup/dup_const.tca:16-30
    def body(b, v, w):
        f = b.Float32
        t1 = b.Mul(b.Mul(f(0.5), b.Add(v, b.Mul(b.Mul(f(0.5), v), v))), b.Add(f(1.0), b.Mul(f(0.044715), v)))
        arg = b.Add(b.Mul(f(0.79788456), b.Add(v, b.Mul(f(0.044715), v))), b.Mul(b.Mul(f(0.79788456), f(0.5)), v))
        t2 = b.Mul(Call("tanhf", arg), b.Sub(f(1.0), f(0.5)))
        return b.Mul(b.Add(t1, t2), w)
    return _rank3_reduce("dup_const", 8, body)


def suite_axpy3():
    # testing/kernels/fusion/axpy3.tca:14-36
    return _rank3_reduce(
        "axpy3", 4, lambda b, v, w, alpha, beta: b.Add(b.Mul(alpha, v), b.Mul(beta, w)),
        scalars=("alpha", "beta"),
        piped=lambda b, v, gamma: b.Add(v, b.Mul(gamma, Call("tanhf", v))), piped_scalars=("gamma",))


def suite_scale_copy():
    # testing/kernels/runtime/scale_copy.tca:16-33
    return _rank3_reduce("scale_copy", 4, lambda b, v, w, gain, bias: b.Mul(b.Add(b.Mul(gain, v), bias), w),
                         scalars=("gain", "bias"))


def suite_row_sum():
    # testing/kernels/runtime/row_sum.tca:17-33 (reduce over the middle axis)
    return _rank3_reduce("row_sum", 4, lambda b, v, w: b.Mul(v, w), middle=True)


def suite_softmax():
    # testing/kernels/fusion/softmax.tca:24-41 (reduce over the middle axis)
    return _rank3_reduce("softmax", 8, lambda b, v, w: b.Mul(Call("expf", v), w), middle=True)


def suite_transpose():
    # testing/kernels/tiling/transpose.tca:24-40 (dynamic K, written as clause)
    return _rank3_reduce("transpose", 0, lambda b, v, w: b.Mul(v, w))


def suite_layernorm():
    # testing/kernels/llm/layernorm.tca:17-40 (RMS-flavoured core, dynamic K)
    return _rank3_reduce("layernorm", 0, lambda b, v, w: b.Mul(b.Mul(v, v), w),
                         piped=lambda b, v, inv_n, eps: b.Mul(v, Call("rsqrtf", b.Add(b.Mul(v, inv_n), eps))),
                         piped_scalars=("inv_n", "eps"))


def _gelu(b, v):
    f = b.Float32
    inner = b.Mul(f(0.79788456), b.Add(v, b.Mul(b.Mul(b.Mul(f(0.044715), v), v), v)))
    return b.Mul(b.Mul(f(0.5), v), b.Add(f(1.0), Call("tanhf", inner)))


def suite_gemm(name="gemm"):
    # testing/kernels/llm/gemm.tca:7-22 (also mm_small / mm_mid / mm_splitk)
    return _matmul(name, TF32)


def suite_mlp():
    # testing/kernels/fusion/mlp.tca:10-32
    return _matmul("mlp", TF32, epilogue=lambda b, v: _gelu(b, v))


def suite_qk_score():
    # testing/kernels/llm/qk_score.tca:7-31 (kk indexed [n][k])
    return _matmul("qk_score", TF32, b_nk=True, epilogue=lambda b, v, scale: b.Mul(v, scale), scalars=("scale",),
                   names=("H", "D", "N", "q", "kk"))


# name -> (builder, suite dims [d0, d1, d2], scalars) ; dims/scalars from testing/suite.toml
SUITE = {
    "dup_expr": (suite_dup_expr, [256, 256, 8], {"gain": 1.5, "bias": 0.25}),
    "dup_const": (suite_dup_const, [256, 256, 8], {}),
    "axpy3": (suite_axpy3, [512, 512, 4], {"alpha": 2.0, "beta": 0.5, "gamma": 0.75}),
    "mlp": (suite_mlp, [64, 128, 64], {}),
    "softmax": (suite_softmax, [128, 8, 256], {}),
    "mm_small": (lambda: suite_gemm("mm_small"), [32, 32, 32], {}),
    "mm_mid": (lambda: suite_gemm("mm_mid"), [128, 256, 64], {}),
    "mm_splitk": (lambda: suite_gemm("mm_splitk"), [64, 128, 64], {}),
    "transpose": (suite_transpose, [192, 96, 8], {}),
    "row_sum": (suite_row_sum, [512, 4, 1024], {}),
    "scale_copy": (suite_scale_copy, [512, 512, 4], {"gain": 1.25, "bias": -0.125}),
    "gemm": (suite_gemm, [128, 128, 96], {}),
    "qk_score": (suite_qk_score, [128, 64, 192], {"scale": 0.125}),
    "layernorm": (suite_layernorm, [128, 256, 64], {"inv_n": 0.015625, "eps": 0.00001}),
}

# Programs build() precompiles: (factory, emit flags). The generic-family
# variants (fusion and MFMA disabled) exist so tests can check every family
# against the same oracle.
def ew_bias_tr():
    """y[r][c] = x[r][c] * g[c] + b[r] + z[c][r]: an elementwise map with an
    aligned, a column-broadcast, a row-broadcast and a transposed operand (the
    transposed one staged through LDS tiles)."""
    b = NewBuilder("ew_bias_tr")
    R, C = b.Dim("R", 0), b.Dim("C", 0)
    x, z = b.Tensor("x", TF32, R, C), b.Tensor("z", TF32, C, R)
    g, bb = b.Tensor("g", TF32, C), b.Tensor("b", TF32, R)
    y = b.Tensor("y", TF32, R, C)
    (b.Stmt().Iter(R, C)
     .Map([At(x, R, C), At(g, C), At(bb, R), At(z, C, R)], lambda v, w, u, t: b.Add(b.Add(b.Mul(v, w), u), t))
     .As(R, C).Store(y, R, C))
    return b.Build()


# ---- the reference's own end-to-end programs (internal/e2e, pkg) ---------
# Each is the graph of one of the reference's numerical e2e tests, written
# through the pkg rungs; tests/test_gpu_e2e.py runs them on the reference's
# shapes and inputs (elem(i), testing/runners/common.cuh:19-21) against its
# CPU references and tolerance (internal/e2e/e2e_test.go:20, reduceTol 2e-3).

def e2e_redwarp():
    """out[r] = sum_c lhs[r][c]: the reduce_warp golden's graph
    (internal/e2e/e2e_test.go:134-179 runner, reduceReference :227-240), which
    TestReduceT1E2E also lowers (internal/e2e/reduce3_test.go:255-266)."""
    b = NewBuilder("redwarp")
    R, C = b.Dim("d0", 0), b.Dim("d1", 0)
    lhs = b.Tensor("lhs", TF32, R, C)
    out = b.Tensor("out", TF32, R)
    b.Stmt().Iter(R, C).Map([At(lhs, R, C)], lambda v: v).As(R, C).Reduce(b.Float32(0), _sum(b)).Store(out, R)
    return b.Build()


def e2e_reduce3():
    """out[i][j] = sum_k lhs[i][j][k], the rank-3 last-axis reduce
    (internal/e2e/reduce3_test.go:81-117 graph, reduce3Reference :288-300)."""
    b = NewBuilder("red3")
    d0, d1, d2 = b.Dim("d0", 0), b.Dim("d1", 0), b.Dim("d2", 0)
    lhs = b.Tensor("lhs", TF32, d0, d1, d2)
    out = b.Tensor("out", TF32, d0, d1)
    (b.Stmt().Iter(d0, d1, d2).Map([At(lhs, d0, d1, d2)], lambda v: v).As(d0, d1, d2)
     .Reduce(b.Float32(0), _sum(b)).Store(out, d0, d1))
    return b.Build()


def e2e_matmul_store():
    """out[m][n][k] = lhs[m][k] * rhs[n][k]: the matmul_store golden's graph
    (the MmLaunch signature, internal/e2e/e2e_test.go:69-71; matmulReference
    :202-225), a rank-3 map with broadcast operands and no reduction."""
    b = NewBuilder("mm")
    d0, d1, d2 = b.Dim("d0", 0), b.Dim("d1", 0), b.Dim("d2", 0)
    lhs = b.Tensor("lhs", TF32, d0, d2)
    rhs = b.Tensor("rhs", TF32, d1, d2)
    out = b.Tensor("out", TF32, d0, d1, d2)
    (b.Stmt().Iter(d0, d1, d2).Map([At(lhs, d0, d2), At(rhs, d1, d2)], lambda l, r: b.Mul(l, r))
     .As(d0, d1, d2).Store(out, d0, d1, d2))
    return b.Build()


def e2e_matmul_scale():
    """output[m][k] = scale * sum_n lhs[m][n] * rhs[n][k]: the doc-pinned
    oracle program built through the public builder (pkg/oracle_test.go:17-53),
    the frontend matmul_scale's semantics (internal/e2e/frontend_test.go:
    194-208)."""
    b = NewBuilder("matmul_scale")
    m, k, n = b.Dim("m", 0), b.Dim("k", 0), b.Dim("n", 0)
    lhs, rhs = b.Tensor("lhs", TF32, m, n), b.Tensor("rhs", TF32, n, k)
    out = b.Tensor("output", TF32, m, k)
    scale = b.ScalarParam("scale", TF32)
    (b.Stmt().Iter(m, k, n).Map([At(lhs, m, n), At(rhs, n, k)], lambda l, r: b.Mul(l, r)).As(m, k, n)
     .Reduce(b.Float32(0), lambda a, v: b.Add(a, v)).Map([], lambda v: b.Mul(v, scale)).As(m, k)
     .Store(out, m, k))
    return b.Build()


def _tca_kernel(path):
    def build():
        from . import syntax
        return syntax.ParseModule(path).Kernels[0].Build()
    return build


E2E_TCA_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tca", "e2e")

E2E = {
    "redwarp": e2e_redwarp,
    "red3": e2e_reduce3,
    "mm": e2e_matmul_store,
    "matmul_scale_pkg": e2e_matmul_scale,
    # the frontend fixture in both forms of its root map (as clause written,
    # and inferred), compiled from .tca text (internal/e2e/frontend_test.go:
    # 340-396)
    "matmul_scale_written": _tca_kernel(os.path.join(E2E_TCA_DIR, "matmul_scale_written.tca")),
    "matmul_scale_omitted": _tca_kernel(os.path.join(E2E_TCA_DIR, "matmul_scale_omitted.tca")),
}


CONFIG_PROGRAMS = {
    "chain_sum_max": chain_sum_max,
    "chain_total": chain_total,
    "chain3_max_total": chain3_max_total,
    "chain_halving": chain_halving,
    "col_sum_max_dyn": col_sum_max,
    "col_mean_bf16": col_mean_bf16,
    "col_mean_var_dyn": col_mean_var,
    "col_mean_var_l_dyn": lambda: col_mean_var(True),
    "col_mean_var_bf16": col_mean_var_bf16,
    "col_sum_u8": col_sum_u8,
    "scale_relu": scale_relu,
    "scale_relu_map": scale_relu_map,
    "row_sum_max_8192": lambda: row_sum_max(8192),
    "softmax_4096": lambda: softmax(4096),
    "layernorm_1024": lambda: layernorm(1024),
    "gemm_f32": gemm_f32,
    "gemm_bf16": gemm_bf16,
    "gemm_bf16_nt": gemm_bf16_nt,
    "gemm_f32_nt": gemm_f32_nt,
    "gemm_f16": gemm_f16,
    "gemm_f16_nt": gemm_f16_nt,
    # batched contractions: one (m, n) grid of tiles per batch
    "bmm_f32": bmm_f32,
    "bmm_bf16_nt": bmm_bf16_nt,
    "bmm_f16_shared_scale": bmm_f16_shared_scale,
    "bmm_f32_nt_shared_a": bmm_f32_nt_shared_a,
    "bmm_bf16": bmm_bf16,
    # small-row variants exercised by the parity tests (tails, few lanes per row)
    "row_sum_max_1000": lambda: row_sum_max(1000),
    "row_sum_max_64": lambda: row_sum_max(64),
    "softmax_200": lambda: softmax(200),
    "layernorm_96": lambda: layernorm(96),
    "softmax_16384": lambda: softmax(16384),
    "copy_f32": copy_f32,
    # an elementwise map with broadcast and transposed operands
    "ew_bias_tr": ew_bias_tr,
    # the same nests with the row length a run-time dim: the streaming family
    "row_sum_max_dyn": lambda: row_sum_max(0),
    "softmax_dyn": lambda: softmax(0),
    "layernorm_dyn": lambda: layernorm(0),
    "vec_sum_max": vec_sum_max,
    # a per-row chain fused between the reductions and the row map
    "layernorm_rstd_1024": lambda: layernorm_rstd(1024),
    "layernorm_rstd_dyn": lambda: layernorm_rstd(0),
    "row_stats_shift_dyn": lambda: row_stats_shift(0),
    "softmax_affine_dyn": lambda: softmax_affine(0),
    "row_moments_affine_dyn": lambda: row_moments_affine(0),
    "softmax_bf16_dyn": lambda: softmax_bf16(0),
    # the expression layer: every operator, builtin and cast on the device
    "expr_f32": lambda: _expr_program("expr_f32", TF32, EXPR_F32),
    "expr_i32": lambda: _expr_program("expr_i32", TI32, EXPR_I32),
    "expr_u32": lambda: _expr_program("expr_u32", TU32, EXPR_U32),
    "expr_casts": expr_casts,
    # other element types through the row and streaming families
    "row_stats_u32_1000": lambda: row_stats_u32(1000),
    "row_stats_u32_dyn": lambda: row_stats_u32(0),
    "row_sum_bf16_1000": lambda: row_sum_bf16(1000),
    "row_sum_bf16_dyn": lambda: row_sum_bf16(0),
    "row_sum_u8_1000": lambda: row_sum_u8(1000),
    "row_sum_u8_dyn": lambda: row_sum_u8(0),
}


def all_builds():
    """(program factory, flags) pairs for every code object build() makes."""
    from .pkg import EMIT_NO_FUSION, EMIT_NO_GEMM, EMIT_NO_GEMM_SPLIT, EMIT_NO_PASS_FUSION
    out = []
    for name, f in sorted(CONFIG_PROGRAMS.items()):
        out.append((name, f, 0))
    for name, (f, _, _) in sorted(SUITE.items()):
        out.append(("suite_" + name, f, 0))
    for name, f in sorted(E2E.items()):
        out.append(("e2e_" + name, f, 0))
    # generic-family lowering of the configs (cross-family parity)
    for name in ("scale_relu", "row_sum_max_1000", "softmax_200", "layernorm_96", "gemm_f32", "chain_sum_max",
                 "chain_total", "chain3_max_total"):
        out.append((name + "_generic", CONFIG_PROGRAMS[name], EMIT_NO_FUSION | EMIT_NO_GEMM))
    # the contractions on their tile kernels alone: small output planes take
    # the small-tile kernel otherwise, and the tests hold both to the oracle
    for name in TILE_ONLY:
        out.append((name + "_tiles", CONFIG_PROGRAMS[name], EMIT_NO_GEMM_SPLIT))
    # multi-pass nests with each pass reading its input (the one-read
    # fusions' unfused lowering, held to the same oracle)
    for name in PASS_FUSED:
        out.append((name + "_passes", CONFIG_PROGRAMS[name], EMIT_NO_PASS_FUSION))
    return out


# Programs whose passes fuse into one read by default (online softmax
# normaliser, pairwise mean/variance); the tests also run them unfused.
PASS_FUSED = ("softmax_dyn", "layernorm_dyn", "row_stats_shift_dyn", "col_mean_var_dyn", "col_mean_var_l_dyn",
              "col_mean_var_bf16", "softmax_affine_dyn", "row_moments_affine_dyn", "softmax_bf16_dyn")


# Contractions the tests also run with EMIT_NO_GEMM_SPLIT (the 128/256 tile
# kernels at every shape).
TILE_ONLY = ("gemm_f32", "gemm_f32_nt", "gemm_bf16", "gemm_bf16_nt", "gemm_f16", "gemm_f16_nt", "bmm_f32",
             "bmm_bf16_nt", "bmm_f16_shared_scale", "bmm_f32_nt_shared_a", "bmm_bf16")
