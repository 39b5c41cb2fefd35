"""The .tca text frontend (include/tca_syntax.h): lexer, parser, semantic
rules, include resolution and the lowering into the builder.

Parity anchors, all host-only:
  - the reference's parser golden (internal/syntax/parser/testdata/
    appendix_a.txt) against this parser's dump of the same source;
  - the reference's own 14-program corpus (testing/kernels/**.tca) compiled
    unchanged to IR identical to the pkg-API restatements in programs.SUITE;
  - tcacomp_amd/tca/configs.tca (the configurations written in .tca) to IR
    identical to programs.CONFIG_PROGRAMS.
The first two read the reference tree when it is mounted and skip otherwise.
Rule tests follow the reference's per-rule-family strategy
(internal/syntax/semacheck/semacheck_test.go): one valid kernel, one edit
per rule, exactly one error mentioning the rule's wording.
"""
import glob
import os
import re

import pytest

from tcacomp_amd import programs, syntax
from tcacomp_amd.pkg import BuildError

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
CONFIGS_TCA = os.path.join(REPO, "tcacomp_amd", "tca", "configs.tca")
needs_ref = pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "internal", "syntax")),
                               reason="reference tree not mounted")

# A valid kernel exercising a root map, a reduction and a piped map with a
# capture (this build's own fixture).
VALID = """kernel scaled(
  a: tensor<dtype=f32, shape=[P, Q]>,
  w: tensor<dtype=f32, shape=[Q, S]>,
  k: f32,
) -> tensor<dtype=f32, shape=[P, S]>
{
  dimvar (p, q, s);
  let r = map on(a[p][q], w[q][s]) as (p, q, s) (u: f32, v: f32) -> f32: u * v
    | reduce(init = 0.0f) on(acc: f32, %0: f32) as (p, s) -> f32: acc + %0
    | map on() [k] (t: f32) -> f32: t * k
    ;
  return r;
}"""


def errors_of(src, check=True):
    """The error lines of a failing parse ([] when it succeeds)."""
    try:
        syntax.ParseSource(src, "t.tca", check=check)
    except BuildError as e:
        return [l for l in str(e).splitlines() if ": error: " in l]
    return []


def want_error(src, needle):
    errs = errors_of(src)
    assert len(errs) == 1, errs
    assert needle in errs[0], errs[0]


# ------------------------------------------------------------ parity anchors

@needs_ref
def test_parse_tree_matches_reference_golden():
    text = open(os.path.join(REF, "internal/syntax/parser/appendix_a_test.go")).read()
    src = re.search(r"appendixASource\s*=\s*`(.*?)`", text, re.S).group(1)
    want = open(os.path.join(REF, "internal/syntax/parser/testdata/appendix_a.txt")).read()
    assert syntax.ParseSource(src, "appendix_a.tca", check=False).Dump() == want


@needs_ref
@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(REF, "testing/kernels/*/*.tca"))),
                         ids=lambda p: os.path.basename(p))
def test_reference_corpus_compiles_unchanged(path):
    name = os.path.basename(path)[:-4]
    m = syntax.ParseModule(path)
    assert m.Runtime == "runtime/tca_runtime.h"
    assert len(m.Kernels) == 1 and m.Kernels[0].CxxName()
    assert m.Kernels[0].Build().IRFull() == programs.SUITE[name][0]().IRFull()


def test_config_sources_build_the_config_programs():
    m = syntax.ParseModule(CONFIGS_TCA)
    assert m.Diagnostics == ""
    factories = {"scale_relu": programs.scale_relu, **programs.CONFIG_PROGRAMS}
    names = [k.Name() for k in m.Kernels]
    assert set(names) >= {"scale_relu_map", "row_sum_max_8192", "softmax_4096", "layernorm_1024",
                          "gemm_f32", "gemm_bf16"}
    for k in m.Kernels:
        p = k.Build()
        ref = factories[k.Name()]()
        assert p.IRFull() == ref.IRFull(), k.Name()
        assert p.emit().families() == ref.emit().families(), k.Name()


# --------------------------------------------------------------------- lexer

@pytest.mark.parametrize("expr,needle", [
    ("u * 1.5", "requires the f/F suffix"),
    ("u * 1.f", "expected digits after '.'"),
    ("u * 1e+f", "exponent has no digits"),
    ("u * 12abc", "malformed numeric literal \"12abc\""),
    ("u * 1.5fx", "malformed numeric literal \"1.5fx\""),
    ("u * 2147483648", "does not fit i32"),
    ("u * 4294967296u", "does not fit u32"),
    ("u $ v", "unexpected character '$'"),
])
def test_lexer_literal_errors(expr, needle):
    src = VALID.replace("u * v", expr)
    errs = errors_of(src, check=False)
    assert errs and needle in errs[0], errs


def test_lexer_positions_and_comments():
    src = "// line one\n/* block\n comment */ kernel k( x: tensor<dtype=f32, shape=[N]> ) -> f32 { $ }"
    errs = errors_of(src, check=False)
    assert errs and errs[0].startswith("t.tca:3:") and "unexpected character" in errs[0], errs
    assert "block comment not terminated" in errors_of("/* open", check=False)[0]
    assert "string literal not terminated" in errors_of('@runtime(cxx_path="abc\n);', check=False)[0]


def test_literal_values():
    src = VALID.replace("init = 0.0f", "init = 1.5e-3f").replace("t * k", "t * k + 0.1f")
    ir = syntax.ParseSource(src).Kernels[0].Build().IR()
    # the reference's constant spelling: shortest float32 digits, %f form
    assert "reduce(init=0.0015, %0," in ir and "+ 0.1)" in ir, ir


# -------------------------------------------------------------------- parser

def test_pipe_escape_and_bitwise_or():
    # '|' before map/reduce ends the stage; elsewhere it is bitwise-or
    src = """kernel k(x: tensor<dtype=u32, shape=[R, C]>, y: tensor<dtype=u32, shape=[R, C]>) -> tensor<dtype=u32, shape=[R]>
{
  dimvar (r, c);
  let o = map on(x[r][c], y[r][c]) (a: u32, b: u32) -> u32: a | b & (a ^ b)
    | reduce(init = 0u) on(acc: u32, %0: u32) -> u32: acc | %0;
  return o;
}"""
    dump = syntax.ParseSource(src, check=False).Dump()
    assert "(| name(a) (& name(b) (^ name(a) name(b))))" in dump
    assert "reduce(init=0u) on(acc:u32, %0:u32) -> u32: (| name(acc) %0)" in dump
    syntax.ParseSource(src).Kernels[0].Build()


def test_precedence_and_forms():
    body = "c ? -u * v + f32(i) : fmaxf(u, v) / 2.0f"
    src = VALID.replace("(u: f32, v: f32) -> f32: u * v", "(u: f32, v: f32) -> f32: " + body)
    dump = syntax.ParseSource(src, check=False).Dump()
    assert ("(select name(c) (+ (* (- name(u)) name(v)) (cast f32 name(i))) "
            "(/ call(fmaxf name(u), name(v)) 2.0f))") in dump


def test_shift_operators_parse_at_c_precedence():
    src = VALID.replace("u * v", "u * v").replace("t * k", "t * k")
    src = src.replace("dtype=f32, shape=[P, Q]", "dtype=u32, shape=[P, Q]").replace(
        "dtype=f32, shape=[Q, S]", "dtype=u32, shape=[Q, S]").replace(
        "(u: f32, v: f32) -> f32: u * v", "(u: u32, v: u32) -> f32: f32(u << 2u + v >> 1u)")
    dump = syntax.ParseSource(src, check=False).Dump()
    assert "(>> (<< name(u) (+ 2u name(v))) 1u)" in dump
    syntax.ParseSource(src).Kernels[0].Build()


def test_parser_reports_and_recovers():
    errs = errors_of("kernel k( -> f32 { let = ; } kernel j() -> f32 { return ; }", check=False)
    assert len(errs) >= 2
    assert any("expected" in e for e in errs)
    assert "does not precede a kernel" in errors_of('kernel k() -> f32 { return x; }\n@name(cxx="K")', check=False)[0]


# Findings of the .tca fuzzer (tests/c/fuzz.cpp under AddressSanitizer and
# UBSan, tests/sanitize.py), kept as regression cases. The recovery skips to a
# ';', '}', 'kernel' or '@' without consuming the last three, so a stray '}'
# at module level, or a statement failing on 'kernel' or '@', recovered to the
# same token forever (the reference's recovery has the same loop,
# internal/syntax/parser/parser.go:105-140); each now reports once and parsing
# goes on past it.
@pytest.mark.parametrize("src,want", [
    ("}", ["1:1: error: expected declaration, found }"]),
    ("} } kernel", ["1:1: error: expected declaration, found }", "1:3: error: expected declaration, found }"]),
    ("kernel k() -> f32 { @ }", ["1:21: error: expected statement, found @"]),
    ("kernel k() -> f32 { kernel k2() -> f32 { return x; } }", ["1:21: error: expected statement, found kernel"]),
])
def test_parser_recovery_always_advances(src, want):
    errs = errors_of(src, check=False)
    for w in want:
        assert any(w in e for e in errs), errs
    assert len(errs) < 10, errs


def test_unchecked_dump_keeps_omitted_cells_empty_and_check_fills_them():
    # root `as` omitted (inferred from the bindings), piped `as` omitted (the
    # live axes), lambda return omitted (the body's type)
    src = VALID.replace(" as (p, q, s)", "").replace("(u: f32, v: f32) -> f32:", "(u: f32, v: f32):")
    raw = syntax.ParseSource(src, check=False).Dump()
    assert "as(p,q,s)" not in raw and "(u:f32, v:f32): " in raw
    filled = syntax.ParseSource(src).Dump()
    assert "map on(a[p][q], w[q][s]) as(p,q,s)" in filled and "map on() as(p,s)" in filled
    assert "(u:f32, v:f32) -> f32: " in filled and "let r: tensor<f32,[P,S]>" in filled
    # with the reduce `as` omitted too, the reduction drops the last live axis
    # (s), so the declared return shape no longer matches
    want_error(src.replace(" as (p, s)", ""), 'bound to shape dim "Q", annotated "S"')


# ------------------------------------------------------------ semantic rules

def test_valid_fixture_is_clean():
    m = syntax.ParseSource(VALID)
    assert m.Diagnostics == ""
    ir = m.Kernels[0].Build().IRFull()
    assert "statement #0 iter(@P, @S, @Q)" in ir


@pytest.mark.parametrize("old,new,needle", [
    ("dimvar (p, q, s);", "dimvar (p, q, s, a);", 'duplicate name "a"'),                       # 5
    ("shape=[P, S]>\n{", "shape=[P, Z]>\n{", '"Z"'),                                            # 6
    ("(u: f32, v: f32)", "(u: i32, v: f32)", "param annotation"),                               # 8
    ("on(a[p][q], w[q][s])", "on(a[p][Q], w[q][s])", "rule 10"),                                # 10
    ("as (p, s) -> f32", "as (p) -> f32", "minus exactly one"),                                 # 11
    ("as (p, s) -> f32", "as (s, p) -> f32", "preserve the live axes"),                         # 11
    ("[k] (t: f32) -> f32:", "[k] (t: f32, x: f32) -> f32:", "rule 13"),                        # 13
    ("[k] (t: f32) -> f32: t * k", "[a] (t: f32) -> f32: t", "not a kernel scalar param"),      # 14
    ("u * v", "u + 1", "operand types differ"),                                                 # 17
    ("u * v", "f32(u)", "redundant cast"),                                                      # 19
    ("u * v", "nosuch(u)", "not a registered pure scalar builtin"),                             # 20
    ("u * v", "u ? u : v", "must be bool"),                                                     # 18
    ("u * v", "u * %0", "no pipe slot"),
    ("return r;", "return k;", "not a let-bound tensor"),                                       # 25
    ("acc + %0", "acc + 1", "operand types differ"),
    ("init = 0.0f", "init = 0", "reduce init has type i32"),
])
def test_rule_families(old, new, needle):
    src = VALID.replace(old, new, 1)
    assert src != VALID
    want_error(src, needle)


def test_binding_rank_rule_9():
    # the unbound dimvar then cascades into the `as` checks; rule 9 comes first
    errs = errors_of(VALID.replace("on(a[p][q], w[q][s])", "on(a[p][q], w[q])", 1))
    assert errs and "subscript count 1 does not match tensor rank 2" in errs[0] and "rule 9" in errs[0]


def test_root_as_must_cover_the_bound_dimvars():
    src = """kernel k(t: tensor<dtype=f32, shape=[M, N]>) -> tensor<dtype=f32, shape=[M]> {
  dimvar (a, b);
  let out = map on(t[a][b]) as (a) (x: f32) -> f32: x;
  return out;
}"""
    want_error(src, "rule 11")


def test_chain_must_open_with_a_root_map():
    src = VALID.replace(
        "let r = map on(a[p][q], w[q][s]) as (p, q, s) (u: f32, v: f32) -> f32: u * v",
        "let r = map on() [k] (t: f32) -> f32: t * k", 1)
    want_error(src, "rule 26")


def test_unused_capture_is_a_warning():
    m = syntax.ParseSource(VALID.replace("[k] (t: f32) -> f32: t * k", "[k] (t: f32) -> f32: t"))
    assert "warning" in m.Diagnostics and "never used" in m.Diagnostics


def test_module_rules():
    assert "duplicate kernel name" in errors_of(
        "kernel a() -> f32 { return x; }\nkernel a() -> f32 { return x; }")[0]
    assert any("string literal" in e for e in errors_of("@runtime(cxx_path=3);\nkernel a() -> f32 { return x; }"))
    assert any("unknown annotation" in e for e in errors_of("@bogus() kernel a() -> f32 { return x; }"))


# ------------------------------------------------------------------- modules

def _write(tmp_path, name, text):
    p = tmp_path / name
    p.parent.mkdir(parents=True, exist_ok=True)
    p.write_text(text)
    return str(p)


def _kernel(name):
    return VALID.replace("kernel scaled(", "kernel %s(" % name)


def test_includes_merge_in_order(tmp_path):
    _write(tmp_path, "lib/b.tca", '@runtime(cxx_path="from_b.h");\n' + _kernel("kb"))
    _write(tmp_path, "a.tca", '@include "lib/b.tca";\n' + _kernel("ka"))
    root = _write(tmp_path, "main.tca", '@include "a.tca";\n' + _kernel("km"))
    m = syntax.ParseModule(root)
    assert [k.Name() for k in m.Kernels] == ["km", "ka", "kb"]
    assert m.Runtime == "from_b.h"  # inherited from the first include that declares one
    assert m.Kernels[2].Build().IR()


def test_include_diamond_merges_once(tmp_path):
    _write(tmp_path, "d.tca", _kernel("kd"))
    _write(tmp_path, "b.tca", '@include "d.tca";\n' + _kernel("kb"))
    _write(tmp_path, "c.tca", '@include "d.tca";\n' + _kernel("kc"))
    root = _write(tmp_path, "a.tca", '@include "b.tca";\n@include "c.tca";\n' + _kernel("ka"))
    assert [k.Name() for k in syntax.ParseModule(root).Kernels] == ["ka", "kb", "kd", "kc"]


@pytest.mark.parametrize("files,root,needle", [
    ({"a.tca": '@include "b.tca";\n', "b.tca": '@include "a.tca";\n'}, "a.tca", "@include cycle"),
    ({"a.tca": '@include "nope.tca";\n'}, "a.tca", "missing include file"),
    ({"sub/a.tca": '@include "../x.tca";\n', "x.tca": ""}, "sub/a.tca", "escapes the including file's directory"),
    ({"a.tca": '@include "/etc/hosts";\n'}, "a.tca", "must be relative"),
    ({"a.tca": '@runtime(cxx_path="x.h");\n@runtime(cxx_path="y.h");\n'}, "a.tca", "at most one @runtime"),
])
def test_include_policy(tmp_path, files, root, needle):
    for n, t in files.items():
        _write(tmp_path, n, t)
    with pytest.raises(BuildError, match=re.escape(needle)):
        syntax.ParseModule(str(tmp_path / root))


def test_missing_root_file(tmp_path):
    with pytest.raises(BuildError, match="cannot read source file"):
        syntax.ParseModule(str(tmp_path / "absent.tca"))


def test_include_needs_a_file_backed_module():
    with pytest.raises(BuildError, match="file-backed"):
        syntax.ParseSource('@include "x.tca";\n' + VALID)


# ---------------------------------------------------------------- extensions

def test_map_only_let_lowers_as_an_elementwise_chain():
    src = """kernel axpy(x: tensor<dtype=f32, shape=[N]>, y: tensor<dtype=f32, shape=[N]>, a: f32)
  -> tensor<dtype=f32, shape=[N]>
{
  dimvar i;
  let z = map on(x[i], y[i]) [a] (p: f32, q: f32) -> f32: a * p + q;
  return z;
}"""
    p = syntax.ParseSource(src).Kernels[0].Build()
    assert "store z[@N]" in p.IRFull()
    assert p.emit().families() == ["elementwise"]


def test_several_outputs():
    m = syntax.ParseModule(CONFIGS_TCA)
    p = m.Kernel("row_sum_max_8192").Build()
    e = p.emit()
    assert e.families() == ["row"]
    assert "tensor sum f32 out" in e.plan and "tensor max f32 out" in e.plan
    two = VALID.replace("-> tensor<dtype=f32, shape=[P, S]>", "-> (tensor<dtype=f32, shape=[P, S]>)")
    syntax.ParseSource(two).Kernels[0].Build()
    want_error(VALID.replace("return r;", "return r, r;").replace(
        "-> tensor<dtype=f32, shape=[P, S]>", "-> (tensor<dtype=f32, shape=[P, S]>, tensor<dtype=f32, shape=[P, S]>)"),
        "twice")
    want_error(VALID.replace("return r;", "return r, r;"), "signature declares 1")


def test_build_needs_a_checked_module():
    m = syntax.ParseSource(VALID, check=False)
    with pytest.raises(BuildError, match="without checks"):
        m.Kernels[0].Build()
