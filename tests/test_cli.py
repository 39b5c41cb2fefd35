"""The compiler driver (tcacomp_amd/cmd/tcacomp.c, built by build() into
tcacomp_amd/bin/tcacomp), host only.

It follows cmd/tcacomp/main.go:28-113: `tcacomp compile [-o DIR] <input.tca>`
compiles every kernel of the module, writes its files into DIR and prints
"tcacomp: compiled <kernel> -> <DIR>"; exit status 2 for usage errors, 1 for
compile errors. What it writes must be what the library's own emitter gives
for the same program through the pkg API, so the code objects its Makefile
builds are the ones the GPU tests already pin (tests/test_gpu_cli.py launches
them)."""
import glob
import os
import shlex
import subprocess

import pytest

from tcacomp_amd import build as tb
from tcacomp_amd import compiler, programs

REF = "/root/reference"


def cli(*args, cwd=None):
    if not os.path.exists(tb.CLI):
        pytest.fail("tcacomp_amd/bin/tcacomp is not built (run build())")
    return subprocess.run([tb.CLI] + list(args), capture_output=True, text=True, cwd=cwd)


def test_usage_and_exit_codes(tmp_path):
    r = cli()
    assert r.returncode == 2 and "usage:" in r.stderr and "tcacomp compile" in r.stderr
    r = cli("help")
    assert r.returncode == 0 and "usage:" in r.stderr
    r = cli("frob")
    assert r.returncode == 2 and 'tcacomp: unknown command "frob"' in r.stderr
    r = cli("compile")
    assert r.returncode == 2 and "tcacomp compile: exactly one input file required" in r.stderr
    r = cli("compile", "a.tca", "b.tca")
    assert r.returncode == 2 and "exactly one input file required" in r.stderr
    r = cli("compile", "-x", "a.tca")
    assert r.returncode == 2 and "flag provided but not defined: -x" in r.stderr
    r = cli("compile", "-o")
    assert r.returncode == 2 and "flag needs an argument" in r.stderr
    # Flags end at the first argument that is not one (Go's flag package):
    # a later -o is a second input file.
    r = cli("compile", tb.CONFIGS_TCA, "-o", str(tmp_path))
    assert r.returncode == 2 and "exactly one input file required" in r.stderr


def test_compile_errors(tmp_path):
    r = cli("compile", "-o", str(tmp_path / "o"), str(tmp_path / "missing.tca"))
    assert r.returncode == 1 and r.stderr.startswith("tcacomp: ")
    bad = tmp_path / "bad.tca"
    bad.write_text("kernel k(x: tensor<dtype=f32, shape=[M]>) -> tensor<dtype=f32, shape=[M]>\n{\n  return y;\n}\n")
    r = cli("compile", "-o", str(tmp_path / "o"), str(bad))
    assert r.returncode == 1 and r.stderr.startswith("tcacomp: ") and "bad.tca:3:" in r.stderr, r.stderr
    empty = tmp_path / "empty.tca"
    empty.write_text("// nothing here\n")
    r = cli("compile", "-o", str(tmp_path / "o"), str(empty))
    assert r.returncode == 1 and "tcacomp: %s: no kernels" % empty in r.stderr, r.stderr
    r = cli("compile", "-target", "sm_86", "-o", str(tmp_path / "o"), tb.CONFIGS_TCA)
    assert r.returncode == 1 and "unsupported target sm_86" in r.stderr, r.stderr


def _kernel_names(path):
    from tcacomp_amd import syntax
    return [k.Name() for k in syntax.ParseModule(path).Kernels]


def test_configs_emit_what_the_pkg_path_emits(tmp_path):
    out = tmp_path / "out"
    r = cli("compile", "-o", str(out), tb.CONFIGS_TCA)
    assert r.returncode == 0, r.stderr
    names = _kernel_names(tb.CONFIGS_TCA)
    assert r.stdout.splitlines() == ["tcacomp: compiled %s -> %s" % (n, out) for n in names]
    for n in names:
        want = programs.CONFIG_PROGRAMS[n]().emit()
        assert (out / (n + ".hip")).read_text() == want.source, n
        assert (out / (n + ".plan")).read_text() == want.plan, n


def test_makefile_builds_with_the_emitters_hipcc_line(tmp_path):
    out = tmp_path / "out"
    assert cli("compile", "--target=gfx950", "--o=" + str(out), tb.CONFIGS_TCA).returncode == 0
    names = _kernel_names(tb.CONFIGS_TCA)
    r = subprocess.run(["make", "-n", "-C", str(out)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    cmds = [line for line in r.stdout.splitlines() if "hipcc" in line]
    assert len(cmds) == len(names)
    for n, line in zip(names, cmds):
        argv = shlex.split(line.split(" && ")[0])
        want = programs.CONFIG_PROGRAMS[n]().emit().hipcc
        assert argv[0].endswith("hipcc")
        assert argv[1:1 + len(want)] == want, n
        assert argv[1 + len(want):] == ["-I", os.path.realpath(compiler.INCLUDE_DIR), "-o", n + ".hsaco.tmp",
                                        n + ".hip"]


def test_rerun_leaves_unchanged_files_untouched(tmp_path):
    out = tmp_path / "out"
    assert cli("compile", "-o", str(out), tb.CONFIGS_TCA).returncode == 0
    stamps = {p: os.stat(p).st_mtime_ns for p in glob.glob(str(out / "*.hip")) + glob.glob(str(out / "*.plan"))}
    os.utime(next(iter(stamps)), ns=(1, 1))
    first = next(iter(stamps))
    stamps[first] = 1
    assert cli("compile", "-o", str(out), tb.CONFIGS_TCA).returncode == 0
    assert {p: os.stat(p).st_mtime_ns for p in stamps} == stamps


def test_prebuilt_output_matches_the_configs():
    # build() ran the driver and its Makefile into tcacomp_amd/_cli_out; the
    # GPU test launches those code objects.
    for n in _kernel_names(tb.CONFIGS_TCA):
        for ext in (".hip", ".plan", ".hsaco"):
            assert os.path.exists(os.path.join(tb.CLI_OUT, n + ext)), n + ext
        with open(os.path.join(tb.CLI_OUT, n + ".hip")) as f:
            assert f.read() == programs.CONFIG_PROGRAMS[n]().emit().source, n


@pytest.mark.skipif(not os.path.isdir(REF), reason="reference tree not mounted")
@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(REF, "testing/kernels/*/*.tca"))),
                         ids=lambda p: os.path.basename(p))
def test_reference_corpus_compiles(tmp_path, path):
    # The reference's own corpus, unchanged, through the driver.
    r = cli("compile", "-o", str(tmp_path), path)
    assert r.returncode == 0, r.stderr
    for n in _kernel_names(path):
        assert (tmp_path / (n + ".hip")).stat().st_size > 0
        assert (tmp_path / (n + ".plan")).stat().st_size > 0
