"""The C ABI as a C or cgo caller sees it.

- Every public header compiles alone and together under
  `gcc -std=c99 -pedantic -Werror` and `g++ -std=c++11 -pedantic -Werror`.
- Each opaque handle type names its own struct, declared in one header and
  defined in one source file; built at -O0 (where nothing is inlined), no
  handle struct's constructor is emitted by two objects of the library.
- `tests/c/abi_consumer.c`, a plain C99 program, builds C2 through the
  builder rungs, emits it, parses the plan and checks the shape contract and
  kernel selection (host), then loads and launches the prebuilt code object
  and compares it with the C oracle (GPU).
"""
import collections
import os
import re
import subprocess
import tempfile

import pytest

from tcacomp_amd import build as tbuild
from tcacomp_amd import compiler, programs

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(REPO, "include")
HEADERS = sorted(h for h in os.listdir(INCLUDE) if h.endswith(".h"))
CDIR = os.path.join(REPO, "tests", "c")
CONSUMER = os.path.join(CDIR, "_build", "abi_consumer")
CONFIGS_TCA = os.path.join(REPO, "tcacomp_amd", "tca", "configs.tca")


def _syntax_only(compiler_argv, text):
    with tempfile.TemporaryDirectory() as d:
        ext = ".c" if compiler_argv[0] == "gcc" else ".cpp"
        src = os.path.join(d, "tu" + ext)
        with open(src, "w") as f:
            f.write(text)
        r = subprocess.run(compiler_argv + ["-fsyntax-only", "-I", INCLUDE, src], capture_output=True, text=True)
        return r.returncode, r.stderr


@pytest.mark.parametrize("cc", [["gcc", "-std=c99"], ["gcc", "-std=c11"], ["g++", "-std=c++11"]])
def test_headers_compile_strict(cc):
    argv = cc + ["-pedantic", "-Wall", "-Wextra", "-Werror"]
    for h in HEADERS:
        rc, err = _syntax_only(argv, '#include "%s"\nint main(void) { return 0; }\n' % h)
        assert rc == 0, "%s alone: %s" % (h, err)
    for order in (HEADERS, HEADERS[::-1]):
        text = "".join('#include "%s"\n' % h for h in order) + "int main(void) { return 0; }\n"
        rc, err = _syntax_only(argv, text)
        assert rc == 0, "%s together: %s" % (order, err)


def _handle_typedefs():
    found = []
    for h in HEADERS:
        text = open(os.path.join(INCLUDE, h)).read()
        for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\*\s*(\w+)\s*;", text):
            found.append((h, m.group(1), m.group(2)))
    return found


def test_handle_types_are_distinct():
    found = _handle_typedefs()
    assert len(found) >= 6
    structs = collections.Counter(s for _, s, _ in found)
    names = collections.Counter(n for _, _, n in found)
    assert all(c == 1 for c in structs.values()), "struct declared by two handle typedefs: %s" % structs
    assert all(c == 1 for c in names.values()), "handle typedef declared twice: %s" % names
    # Each handle struct is defined in exactly one source file of the library.
    csrc = os.path.join(REPO, "tcacomp_amd", "csrc")
    defs = collections.defaultdict(list)
    for root, _, files in os.walk(csrc):
        for f in files:
            if f.endswith((".cpp", ".h")):
                text = open(os.path.join(root, f)).read()
                for _, s, _ in found:
                    if re.search(r"^struct\s+%s\s*\{" % s, text, flags=re.M):
                        defs[s].append(f)
    for _, s, _ in found:
        assert len(defs[s]) == 1, "struct %s defined in %s" % (s, defs[s])


def _weak_body(obj, mangled):
    """Disassembly of a weak function's own COMDAT section (`.text.<name>`),
    addresses and the section's label stripped, relocations kept."""
    out = subprocess.run(["objdump", "-d", "-r", "--no-show-raw-insn", "-j", ".text." + mangled, obj],
                         capture_output=True, text=True, check=True).stdout
    body = out.split("Disassembly of section .text.%s:" % mangled, 1)[1]
    lines = [re.sub(r"^\s*[0-9a-f]+:\s*", "", l).strip() for l in body.splitlines() if l.strip()]
    lines = [re.sub(r"<[^>]*>", "<>", l) for l in lines]
    assert lines, "no code in section .text.%s of %s" % (mangled, obj)
    return lines


def test_no_handle_constructor_defined_twice_at_O0():
    """At -O0 every inline member function becomes a weak symbol. A handle
    struct name given two different definitions in two translation units
    shows up as one weak constructor with two different bodies (the linker
    keeps either); a struct from one shared header emits the same body in
    every object that includes it."""
    flags = [f for f in tbuild.CXXFLAGS if f != "-O2"] + ["-O0"]
    bodies = collections.defaultdict(dict)  # struct -> {mangled+object: body}
    with tempfile.TemporaryDirectory() as d:
        for s in tbuild.SOURCES:
            obj = os.path.join(d, s.replace("/", "_") + ".o")
            subprocess.run(["g++"] + flags + ["-c", os.path.join(tbuild.CSRC, s), "-o", obj], check=True)
            out = subprocess.run(["nm", "--defined-only", obj], capture_output=True, text=True, check=True).stdout
            for line in out.splitlines():
                parts = line.split()
                if len(parts) == 3 and parts[1] in ("W", "V"):
                    m = re.match(r"_ZN(\d+)(tca_\w+_s)[CD]2E", parts[2])
                    if m and len(m.group(2)) == int(m.group(1)):
                        bodies[m.group(2)][(parts[2], s)] = _weak_body(obj, parts[2])
    assert bodies, "expected inline handle constructors at -O0"
    for struct, per in bodies.items():
        by_symbol = collections.defaultdict(set)
        for (mangled, src), body in per.items():
            by_symbol[mangled].add(tuple(body))
        for mangled, variants in by_symbol.items():
            srcs = sorted(src for (m, src) in per if m == mangled)
            assert len(variants) == 1, "%s: %s has %d different bodies across %s" % (
                struct, mangled, len(variants), srcs)


def _prebuilt_c2():
    prog = compiler.compile_program(programs.CONFIG_PROGRAMS["row_sum_max_8192"]())
    hip = prog.hsaco[: -len(".hsaco")] + ".hip"
    return hip, prog.hsaco


def test_c_consumer_host():
    r = subprocess.run(["make", "-s", "-C", CDIR], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    hip, _ = _prebuilt_c2()
    r = subprocess.run([CONSUMER, "host", hip, CONFIGS_TCA], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "ok host" in r.stdout, r.stdout + r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1000, 8192])
def test_c_consumer_gpu(gpu, rows):
    if not os.path.exists(CONSUMER):
        raise RuntimeError("%s is not built (run build())" % CONSUMER)
    hip, hsaco = _prebuilt_c2()
    print("c consumer: C2 rows=%d" % rows, flush=True)
    r = subprocess.run([CONSUMER, "gpu", hip, hsaco, str(rows)], capture_output=True, text=True, timeout=120)
    print(r.stdout + r.stderr)
    assert r.returncode == 0 and "ok gpu" in r.stdout, r.stdout + r.stderr
