"""In-tree build: the host library (libtcacomp.so) and every prebuilt code
object the tests and the bench launch.

The host library holds the runtime (plain HIP host API), the plan
interpreter, the DSL builder, the .tca text frontend and the HIP emitter; it is ordinary C++ built
with g++ against the ROCm headers, plus one hipcc-built source (rt/scratch.hip:
the device array behind the allocation-free launch). Kernels exist only as
emitted code objects, compiled by hipcc for gfx950 into ``_kcache/``.
"""
import concurrent.futures
import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
OBJ_DIR = os.path.join(PKG_DIR, "_build")
LIB = os.path.join(PKG_DIR, "libtcacomp.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

SOURCES = [
    "rt/runtime.cpp",
    "rt/plan.cpp",
    "cg/ir.cpp",
    "cg/builder.cpp",
    "cg/emit_hip.cpp",
    "cg/gemm_emit.cpp",
    "cg/capi.cpp",
    "syntax/lexer.cpp",
    "syntax/parser.cpp",
    "syntax/check.cpp",
    "syntax/lower.cpp",
    "syntax/module.cpp",
    "syntax/capi.cpp",
]

HIP_SOURCES = ["rt/scratch.hip"]

CXXFLAGS = ["-std=c++17", "-O2", "-fPIC", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
            "-I" + os.path.join(ROCM, "include"), "-I" + os.path.join(REPO, "include"),
            "-I" + os.path.join(CSRC, "rt")]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("build step failed: %s\n%s%s" % (" ".join(cmd), r.stdout[-3000:], r.stderr[-3000:]))
    return r


def build_library(jobs=8):
    os.makedirs(OBJ_DIR, exist_ok=True)
    objs = []
    cmds = []
    for s in SOURCES:
        src = os.path.join(CSRC, s)
        obj = os.path.join(OBJ_DIR, s.replace("/", "_").replace(".cpp", ".o"))
        objs.append(obj)
        cmds.append(["g++"] + CXXFLAGS + ["-c", src, "-o", obj])
    # The one device-code source of the library: the allocation-free
    # launch's scratch array (a device global, so hipcc builds it for gfx950).
    for s in HIP_SOURCES:
        src = os.path.join(CSRC, s)
        obj = os.path.join(OBJ_DIR, s.replace("/", "_").replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([os.path.join(ROCM, "bin", "hipcc"), "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC",
                     "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                     "-I" + os.path.join(CSRC, "rt"), "-c", src, "-o", obj])
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB + ".tmp"
    _run(["g++", "-shared", "-o", tmp] + objs +
         ["-L" + os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,-rpath," + os.path.join(ROCM, "lib")])
    os.replace(tmp, LIB)
    return LIB


def build_kernels(jobs=8, force=False, extra=()):
    """Emits and compiles every registered program, plus `extra` (name,
    factory, flags) triples such as the test suite's generated programs,
    into _kcache/; code objects of neither are pruned."""
    from . import compiler, programs

    jobs_list = []
    current = set()
    for name, factory, flags in list(programs.all_builds()) + list(extra):
        prog = factory()
        emitted = prog.emit(flags=flags)
        key = compiler.cache_key(emitted.source, emitted.hipcc)
        os.makedirs(compiler.KCACHE, exist_ok=True)
        base = os.path.join(compiler.KCACHE, "%s-%s" % (prog.name, key))
        current.add(os.path.basename(base))
        with open(base + ".hip", "w") as f:
            f.write(emitted.source)
        with open(base + ".plan", "w") as f:
            f.write(emitted.plan)
        if force or not os.path.exists(base + ".hsaco"):
            jobs_list.append((base + ".hip", base + ".hsaco", emitted.hipcc))

    def one(j):
        compiler.build_code_object(*j)
        return j[1]

    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        done = list(ex.map(one, jobs_list))
    # Drop code objects of earlier sources: the cache travels with the tree.
    for f in os.listdir(compiler.KCACHE):
        stem = f.rsplit(".", 1)[0]
        if stem not in current:
            os.remove(os.path.join(compiler.KCACHE, f))
    return done


def build_all(force_kernels=False, extra=()):
    build_library()
    # The freshly built library must be the one loaded.
    from . import _lib
    _lib._lib = None
    return build_kernels(force=force_kernels, extra=extra)


if __name__ == "__main__":
    sys.path.insert(0, REPO)
    out = build_all(force_kernels="--force" in sys.argv)
    print("built %s and %d code object(s)" % (LIB, len(out)))


CLI = os.path.join(PKG_DIR, "bin", "tcacomp")
CLI_OUT = os.path.join(PKG_DIR, "_cli_out")
CONFIGS_TCA = os.path.join(PKG_DIR, "tca", "configs.tca")


def build_cli(jobs=8):
    """Builds the compiler driver (cmd/tcacomp.c) and runs it the way a user
    would: `tcacomp compile -o _cli_out tca/configs.tca`, then `make` in the
    output directory, leaving <kernel>.{hip,plan,hsaco} for every kernel of
    the configurations' .tca module."""
    _run(["make", "-s", "-C", os.path.join(CSRC, "..", "cmd")])
    _run([CLI, "compile", "-o", CLI_OUT, CONFIGS_TCA])
    _run(["make", "-s", "-j%d" % jobs, "-C", CLI_OUT])
    return CLI_OUT
