"""The CPU half of the reference's sanitizer gate (its e2e runs pass through
memcheck and racecheck: internal/e2e/e2e_test.go:332-385,
testing/orchestrator.py:295-316). GPU sanitizers do not run on this pool,
so the gate covers the host library: every C++ source of libtcacomp.so is
built with AddressSanitizer and UndefinedBehaviorSanitizer into
tcacomp_amd/_asan/, and then

  - tests/c/fuzz.cpp mutates launch plans (the emitter's .plan files) and
    .tca sources (this repository's) and feeds them to the parsers, the
    shape contract, the builder and the emitter, stopping at the first
    finding;
  - the plain-C consumer's host leg (tests/c/abi_consumer.c) runs against
    that library;
  - with --pytest, the whole CPU test suite runs against it
    (pytest -m "not gpu", TCA_LIB naming the sanitized library, the ASan
    runtime preloaded into Python).

A finding is a sanitizer report (the run aborts: halt_on_error, no UBSan
recovery) or any other crash. Test infrastructure: nothing in the product
imports this file.

    python tests/sanitize.py [--fuzz-seconds S] [--pytest]
"""
import argparse
import glob
import hashlib
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)
from tcacomp_amd import build as tb  # noqa: E402

ASAN_DIR = os.path.join(REPO, "tcacomp_amd", "_asan")
ASAN_LIB = os.path.join(ASAN_DIR, "libtcacomp.so")
CDIR = os.path.join(REPO, "tests", "c")
FUZZ = os.path.join(ASAN_DIR, "fuzz")
CONSUMER = os.path.join(ASAN_DIR, "abi_consumer")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-g"]
ENV = {"ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=1:detect_stack_use_after_return=1",
       "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


def _run(cmd, **kw):
    r = subprocess.run(cmd, capture_output=True, text=True, **kw)
    if r.returncode != 0:
        raise RuntimeError("failed (%d): %s\n%s%s" % (r.returncode, " ".join(cmd), r.stdout[-4000:], r.stderr[-8000:]))
    return r


def _digest(paths, extra=""):
    h = hashlib.sha256(extra.encode())
    for p in sorted(paths):
        h.update(p.encode())
        with open(p, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def build(jobs=8):
    """The sanitized library, the fuzzer and the C consumer (rebuilt only
    when a source or header changed)."""
    import concurrent.futures
    os.makedirs(ASAN_DIR, exist_ok=True)
    srcs = [os.path.join(tb.CSRC, s) for s in tb.SOURCES]
    # The host library's own headers (the device headers under csrc/include
    # go into emitted kernels, never into the library).
    headers = [h for h in glob.glob(os.path.join(tb.CSRC, "**", "*.h"), recursive=True)
               if os.sep + "include" + os.sep not in h] + glob.glob(os.path.join(REPO, "include", "*.h"))
    tests_src = [os.path.join(CDIR, "fuzz.cpp"), os.path.join(CDIR, "abi_consumer.c")]
    key = _digest(srcs + headers + tests_src + [os.path.join(tb.CSRC, s) for s in tb.HIP_SOURCES], " ".join(SAN))
    stamp = os.path.join(ASAN_DIR, "stamp")
    if os.path.exists(stamp) and open(stamp).read() == key and all(os.path.exists(p) for p in (ASAN_LIB, FUZZ, CONSUMER)):
        return
    flags = [f for f in tb.CXXFLAGS if f != "-O2"] + ["-O1"] + SAN
    objs, cmds = [], []
    for s in tb.SOURCES:
        obj = os.path.join(ASAN_DIR, s.replace("/", "_").replace(".cpp", ".o"))
        objs.append(obj)
        cmds.append(["g++"] + flags + ["-c", os.path.join(tb.CSRC, s), "-o", obj])
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    # The library's one device-code object (the allocation-free launch's
    # scratch array) comes from the regular build, without sanitizers.
    tb.build_library()
    objs += [os.path.join(tb.OBJ_DIR, s.replace("/", "_").replace(".hip", ".o")) for s in tb.HIP_SOURCES]
    rocm_lib = os.path.join(tb.ROCM, "lib")
    _run(["g++", "-shared"] + SAN + ["-o", ASAN_LIB + ".tmp"] + objs +
         ["-L" + rocm_lib, "-lamdhip64", "-Wl,-rpath," + rocm_lib])
    os.replace(ASAN_LIB + ".tmp", ASAN_LIB)
    link = ["-L" + ASAN_DIR, "-ltcacomp", "-Wl,-rpath," + ASAN_DIR]
    _run(["g++", "-std=c++17", "-O1", "-I" + os.path.join(REPO, "include")] + SAN +
         [os.path.join(CDIR, "fuzz.cpp"), "-o", FUZZ] + link)
    oracle_dir = os.path.join(REPO, "oracle", "_build")
    _run(["gcc", "-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror", "-O1", "-I" + os.path.join(REPO, "include")] +
         SAN + [os.path.join(CDIR, "abi_consumer.c"), "-o", CONSUMER] + link +
         ["-L" + oracle_dir, "-loracle", "-lm", "-Wl,-rpath," + oracle_dir])
    with open(stamp, "w") as f:
        f.write(key)


def corpus(mode):
    if mode == "plan":
        return sorted(glob.glob(os.path.join(REPO, "tcacomp_amd", "_kcache", "*.plan")))
    return sorted(glob.glob(os.path.join(REPO, "tcacomp_amd", "tca", "**", "*.tca"), recursive=True))


def fuzz(mode, seconds, seed=1, iterations=10 ** 9):
    """Runs the fuzzer; returns its summary line. Raises with the sanitizer
    report and the input on disk at the first finding."""
    out = os.path.join(ASAN_DIR, "fuzz_out")
    os.makedirs(out, exist_ok=True)
    files = corpus(mode)
    if not files:
        raise RuntimeError("no %s corpus (build() writes the .plan files)" % mode)
    env = dict(os.environ, **ENV)
    r = subprocess.run([FUZZ, mode, str(iterations), str(seconds), str(seed), out] + files, capture_output=True,
                       text=True, env=env, timeout=seconds + 300)
    if r.returncode != 0 or not r.stdout.startswith("ok "):
        raise RuntimeError("fuzz %s finding (rc %d); input in %s/current.%s\n%s%s" % (
            mode, r.returncode, out, mode, r.stdout[-2000:], r.stderr[-8000:]))
    return r.stdout.strip()


def consumer_host():
    from tcacomp_amd import compiler, programs
    prog = compiler.compile_program(programs.CONFIG_PROGRAMS["row_sum_max_8192"]())
    hip = prog.hsaco[: -len(".hsaco")] + ".hip"
    r = subprocess.run([CONSUMER, "host", hip, os.path.join(REPO, "tcacomp_amd", "tca", "configs.tca")],
                       capture_output=True, text=True, env=dict(os.environ, **ENV), timeout=300)
    if r.returncode != 0 or "ok host" not in r.stdout:
        raise RuntimeError("consumer host leg under ASan failed (rc %d)\n%s%s" % (r.returncode, r.stdout, r.stderr[-8000:]))
    return r.stdout.strip()


def pytest_cpu():
    """pytest -m "not gpu" against the sanitized library; returns its summary."""
    asan_rt = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    env = dict(os.environ, **ENV, TCA_LIB=ASAN_LIB, LD_PRELOAD=asan_rt)
    r = subprocess.run([sys.executable, "-m", "pytest", os.path.join(REPO, "tests"), "-x", "-q", "-m", "not gpu",
                        "-p", "no:cacheprovider", "--deselect", "tests/test_sanitize.py"],
                       capture_output=True, text=True, env=env, cwd=REPO, timeout=3600)
    tail = (r.stdout + r.stderr)[-3000:]
    if r.returncode != 0:
        raise RuntimeError("pytest under ASan failed (rc %d)\n%s" % (r.returncode, tail))
    return r.stdout.strip().splitlines()[-1]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--fuzz-seconds", type=float, default=60.0)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--pytest", action="store_true", help="also run pytest -m 'not gpu' against the sanitized library")
    a = ap.parse_args()
    build()
    print("built", ASAN_LIB, flush=True)
    for mode in ("plan", "tca"):
        print("fuzz:", fuzz(mode, a.fuzz_seconds, a.seed), flush=True)
    print("consumer:", consumer_host(), flush=True)
    if a.pytest:
        print("pytest:", pytest_cpu(), flush=True)
    print("no sanitizer reports")


if __name__ == "__main__":
    main()
