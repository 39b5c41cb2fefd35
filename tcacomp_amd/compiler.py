"""Compile driver: program -> emitted HIP -> code object (.hsaco) -> launchable.

The reference compiler emits a .cu plus a CMakeLists.txt and leaves the
toolchain to a harness (CLAUDE.md:18, internal/e2e/harness.go:87-127, with a
content-addressed fixture cache keyed by the emitted source). This driver is
that harness for the HIP path: the code object is cached under
``tcacomp_amd/_kcache/`` by the SHA-256 of the emitted source, the hipcc
argv and the device headers the source includes, so ``build()`` can prebuild every kernel the
tests and the bench use and a GPU box never compiles. ``TCA_JIT=0`` turns a
cache miss into an error instead of a hipcc run.
"""
import ctypes
import hashlib
import re
import os
import subprocess

from . import _lib
from .pkg import EMIT_NO_FUSION, EMIT_NO_GEMM, EMIT_NO_GEMM_SPLIT, EMIT_NO_PASS_FUSION  # noqa: F401  (re-exported)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
INCLUDE_DIR = os.path.join(PKG_DIR, "csrc", "include")
KCACHE = os.path.join(PKG_DIR, "_kcache")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


_INCLUDE_RE = re.compile(r'^\s*#\s*include\s*"([^"]+)"', re.M)


def _header_digest(source):
    """sha256 over the headers under csrc/include that `source` includes,
    followed transitively (path and contents, in a fixed order): a code
    object depends on those files only, so a change to one header leaves the
    keys of kernels that do not include it unchanged."""
    seen = set()
    todo = list(_INCLUDE_RE.findall(source))
    while todo:
        rel = todo.pop()
        p = os.path.join(INCLUDE_DIR, rel)
        if rel in seen or not os.path.isfile(p):
            continue
        seen.add(rel)
        with open(p, "r") as fh:
            todo.extend(_INCLUDE_RE.findall(fh.read()))
    h = hashlib.sha256()
    for rel in sorted(seen):
        h.update(rel.encode())
        with open(os.path.join(INCLUDE_DIR, rel), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()


def cache_key(source, hipcc_args):
    h = hashlib.sha256()
    h.update(source.encode())
    h.update(b"\0")
    h.update(" ".join(hipcc_args).encode())
    h.update(b"\0")
    h.update(_header_digest(source).encode())
    return h.hexdigest()[:20]


def jit_allowed():
    return os.environ.get("TCA_JIT", "1") != "0"


def build_code_object(src_path, out_path, hipcc_args):
    cmd = [HIPCC] + list(hipcc_args) + ["-I", INCLUDE_DIR, "-o", out_path + ".tmp", src_path]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed (%d) for %s:\n%s\n%s" % (r.returncode, src_path, " ".join(cmd),
                                                                   r.stderr[-4000:]))
    os.replace(out_path + ".tmp", out_path)


class CompiledProgram:
    """An emitted program bound to its code object. Loading (and every
    launch) needs a GPU; parsing and the shape contract do not."""

    def __init__(self, name, emitted, hsaco):
        self.name = name
        self.source = emitted.source
        self.plan = emitted.plan
        self.report = emitted.report
        self.hsaco = hsaco
        self._h = None
        self._parsed = None

    def families(self):
        return [line.split()[1] for line in self.report.splitlines() if line.strip()]

    def kernel_symbols(self):
        return [line.split()[0] for line in self.report.splitlines() if line.strip()]

    # -- host-only: plan parse + shape contract
    def parsed(self):
        if self._parsed is None:
            h = ctypes.c_void_p()
            _lib.check(_lib.lib().tca_program_parse(self.plan.encode(), ctypes.byref(h)))
            self._parsed = h
        return self._parsed

    def signature(self):
        n = [ctypes.c_uint32() for _ in range(4)]
        _lib.check(_lib.lib().tca_program_signature(self.parsed(), *[ctypes.byref(x) for x in n]))
        return tuple(x.value for x in n)

    def check(self, tensors, free_dims=()):
        arr = _descriptors(tensors)
        fd = (ctypes.c_uint32 * max(1, len(free_dims)))(*free_dims)
        return _lib.lib().tca_program_check(self.parsed(), arr, len(tensors), fd, len(free_dims))

    def selected_symbols(self, tensors, free_dims=()):
        """The kernels a launch with these tensors runs, in launch order:
        launch guards applied, and kernels whose grid is empty (no outputs,
        or a split kernel the row-chunk count leaves out) dropped."""
        syms = self.kernel_symbols()
        arr = _descriptors(tensors)
        fd = (ctypes.c_uint32 * max(1, len(free_dims)))(*free_dims)
        out = (ctypes.c_uint8 * max(1, len(syms)))()
        grids = (ctypes.c_uint64 * max(1, len(syms)))()
        _lib.check(_lib.lib().tca_program_selected(self.parsed(), arr, len(tensors), fd, len(free_dims), out,
                                                   grids, None, len(syms)))
        return [s for s, f, g in zip(syms, out, grids) if f and g]

    # -- GPU
    def load(self):
        if self._h is None:
            if not os.path.exists(self.hsaco):
                raise RuntimeError("code object %s is missing; build it first" % self.hsaco)
            h = ctypes.c_void_p()
            _lib.check(_lib.lib().tca_program_load(self.hsaco.encode(), self.plan.encode(), ctypes.byref(h)))
            self._h = h
        return self._h

    def launch(self, tensors, free_dims=(), scalars=(), stream=None, noalloc=False):
        """Launches every kernel of the program on `stream` (a hipStream_t
        handle as int, or None for the current torch stream). noalloc takes
        the workspace from the device's scratch array
        (tca_program_launch_noalloc) instead of allocating one."""
        h = self.load()
        arr = _descriptors(tensors)
        fd = (ctypes.c_uint32 * max(1, len(free_dims)))(*free_dims)
        sc = (ctypes.c_double * max(1, len(scalars)))(*[float(s) for s in scalars])
        if stream is None:
            stream = _current_stream()
        fn = _lib.lib().tca_program_launch_noalloc if noalloc else _lib.lib().tca_program_launch
        _lib.check(fn(h, arr, len(tensors), fd, len(free_dims), sc, len(scalars), ctypes.c_void_p(stream)))

    def __del__(self):
        try:
            L = _lib.lib()
            if self._h is not None:
                L.tca_program_unload(self._h)
            if self._parsed is not None:
                L.tca_program_unload(self._parsed)
        except Exception:
            pass


_TORCH_DTYPES = None


def _dtype_code(t):
    global _TORCH_DTYPES
    import torch
    if _TORCH_DTYPES is None:
        _TORCH_DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.int32: 3,
                         torch.int8: 5, torch.int16: 6, torch.uint8: 7, torch.bool: 9}
        if hasattr(torch, "uint32"):
            _TORCH_DTYPES[torch.uint32] = 4
        if hasattr(torch, "uint16"):
            _TORCH_DTYPES[torch.uint16] = 8
    return _TORCH_DTYPES[t.dtype]


class TensorDesc:
    """A raw descriptor (device pointer, shape, dtype code) for callers that
    do not hold torch tensors."""

    def __init__(self, ptr, shape, dtype):
        self.ptr, self.shape, self.dtype = ptr, tuple(shape), dtype


def _descriptors(tensors):
    arr = (_lib.tca_tensor * max(1, len(tensors)))()
    for i, t in enumerate(tensors):
        if isinstance(t, TensorDesc):
            ptr, shape, code = t.ptr, t.shape, t.dtype
        else:
            if not t.is_contiguous():
                raise ValueError("tensor %d is not contiguous (tca tensors are row-major)" % i)
            ptr, shape, code = t.data_ptr(), tuple(t.shape), _dtype_code(t)
        arr[i].data = ptr
        arr[i].rank = len(shape)
        for a, d in enumerate(shape[:8]):
            arr[i].dims[a] = d
        arr[i].dtype = code
    return arr


def _current_stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def compile_program(prog, kernel_name=None, flags=0, jit=None):
    """Emits `prog` (a built pkg.Program) and returns its CompiledProgram,
    building the code object on a cache miss when JIT is allowed."""
    emitted = prog.emit(kernel_name=kernel_name, flags=flags)
    key = cache_key(emitted.source, emitted.hipcc)
    os.makedirs(KCACHE, exist_ok=True)
    base = os.path.join(KCACHE, "%s-%s" % (prog.name, key))
    hsaco = base + ".hsaco"
    if not os.path.exists(hsaco):
        allowed = jit_allowed() if jit is None else jit
        if not allowed:
            raise RuntimeError("code object for %s (%s) is not prebuilt and TCA_JIT=0" % (prog.name, key))
        with open(base + ".hip", "w") as f:
            f.write(emitted.source)
        build_code_object(base + ".hip", hsaco, emitted.hipcc)
        with open(base + ".plan", "w") as f:
            f.write(emitted.plan)
    return CompiledProgram(prog.name, emitted, hsaco)
