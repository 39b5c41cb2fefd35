"""The .tca text frontend, Python face (names follow internal/syntax/api.go).

    m = ParseModule("softmax.tca")        # load + @include + checks
    for k in m.Kernels:
        prog = k.Build()                  # a built pkg.Program (IR(), emit())

ParseModule fails with pkg.BuildError carrying every error diagnostic
("file:line:col: error: ..."); warnings stay on Module.Diagnostics.
ParseSource does the same for text held in memory (no @include); with
check=False it stops after parsing, so Dump() shows the tree as written.
The work is done by the C++ frontend behind include/tca_syntax.h.
"""
import ctypes

from . import _lib
from .pkg import Builder, BuildError, Program


class Kernel:
    """One checked kernel of a module (internal/syntax/api.go:31-49)."""

    def __init__(self, module, index):
        self._m = module
        self._i = index

    def Name(self):
        return _lib.lib().tca_syntax_module_kernel_name(self._m._h, self._i).decode()

    def CxxName(self):
        """@name(cxx="...") or None."""
        s = _lib.lib().tca_syntax_module_kernel_cxx_name(self._m._h, self._i)
        return s.decode() if s else None

    def Build(self):
        """Lowers the kernel through the builder rungs and builds it."""
        L = _lib.lib()
        out = ctypes.c_void_p()
        if L.tca_syntax_module_build_kernel(self._m._h, self._i, ctypes.byref(out)) != 0:
            raise BuildError(L.tca_syntax_last_error().decode())
        return Program(Builder._adopt(self.Name(), out.value))


class Module:
    """A loaded module: Kernels in merge order, Runtime (@runtime cxx_path or
    None), Source (the root path) and Diagnostics (warnings)."""

    def __init__(self, handle, source):
        self._h = handle
        self.Source = source
        L = _lib.lib()
        self.Kernels = [Kernel(self, i) for i in range(L.tca_syntax_module_kernel_count(handle))]
        rt = L.tca_syntax_module_runtime_path(handle)
        self.Runtime = rt.decode() if rt else None
        self.Diagnostics = L.tca_syntax_module_diagnostics(handle).decode()

    def Kernel(self, name):
        for k in self.Kernels:
            if k.Name() == name:
                return k
        raise KeyError(name)

    def Dump(self):
        return _lib.lib().tca_syntax_module_dump(self._h).decode()

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.lib().tca_syntax_module_free(h)
            except Exception:
                pass
            self._h = None


def ParseModule(path):
    L = _lib.lib()
    out = ctypes.c_void_p()
    if L.tca_syntax_parse_module(str(path).encode(), ctypes.byref(out)) != 0:
        raise BuildError(L.tca_syntax_last_error().decode())
    return Module(out.value, str(path))


def ParseSource(src, name="<source>", check=True):
    L = _lib.lib()
    out = ctypes.c_void_p()
    if L.tca_syntax_parse_source(name.encode(), src.encode(), 1 if check else 0, ctypes.byref(out)) != 0:
        raise BuildError(L.tca_syntax_last_error().decode())
    return Module(out.value, name)
