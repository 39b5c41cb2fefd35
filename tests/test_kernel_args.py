"""Host-only checks of the argument blocks a launch passes to its kernels
(tca_program_kernel_args, which shares its layout and slot filling with
tca_program_launch): every byte equal to a packing of the plan's arg records
written here independently (the HIP kernarg layout: natural alignment,
pointers 8 bytes, dims u32, f32 scalars 4 bytes), with locals at their
offsets in a workspace at address 0 (256-byte aligned, in declaration order,
only the locals the selected kernels take). Programs with locals, split
scratch, scalars and several kernels per launch."""
import ctypes
import struct

import pytest

from tcacomp_amd import _lib, compiler, programs
from tcacomp_amd.compiler import TensorDesc

DT_BYTES = {"f32": 4, "f16": 2, "bf16": 2, "i32": 4, "u32": 4, "i8": 1, "i16": 2, "u8": 1, "u16": 2, "bool": 1}
DT_CODE = {"f32": 0, "f16": 1, "bf16": 2, "i32": 3, "u32": 4, "i8": 5, "i16": 6, "u8": 7, "u16": 8, "bool": 9}


def _plan(text):
    dims, tensors, scalars, kernels = {}, [], [], []
    for line in text.splitlines():
        f = line.split()
        if not f:
            continue
        if f[0] == "dim":
            dims[f[1]] = int(f[2])
        elif f[0] == "tensor":
            tensors.append((f[1], f[2], f[3], f[5:5 + int(f[4])]))
        elif f[0] == "scalar":
            scalars.append((f[1], f[2]))
        elif f[0] == "kernel":
            kernels.append({"symbol": f[1], "args": []})
        elif f[0] == "arg":
            kernels[-1]["args"].append((f[1], f[2]))
    return dims, tensors, scalars, kernels


def _pack(args, ptr_of, dimval, scal):
    out = bytearray()

    def put(b, n):
        while len(out) % n:
            out.append(0)
        out.extend(b)
    for kind, name in args:
        if kind == "ptr":
            put(struct.pack("<Q", ptr_of[name]), 8)
        elif kind == "dim":
            put(struct.pack("<I", dimval[name]), 4)
        else:
            put(struct.pack("<f", scal[name]), 4)
    return bytes(out)


CASES = [
    ("bmm_f32", [(2, 64, 4096), (2, 4096, 64), (2, 64, 64)], []),              # small kernel + merge, split scratch
    ("qk_score", [(128, 64), (192, 64), (128, 192)], [0.125]),                # a scalar in the epilogue
    ("layernorm_dyn", [(3, 8193), (8193,), (8193,), (3, 8193)], [1 / 8193, 1e-5]),
    ("softmax_dyn", [(2, 1 << 20), (2, 1 << 20)], []),                        # split passes: plan-only locals
    ("col_mean_var_dyn", [(1, 8192, 8192), (1, 8192), (1, 8192)], [1 / 8192]),
    ("gemm_bf16", [(4096, 4096), (4096, 4096), (4096, 4096)], []),
]


@pytest.mark.parametrize("name,shapes,scalars", CASES)
def test_kernel_args_match_an_independent_packing(name, shapes, scalars):
    factory = programs.SUITE[name][0] if name in programs.SUITE else programs.CONFIG_PROGRAMS[name]
    e = factory().emit()
    dims, tensors, scal_decl, kernels = _plan(e.plan)
    params = [t for t in tensors if t[2] != "local"]
    assert len(params) == len(shapes)
    base = 0x7f0000000000
    descs, ptr_of, dimval = [], {}, dict((k, v) for k, v in dims.items() if v)
    for i, ((tname, dt, _, tdims), shp) in enumerate(zip(params, shapes)):
        ptr_of[tname] = base + i * (1 << 32)
        descs.append(TensorDesc(ptr_of[tname], shp, DT_CODE[dt]))
        for dn, v in zip(tdims, shp):
            dimval.setdefault(dn, v)
    h = ctypes.c_void_p()
    assert _lib.lib().tca_program_parse(e.plan.encode(), ctypes.byref(h)) == 0, _lib.last_error()
    arr = compiler._descriptors(descs)
    n = len(kernels)
    sel = (ctypes.c_uint8 * n)()
    grids = (ctypes.c_uint64 * n)()
    assert _lib.lib().tca_program_selected(h, arr, len(descs), None, 0, sel, grids, None, n) == 0, _lib.last_error()
    # the workspace: locals the guard-selected kernels take, in declaration order
    used = set()
    for k, s in zip(kernels, sel):
        if s:
            used |= {nm for kind, nm in k["args"] if kind == "ptr"}
    off = 0
    for tname, dt, role, tdims in tensors:
        if role == "local" and tname in used:
            ptr_of[tname] = off
            size = DT_BYTES[dt]
            for dn in tdims:
                size *= dimval[dn]
            off += (size + 255) // 256 * 256
    scal = dict(zip([s[0] for s in scal_decl], [struct.unpack("<f", struct.pack("<f", v))[0] for v in scalars]))
    sc = (ctypes.c_double * max(1, len(scalars)))(*scalars)
    ran = 0
    for i, k in enumerate(kernels):
        buf = (ctypes.c_ubyte * 512)()
        size = ctypes.c_size_t()
        rc = _lib.lib().tca_program_kernel_args(h, arr, len(descs), None, 0, sc, len(scalars), i, buf, 512,
                                                ctypes.byref(size))
        if not (sel[i] and grids[i]):
            assert rc != 0 and "does not run" in _lib.last_error()
            continue
        assert rc == 0, _lib.last_error()
        want = _pack(k["args"], ptr_of, dimval, scal)
        assert bytes(buf[:size.value]) == want, (k["symbol"], bytes(buf[:size.value]).hex(), want.hex())
        ran += 1
    assert ran >= 1
    _lib.lib().tca_program_unload(h)


def test_kernel_args_errors():
    e = programs.CONFIG_PROGRAMS["row_sum_max_8192"]().emit()
    h = ctypes.c_void_p()
    assert _lib.lib().tca_program_parse(e.plan.encode(), ctypes.byref(h)) == 0
    arr = compiler._descriptors([TensorDesc(0x1000, (4, 8192), 0), TensorDesc(0x1000, (4,), 0),
                                 TensorDesc(0x1000, (4,), 0)])
    size = ctypes.c_size_t()
    buf = (ctypes.c_ubyte * 8)()
    assert _lib.lib().tca_program_kernel_args(h, arr, 3, None, 0, None, 0, 0, buf, 8, ctypes.byref(size)) != 0
    assert size.value == 32 and "32 bytes needed" in _lib.last_error()
    assert _lib.lib().tca_program_kernel_args(h, arr, 3, None, 0, None, 0, 1, buf, 8, ctypes.byref(size)) != 0
    bad = compiler._descriptors([TensorDesc(0x1000, (4, 8000), 0), TensorDesc(0x1000, (4,), 0),
                                 TensorDesc(0x1000, (4,), 0)])
    assert _lib.lib().tca_program_kernel_args(h, bad, 3, None, 0, None, 0, 0, buf, 8, ctypes.byref(size)) == 2
    _lib.lib().tca_program_unload(h)
