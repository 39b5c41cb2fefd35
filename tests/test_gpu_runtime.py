"""The run-time C ABI on the device with no torch in the data path (the
boundary a cgo caller uses, include/tca_rt.h): device query, memory, copies,
memset, streams, events, programs launched on a created stream, raw
code-object launches with a hand-packed kernarg blob, and the error paths
(every failure is a status code plus a message, never a crash).
Results against the oracle's scale_relu (bit-identical: elementwise,
contraction off on both sides)."""
import ctypes
import os
import struct

import numpy as np
import pytest

import oracle
from helpers import compiled
from tcacomp_amd import _lib, inputs
from tcacomp_amd.compiler import TensorDesc

pytestmark = pytest.mark.gpu
L = None


@pytest.fixture(scope="module")
def rt(gpu):
    global L
    L = _lib.lib()
    return L


class Dev:
    """A device buffer owned through tca_rt_malloc / tca_rt_free."""

    def __init__(self, nbytes):
        self.p = ctypes.c_void_p()
        _lib.check(L.tca_rt_malloc(ctypes.byref(self.p), nbytes))
        self.nbytes = nbytes

    def put(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        _lib.check(L.tca_rt_memcpy_h2d(self.p, a.ctypes.data_as(ctypes.c_void_p), a.nbytes))

    def get(self, shape, dtype):
        out = np.empty(shape, dtype)
        _lib.check(L.tca_rt_memcpy_d2h(out.ctypes.data_as(ctypes.c_void_p), self.p, out.nbytes))
        return out

    def free(self):
        _lib.check(L.tca_rt_free(self.p))


def test_device_info(rt):
    info = _lib.tca_device_info()
    _lib.check(rt.tca_rt_device_info(0, ctypes.byref(info)))
    assert info.arch.decode().startswith("gfx950")
    assert info.wavefront_size == 64
    assert info.compute_units >= 256
    assert info.max_lds_per_block >= 64 * 1024
    assert info.total_global_mem > (200 << 30)


def test_memory_roundtrip_and_memset(rt):
    n = 1 << 20
    d = Dev(n * 4)
    a = np.arange(n, dtype=np.uint32) * 2654435761
    d.put(a)
    assert np.array_equal(d.get(n, np.uint32), a)
    _lib.check(rt.tca_rt_memset(d.p, 0x5A, n * 4))
    _lib.check(rt.tca_rt_device_sync())
    assert np.all(d.get(n * 4, np.uint8) == 0x5A)
    d.free()


def _scale_relu_case(M=512, N=1024):
    x = inputs.uniform((M, N), -1, 1, 0)
    y = inputs.uniform((M, N), -1, 1, 1)
    return x, y, oracle.scale_relu(x, y, 1.5)


def test_program_on_created_stream_with_events(rt):
    M, N = 512, 1024
    x, y, want = _scale_relu_case(M, N)
    dx, dy, dz = Dev(x.nbytes), Dev(y.nbytes), Dev(x.nbytes)
    dx.put(x)
    dy.put(y)
    prog = compiled("scale_relu_map")
    h = prog.load()
    s = ctypes.c_void_p()
    e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
    _lib.check(rt.tca_rt_stream_create(ctypes.byref(s)))
    _lib.check(rt.tca_rt_event_create(ctypes.byref(e0)))
    _lib.check(rt.tca_rt_event_create(ctypes.byref(e1)))
    ts = [TensorDesc(dx.p.value, (M, N), 0), TensorDesc(dy.p.value, (M, N), 0), TensorDesc(dz.p.value, (M, N), 0)]
    from tcacomp_amd.compiler import _descriptors
    arr = _descriptors(ts)
    sc = (ctypes.c_double * 1)(1.5)
    _lib.check(rt.tca_rt_event_record(e0, s))
    for _ in range(3):
        _lib.check(rt.tca_program_launch(h, arr, 3, None, 0, sc, 1, s))
    _lib.check(rt.tca_rt_event_record(e1, s))
    _lib.check(rt.tca_rt_stream_sync(s))
    ms = ctypes.c_float()
    _lib.check(rt.tca_rt_event_elapsed_ms(e0, e1, ctypes.byref(ms)))
    assert ms.value > 0.0
    got = dz.get((M, N), np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for e in (e0, e1):
        _lib.check(rt.tca_rt_event_destroy(e))
    _lib.check(rt.tca_rt_stream_destroy(s))
    for d in (dx, dy, dz):
        d.free()


def test_raw_module_launch(rt):
    """tca_rt_module_load + tca_rt_launch: the code object and a kernarg blob
    packed by hand in the plan's argument order (ptr x, ptr y, ptr z, dim M,
    dim N, scalar a: natural alignment, 4-byte scalar slots)."""
    M, N = 256, 4096
    x, y, want = _scale_relu_case(M, N)
    dx, dy, dz = Dev(x.nbytes), Dev(y.nbytes), Dev(x.nbytes)
    dx.put(x)
    dy.put(y)
    prog = compiled("scale_relu_map")
    kernel = prog.kernel_symbols()[0]
    mod = ctypes.c_void_p()
    _lib.check(rt.tca_rt_module_load(prog.hsaco.encode(), ctypes.byref(mod)))
    blob = struct.pack("<QQQIIf", dx.p.value, dy.p.value, dz.p.value, M, N, 1.5)
    buf = ctypes.create_string_buffer(blob, len(blob))
    grid = (M * N + 4095) // 4096
    _lib.check(rt.tca_rt_launch(mod, kernel.encode(), grid, 256, 0, ctypes.cast(buf, ctypes.c_void_p), len(blob), None))
    _lib.check(rt.tca_rt_device_sync())
    got = dz.get((M, N), np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # an unknown kernel name is an error with a message, not a crash
    rc = rt.tca_rt_launch(mod, b"no_such_kernel", 1, 256, 0, ctypes.cast(buf, ctypes.c_void_p), len(blob), None)
    assert rc != 0 and "no_such_kernel" in _lib.last_error()
    # a geometry the wave64 grammar refuses is refused before any launch
    rc = rt.tca_rt_launch(mod, kernel.encode(), grid, 96, 0, ctypes.cast(buf, ctypes.c_void_p), len(blob), None)
    assert rc == _lib.TCA_ERR_LAUNCH
    _lib.check(rt.tca_rt_module_unload(mod))
    for d in (dx, dy, dz):
        d.free()


def test_error_paths(rt):
    mod = ctypes.c_void_p()
    rc = rt.tca_rt_module_load(b"/nonexistent/k.hsaco", ctypes.byref(mod))
    assert rc == _lib.TCA_ERR_NOT_FOUND and "nonexistent" in _lib.last_error()
    rc = rt.tca_rt_memcpy_h2d(None, None, 16)
    assert rc == _lib.TCA_ERR_INVALID and _lib.last_error()
    p = ctypes.c_void_p()
    rc = rt.tca_rt_malloc(ctypes.byref(p), 1 << 62)  # more than the device holds
    assert rc != 0 and _lib.last_error()
    # the failure is reported here and not left in HIP's last-error slot for
    # the next HIP user in the process (torch checks it after its launches)
    import torch
    torch.full((16,), 1.0, device="cuda:0")
    torch.cuda.synchronize()
    # a program launch whose tensors disagree with the plan
    prog = compiled("scale_relu_map")
    h = prog.load()
    from tcacomp_amd.compiler import _descriptors
    arr = _descriptors([TensorDesc(0x1000, (4, 8), 0), TensorDesc(0x1000, (4, 9), 0), TensorDesc(0x1000, (4, 8), 0)])
    sc = (ctypes.c_double * 1)(1.0)
    rc = rt.tca_program_launch(h, arr, 3, None, 0, sc, 1, None)
    assert rc == _lib.TCA_ERR_SHAPE and "N" in _lib.last_error()
    _lib.check(rt.tca_rt_device_sync())  # the device is still healthy


def test_one_program_on_two_streams(rt):
    """A program whose kernels use its workspace (the column family's
    partials) launched on two streams that overlap: each stream has a
    workspace of its own, so both results are exact."""
    R, C = 8192, 1024  # P = 256 row chunks per column block: partials, then the merge
    rng = np.random.default_rng(11)
    xs = [rng.integers(-8, 9, size=(R, C)).astype(np.float32) for _ in range(2)]
    want = [(x.astype(np.float64).sum(axis=0).astype(np.float32), x.max(axis=0)) for x in xs]
    prog = compiled("col_sum_max_dyn")
    h = prog.load()
    from tcacomp_amd.compiler import _descriptors
    streams, bufs, descs = [], [], []
    for x in xs:
        s = ctypes.c_void_p()
        _lib.check(rt.tca_rt_stream_create(ctypes.byref(s)))
        dx, ds, dm = Dev(x.nbytes), Dev(C * 4), Dev(C * 4)
        dx.put(x)
        streams.append(s)
        bufs.append((dx, ds, dm))
        descs.append(_descriptors([TensorDesc(dx.p.value, (R, C), 0), TensorDesc(ds.p.value, (C,), 0),
                                   TensorDesc(dm.p.value, (C,), 0)]))
    for _ in range(20):  # interleaved, never synchronized in between
        for s, arr in zip(streams, descs):
            _lib.check(rt.tca_program_launch(h, arr, 3, None, 0, None, 0, s))
    for s in streams:
        _lib.check(rt.tca_rt_stream_sync(s))
    for (dx, ds, dm), (ws, wm) in zip(bufs, want):
        np.testing.assert_array_equal(ds.get((C,), np.float32), ws)
        np.testing.assert_array_equal(dm.get((C,), np.float32), wm)
    for s in streams:
        _lib.check(rt.tca_rt_stream_destroy(s))
    for b in bufs:
        for d in b:
            d.free()
