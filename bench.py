#!/usr/bin/env python3
"""Benchmark of the map+reduce hot path on one MI355X.

Runs the BASELINE.json configurations through the HIP emitter's kernels
(tca_program_launch, the C ABI) and prints ONE JSON line. The headline
`value` is configs[1] (C2: fused row sum + row max over fp32 [8192, 8192]),
in achieved HBM GB/s; every configuration is reported under "kernels" with
its own roofline entry. A "step" is one launch of the compiled program over
one batch of inputs already resident in HBM. Inputs rotate over enough
buffer sets (>= 768 MB) that the 256 MB Infinity Cache cannot serve a
repeat. Timing: hipEvents on the launch stream around the timed steps.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c1,c2,...]
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, AMD published
MFMA_PEAK_TFLOPS = {"f32": 157.3, "bf16": 2500.0, "f16": 2500.0}  # dense, AMD published
MALL_DEFEAT_BYTES = 768 << 20

CONFIGS = {
    # key: (program, description)
    "c1": ("scale_relu", "C1 z=max(a*x+y,0) f32 [4096,4096]"),
    "c2": ("row_sum_max_8192", "C2 row sum+max f32 [8192,8192]"),
    "c3": ("softmax_4096", "C3 row softmax f32 [16384,4096]"),
    "c4": ("layernorm_1024", "C4 layernorm f32 [32768,1024]"),
    "c5f": ("gemm_f32", "C5 gemm f32 4096^3"),
    "c5b": ("gemm_bf16", "C5 gemm bf16-in f32-acc 4096^3"),
    # C5's contraction on f16 inputs: not a configuration (the bf16 kernels with the f16 MFMAs)
    "c5h": ("gemm_f16", "gemm f16-in f32-acc 4096^3 (not a configuration)"),
    # C2-C4 with the row length a run-time dim (streaming row family); same
    # data and algorithmic bytes, not configurations of their own
    "c2s": ("row_sum_max_dyn", "C2 with run-time row length (streaming family)"),
    "c3s": ("softmax_dyn", "C3 with run-time row length (streaming family)"),
    "c4s": ("layernorm_dyn", "C4 with run-time row length (streaming family)"),
    # C2's reductions on few long rows (the streaming family's split rows):
    # not configurations; shown because one workgroup per row would idle the GPU
    "c2v": ("vec_sum_max", "sum+max of one f32 vector [67108864] (split rows, full reduction)"),
    "c2r": ("row_sum_max_dyn", "row sum+max f32 [16,4194304] (split rows)"),
    # C3's softmax on few long rows: each of its three passes over a grid of
    # row chunks (partial + merge per reduction pass, a chunked row map)
    "c3r": ("softmax_dyn", "row softmax f32 [64,1048576] (few long rows: passes split over row chunks)"),
    "c4r": ("layernorm_dyn", "row layernorm f32 [64,1048576] (few long rows: passes split over row chunks)"),
    "c3v": ("softmax_dyn", "row softmax f32 [4096,40000] (streamed rows: max and exp-sum in one read, then the row map)"),
    "c4v": ("layernorm_dyn", "row layernorm f32 [4096,40000] (streamed rows: mean and centred squares in one read, then the row map)"),
    # C2's reductions over narrow element types (16-byte vectors of 8 bf16 /
    # 16 u8 elements): not configurations, the same family on other dtypes
    "c2h": ("row_sum_bf16_dyn", "row sum+max bf16 -> f32 [8192,16384] (streaming family)"),
    "c2u": ("row_sum_u8_dyn", "row sum u8 -> u32 -> f32 scaled [8192,32768] (streaming family)"),
    # C2's reductions over the non-contiguous axis (the column family): the
    # reference's middle-axis reduction form; not a configuration
    "c2c": ("col_sum_max_dyn", "column sum+max f32 [8192,8192] (column family)"),
    # dependent reductions over the non-contiguous axis (a variance reading
    # its mean): one column nest of two passes, lowered as a partial + merge
    # pair per pass ([8192, 8192]: 32 row chunks) or as one whole-column
    # kernel (64 rows: one chunk); not configurations
    "c2mv": ("col_mean_var_dyn", "column mean+variance f32 [1,8192,8192] (column family, one read: pairwise "
                                 "mean and centred sum of squares, partial + merge)"),
    "c2mw": ("col_mean_var_dyn", "column mean+variance f32 [1,64,1048576] (column family, one read: pairwise "
                                 "mean and centred sum of squares, one chunk)"),
    # C5 bf16 at 8192^3: not a configuration; four tiles per CU instead of one, so the C epilogue
    # and the ring's fill weigh a quarter as much
    "c5b8": ("gemm_bf16", "gemm bf16 -> f32 8192^3 (not a configuration)"),
    # elementwise maps whose operands are not aligned with the store: not
    # configurations. y = x*g + b + z^T (z read transposed through LDS tiles),
    # and the reference's matmul_store e2e program out[m][n][k] = lhs[m][k] *
    # rhs[n][k] (broadcast operands read per vector; 4 GiB written)
    "c1t": ("ew_bias_tr", "y = x*g[c] + b[r] + z^T f32 [8192,8192] (elementwise, transposed operand via LDS tiles)"),
    "c1m": ("e2e:mm", "out[m][n][k] = lhs[m][k]*rhs[n][k] f32 1024^3 (elementwise, broadcast operands)"),
    # not a configuration: the plain copy used to calibrate rocprof counters
    "copy": ("copy_f32", "copy f32 [8192,8192] (counter calibration)"),
}
STREAM_OF = {"c2s": "c2", "c3s": "c3", "c4s": "c4"}


def _events():
    from tcacomp_amd import _lib
    L = _lib.lib()
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    _lib.check(L.tca_rt_event_create(ctypes.byref(a)))
    _lib.check(L.tca_rt_event_create(ctypes.byref(b)))
    return a, b


def _setup(key, dev):
    """Returns (program, list of argument sets, scalars, work dict)."""
    import numpy as np
    import torch
    from tcacomp_amd import inputs, programs, compiler

    name = CONFIGS[key][0]
    factory = programs.E2E[name[4:]] if name.startswith("e2e:") else programs.CONFIG_PROGRAMS[name]
    prog = compiler.compile_program(factory(), jit=os.environ.get("TCA_JIT", "0") != "0")
    streamed = key in STREAM_OF
    key = STREAM_OF.get(key, key)

    def dev_f32(a):
        return torch.from_numpy(a).to(dev)

    if key == "c2c":
        R = C = 8192
        x = inputs.normal((R, C), 1.0, 0)
        algo = R * C * 4 + 2 * C * 4
        per_set = algo
        make = lambda i: [dev_f32(x), torch.empty(C, device=dev), torch.empty(C, device=dev)]  # noqa: E731
        scalars = []
        work = {"bytes": algo, "bound": "hbm", "shape": [R, C]}
        cpu = None
    elif key in ("c2mv", "c2mw"):
        R, C = (8192, 8192) if key == "c2mv" else (64, 1 << 20)
        x = inputs.normal((1, R, C), 1.0, 0)
        # the tile read once (the two reductions fused into one read), plus
        # the two [C] results
        algo = R * C * 4 + 2 * C * 4
        per_set = algo
        make = lambda i: [dev_f32(x), torch.empty((1, C), device=dev), torch.empty((1, C), device=dev)]  # noqa: E731
        scalars = [1.0 / R]
        work = {"bytes": algo, "bound": "hbm", "shape": [1, R, C], "single_read_bytes": R * C * 4 + 2 * C * 4}
        per_set = R * C * 4  # the footprint
        cpu = None
    elif key in ("c2v", "c2r"):
        R, C = (1, 64 << 20) if key == "c2v" else (16, 4 << 20)
        x = inputs.normal((R, C), 1.0, 0)
        algo = R * C * 4 + 2 * R * 4
        per_set = algo
        if key == "c2v":
            make = lambda i: [dev_f32(x.reshape(C)), torch.empty((), device=dev), torch.empty((), device=dev)]  # noqa: E731
        else:
            make = lambda i: [dev_f32(x), torch.empty(R, device=dev), torch.empty(R, device=dev)]  # noqa: E731
        scalars = []
        work = {"bytes": algo, "bound": "hbm", "shape": [R, C]}
        cpu = None
    elif key in ("c2h", "c2u"):
        R, C = (8192, 16384) if key == "c2h" else (8192, 32768)
        if key == "c2h":
            xd = torch.from_numpy(inputs.normal((R, C), 1.0, 0)).to(dev).to(torch.bfloat16)
            algo = R * C * 2 + 2 * R * 4
            make = lambda i: [xd.clone(), torch.empty(R, device=dev), torch.empty(R, device=dev)]  # noqa: E731
            scalars = []
        else:
            xd = torch.from_numpy(np.random.default_rng(0).integers(0, 256, size=(R, C), dtype=np.uint8)).to(dev)
            algo = R * C + R * 4
            make = lambda i: [xd.clone(), torch.empty(R, device=dev)]  # noqa: E731
            scalars = [0.37]
        per_set = algo
        work = {"bytes": algo, "bound": "hbm", "shape": [R, C]}
        cpu = None
    elif key == "c1t":
        R = C = 8192
        x, z = inputs.uniform((R, C), -1, 1, 0), inputs.uniform((C, R), -1, 1, 1)
        g, bt = inputs.uniform((C,), -1, 1, 2), inputs.uniform((R,), -1, 1, 3)
        algo = 3 * R * C * 4 + (R + C) * 4
        per_set = algo
        make = lambda i: [dev_f32(x), dev_f32(z), dev_f32(g), dev_f32(bt), torch.empty((R, C), device=dev)]  # noqa: E731
        scalars = []
        work = {"bytes": algo, "bound": "hbm", "shape": [R, C]}
        cpu = None
    elif key == "c1m":
        d = 1024
        lhs, rhs = inputs.uniform((d, d), 0, 1, 0), inputs.uniform((d, d), 0, 1, 1)
        algo = d * d * d * 4 + 2 * d * d * 4
        per_set = algo
        make = lambda i: [dev_f32(lhs), dev_f32(rhs), torch.empty((d, d, d), device=dev)]  # noqa: E731
        scalars = []
        work = {"bytes": algo, "bound": "hbm", "shape": [d, d, d]}
        cpu = None
    elif key == "copy":
        R = C = 8192
        x = inputs.uniform((R, C), -1, 1, 0)
        algo = 2 * R * C * 4
        per_set = algo
        make = lambda i: [dev_f32(x), torch.empty((R, C), device=dev)]  # noqa: E731
        scalars = []
        work = {"bytes": algo, "bound": "hbm", "shape": [R, C]}
        cpu = None
    elif key == "c1":
        M = N = 4096
        x, y = inputs.uniform((M, N, 1), -1, 1, 0), inputs.uniform((M, N, 1), -1, 1, 1)
        algo = 3 * M * N * 4
        per_set = algo
        make = lambda i: [dev_f32(x), dev_f32(y), torch.empty((M, N), device=dev)]  # noqa: E731
        scalars = [1.5]
        work = {"bytes": algo, "bound": "hbm", "shape": [M, N]}
        cpu = ("c1", (x, y))
    elif key == "c2":
        R = C = 8192
        x = inputs.normal((R, C), 1.0, 0)
        algo = R * C * 4 + 2 * R * 4
        per_set = algo
        make = lambda i: [dev_f32(x), torch.empty(R, device=dev), torch.empty(R, device=dev)]  # noqa: E731
        scalars = []
        work = {"bytes": algo, "bound": "hbm", "shape": [R, C]}
        cpu = ("c2", (x,))
    elif key == "c3r":
        R, C = 64, 1 << 20
        x = inputs.normal((R, C), 2.0, 0)
        algo = 2 * R * C * 4
        per_set = algo
        make = lambda i: [dev_f32(x), torch.empty((R, C), device=dev)]  # noqa: E731
        scalars = []
        work = {"bytes": algo, "bound": "hbm", "shape": [R, C]}
        cpu = None
    elif key == "c4r":
        R, C = 64, 1 << 20
        x = inputs.normal((R, C), 1.0, 0)
        g = inputs.uniform((C,), 0.5, 1.5, 1)
        bt = inputs.uniform((C,), -0.1, 0.1, 2)
        algo = 2 * R * C * 4 + 2 * C * 4
        per_set = algo
        make = lambda i: [dev_f32(x), dev_f32(g), dev_f32(bt), torch.empty((R, C), device=dev)]  # noqa: E731
        scalars = [1.0 / C, 1e-5]
        work = {"bytes": algo, "bound": "hbm", "shape": [R, C]}
        cpu = None
    elif key == "c3v":
        R, C = 4096, 40000
        x = inputs.normal((R, C), 2.0, 0)
        algo = 2 * R * C * 4
        per_set = algo
        make = lambda i: [dev_f32(x), torch.empty((R, C), device=dev)]  # noqa: E731
        scalars = []
        work = {"bytes": algo, "bound": "hbm", "shape": [R, C]}
        cpu = None
    elif key == "c4v":
        R, C = 4096, 40000
        x = inputs.normal((R, C), 1.0, 0)
        g = inputs.uniform((C,), 0.5, 1.5, 1)
        bt = inputs.uniform((C,), -0.1, 0.1, 2)
        algo = 2 * R * C * 4 + 2 * C * 4
        per_set = algo
        make = lambda i: [dev_f32(x), dev_f32(g), dev_f32(bt), torch.empty((R, C), device=dev)]  # noqa: E731
        scalars = [1.0 / C, 1e-5]
        work = {"bytes": algo, "bound": "hbm", "shape": [R, C]}
        cpu = None
    elif key == "c3":
        R, C = 16384, 4096
        x = inputs.normal((R, C), 2.0, 0)
        algo = 2 * R * C * 4
        per_set = algo
        make = lambda i: [dev_f32(x), torch.empty((R, C), device=dev)]  # noqa: E731
        scalars = []
        work = {"bytes": algo, "bound": "hbm", "shape": [R, C]}
        cpu = ("c3", (x,))
    elif key == "c4":
        R, C = 32768, 1024
        x = inputs.normal((R, C), 1.0, 0)
        g = inputs.uniform((C,), 0.5, 1.5, 1)
        bt = inputs.uniform((C,), -0.1, 0.1, 2)
        algo = 2 * R * C * 4 + 2 * C * 4
        per_set = algo
        make = lambda i: [dev_f32(x), dev_f32(g), dev_f32(bt), torch.empty((R, C), device=dev)]  # noqa: E731
        scalars = [1.0 / C, 1e-5]
        work = {"bytes": algo, "bound": "hbm", "shape": [R, C]}
        cpu = ("c4", (x, g, bt))
    else:
        M = N = K = 8192 if key == "c5b8" else 4096
        a = inputs.uniform((M, K), -1, 1, 0)
        b = inputs.uniform((K, N), -1, 1, 1)
        if key in ("c5b", "c5b8"):
            ta = torch.from_numpy(a).to(dev).to(torch.bfloat16)
            tb = torch.from_numpy(b).to(dev).to(torch.bfloat16)
            elt = 2
            dt = "bf16"
        elif key == "c5h":
            ta = torch.from_numpy(a).to(dev).to(torch.float16)
            tb = torch.from_numpy(b).to(dev).to(torch.float16)
            elt = 2
            dt = "f16"
        else:
            ta, tb = dev_f32(a), dev_f32(b)
            elt = 4
            dt = "f32"
        per_set = (M * K + K * N) * elt + M * N * 4
        make = lambda i: [ta.clone(), tb.clone(), torch.empty((M, N), device=dev)]  # noqa: E731
        scalars = []
        work = {"flops": 2 * M * N * K, "bound": "mfma", "dtype": dt, "shape": [M, N, K],
                "bytes": per_set}
        cpu = (key, (a, b)) if key not in ("c5b8", "c5h") else None
    nsets = max(2, math.ceil(MALL_DEFEAT_BYTES / per_set))
    sets = [make(i) for i in range(nsets)]
    if streamed:
        cpu = None  # the same CPU figure as the register-resident line
    return prog, sets, scalars, work, cpu


def _time(prog, sets, scalars, steps, warmup, settle_ms):
    import torch
    from tcacomp_amd import _lib
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    # Settle: the same launches, untimed, until settle_ms of wall time has
    # passed. The GPU's clocks ramp over the first few hundred milliseconds of
    # sustained load; a 20-step timed region (2.5 ms for the bf16 GEMM) would
    # otherwise measure the ramp rather than the kernel.
    t_end = time.perf_counter() + settle_ms * 1e-3
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(8):
            prog.launch(sets[i % len(sets)], scalars=scalars, stream=stream)
            i += 1
        torch.cuda.synchronize()
    for i in range(warmup):
        prog.launch(sets[i % len(sets)], scalars=scalars, stream=stream)
    torch.cuda.synchronize()
    e0, e1 = _events()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    _lib.check(L.tca_rt_event_record(e0, ctypes.c_void_p(stream)))
    for i in range(steps):
        prog.launch(sets[i % len(sets)], scalars=scalars, stream=stream)
    _lib.check(L.tca_rt_event_record(e1, ctypes.c_void_p(stream)))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ctypes.c_float()
    _lib.check(L.tca_rt_event_elapsed_ms(e0, e1, ctypes.byref(ms)))
    L.tca_rt_event_destroy(e0)
    L.tca_rt_event_destroy(e1)
    return ms.value / steps, wall * 1e3 / steps


def _cpu_baseline(key, args, threads):
    """The CPU oracle timed on this host on a bounded sample (best of 3).
    Returns (value, unit, sample description)."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import numpy as np
    import oracle

    def best(f, reps=3):
        t = []
        for _ in range(reps):
            s = time.perf_counter()
            f()
            t.append(time.perf_counter() - s)
        return min(t)

    if key == "c1":
        x, y = args
        xs, ys = x.reshape(-1), y.reshape(-1)
        dt = best(lambda: oracle.scale_relu(xs, ys, 1.5, threads))
        return 3 * xs.size * 4 / dt / 1e9, "GB/s", "full [4096,4096]"
    if key == "c2":
        (x,) = args
        dt = best(lambda: oracle.row_sum_max(x, threads))
        return (x.size * 4 + 2 * x.shape[0] * 4) / dt / 1e9, "GB/s", "full [8192,8192]"
    if key == "c3":
        (x,) = args
        dt = best(lambda: oracle.softmax(x, threads))
        return 2 * x.size * 4 / dt / 1e9, "GB/s", "full [16384,4096]"
    if key == "c4":
        x, g, b = args
        dt = best(lambda: oracle.layernorm(x, g, b, 1.0 / 1024, 1e-5, threads))
        return (2 * x.size * 4 + 2 * 1024 * 4) / dt / 1e9, "GB/s", "full [32768,1024]"
    a, b = args
    rows = 16 * max(1, threads)
    asub = np.ascontiguousarray(a[:rows])
    if key == "c5b":
        asub, b = oracle.to_bf16_bits(asub), oracle.to_bf16_bits(b)
    dt = best(lambda: oracle.gemm(asub, b, threads=threads), reps=1)
    return 2 * rows * 4096 * 4096 / dt / 1e12, "TFLOP/s", "%d of 4096 rows" % rows


# Configurations launching one kernel at two shapes: profiles/traffic.json
# keys their figures `symbol@config`, and a plain `symbol` entry is another
# shape's.
TRAFFIC_SHARED = ("c5b", "c5b8", "c2mv", "c2mw")


def _traffic(symbol, prog, key=None):
    """HBM bytes per launch of `symbol` from profiles/traffic.json (rocprof
    FETCH_SIZE + WRITE_SIZE, calibration-scaled), with where they come from.
    The file records the code-object key (a hash of the emitted source, the
    hipcc flags and the device headers) each figure was profiled with; when
    the kernel launched here has another key the figure is stale and is not
    reported."""
    p = os.path.join(REPO, "profiles", "traffic.json")
    if not os.path.exists(p):
        return None, "no profiles/traffic.json"
    with open(p) as f:
        t = json.load(f)
    e = t.get("%s@%s" % (symbol, key))
    if e is None and key in TRAFFIC_SHARED:
        return None, "kernel not profiled at this configuration's shape"
    if e is None:
        e = t.get(symbol)
    if e is None:
        return None, "kernel not profiled"
    if not isinstance(e, dict):
        return None, "profiled without a code-object key: provenance unknown"
    key = os.path.basename(prog.hsaco).rsplit("-", 1)[-1].split(".")[0]
    if e.get("code_object") != key:
        return None, "stale: kernel changed since it was profiled (%s, now %s)" % (e.get("code_object"), key)
    return e["bytes"], "profiles/traffic.json (%s, code object %s)" % (t.get("_profiled", "?"), key)


def _window_us(prog, args, sc, stream, steps, hold_cycles=0):
    """Microseconds per launch between two events around `steps` launches.
    With hold_cycles > 0 a spin kernel of that many clock cycles is queued
    first, so the launches are all queued before the GPU reaches them and
    run back to back: the window is then device time per launch (kernel
    durations and the dispatch gaps between them), not the host's launch
    rate."""
    import torch
    from tcacomp_amd import _lib
    L = _lib.lib()
    e0, e1 = _events()
    torch.cuda.synchronize()
    if hold_cycles:
        torch.cuda._sleep(int(hold_cycles))
    _lib.check(L.tca_rt_event_record(e0, ctypes.c_void_p(stream)))
    for _ in range(steps):
        prog.launch(args, scalars=sc, stream=stream)
    _lib.check(L.tca_rt_event_record(e1, ctypes.c_void_p(stream)))
    torch.cuda.synchronize()
    ms = ctypes.c_float()
    _lib.check(L.tca_rt_event_elapsed_ms(e0, e1, ctypes.byref(ms)))
    L.tca_rt_event_destroy(e0)
    L.tca_rt_event_destroy(e1)
    return ms.value * 1e3 / steps


def _suite(dev, steps):
    """The reference's 14 suite kernels at testing/suite.toml's dims, inputs
    from elem(i): kernel_us, the device time per launch (`steps` launches
    queued behind a spin kernel, so they run back to back: the kernels'
    durations plus the dispatch gaps between them); launch_rate_us, the
    same event window without the hold (bounded by the host's launch rate);
    the reference runner's BenchReport (host launch + synchronize per
    iteration, 20 iterations); the achieved rate over suite.toml's
    bench_bytes (and flops for contractions) at kernel_us; and the
    reference's own A6000 figures. A kernel trace (rocprofv3) of the same
    window reports longer durations for these microsecond kernels: its
    back-to-back dispatches tile the window with no gap, and the window
    itself takes 0.4-1 us more per launch under the profiler (its
    per-dispatch completion signal)."""
    import torch
    from tcacomp_amd import compiler, programs, suite
    stream = torch.cuda.current_stream().cuda_stream
    out = {}
    for name in sorted(suite.REGISTRY):
        prog = compiler.compile_program(programs.SUITE[name][0](), jit=os.environ.get("TCA_JIT", "0") != "0")
        ins, oshape = suite.host_inputs(name)
        args = [torch.from_numpy(a).to(dev) for a in ins] + [torch.empty(oshape, device=dev)]
        sc = suite.scalars(name)
        for _ in range(20):
            prog.launch(args, scalars=sc, stream=stream)
        torch.cuda.synchronize()
        rate_us = _window_us(prog, args, sc, stream, steps)
        # Hold the queue for three times the host's enqueue time (clock
        # cycles at up to 2.4 GHz), so every launch is queued before the
        # first one runs.
        t0 = time.perf_counter()
        for _ in range(steps):
            prog.launch(args, scalars=sc, stream=stream)
        enqueue_s = time.perf_counter() - t0
        torch.cuda.synchronize()
        dev_us = _window_us(prog, args, sc, stream, steps, hold_cycles=3 * enqueue_s * 2.4e9)
        host = []
        for _ in range(20):
            t0 = time.perf_counter()
            prog.launch(args, scalars=sc, stream=stream)
            torch.cuda.synchronize()
            host.append((time.perf_counter() - t0) * 1e6)
        cat, dims, tol, bench_bytes = suite.REGISTRY[name]
        ref_avg, ref_min = suite.REFERENCE_A6000_US[name]
        e = {"dims": list(dims), "kernels": prog.selected_symbols(args), "kernel_us": dev_us,
             "launch_rate_us": rate_us, "bench_us": {"avg": sum(host) / len(host), "min": min(host)},
             "bench_bytes": bench_bytes, "achieved_GBps": bench_bytes / (dev_us * 1e-6) / 1e9,
             "reference_a6000_bench_us": {"avg": ref_avg, "min": ref_min},
             "speedup_vs_reference_min": ref_min / min(host)}
        if suite.flops(name):
            e["achieved_GFLOPs"] = suite.flops(name) / (dev_us * 1e-6) / 1e9
        out[name] = e
        print("[bench] suite %s %.2f us per launch on the device, %.2f us launch rate, %.1f us launch+sync "
              "(reference A6000 %.1f us)" % (name, dev_us, rate_us, min(host), ref_min), file=sys.stderr, flush=True)
    return out


def _gemm_sweep(dev, steps):
    """Contractions at small and medium output planes (the small-tile K-split
    kernel up to M*N = 2^20, the tile kernels above): M, N in {64, 256, 1024,
    2048}, K in {64, 4096}, f32 and bf16 inputs, B as [K][N] and [N][K];
    device time per launch from the held window (kernels back to back)."""
    import torch
    from tcacomp_amd import compiler, programs
    stream = torch.cuda.current_stream().cuda_stream
    out = []
    for pname in ("gemm_f32", "gemm_f32_nt", "gemm_bf16", "gemm_bf16_nt"):
        prog = compiler.compile_program(programs.CONFIG_PROGRAMS[pname](), jit=os.environ.get("TCA_JIT", "0") != "0")
        nt, bf = pname.endswith("_nt"), "bf16" in pname
        for M in (64, 256, 1024, 2048):
            for N in (64, 256, 1024, 2048):
                for K in (64, 4096):
                    g = torch.Generator(device=dev).manual_seed(M + N + K)
                    a = torch.rand((M, K), device=dev, generator=g) * 2 - 1
                    b = torch.rand((N, K) if nt else (K, N), device=dev, generator=g) * 2 - 1
                    if bf:
                        a, b = a.to(torch.bfloat16), b.to(torch.bfloat16)
                    args = [a, b, torch.empty((M, N), device=dev)]
                    for _ in range(10):
                        prog.launch(args, stream=stream)
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                    for _ in range(steps):
                        prog.launch(args, stream=stream)
                    enq = time.perf_counter() - t0
                    torch.cuda.synchronize()
                    us = _window_us(prog, args, [], stream, steps, hold_cycles=3 * enq * 2.4e9)
                    e = {"program": pname, "M": M, "N": N, "K": K, "kernels": prog.selected_symbols(args),
                         "us": us, "TFLOPs": 2.0 * M * N * K / (us * 1e-6) / 1e12}
                    out.append(e)
                    print("[bench] sweep %s %dx%dx%d %.2f us %.2f TFLOP/s %s" % (
                        pname, M, N, K, us, e["TFLOPs"], [s.split("_k0")[-1] for s in e["kernels"]]),
                        file=sys.stderr, flush=True)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="c1,c2,c3,c4,c5f,c5b,c2s,c3s,c4s,c2v,c2r,c3r,c4r,c3v,c4v,c2h,c2u,c2c,c2mv,c2mw,c5b8,c5h,c1t,c1m")
    ap.add_argument("--settle-ms", type=float, default=1000.0,
                    help="untimed launches per config before the warmup steps, in wall-clock ms")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline")
    ap.add_argument("--no-suite", action="store_true", help="skip the reference suite's 14 kernels")
    ap.add_argument("--gemm-sweep", action="store_true",
                    help="only the contraction sweep (M, N in 64..2048, K in 64, 4096; one JSON line of its own)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the row configurations would "
              "shard by rows with no exchange, the GEMM by row panels of A after an all-gather of B, and each "
              "GPU would run these same kernels at its shard shape). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    from tcacomp_amd import _lib
    dev = torch.device("cuda:0")
    _lib.check(_lib.lib().tca_rt_init(0))
    if args.gemm_sweep:
        print(json.dumps({"gemm_sweep": _gemm_sweep(dev, args.steps)}))
        return
    keys = [k for k in args.configs.split(",") if k]
    # The N-core CPU figure uses the host's cores (the box's CPU share: its
    # OMP_NUM_THREADS), overridable with TCA_CPU_THREADS.
    ncpu = os.cpu_count() or 1
    threads = int(os.environ.get("TCA_CPU_THREADS") or os.environ.get("OMP_NUM_THREADS") or ncpu)
    threads = max(1, min(threads, ncpu))
    results = {}
    for key in keys:
        prog, sets, scalars, work, cpu = _setup(key, dev)
        ms, wall_ms = _time(prog, sets, scalars, args.steps, args.warmup, args.settle_ms)
        sym = prog.selected_symbols(sets[0])[0]
        entry = {"config": CONFIGS[key][1], "kernel": sym, "family": prog.families()[0], "ms": ms,
                 "host_wall_ms": wall_ms}
        if work["bound"] == "hbm":
            gbs = work["bytes"] / (ms * 1e-3) / 1e9
            traffic, source = _traffic(sym, prog, key)
            entry["roofline"] = {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                 "frac": gbs / HBM_PEAK_GBS, "traffic": traffic, "traffic_source": source}
            entry["algorithmic_bytes"] = work["bytes"]
            if "single_read_bytes" in work:  # the tile read once: the bound a fused single read would meet
                entry["single_read_GBps"] = work["single_read_bytes"] / (ms * 1e-3) / 1e9
        else:
            tf = work["flops"] / (ms * 1e-3) / 1e12
            peak = MFMA_PEAK_TFLOPS[work["dtype"]]
            traffic, source = _traffic(sym, prog, key)
            entry["roofline"] = {"bound": "mfma", "achieved": tf, "peak": peak, "unit": "TFLOP/s",
                                 "frac": tf / peak, "traffic": traffic, "traffic_source": source}
            entry["algorithmic_flops"] = work["flops"]
        if not args.no_cpu and cpu is not None:
            v1, unit, sample = _cpu_baseline(key, cpu[1], 1)
            entry["cpu_baseline"] = {"value": v1, "unit": unit, "cores": 1, "kind": "port", "sample": sample}
            vn, _, sample_n = _cpu_baseline(key, cpu[1], threads)
            entry["cpu_baseline_ncores"] = {"value": vn, "unit": unit, "cores": threads, "kind": "port",
                                            "sample": sample_n + " (rows split over the cores, each row's fold order "
                                            "unchanged: results bit-identical to 1 core)"}
        results[key] = entry
        print("[bench] %s %s %.4f ms %s" % (key, sym, ms, json.dumps(entry["roofline"])), file=sys.stderr,
              flush=True)
        del sets
        torch.cuda.empty_cache()
    head = results.get("c2") or next(iter(results.values()))
    line = {
        "metric": "achieved HBM GB/s (% of peak) per kernel; matmul TFLOP/s (% MFMA peak)",
        "value": head["roofline"]["achieved"],
        "unit": head["roofline"]["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded counter-based U/N generators, host-generated, resident in HBM)",
        "config": {"workload": head["config"], "kernel": head["kernel"]},
        "roofline": head["roofline"],
        "cpu_baseline": head.get("cpu_baseline"),
        "cpu_baseline_ncores": head.get("cpu_baseline_ncores"),
        "kernels": results,
    }
    if not args.no_suite:
        line["suite"] = _suite(dev, 200)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
