"""The reference's 14-kernel suite as data, its inputs and its runner
protocol.

REGISTRY restates testing/suite.toml (dims, tolerances, scalars,
bench_bytes per kernel); the programs are the pkg-API restatements in
programs.SUITE (the same IR the .tca sources build). inputs() fills every
input from the runners' elem(i) formula (testing/runners/common.cuh:19-21)
and allocates the output pre-filled with the runners' canary. protocol()
prints the machine-parseable lines the runners print
(testing/runners/common.cuh:50-90: CANARY, CHECKSUM, REF_CHECKSUM, MAXDIFF,
SAMPLES, BENCH_US) and parse_protocol() reads them back the way the
orchestrator does (testing/orchestrator.py:140-164); verify() applies its
pass rule (canary == 0 and maxdiff <= tolerance, :319-345). The expected
values come from the caller: this module computes no reference result.
"""
import math

import numpy as np

from . import inputs as _inputs
from . import programs

CANARY = -12345.0  # testing/runners/softmax.cu:24

# name: (category, dims, tolerance, bench_bytes)  -- testing/suite.toml:15-153
REGISTRY = {
    "dup_expr": ("dedup", (256, 256, 8), 1e-5, 4456448),
    "dup_const": ("dedup", (256, 256, 8), 1e-5, 4456448),
    "axpy3": ("fusion", (512, 512, 4), 1e-5, 9437184),
    "mlp": ("fusion", (64, 128, 64), 2e-3, 98304),
    "softmax": ("fusion", (128, 8, 256), 2e-3, 2228224),
    "mm_small": ("tiling", (32, 32, 32), 2e-3, 16384),
    "mm_mid": ("tiling", (128, 256, 64), 2e-3, 262144),
    "mm_splitk": ("tiling", (64, 128, 64), 2e-3, 98304),
    "transpose": ("tiling", (192, 96, 8), 1e-5, 1253376),
    "row_sum": ("runtime", (512, 4, 1024), 2e-3, 18874368),
    "scale_copy": ("runtime", (512, 512, 4), 1e-5, 9437184),
    "gemm": ("llm", (128, 128, 96), 2e-3, 212992),
    "qk_score": ("llm", (128, 64, 192), 2e-3, 278528),
    "layernorm": ("llm", (128, 256, 64), 1e-5, 16908288),
}

# The reference's own timings of these kernels on its A6000 (sm_86), BENCH_US
# avg / min over its 4-run table, in microseconds
# (.planning/quick/261101-oqg-fix7-5-slice-1c-effect-chain-vectorizati/after-bench.txt:97-110).
REFERENCE_A6000_US = {
    "dup_expr": (1748.7, 1740.4), "dup_const": (2600.6, 2588.0), "axpy3": (3808.3, 3524.7),
    "mlp": (6924.2, 6315.6), "softmax": (839.3, 837.9), "mm_small": (3585.7, 3007.1),
    "mm_mid": (6950.6, 6508.7), "mm_splitk": (6527.6, 6128.6), "transpose": (950.7, 950.0),
    "row_sum": (5355.7, 5242.2), "scale_copy": (3571.8, 3288.4), "gemm": (10487.2, 9780.5),
    "qk_score": (18354.1, 17424.4), "layernorm": (9475.6, 8971.8),
}

# Rank-3 kernels: x, z [R, C, K] (K innermost, reduced) or, for the
# middle-axis reductions, [R, K, C].
RANK3_MIDDLE = {"dup_expr": False, "dup_const": False, "axpy3": False, "scale_copy": False, "transpose": False,
                "layernorm": False, "row_sum": True, "softmax": True}
MATMULS = ("mlp", "mm_small", "mm_mid", "mm_splitk", "gemm", "qk_score")


def flops(name):
    """Multiply-add flops of a contraction kernel (2 per term), else 0."""
    if name not in MATMULS:
        return 0
    a, b, c = REGISTRY[name][1]
    return 2 * a * b * c


def host_inputs(name):
    """(input arrays, output shape) in the runner's layout, from elem(i)."""
    dims = REGISTRY[name][1]
    if name in RANK3_MIDDLE:
        if RANK3_MIDDLE[name]:
            R, K, C = dims
            shape = (R, K, C)
        else:
            R, C, K = dims
            shape = (R, C, K)
        n = R * C * K
        x = _inputs.elem(n).reshape(shape)
        return [x, x.copy()], (R, C)  # the runners fill both operands from elem(i)
    if name == "qk_score":
        H, D, N = dims  # q [H, D], k [N, D] (testing/runners/qk_score.cu:10)
        return [_inputs.elem(H * D).reshape(H, D), _inputs.elem(N * D).reshape(N, D)], (H, N)
    M, K, N = dims
    return [_inputs.elem(M * K).reshape(M, K), _inputs.elem(K * N).reshape(K, N)], (M, N)


def scalars(name):
    return list(programs.SUITE[name][2].values())


def protocol(got, want, canaries, bench_us=None):
    """The runner's stdout protocol lines for one run."""
    g = np.asarray(got, dtype=np.float32).reshape(-1)
    w = np.asarray(want, dtype=np.float32).reshape(-1)
    lines = ["CANARY %d" % canaries,
             "CHECKSUM %.17g" % float(g.astype(np.float64).sum()),
             "REF_CHECKSUM %.17g" % float(w.astype(np.float64).sum()),
             "MAXDIFF %.17g" % (float(np.abs(g.astype(np.float64) - w.astype(np.float64)).max()) if g.size else 0.0),
             "SAMPLES" + "".join(" " + float(v).hex() for v in g[:8])]
    if bench_us is not None:
        lines.append("BENCH_US %g %g %g" % (sum(bench_us) / len(bench_us), min(bench_us), max(bench_us)))
    return "\n".join(lines) + "\n"


def parse_protocol(text):
    """CANARY/CHECKSUM/REF_CHECKSUM/MAXDIFF/SAMPLES/BENCH_US fields of a
    protocol text (testing/orchestrator.py:140-164)."""
    out = {}
    for line in text.splitlines():
        f = line.split()
        if not f:
            continue
        try:
            if f[0] == "CANARY" and len(f) >= 2:
                out["canary"] = int(f[1])
            elif f[0] == "CHECKSUM" and len(f) >= 2:
                out["checksum"] = float(f[1])
            elif f[0] == "REF_CHECKSUM" and len(f) >= 2:
                out["ref_checksum"] = float(f[1])
            elif f[0] == "MAXDIFF" and len(f) >= 2:
                out["maxdiff"] = float(f[1])
            elif f[0] == "SAMPLES":
                out["samples"] = f[1:9]
            elif f[0] == "BENCH_US" and len(f) >= 4:
                out["bench"] = (float(f[1]), float(f[2]), float(f[3]))
        except ValueError:
            out.setdefault("malformed", []).append(line)
    return out


def verify(name, proto):
    """The orchestrator's verdict (testing/orchestrator.py:319-345): a list
    of failure strings, empty when the run passes."""
    fails = []
    if "canary" not in proto or "maxdiff" not in proto:
        fails.append("protocol lines missing")
        return fails
    if proto["canary"] != 0:
        fails.append("canary: %d unwritten output(s)" % proto["canary"])
    tol = REGISTRY[name][2]
    if not (proto["maxdiff"] <= tol) or math.isnan(proto["maxdiff"]):
        fails.append("maxdiff %g > tolerance %g" % (proto["maxdiff"], tol))
    return fails
