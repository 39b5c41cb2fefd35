"""The code objects the compiler driver's output builds (build() runs
`tcacomp compile -o tcacomp_amd/_cli_out tcacomp_amd/tca/configs.tca` and
`make` there), loaded from those files only — <kernel>.hsaco and the
<kernel>.plan beside it, through tca_program_load — and checked against the
CPU oracle with the tolerances of test_gpu_configs.py. This is the user's
path of cmd/tcacomp/main.go: compile a .tca file, build what it wrote, launch
it through the runtime."""
import os
import sys

import numpy as np
import pytest

import oracle
from helpers import assert_layernorm_close, assert_reduce_close, canaries, host, out_dev, reduce_tol, run, to_dev
from tcacomp_amd import build as tb
from tcacomp_amd import compiler, inputs
from tcacomp_amd.pkg import EmitResult

pytestmark = pytest.mark.gpu
_progs = {}


def cli_program(name):
    """A program made of the driver's files alone (no emitter call)."""
    if name not in _progs:
        base = os.path.join(tb.CLI_OUT, name)
        with open(base + ".hip") as f:
            src = f.read()
        with open(base + ".plan") as f:
            plan = f.read()
        _progs[name] = compiler.CompiledProgram(name, EmitResult(src, plan, "", []), base + ".hsaco")
    return _progs[name]


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_cli_c1_scale_relu_map_bitwise(gpu):
    M, N = 129, 2051
    _say("cli C1", M, N)
    x, y = inputs.uniform((M, N), -1, 1, 3), inputs.uniform((M, N), -1, 1, 4)
    want = oracle.scale_relu(x.reshape(-1), y.reshape(-1), 1.5).reshape(M, N)
    z = out_dev((M, N), gpu)
    run(cli_program("scale_relu_map"), [to_dev(x, gpu), to_dev(y, gpu), z], scalars=[1.5])
    got = host(z)
    assert canaries(got) == 0 and np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_cli_c2_row_sum_max(gpu):
    R, C = 41, 8192
    _say("cli C2", R)
    x = inputs.normal((R, C), 1.0, 3)
    ws, wm = oracle.row_sum_max(x)
    s, m = out_dev((R,), gpu), out_dev((R,), gpu)
    run(cli_program("row_sum_max_8192"), [to_dev(x, gpu), s, m])
    assert canaries(host(s)) == 0 and canaries(host(m)) == 0
    assert np.array_equal(host(m).view(np.uint32), wm.view(np.uint32))
    assert_reduce_close(host(s), ws, np.sqrt((x.astype(np.float64) ** 2).sum(1)), C, "row sum")


def test_cli_c3_softmax(gpu):
    R, C = 21, 4096
    _say("cli C3", R)
    x = inputs.normal((R, C), 2.0, 3)
    want = oracle.softmax(x)
    y = out_dev((R, C), gpu)
    run(cli_program("softmax_4096"), [to_dev(x, gpu), y])
    got = host(y)
    assert canaries(got) == 0
    rel = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want), np.finfo(np.float32).tiny)
    assert rel.max() <= reduce_tol(C), rel.max()


def test_cli_c4_layernorm(gpu):
    R, C = 27, 1024
    _say("cli C4", R)
    x = inputs.normal((R, C), 1.0, 3)
    g, b = inputs.uniform((C,), 0.5, 1.5, 4), inputs.uniform((C,), -0.1, 0.1, 5)
    want = oracle.layernorm(x, g, b, 1.0 / C, 1e-5)
    y = out_dev((R, C), gpu)
    run(cli_program("layernorm_1024"), [to_dev(x, gpu), to_dev(g, gpu), to_dev(b, gpu), y],
        scalars=[1.0 / C, 1e-5])
    got = host(y)
    assert canaries(got) == 0
    assert_layernorm_close(got, want, x, g, b, 1e-5, "cli C4")


@pytest.mark.parametrize("name", ["gemm_f32", "gemm_bf16"])
def test_cli_c5_gemm(gpu, name):
    import torch
    # Whole 256x256 tiles plus ragged edges, K a multiple of 64 from 256 on:
    # the bf16 launch takes its whole-tile kernel and the edge kernel.
    M, N, K = 520, 264, 512
    _say("cli C5", name, M, N, K)
    a, b = inputs.uniform((M, K), -1, 1, 3), inputs.uniform((K, N), -1, 1, 4)
    if name == "gemm_bf16":
        a, b = oracle.to_bf16_bits(a), oracle.to_bf16_bits(b)
        ta = to_dev(a.view(np.int16), gpu).view(torch.bfloat16)
        tb_ = to_dev(b.view(np.int16), gpu).view(torch.bfloat16)
    else:
        ta, tb_ = to_dev(a, gpu), to_dev(b, gpu)
    want = oracle.gemm(a, b)
    c = out_dev((M, N), gpu)
    run(cli_program(name), [ta, tb_, c])
    got = host(c)
    assert canaries(got) == 0
    af = a if a.dtype == np.float32 else oracle.bf16_bits_to_f32(a)
    bf = b if b.dtype == np.float32 else oracle.bf16_bits_to_f32(b)
    bound = np.sqrt((af.astype(np.float64) ** 2).sum(1))[:, None] * np.sqrt((bf.astype(np.float64) ** 2).sum(0))[None, :]
    assert_reduce_close(got, want, bound, K, name)
