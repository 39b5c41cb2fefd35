"""The configurations compiled from .tca source (tcacomp_amd/tca/configs.tca)
through the text frontend, the emitter and the runtime, checked against the
CPU oracle with the same tolerances as test_gpu_configs.py. The frontend
builds the same IR as the pkg-API programs, so these launches use the
prebuilt code objects."""
import os
import sys

import numpy as np
import pytest

import oracle
from helpers import assert_layernorm_close, assert_reduce_close, canaries, host, out_dev, reduce_tol, run, to_dev
from tcacomp_amd import compiler, inputs, syntax

pytestmark = pytest.mark.gpu
CONFIGS_TCA = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "tcacomp_amd", "tca",
                           "configs.tca")
_progs = {}


def tca(name):
    if name not in _progs:
        _progs[name] = compiler.compile_program(syntax.ParseModule(CONFIGS_TCA).Kernel(name).Build())
    return _progs[name]


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_tca_c1_scale_relu_map_bitwise(gpu):
    M, N = 257, 1031
    _say("tca C1", M, N)
    x, y = inputs.uniform((M, N), -1, 1, 0), inputs.uniform((M, N), -1, 1, 1)
    want = oracle.scale_relu(x.reshape(-1), y.reshape(-1), 1.5).reshape(M, N)
    z = out_dev((M, N), gpu)
    run(tca("scale_relu_map"), [to_dev(x, gpu), to_dev(y, gpu), z], scalars=[1.5])
    got = host(z)
    assert canaries(got) == 0 and np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_tca_c2_row_sum_max(gpu):
    R, C = 37, 8192
    _say("tca C2", R)
    x = inputs.normal((R, C), 1.0, 0)
    ws, wm = oracle.row_sum_max(x)
    s, m = out_dev((R,), gpu), out_dev((R,), gpu)
    run(tca("row_sum_max_8192"), [to_dev(x, gpu), s, m])
    assert np.array_equal(host(m).view(np.uint32), wm.view(np.uint32))
    assert_reduce_close(host(s), ws, np.sqrt((x.astype(np.float64) ** 2).sum(1)), C, "row sum")


def test_tca_c3_softmax(gpu):
    R, C = 19, 4096
    _say("tca C3", R)
    x = inputs.normal((R, C), 2.0, 0)
    want = oracle.softmax(x)
    y = out_dev((R, C), gpu)
    run(tca("softmax_4096"), [to_dev(x, gpu), y])
    got = host(y)
    assert canaries(got) == 0
    rel = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want), np.finfo(np.float32).tiny)
    assert rel.max() <= reduce_tol(C), rel.max()


def test_tca_c4_layernorm(gpu):
    R, C = 23, 1024
    _say("tca C4", R)
    x = inputs.normal((R, C), 1.0, 0)
    g, b = inputs.uniform((C,), 0.5, 1.5, 1), inputs.uniform((C,), -0.1, 0.1, 2)
    want = oracle.layernorm(x, g, b, 1.0 / C, 1e-5)
    y = out_dev((R, C), gpu)
    run(tca("layernorm_1024"), [to_dev(x, gpu), to_dev(g, gpu), to_dev(b, gpu), y], scalars=[1.0 / C, 1e-5])
    got = host(y)
    assert canaries(got) == 0
    assert_layernorm_close(got, want, x, g, b, 1e-5, "tca C4")


@pytest.mark.parametrize("name", ["gemm_f32", "gemm_bf16"])
def test_tca_c5_gemm(gpu, name):
    import torch
    M, N, K = 200, 136, 300
    _say("tca C5", name)
    a, b = inputs.uniform((M, K), -1, 1, 0), inputs.uniform((K, N), -1, 1, 1)
    if name == "gemm_bf16":
        a, b = oracle.to_bf16_bits(a), oracle.to_bf16_bits(b)
        ta = to_dev(a.view(np.int16), gpu).view(torch.bfloat16)
        tb = to_dev(b.view(np.int16), gpu).view(torch.bfloat16)
    else:
        ta, tb = to_dev(a, gpu), to_dev(b, gpu)
    want = oracle.gemm(a, b)
    c = out_dev((M, N), gpu)
    run(tca(name), [ta, tb, c])
    got = host(c)
    assert canaries(got) == 0
    af = a if a.dtype == np.float32 else oracle.bf16_bits_to_f32(a)
    bf = b if b.dtype == np.float32 else oracle.bf16_bits_to_f32(b)
    bound = np.sqrt((af.astype(np.float64) ** 2).sum(1))[:, None] * np.sqrt((bf.astype(np.float64) ** 2).sum(0))[None, :]
    assert_reduce_close(got, want, bound, K, name)
