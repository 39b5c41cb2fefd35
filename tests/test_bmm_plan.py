"""Host-only checks of the batched contraction lowering (tests/test_gpu_bmm.py
runs it): which chains take the MFMA family with a batch axis, the grid it
plans (one (m, n) grid of tiles per batch), the per-batch operand offsets
the wrappers apply, and the launch contract for shared operands."""
import pytest

from tcacomp_amd import compiler, programs
from tcacomp_amd.compiler import TensorDesc
from tcacomp_amd.pkg import At, NewBuilder, TF32

P = 1 << 20  # any non-null address: nothing is dereferenced host-side


def _kernels(plan):
    return [line.split() for line in plan.splitlines() if line.startswith("kernel ")]


@pytest.mark.parametrize("name", ["bmm_f32", "bmm_bf16_nt", "bmm_f16_shared_scale"])
def test_batched_contractions_take_the_mfma_family(name):
    e = programs.CONFIG_PROGRAMS[name]().emit()
    assert set(e.families()) == {"gemm"}
    for k in _kernels(e.plan):
        assert k[4] == "3" and k[5] == "B/1", k  # batch x tiles_m x tiles_n
    assert "batched (over @B) contraction" in e.source
    # The wrapper offsets C, and each operand led by the batch axis, to its batch.
    assert "(t2 + (size_t)bb * M * N)" in e.source
    assert "(t0 + (size_t)bb * M * K)" in e.source
    if name == "bmm_f16_shared_scale":
        assert "(t1 + (size_t)bb" not in e.source  # rhs shared by every batch
    else:
        assert "(t1 + (size_t)bb * K * N)" in e.source


def test_unbatched_contractions_emit_no_batch_split():
    e = programs.CONFIG_PROGRAMS["gemm_bf16"]().emit()
    assert "bb = blockIdx.x" not in e.source
    assert all(k[4] == "2" for k in _kernels(e.plan))


def test_epilogue_read_per_batch_is_not_a_contraction():
    # A piped operand indexed by the batch axis is outside the epilogue's
    # (m, n) contract: the chain lowers elsewhere, never to a wrong GEMM.
    b = NewBuilder("bmm_bias_per_batch")
    B, M, K, N = b.Dim("B", 0), b.Dim("M", 0), b.Dim("K", 0), b.Dim("N", 0)
    lhs, rhs = b.Tensor("lhs", TF32, B, M, K), b.Tensor("rhs", TF32, B, K, N)
    bias = b.Tensor("bias", TF32, B, N)
    out = b.Tensor("out", TF32, B, M, N)
    (b.Stmt().Iter(B, M, N, K).Map([At(lhs, B, M, K), At(rhs, B, K, N)], lambda l, r: b.Mul(l, r)).As(B, M, N, K)
     .Reduce(b.Float32(0), programs._sum(b))
     .Map([At(bias, B, N)], lambda v, z: b.Add(v, z)).As(B, M, N).Store(out, B, M, N))
    fam = b.Build().emit().families()
    assert "gemm" not in fam and fam


# Descriptor dtype codes: f32 0, f16 1, bf16 2 (the inputs); outputs are f32.
IN_CODE = {"bmm_f32": 0, "bmm_f16_shared_scale": 1, "bmm_bf16_nt": 2}


@pytest.mark.parametrize("name,shapes,ok", [
    ("bmm_f32", [(2, 64, 32), (2, 32, 48), (2, 64, 48)], True),
    ("bmm_f32", [(2, 64, 32), (3, 32, 48), (2, 64, 48)], False),
    ("bmm_f16_shared_scale", [(2, 64, 32), (32, 48), (2, 64, 48)], True),
    ("bmm_f16_shared_scale", [(2, 64, 32), (2, 32, 48), (2, 64, 48)], False),
    ("bmm_bf16_nt", [(2, 64, 32), (2, 48, 32), (2, 64, 48)], True),
    ("bmm_bf16_nt", [(2, 64, 32), (2, 32, 48), (2, 64, 48)], False),
])
def test_launch_contract(name, shapes, ok):
    prog = compiler.CompiledProgram(name, programs.CONFIG_PROGRAMS[name]().emit(), "")
    codes = [IN_CODE[name], IN_CODE[name], 0]
    rc = prog.check([TensorDesc(P, s, c) for s, c in zip(shapes, codes)])
    assert (rc == 0) == ok, rc
