"""tca_program_launch_noalloc: the allocation-free launch against
tca_program_launch, through the C ABI.

Each case uses a kernel family with a scratch workspace: split-row partials,
column-reduction partials, HBM-resident locals (the generic lowering) and a
chained reduction's local. Two calls in a row, the second with a smaller
input, each compared bit for bit with the allocating launch of the same
program on the same inputs (the same kernels run on the same data, so the
outputs are identical). A workspace beyond the 32 MiB scratch is refused
before anything is queued.
"""
import sys

import numpy as np
import pytest
import torch

from helpers import CANARY, compiled
from tcacomp_amd import _lib, inputs
from tcacomp_amd.pkg import EMIT_NO_FUSION, EMIT_NO_GEMM

pytestmark = pytest.mark.gpu
GENERIC = EMIT_NO_FUSION | EMIT_NO_GEMM

CASES = [
    # (program, emit flags, [first shape, smaller second shape], outputs' shapes, scalars)
    ("row_sum_max_dyn", 0, [(3, 1_000_000), (2, 200_000)], lambda R, C: [(R,), (R,)], ()),
    ("col_sum_max_dyn", 0, [(8192, 1024), (300, 512)], lambda R, C: [(C,), (C,)], ()),
    ("softmax_200", GENERIC, [(257, 200), (5, 200)], lambda R, C: [(R, C)], ()),
    ("chain_sum_max", 0, [(6, 40, 96), (3, 17, 96)], None, (-0.5,)),
]


def _workspace_used(prog, tensors):
    """The program's plan has locals and a selected kernel takes one."""
    locals_ = [l.split()[1] for l in prog.plan.splitlines() if l.startswith("tensor ") and l.split()[3] == "local"]
    assert locals_, "program has no workspace locals"
    return locals_


def _run(prog, x, out_shapes, scalars, noalloc):
    outs = [torch.full(s, CANARY, device=x.device) for s in out_shapes]
    prog.launch([x] + outs, scalars=scalars, noalloc=noalloc)
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in outs]


@pytest.mark.parametrize("name,flags,shapes,outs,scalars", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_allocating_launch(gpu, name, flags, shapes, outs, scalars):
    prog = compiled(name, flags)
    for shape in shapes:  # two calls in a row, the second smaller
        print("noalloc", name, shape, flush=True)
        sys.stdout.flush()
        x = torch.from_numpy(inputs.normal(shape, 1.0, 3)).to(gpu)
        if outs is None:  # chained reduction: x [B, R, C] -> out [B]
            out_shapes = [(shape[0],)]
        else:
            out_shapes = outs(*shape)
        _workspace_used(prog, [x])
        want = _run(prog, x, out_shapes, scalars, noalloc=False)
        got = _run(prog, x, out_shapes, scalars, noalloc=True)
        for g, w in zip(got, want):
            assert not np.any(g == np.float32(CANARY))
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), (name, shape)


def test_noalloc_refuses_oversized_workspace(gpu):
    """Locals of 2 x 4.3 M floats (34.4 MB) exceed the 32 MiB scratch: the
    call fails before queueing a kernel; the output keeps its canary."""
    prog = compiled("softmax_200", GENERIC)
    R, C = 4_300_000, 200
    x = torch.zeros((R, C), device=gpu)
    y = torch.full((8,), CANARY, device=gpu)  # sentinel: nothing may run
    out = torch.empty((R, C), device=gpu)
    out[:8, 0] = y
    with pytest.raises(_lib.TcaError) as e:
        prog.launch([x, out], noalloc=True)
    assert "32" in str(e.value) or "scratch" in str(e.value)
    torch.cuda.synchronize()
    assert torch.equal(out[:8, 0], y)
