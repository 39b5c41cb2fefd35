"""tca_program_launch_noalloc: the allocation-free launch against
tca_program_launch, through the C ABI.

Each case uses a kernel family with a scratch workspace: split-row partials,
column-reduction partials, HBM-resident locals (the generic lowering), a
chained reduction's local, split softmax and layernorm rows and the one-read
column mean and variance. Two calls in a row, the second with a smaller
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
    # split softmax rows (online max/exp-sum partials, plan-only row locals)
    ("softmax_dyn", 0, [(4, 1_000_000), (2, 300_000)], lambda R, C: [(R, C)], ()),
    # one-read column mean + variance (sum and centred-square partials)
    ("col_mean_var_dyn", 0, [(2, 8192, 1024), (1, 700, 512)], lambda B, R, C: [(B, C), (B, C)], (1.0 / 8192,)),
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


def test_noalloc_split_layernorm(gpu):
    """Split layernorm rows (the mean and the centred sum of squares in one
    read: sum and sum-of-squares partials, plan-only row locals), long rows
    then shorter ones (the 4x-chunk row map, then the 1x one)."""
    prog = compiled("layernorm_dyn")
    for R, C in ((3, 1_000_000), (2, 200_000)):
        print("noalloc layernorm_dyn", (R, C), flush=True)
        x = torch.from_numpy(inputs.normal((R, C), 1.0, 3)).to(gpu)
        g = torch.from_numpy(inputs.uniform((C,), 0.5, 1.5, 4)).to(gpu)
        b = torch.from_numpy(inputs.uniform((C,), -0.1, 0.1, 5)).to(gpu)
        _workspace_used(prog, [x])
        res = []
        for noalloc in (False, True):
            y = torch.full((R, C), CANARY, device=gpu)
            prog.launch([x, g, b, y], scalars=(1.0 / C, 1e-5), noalloc=noalloc)
            torch.cuda.synchronize()
            res.append(y.cpu().numpy())
        assert not np.any(res[1] == np.float32(CANARY))
        assert np.array_equal(res[1].view(np.uint32), res[0].view(np.uint32)), (R, C)


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


_NO_INIT = r"""
import sys
sys.path[:0] = [{repo!r}, {tests!r}]
import numpy as np
import torch
from helpers import compiled
from tcacomp_amd import _lib, inputs
# tca_rt_init is never called in this process: torch sets the device up.
x = torch.from_numpy(inputs.normal((64, 8192), 1.0, 3)).to("cuda:0")
p = compiled("row_sum_max_8192")  # no workspace
outs = [torch.empty(64, device="cuda:0") for _ in range(2)]
p.launch([x] + outs, noalloc=True)
torch.cuda.synchronize()
s, m = (o.cpu().numpy() for o in outs)
xs = x.cpu().numpy()
assert np.array_equal(m, xs.max(1)), "max"
assert np.allclose(s, xs.astype(np.float64).sum(1), rtol=0, atol=1e-3), "sum"
q = compiled("row_sum_max_dyn")  # split rows at 3 x 1 M: a partial scratch
y = torch.zeros((3, 1 << 20), device="cuda:0")
try:
    q.launch([y, torch.empty(3, device="cuda:0"), torch.empty(3, device="cuda:0")], noalloc=True)
except _lib.TcaError as e:
    assert "has not set up this device" in str(e), str(e)
    print("ok no-init")
else:
    raise SystemExit("a launch that needs scratch ran without tca_rt_init")
"""


def test_noalloc_without_init_needs_no_scratch(gpu):
    """A program with no workspace launches allocation-free in a process that
    never called tca_rt_init (nothing of the scratch array is needed); one
    that needs scratch there fails with the init error, before any kernel
    is queued. A fresh process: this one has called tca_rt_init."""
    import os
    import subprocess
    here = os.path.dirname(os.path.abspath(__file__))
    code = _NO_INIT.format(repo=os.path.dirname(here), tests=here)
    print("noalloc without init (subprocess)", flush=True)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=110,
                       env=dict(os.environ, TCA_JIT="0"))
    assert r.returncode == 0 and "ok no-init" in r.stdout, r.stdout + r.stderr[-3000:]
