"""Element types other than f32 through the row family (compile-time row
length) and the streaming row family (run-time row length): u32 rows reduced
with the integer monoid combiners (wrapping +, ^, umax), bf16 rows cast to f32
and reduced (+, fmaxf), u8 rows cast to u32, summed and scaled by a piped map.

Expected values: the integer results are exact closed forms (a sum mod 2^32,
an xor, a max: order-independent, so numpy's reductions fix them bit for
bit); the bf16 rows go through the oracle's sequential f32 fold on the
exactly widened values; u8: f32(sum) * scale, one correctly rounded multiply
on both sides. Empty rows yield each reduction's init."""
import numpy as np
import pytest

import oracle
from helpers import CANARY, assert_reduce_close, compiled, run
from tcacomp_amd.compiler import TensorDesc

pytestmark = pytest.mark.gpu

U32 = 4  # tca dtype codes (include/tca_rt.h)


def _rng(seed):
    return np.random.default_rng(0x7CA0C0DE + seed)


def _u32_dev(a, dev):
    """A u32 array on the device (stored in an int32 torch tensor) and its
    descriptor."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)
    return t, TensorDesc(t.data_ptr() if t.numel() else 0, a.shape, U32)


def _u32_out(shape, dev):
    import torch
    t = torch.full(shape, int(np.float32(CANARY).view(np.int32)), dtype=torch.int32, device=dev)
    return t, TensorDesc(t.data_ptr() if t.numel() else 0, shape, U32)


STATIC_C = 1000
# Row lengths covering every vector width of each element type (u8: 16, 8,
# 4, 2, 1 elements; bf16: 8, 4, 2, 1; u32: 4, 2, 1), register-cached and
# streamed rows, and (<= 255 rows) split rows.
DYN_C = [0, 1, 3, 6, 12, 20, 1000, 4096, 5003, 20000, 40004, 65544, 70000, 140000]
LONG_C = [40004, 70000]  # also with > 255 rows: streamed without a split


def _cases():
    out = [("_1000", STATIC_C, 37)]
    out += [("_dyn", c, r) for c in DYN_C for r in (1, 37)]
    out += [("_dyn", c, 300) for c in LONG_C]
    return out


@pytest.mark.parametrize("suffix,C,R", _cases())
def test_row_stats_u32(gpu, suffix, C, R):
    x = _rng(C).integers(0, 2**32, size=(R, C), dtype=np.uint64).astype(np.uint32)
    xt, xd = _u32_dev(x, gpu)
    outs = [_u32_out((R,), gpu) for _ in range(3)]
    run(compiled("row_stats_u32" + suffix), [xd] + [o[1] for o in outs])
    got = [o[0].cpu().numpy().view(np.uint32) for o in outs]
    want_sum = (x.astype(np.uint64).sum(axis=1) % (1 << 32)).astype(np.uint32)
    want_xor = np.bitwise_xor.reduce(x, axis=1) if C else np.zeros(R, np.uint32)
    want_max = x.max(axis=1) if C else np.zeros(R, np.uint32)
    assert np.array_equal(got[0], want_sum), "u32 wrapping sum"
    assert np.array_equal(got[1], want_xor), "u32 xor"
    assert np.array_equal(got[2], want_max), "u32 umax"
    del xt


@pytest.mark.parametrize("suffix,C,R", _cases())
def test_row_sum_bf16(gpu, suffix, C, R):
    import torch
    from tcacomp_amd import inputs
    xb = oracle.to_bf16_bits(inputs.normal((R, C), 1.0, 5))
    xt = torch.from_numpy(xb.view(np.int16)).to(gpu).view(torch.bfloat16)
    s = torch.full((R,), CANARY, device=gpu)
    m = torch.full((R,), CANARY, device=gpu)
    run(compiled("row_sum_bf16" + suffix), [xt, s, m])
    xf = oracle.bf16_bits_to_f32(xb)
    ws, wm = oracle.row_sum_max(np.ascontiguousarray(xf))
    gs, gm = s.cpu().numpy(), m.cpu().numpy()
    assert np.array_equal(gm.view(np.uint32), wm.view(np.uint32)), "bf16 row max is not bit-identical"
    assert_reduce_close(gs, ws, np.sqrt((xf.astype(np.float64) ** 2).sum(1)), C, "bf16 row sum")


@pytest.mark.parametrize("suffix,C,R", _cases())
def test_row_sum_u8(gpu, suffix, C, R):
    import torch
    x = _rng(C + 1).integers(0, 256, size=(R, C), dtype=np.uint8)
    xt = torch.from_numpy(x).to(gpu)
    out = torch.full((R,), CANARY, device=gpu)
    scale = 0.37
    run(compiled("row_sum_u8" + suffix), [xt, out], scalars=[scale])
    want = x.astype(np.uint64).sum(axis=1).astype(np.uint32).astype(np.float32) * np.float32(scale)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32)), "u8 row sum"
