"""Seeded random row programs (tests/randprog.py) on the device
against the CPU evaluation of the same spec (oracle/dsl_eval.py).

Each program runs over row counts and row lengths that reach every variant
its family has: static lengths of every vector width, run-time lengths from
empty rows to rows streamed past the register cache, split rows, one and
two row axes. f32 inputs are small integers, so every float sum is exact
(the evaluator checks it) and every output must match bit for bit up to the
sign of zero: elementwise arithmetic is correctly rounded on both sides
under -ffp-contract=off, and an exact sum does not depend on the fold
order. u32 programs are exact by construction (wrapping arithmetic).
"""
import sys
import zlib

import numpy as np
import pytest

from dsl_eval import evaluate, evaluate_grid
from helpers import CANARY
import randprog
from tcacomp_amd import compiler
from tcacomp_amd.compiler import TensorDesc
from tcacomp_amd.pkg import EMIT_NO_FUSION, EMIT_NO_GEMM

pytestmark = pytest.mark.gpu

U32 = 4  # tca dtype code (include/tca_rt.h)
DYN_C = [0, 1, 3, 6, 64, 1000, 4100, 20000, 70001, 140000]
ROWS = {1: [(1,), (37,), (300,)], 2: [(1, 1), (3, 37), (20, 15)]}


# Chained reductions over rows: segments B from 1 to past the segment
# kernel's 1024, every vector width and long rows; (B, R, C) products kept
# small enough that f32 sums stay exact.
ROWC_ROWS = {1: [(1,), (37,), (300,)], 2: [(1, 1), (3, 37), (20, 15), (1024, 3), (1100, 17), (2048, 1), (1024, 0)]}
ROWC_DYN = [(1, 1, 0), (3, 37, 1), (20, 15, 3), (1024, 3, 6), (1100, 17, 64), (2048, 1, 1000), (1024, 9, 4100),
            (3, 37, 20000), (1030, 2, 20000), (1024, 0, 5), (1024, 5, 0), (1100, 17, 7), (1024, 3, 70001)]


def _shapes(spec, generic):
    if spec.name.startswith("rowc"):
        if spec.outer == 1:
            return [r + (c,) for r in ROWC_ROWS[1] for c in ((spec.c,) if spec.c else (0, 5, 1000, 70001))]
        if spec.c:
            return [r[:2] + (spec.c,) for r in ROWC_ROWS[2] if r[0] * max(r[1], 1) * spec.c <= 1 << 24]
        return ROWC_DYN
    rows = ROWS[spec.outer]
    if spec.c:
        return [r + (spec.c,) for r in rows]
    out = [rows[j % 3] + (c,) for j, c in enumerate(DYN_C)]
    out.append(rows[2] + (70000,))  # > 255 rows of a streamed length: no split
    if generic:  # one thread folds a whole row: keep the rows short
        return [s for s in out if s[-1] <= 70001]
    out.append(rows[0] + (2 << 20,))  # one long row: split over the GPU
    return out


_progs = {}


def _program(spec, generic):
    key = (spec.name, generic)
    if key not in _progs:
        flags = EMIT_NO_FUSION | EMIT_NO_GEMM if generic else 0
        _progs[key] = compiler.compile_program(randprog.build(spec), flags=flags)
    return _progs[key]


def _inputs(spec, shape, bound):
    rng = np.random.default_rng(zlib.crc32(("%s %s %d" % (spec.name, shape, bound)).encode()))
    rows, C = shape[:-1], shape[-1]
    if spec.elem == "f32":
        tiles = {t: rng.integers(-bound, bound + 1, size=shape).astype(np.float32) for t, _ in spec.tiles}
        col = rng.integers(-2, 3, size=(C,)).astype(np.float32) if spec.col else None
        row = rng.integers(-bound, bound + 1, size=rows).astype(np.float32) if spec.row else None
    else:
        tiles = {}
        for t, st in spec.tiles:
            hi = 256 if st == "u8" else 1 << 32
            tiles[t] = rng.integers(0, hi, size=shape, dtype=np.uint64).astype(np.uint32)
        col = rng.integers(0, 1 << 32, size=(C,), dtype=np.uint64).astype(np.uint32) if spec.col else None
        row = rng.integers(0, 1 << 32, size=rows, dtype=np.uint64).astype(np.uint32) if spec.row else None
    return tiles, col, row


def _dev(a, storage, dev):
    """A device tensor (or descriptor) holding `a` in the storage type."""
    import torch
    if storage == "f32":
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev), None
    if storage == "bf16":
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(torch.bfloat16), None
    if storage == "u8":
        return torch.from_numpy(np.ascontiguousarray(a.astype(np.uint8))).to(dev), None
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)
    return t, TensorDesc(t.data_ptr() if t.numel() else 0, a.shape, U32)


def _check(spec, generic, gpu):
    import torch
    prog = _program(spec, generic)
    for shape in _shapes(spec, generic):
        rows = shape[:-1]
        print("random", spec.name, "generic" if generic else "fused", shape, flush=True)
        sys.stdout.flush()
        for bound in (8, 3, 1):
            tiles, col, row = _inputs(spec, shape, bound)
            want, exact = evaluate(spec, tiles, col, row, dict(spec.scalars))
            if exact:
                break
        assert exact, "no input range keeps the f32 sums of %s exact at %s" % (spec.name, shape)
        keep, args = [], []
        for t, st in spec.tiles:
            d, desc = _dev(tiles[t], st, gpu)
            keep.append(d)
            args.append(desc or d)
        for a in ([col] if spec.col else []) + ([row] if spec.row else []):
            d, desc = _dev(a, spec.elem, gpu)
            keep.append(d)
            args.append(desc or d)
        outs = {}
        for st in spec.stmts:
            if st["local"]:
                continue
            oshape = shape if st["kind"] == "map" else rows[:-1] if st["kind"] in ("chain", "rowreduce") else rows
            if spec.elem == "f32":
                o = torch.full(oshape, CANARY, device=gpu)
                args.append(o)
            else:
                o = torch.full(oshape, 0x5A5A5A5A, dtype=torch.int32, device=gpu)
                args.append(TensorDesc(o.data_ptr() if o.numel() else 0, oshape, U32))
            outs[st["out"]] = o
        prog.launch(args, scalars=[v for _, v in spec.scalars])
        torch.cuda.synchronize()
        for name, o in outs.items():
            got = o.cpu().numpy()
            if spec.elem == "u32":
                got = got.view(np.uint32)
            np.testing.assert_array_equal(got, want[name], err_msg="%s %s output %s" % (spec.name, shape, name))
        del keep, args, outs


ROW_SPECS = [s for s in randprog.specs() if getattr(s, "kind", "row") == "row"]
GRID_SPECS = [s for s in randprog.specs() if getattr(s, "kind", "row") == "grid"]
GRID_SHAPES = [(1, 0), (0, 5), (1, 1), (37, 3), (300, 64), (37, 1000), (300, 4100), (5, 70001), (1000, 1000)]
# Dependent column programs also run 100 rows of 140000 columns: 547 column
# blocks, so one whole-column kernel runs every pass over all 100 rows (the
# other shapes reach it with <= 64 rows, and the per-pass pairs with more).
COLCHAIN_SHAPES = GRID_SHAPES + [(100, 140000)]


@pytest.mark.parametrize("spec", ROW_SPECS, ids=lambda s: s.name)
def test_random_program(gpu, spec):
    _check(spec, False, gpu)


@pytest.mark.parametrize("spec", GRID_SPECS, ids=lambda s: s.name)
def test_random_grid_program(gpu, spec):
    """Elementwise maps with broadcast and transposed operands, transposed
    stores, reductions over the leading axis (elementwise, streaming,
    column and generic families), and dependent column reductions: a
    reduction reading an earlier one's result at its own column (one
    column nest of several passes: the whole-column kernel, or per-pass
    partial and merge pairs)."""
    import torch
    prog = _program(spec, False)
    shapes = ([(r, spec.c) for r in (1, 37, 300)] if spec.c else
              COLCHAIN_SHAPES if spec.name.startswith("gridc") else GRID_SHAPES)
    lead = (3,) if spec.batch else ()  # batch programs: three batch indices
    for R, C in shapes:
        if spec.batch and R * C > (1 << 22):
            continue
        print("random", spec.name, lead + (R, C), flush=True)
        sys.stdout.flush()
        for bound in (8, 3, 1):
            rng = np.random.default_rng(zlib.crc32(("%s %d %d %d" % (spec.name, R, C, bound)).encode()))
            if spec.elem == "f32":
                gen = lambda *shape: rng.integers(-bound, bound + 1, size=shape).astype(np.float32)  # noqa: E731
            else:
                gen = lambda *shape: rng.integers(0, 1 << 32, size=shape, dtype=np.uint64).astype(np.uint32)  # noqa: E731
            x0 = gen(*lead, R, C)
            if spec.tiles[0][1] == "u8":
                x0 = x0 & np.uint32(0xFF)
            xt = gen(*lead, C, R) if spec.trans else None
            g = gen(C) if spec.col else None
            r = gen(R) if spec.row else None
            want, exact = evaluate_grid(spec, x0, xt, g, r, dict(spec.scalars))
            if exact:
                break
        assert exact, "no input range keeps the f32 sums of %s exact at %s" % (spec.name, (R, C))
        keep, args = [], []
        d, desc = _dev(x0, spec.tiles[0][1], gpu)
        keep.append(d)
        args.append(desc or d)
        for a in [a for a in (xt, g, r) if a is not None]:
            d, desc = _dev(a, spec.elem, gpu)
            keep.append(d)
            args.append(desc or d)
        outs = {}
        for st in spec.stmts:
            if st.get("local"):
                continue
            oshape = lead + {"map": (R, C), "tmap": (C, R), "colreduce": (C,)}[st["kind"]]
            if spec.elem == "f32":
                o = torch.full(oshape, CANARY, device=gpu)
                args.append(o)
            else:
                o = torch.full(oshape, 0x5A5A5A5A, dtype=torch.int32, device=gpu)
                args.append(TensorDesc(o.data_ptr() if o.numel() else 0, oshape, U32))
            outs[st["out"]] = o
        prog.launch(args, scalars=[v for _, v in spec.scalars])
        torch.cuda.synchronize()
        for name, o in outs.items():
            got = o.cpu().numpy()
            if spec.elem == "u32":
                got = got.view(np.uint32)
            np.testing.assert_array_equal(got, want[name], err_msg="%s %s output %s" % (spec.name, lead + (R, C), name))
        del keep, args, outs


@pytest.mark.parametrize("spec", [s for s in ROW_SPECS if s.name in randprog.GENERIC_TOO], ids=lambda s: s.name)
def test_random_program_generic(gpu, spec):
    """The same program lowered with fusion off: one thread per output,
    sequential folds (the generic family)."""
    _check(spec, True, gpu)
