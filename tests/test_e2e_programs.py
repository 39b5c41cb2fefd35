"""Host-only checks of the reference's end-to-end programs
(tcacomp_amd.programs.E2E; tests/test_gpu_e2e.py runs them on the device):
the families they lower to, their launch contract at the reference's shapes,
and that the two .tca fixtures under tcacomp_amd/tca/e2e build the same IR as
the reference's own fixture text (internal/e2e/frontend_test.go:27-70), read
from the reference tree when it is mounted."""
import os
import re

import pytest

from tcacomp_amd import compiler, programs, syntax
from tcacomp_amd.compiler import TensorDesc

REF_FRONTEND_TEST = "/root/reference/internal/e2e/frontend_test.go"
P = 1 << 20  # any non-null address: nothing is dereferenced host-side


def test_families():
    fam = {n: set(f().emit().families()) for n, f in programs.E2E.items()}
    assert fam["redwarp"] == {"stream"} and fam["red3"] == {"stream"}
    assert fam["mm"] == {"elementwise"}
    for n in ("matmul_scale_pkg", "matmul_scale_written", "matmul_scale_omitted"):
        assert fam[n] == {"gemm"}, n


def test_written_and_omitted_fixtures_build_the_same_program():
    w = programs.E2E["matmul_scale_written"]()
    o = programs.E2E["matmul_scale_omitted"]()
    assert w.IR() == o.IR()
    assert w.emit().source == o.emit().source


@pytest.mark.parametrize("name,shapes,ok", [
    ("redwarp", [(1024, 512), (1024,)], True),
    ("redwarp", [(1024, 512), (1023,)], False),
    ("red3", [(64, 32, 512), (64, 32)], True),
    ("red3", [(64, 32, 512), (32, 64)], False),
    ("mm", [(1024, 1024), (1024, 1024), (1024, 1024, 1024)], True),
    ("mm", [(1024, 1024), (1024, 512), (1024, 1024, 1024)], False),
    ("matmul_scale_written", [(64, 128), (128, 64), (64, 64)], True),
    ("matmul_scale_written", [(64, 128), (64, 128), (64, 64)], False),
])
def test_launch_contract(name, shapes, ok):
    prog = compiler.CompiledProgram(name, programs.E2E[name]().emit(), "")
    rc = prog.check([TensorDesc(P, s, 0) for s in shapes])
    assert (rc == 0) == ok, rc


def _go_raw_string(src, const):
    m = re.search(r"const %s = `(.*?)`" % const, src, re.S)
    assert m, const
    return m.group(1)


@pytest.mark.skipif(not os.path.exists(REF_FRONTEND_TEST), reason="reference tree not mounted")
@pytest.mark.parametrize("const,ours", [("frontendMatmulWritten", "matmul_scale_written"),
                                        ("frontendMatmulOmitted", "matmul_scale_omitted")])
def test_fixtures_match_the_reference_fixture_text(tmp_path, const, ours):
    # The reference's fixture text is read from its test file and compiled
    # through this frontend unchanged, @include of its common file included.
    with open(REF_FRONTEND_TEST) as f:
        go = f.read()
    (tmp_path / "tca-common.tca").write_text(_go_raw_string(go, "frontendCommon"))
    (tmp_path / "matmul_scale.tca").write_text(_go_raw_string(go, const))
    ref = syntax.ParseModule(str(tmp_path / "matmul_scale.tca"))
    assert [k.Name() for k in ref.Kernels] == ["matmul_scale"]
    assert ref.Kernels[0].Build().IR() == programs.E2E[ours]().IR()
