"""The CPU sanitizer gate in the CPU suite (tests/sanitize.py does the work):
the host library built with AddressSanitizer and UBSan, a bounded run of the
plan and .tca fuzzers against it, and the plain-C consumer's host leg under
it, each with no report. The full run (longer fuzzing, and the whole CPU
suite against the sanitized library) is `python tests/sanitize.py --pytest`."""
import os
import shutil
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import sanitize  # noqa: E402

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="no host C++ compiler")


@pytest.fixture(scope="module")
def built():
    sanitize.build()


@pytest.mark.parametrize("mode", ["plan", "tca"])
def test_fuzz_finds_nothing(built, mode):
    line = sanitize.fuzz(mode, seconds=8, seed=7)
    assert line.startswith("ok %s " % mode), line


def test_consumer_host_leg_under_asan(built):
    assert "ok host" in sanitize.consumer_host()
