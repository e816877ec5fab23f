"""The C++20 facade (luisacompute-parallelprimitive_amd/include/lcpp/) on the GPU: runs
tests/cpp/facade_test.cpp, which restates the reference's module-level tests as a reference user would
write them (CommandList recording, commit on a stream, host checks with std:: algorithms), in a child
process; each case prints its name before it touches the GPU."""
import pathlib
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = pathlib.Path(__file__).resolve().parent / "cpp" / "bin" / "facade_test"


def test_facade_cases():
    assert BIN.exists(), "tests/cpp/bin/facade_test is missing: run __graft_entry__.build()"
    cases = subprocess.run([str(BIN), "--list"], check=True, capture_output=True, text=True).stdout.split()
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert f"{len(cases)} cases, 0 failures" in r.stdout
