"""The C-ABI example program (sandmuon_amd/examples/abi_example.cpp): a host
program that drives the library without Python (HIP memory, one stream) and
checks its own results against FP64 host sums and the graft invariant."""
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parents[1] / "sandmuon_amd" / "abi_example"


def test_c_abi_example_program(device):
    if not EXE.exists():
        pytest.fail(f"{EXE} is missing: build with python -m sandmuon_amd.build")
    res = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=120)
    sys.stdout.write(res.stdout)
    sys.stderr.write(res.stderr)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "all checks passed" in res.stdout
