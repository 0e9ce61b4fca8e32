"""The C++ host layer (runtimed_amd/host): GgufFile / QMatMul / Weights /
Fp8Weight / HipSubstrate, exercised by tests/cpp/test_host.cpp."""
import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "cpp" / "test_host"


def _run(flag):
    if not BIN.exists():
        from runtimed_amd import build

        build.build_host_tests()
    res = subprocess.run([str(BIN), flag], capture_output=True, text=True, timeout=300)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr


def test_host_layer_cpu():
    _run("--cpu")


@pytest.mark.gpu
def test_host_layer_gpu():
    _run("--gpu")
