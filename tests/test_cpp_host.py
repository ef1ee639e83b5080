"""The C++ host layer (include/dcn/deform_conv.hpp) through its own test program,
tests/cpp/host_tests, whose cases follow the reference's Swift tests
(DeformConvCPUTests.swift, BenchmarkStatisticsTests.swift, MetalNonFiniteFlagTests.swift,
JasnaCLI.swift:68-110). The CPU group builds the program if needed; the GPU group runs
the program built beforehand."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PROGRAM = ROOT / "tests" / "cpp" / "host_tests"


def _run(group: str, timeout: int) -> None:
    r = subprocess.run([str(PROGRAM), group], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 failed" in r.stdout


def test_cpp_host_layer_cpu(dcn, oracle):
    subprocess.run(["make", "-s", "-C", str(ROOT / "tests" / "cpp")], check=True)
    _run("cpu", 120)


@pytest.mark.gpu
def test_cpp_host_layer_gpu():
    assert PROGRAM.exists(), "tests/cpp/host_tests is not built (run __graft_entry__.build())"
    _run("gpu", 120)
