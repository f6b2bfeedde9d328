"""The C++ conformance program (tests/cpp/conformance.cpp) on the GPU.

It runs the reference's conformance clauses and ROCm contract cases through
the C++ host interface hephaestus_amd/host/hephaestus.hpp, one process that
links libhephaestus_amd.so directly.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

CPP = Path(__file__).parent / "cpp"
BIN = CPP / "hx_conformance"


def _binary() -> Path:
    if not BIN.exists():
        subprocess.run(["make", "-s", "-C", str(CPP)], check=True)
    return BIN


def test_cpp_program_skips_cleanly_without_a_device():
    """On a host with no GPU the program reports itself skipped (exit 77)."""
    import hephaestus_amd as hx

    if hx.RocmDevice.device_count() > 0:
        pytest.skip("a GPU is present; the GPU test runs the clauses")
    r = subprocess.run([str(_binary())], capture_output=True, text=True, timeout=60)
    assert r.returncode == 77, r.stdout + r.stderr


@pytest.mark.gpu
def test_cpp_conformance_clauses(device):
    r = subprocess.run([str(_binary())], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failures" in r.stdout
