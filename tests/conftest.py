"""Shared fixtures.

`gpu` marks tests that need an AMD GPU.  Like the reference's device tests
(crates/hephaestus-rocm/tests/full_reduction_contracts.rs:12-25) they skip
when no device can be acquired, unless HEPHAESTUS_ROCM_REQUIRE_DEVICE is set,
in which case a missing device is a failure.
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X / gfx950)")


@pytest.fixture(scope="session")
def device():
    import hephaestus_amd as hx

    hx.load_native()  # a missing library is an error, never a skip
    try:
        dev = hx.RocmDevice.try_default()
    except hx.AdapterUnavailable as exc:
        if os.environ.get("HEPHAESTUS_ROCM_REQUIRE_DEVICE"):
            raise
        pytest.skip(f"no ROCm device: {exc}")
    print(f"\n[device] {dev.topology().name} {dev.topology().arch} "
          f"CUs={dev.topology().compute_units}", flush=True)
    yield dev
    dev.close()


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    o.lib()
    return o
