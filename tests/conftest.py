"""Shared test setup.

Backends: every reference-derived test runs on the CPU oracle (oracle/libkivi_oracle.so,
the C++ restatement of the reference) and, under the ``gpu`` marker, on the HIP library
(kivi-cache-rs_amd/lib/libkivi_amd.so) through the same C ABI.
"""

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "kivi-cache-rs_amd"
ORACLE_SO = ROOT / "oracle" / "libkivi_oracle.so"
sys.path.insert(0, str(PKG))
sys.path.insert(0, str(ROOT / "tests"))

import kivi  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); runs the HIP library")
    config.addinivalue_line("markers", "slow: larger CPU cases")


def oracle_backend():
    if not ORACLE_SO.exists():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    return kivi.Backend.load(ORACLE_SO, prefix="kivi_oracle_", device=False)


def amd_backend():
    return kivi.Backend.amd()


@pytest.fixture(scope="session")
def oracle():
    return oracle_backend()


@pytest.fixture(scope="session")
def amd():
    b = amd_backend()
    n = b["device_count"]()
    assert n >= 1, "no HIP device visible: GPU tests must run on the MI355X box"
    return b


@pytest.fixture(
    params=["oracle", pytest.param("amd", marks=pytest.mark.gpu)], scope="session"
)
def backend(request):
    """The library under test: the oracle on CPU, the HIP library on the GPU box."""
    if request.param == "oracle":
        return oracle_backend()
    b = amd_backend()
    assert b["device_count"]() >= 1, "no HIP device visible"
    return b
