"""C-ABI checks that need no GPU: the HIP library loads, exports every entry point that
include/kivi.h declares, and its host-side argument validation reports the same
KiviError variants, payloads and messages as the oracle (the reference's check order)."""

import re
import subprocess

import numpy as np
import pytest

import kivi
from conftest import ROOT, amd_backend

HEADER = ROOT / "include" / "kivi.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kivi_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = kivi.LIB_PATH
    assert lib.exists(), "build the library first (__graft_entry__.build())"
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    declared = declared_functions()
    assert len(declared) > 60
    missing = [f for f in declared if f not in exported]
    assert not missing, missing
    extra = sorted(s for s in exported if s.startswith("kivi_") and s not in declared)
    assert not extra, extra


def test_library_loads_and_binds():
    b = amd_backend()
    assert b["abi_version"]() == 1
    assert b["device_count"]() >= 0
    assert b["status_name"](7) == b"Shape"


def test_oracle_mirrors_the_host_api(oracle):
    """The oracle exports the host-pointer API under kivi_oracle_ (same signatures)."""
    for name in kivi._SIGS:
        assert hasattr(oracle.lib, "kivi_oracle_" + name), name


def _err(fn):
    with pytest.raises(kivi.KiviError) as e:
        fn()
    return e.value


CASES = [
    ("try_new bits", lambda b: kivi.KiviConfig.try_new(b, 3, 32, 128)),
    ("try_new group 0", lambda b: kivi.KiviConfig.try_new(b, 2, 0, 128)),
    ("try_new misaligned", lambda b: kivi.KiviConfig.try_new(b, 4, 12, 128)),
    ("try_new residual 0", lambda b: kivi.KiviConfig.try_new(b, 2, 32, 0)),
    ("try_new residual", lambda b: kivi.KiviConfig.try_new(b, 8, 32, 48)),
    ("new batch", lambda b: kivi.KiviCache(b, kivi.KiviConfig(), 0, 0, 7)),
    ("new heads", lambda b: kivi.KiviCache(b, kivi.KiviConfig(), 1, 0, 7)),
    ("new head_dim", lambda b: kivi.KiviCache(b, kivi.KiviConfig(), 1, 1, 7)),
    ("new head_dim 0", lambda b: kivi.KiviCache(b, kivi.KiviConfig(), 1, 1, 0)),
    ("new bad config", lambda b: kivi.KiviCache(b, kivi.KiviConfig(4, 4, 8), 1, 1, 32)),
    ("runtime", lambda b: kivi.RuntimeKv(b, kivi.KiviConfig(), 1, 0, 128)),
    ("qpc bits", lambda b: kivi.quantize_per_channel(b, np.zeros(8), 1, 1, 8, 1, 3, 32)),
    ("qpc tokens", lambda b: kivi.quantize_per_channel(b, np.zeros(8), 1, 1, 7, 1, 2, 32)),
    ("qpc shape", lambda b: kivi.quantize_per_channel(b, np.zeros(8), 1, 1, 32, 32, 2, 32)),
    ("qpt head_dim", lambda b: kivi.quantize_per_token(b, np.zeros(8), 1, 1, 4, 2, 2, 32)),
    ("qpt zero", lambda b: kivi.quantize_per_token(b, np.zeros(8), 1, 0, 4, 2, 2, 32)),
    ("qpt shape", lambda b: kivi.quantize_per_token(b, np.zeros(8), 2, 1, 4, 32, 2, 32)),
]


@pytest.mark.parametrize("name,fn", CASES, ids=[c[0] for c in CASES])
def test_host_validation_matches_oracle(oracle, name, fn):
    want = _err(lambda: fn(oracle))
    got = _err(lambda: fn(amd_backend()))
    assert (got.variant, got.payload, got.message) == (want.variant, want.payload, want.message)


def test_compute_without_a_device_fails_loudly():
    """No CPU fallback: a valid cache cannot be created without a HIP device."""
    b = amd_backend()
    if b["device_count"]() > 0:
        pytest.skip("a HIP device is present")
    e = _err(lambda: kivi.KiviCache(b, kivi.KiviConfig(), 1, 1, 128))
    assert e.variant == "Device"
    e = _err(lambda: kivi.quantize_per_channel(b, np.zeros(1024), 1, 1, 32, 32, 2, 32))
    assert e.variant == "Device"


def test_display_texts_match_src_error_rs(oracle):
    """Display strings of src/error.rs:47-95, read off the reference source text."""
    assert _err(lambda: kivi.KiviConfig.try_new(oracle, 4, 12, 128)).message == \
        "group_size 12 * bits 4 must be a multiple of 32"
    assert _err(lambda: kivi.KiviCache(oracle, kivi.KiviConfig(), 1, 0, 7)).message == \
        "num_kv_heads must be greater than zero"
    assert _err(lambda: kivi.KiviCache(oracle, kivi.KiviConfig(), 1, 1, 7)).message == \
        "head_dim 7 must be a positive multiple of group_size 32"
