"""Golden fixtures of tests/golden/ (written by tests/golden/make_golden.py).

* pytorch_golden.json: the reference's PyTorch-KIVI golden vectors
  (examples/pytorch_golden.rs:16-105) on both backends — code words, (scale, zero), dequantize
  and the 1.5 attention output, all exact.
* seeded_streams.npz: frozen oracle outputs on seeded streaming schedules. On CPU the oracle
  must still reproduce them bit for bit (a regression pin on the restatement); under ``gpu``
  the HIP library must match the packed streams and counters bit for bit and the attention
  within max-abs 1e-3 + rel 1e-4.
"""

import json
from pathlib import Path

import numpy as np
import pytest

import kivi
from golden.make_golden import CASES, case_inputs

HERE = Path(__file__).resolve().parent / "golden"
ATOL, RTOL = 1e-3, 1e-4


@pytest.fixture(scope="module")
def golden_json():
    return json.loads((HERE / "pytorch_golden.json").read_text())


@pytest.fixture(scope="module")
def seeded():
    return np.load(HERE / "seeded_streams.npz")


def test_pytorch_golden_fixture(backend, golden_json):
    g = golden_json
    _, _, seq, dim = g["shape"]
    t = np.arange(seq)[:, None]
    d = np.arange(dim)[None, :]
    data = ((t + d) % 4).astype(np.float32).reshape(-1)
    keys = kivi.quantize_per_channel(backend, data, 1, 1, seq, dim, g["bits"], g["group_size"])
    values = kivi.quantize_per_token(backend, data, 1, 1, seq, dim, g["bits"], g["group_size"])
    assert keys.pytorch_codes().tolist() == g["key_pytorch_codes"]
    assert values.pytorch_codes().tolist() == g["value_pytorch_codes"]
    for q in (keys, values):
        assert np.all(q.scale_zero().reshape(-1, 2) == np.array(g["scale_zero"], np.float32))
        assert np.array_equal(q.dequantize(), data)
    cfg = kivi.KiviConfig(g["bits"], g["group_size"], g["residual_length"])
    cache = kivi.KiviCache(backend, cfg, 1, 1, dim)
    cache.append(data, data, seq)
    out = cache.attention(np.ones(dim, np.float32), 1, np.float32(1.0) / np.sqrt(np.float32(dim)))
    assert np.all(out == np.float32(g["attention_expected"]))
    assert cache.quantized_key_tokens() == g["quantized_key_tokens"]
    assert cache.quantized_value_tokens() == g["quantized_value_tokens"]


def replay(backend, case):
    bits, G, R, batch, heads, qh, dim, schedule, seed = case
    total = sum(schedule)
    keys, values, query = case_inputs(case)
    cache = kivi.KiviCache(backend, kivi.KiviConfig(bits, G, R), batch, heads, dim)
    off = 0
    for n in schedule:
        k = keys.reshape(batch, heads, total, dim)[:, :, off:off + n].copy()
        v = values.reshape(batch, heads, total, dim)[:, :, off:off + n].copy()
        cache.append(k, v, n)
        off += n
    out = cache.attention(query, qh, np.float32(1.0) / np.sqrt(np.float32(dim)))
    return cache, out


def check_against_fixture(cache, out, seeded, name, exact_attention):
    counters = [cache.sequence_length(), cache.quantized_key_tokens(),
                cache.quantized_value_tokens(), cache.key_residual_len(), cache.value_residual_len()]
    assert counters == seeded[f"{name}/counters"].tolist()
    got = cache.export_streams()
    for arr, field in zip(got, ("key_codes", "key_params", "value_codes", "value_params")):
        want = seeded[f"{name}/{field}"]
        assert arr.shape == want.shape, field
        assert np.array_equal(arr.view(np.uint32), want.view(np.uint32)), field
    want = seeded[f"{name}/attention"].astype(np.float64)
    if exact_attention:
        assert np.array_equal(out.view(np.uint32), seeded[f"{name}/attention"].view(np.uint32))
    else:
        err = np.abs(out.astype(np.float64) - want)
        assert (err <= ATOL + RTOL * np.abs(want)).all(), f"max err {err.max():.3g}"


@pytest.mark.parametrize("name", list(CASES))
def test_oracle_reproduces_seeded_fixture(oracle, seeded, name):
    cache, out = replay(oracle, CASES[name])
    check_against_fixture(cache, out, seeded, name, exact_attention=True)


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CASES))
def test_hip_matches_seeded_fixture(amd, seeded, name):
    cache, out = replay(amd, CASES[name])
    check_against_fixture(cache, out, seeded, name, exact_attention=False)
