"""Export formats into device memory, and HBM planning for the arenas.

Device forms of ``KiviCache::dequantize`` (src/cache.rs:282-325), the PackedStream read-out
(src/quant.rs:37-44), ``QuantizedTensor::pytorch_codes`` (src/quant.rs:77-112) and
``QuantizedTensor::dequantize`` (src/quant.rs:124-150): each is compared bit for bit with the
oracle's output on the same inputs. The HBM planner is checked against its closed form on the
CPU and against live caches on the GPU; the occupied-byte model it sits beside is pinned by
tests/budget.rs:68-82 in test_cache.py."""

import math

import numpy as np
import pytest

import kivi
from kivi import KiviCache, KiviConfig, KiviError, quantize_per_channel, quantize_per_token
from helpers import DeviceArrays, fill


def _state_cache(backend, bits, group, residual, batch, heads, dim, seq, seed):
    cfg = KiviConfig.try_new(backend, bits, group, residual)
    c = KiviCache(backend, cfg, batch, heads, dim)
    n = batch * heads * seq * dim
    c.append(fill(n, seed) * np.float32(3.0), fill(n, seed + 1), seq)
    return c


EXPORT_CASES = [
    # bits, group, residual, batch, heads, dim, seq
    (2, 32, 128, 2, 4, 128, 1000),
    (4, 32, 64, 1, 2, 128, 333),
    (8, 16, 32, 2, 1, 64, 97),
    (2, 64, 128, 1, 3, 128, 40),  # nothing packed yet: zero-length streams
    # wide heads: the export stages too many words for an output buffer in LDS (stores
    # straight from registers) and the reconstruction asks for more than 64 KB of LDS
    (8, 64, 64, 1, 2, 512, 300),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", EXPORT_CASES)
def test_cache_device_exports_match_oracle(amd, oracle, case):
    bits, group, residual, batch, heads, dim, seq = case
    ca = _state_cache(amd, bits, group, residual, batch, heads, dim, seq, 11)
    co = _state_cache(oracle, bits, group, residual, batch, heads, dim, seq, 11)
    dev = DeviceArrays()
    try:
        n = batch * heads * seq * dim
        dk, dv = dev.empty(n), dev.empty(n)
        ca.dequantize_device(dk, n, dv, n)
        ok, ov = co.dequantize()
        assert np.array_equal(dev.download(dk, n).view(np.uint32), ok.view(np.uint32))
        assert np.array_equal(dev.download(dv, n).view(np.uint32), ov.view(np.uint32))

        lens = ca.stream_lengths()
        ptrs = [dev.empty(x) if x else 0 for x in lens]
        ca.export_streams_device(ptrs, lens)
        want = co.export_streams()
        for p, x, w in zip(ptrs, lens, want):
            got = dev.download(p, x) if x else np.zeros(0, np.float32)
            assert np.array_equal(got.view(np.uint32), np.asarray(w).view(np.uint32))
        # a NULL array is skipped; the others are still written
        ptrs2 = [0, dev.empty(lens[1]) if lens[1] else 0, 0, dev.empty(lens[3]) if lens[3] else 0]
        ca.export_streams_device(ptrs2, lens)
        if lens[3]:
            assert np.array_equal(dev.download(ptrs2[3], lens[3]).view(np.uint32),
                                  np.asarray(want[3]).view(np.uint32))
        with pytest.raises(KiviError) as e:
            ca.dequantize_device(dk, n - 1, dv, n)
        assert e.value.variant == "Shape"
    finally:
        dev.free()


@pytest.mark.gpu
def test_cache_dequantize_device_unaligned_outputs(amd, oracle):
    """Output arrays that are not 16-byte aligned take the one-element-per-thread kernel: the
    same bits as the oracle."""
    bits, group, residual, batch, heads, dim, seq = 4, 32, 64, 1, 2, 128, 333
    ca = _state_cache(amd, bits, group, residual, batch, heads, dim, seq, 21)
    co = _state_cache(oracle, bits, group, residual, batch, heads, dim, seq, 21)
    dev = DeviceArrays()
    try:
        n = batch * heads * seq * dim
        base_k, base_v = dev.empty(n + 1), dev.empty(n + 1)
        ca.dequantize_device(base_k + 4, n, base_v + 4, n)  # one float past the allocation start
        ok, ov = co.dequantize()
        assert np.array_equal(dev.download(base_k, n + 1)[1:].view(np.uint32), ok.view(np.uint32))
        assert np.array_equal(dev.download(base_v, n + 1)[1:].view(np.uint32), ov.view(np.uint32))
    finally:
        dev.free()


QUANT_CASES = [
    # per_channel, bits, group, batch, heads, tokens, dim
    (True, 2, 32, 2, 3, 256, 128),
    (True, 4, 16, 1, 2, 96, 64),
    (False, 8, 32, 2, 2, 50, 128),
    (False, 2, 64, 1, 1, 7, 128),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", QUANT_CASES)
def test_quantized_device_exports_match_oracle(amd, oracle, case):
    per_channel, bits, group, batch, heads, tokens, dim = case
    q = quantize_per_channel if per_channel else quantize_per_token
    data = fill(batch * heads * tokens * dim, 77) * np.float32(2.5)
    qa = q(amd, data, batch, heads, tokens, dim, bits, group)
    qo = q(oracle, data, batch, heads, tokens, dim, bits, group)
    dev = DeviceArrays()
    try:
        nc = qa.code_bytes() // 4
        pc = dev.empty(nc)
        qa.pytorch_codes_device(pc, nc)
        assert np.array_equal(dev.download(pc, nc).view(np.uint32), qo.pytorch_codes())
        n = batch * heads * tokens * dim
        dq = dev.empty(n)
        qa.dequantize_device(dq, n)
        assert np.array_equal(dev.download(dq, n).view(np.uint32), qo.dequantize().view(np.uint32))
        with pytest.raises(KiviError) as e:
            qa.pytorch_codes_device(pc, nc + 1)
        assert e.value.variant == "Shape"
    finally:
        dev.free()


# ------------------------------------------------------------------ HBM planning


def planned_bytes(bits, group, residual, batch, heads, dim, tokens):
    """Closed form of the arena layout: packed capacity C = max(tokens, 256) rounded up to
    lcm(64, G) tokens (0 with no tokens); per unit and token of capacity, key and value codes
    D*bits/8 bytes each, key params D/G*8, value params D/G*8; plus the fp32 key residual and
    value window (R*D*4 each) and the scale maxima, eight 16-byte records per unit."""
    units = batch * heads
    gran = 64 * group // math.gcd(64, group)
    cap = 0 if tokens == 0 else -(-max(tokens, 256) // gran) * gran
    per_token = 2 * dim * bits // 8 + 2 * (dim // group) * 8
    return units * (cap * per_token + 2 * residual * dim * 4 + 8 * 16)


PLAN_CASES = [
    (2, 32, 128, 16, 8, 128, 32768),
    (4, 32, 128, 1, 8, 128, 262144),
    (8, 16, 32, 2, 2, 64, 1),
    (2, 128, 256, 1, 1, 128, 1000),
    (2, 32, 128, 3, 5, 96, 0),
]


@pytest.mark.parametrize("case", PLAN_CASES)
def test_plan_device_bytes_closed_form(case):
    amd = kivi.Backend.amd()
    bits, group, residual, batch, heads, dim, tokens = case
    got = kivi.plan_device_bytes(amd, KiviConfig(bits, group, residual), batch, heads, dim, tokens)
    assert got == planned_bytes(*case)


def test_plan_device_bytes_checks_like_cache_new():
    amd = kivi.Backend.amd()
    with pytest.raises(KiviError) as e:
        kivi.plan_device_bytes(amd, KiviConfig(3, 32, 128), 1, 1, 128, 10)
    assert e.value.variant == "InvalidBits"
    with pytest.raises(KiviError) as e:
        kivi.plan_device_bytes(amd, KiviConfig(2, 32, 128), 0, 1, 128, 10)
    assert e.value.variant == "ZeroDimension"
    with pytest.raises(KiviError) as e:
        kivi.plan_device_bytes(amd, KiviConfig(2, 32, 128), 1, 1, 48, 10)
    assert e.value.variant == "HeadDim"


def test_c2_fits_one_mi355x():
    """The benchmark's C2 shape (16 sequences x 8 KV heads x 32k tokens, 2-bit) per layer, and
    how many such layers 288 GB of HBM holds."""
    amd = kivi.Backend.amd()
    per_layer = kivi.plan_device_bytes(amd, KiviConfig(2, 32, 128), 16, 8, 128, 32768)
    assert per_layer == planned_bytes(2, 32, 128, 16, 8, 128, 32768)
    assert 288 * 10**9 // per_layer >= 32


@pytest.mark.gpu
@pytest.mark.parametrize("case", PLAN_CASES[:4])
def test_live_cache_holds_the_planned_bytes(amd, case):
    bits, group, residual, batch, heads, dim, tokens = case
    cfg = KiviConfig.try_new(amd, bits, group, residual)
    c = KiviCache(amd, cfg, batch, heads, dim)
    assert c.device_bytes() == planned_bytes(bits, group, residual, batch, heads, dim, 0)
    c.reserve(tokens)
    assert c.device_bytes() == kivi.plan_device_bytes(amd, cfg, batch, heads, dim, tokens)
    # occupied bytes (the reference byte model) never exceed what the arenas hold
    seq = min(tokens, 700)
    n = batch * heads * seq * dim
    c.append(fill(n, 5), fill(n, 6), seq)
    assert c.memory().compressed_bytes() <= c.device_bytes()
    assert c.device_bytes() == kivi.plan_device_bytes(amd, cfg, batch, heads, dim, tokens)
