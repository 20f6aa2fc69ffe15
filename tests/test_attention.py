"""Decode attention tests: reference tests/attention.rs, tests/runtime.rs,
examples/pytorch_golden.rs (attention part), examples/passkey_retrieval.rs and
examples/decode_attention.rs. Run on the oracle and, with ``-m gpu``, on the HIP library.

Tolerances: the reference's 1e-4 max-abs against dense attention on the dequantized
cache (tests/attention.rs:59, 98), measured here against an f64 dense brute force.
"""

import numpy as np
import pytest

from kivi import KiviCache, KiviConfig, KiviError, RuntimeKv
from helpers import dense_attend, fill, max_abs, slice_tokens


def assert_matches_dequantized(backend, bits, group, residual, dim, seq):
    """tests/attention.rs:40-60."""
    cfg = KiviConfig.try_new(backend, bits, group, residual)
    cache = KiviCache(backend, cfg, 1, 1, dim)
    keys, values = fill(seq * dim, 21), fill(seq * dim, 22)
    cache.append(keys, values, seq)
    k_hat, v_hat = cache.dequantize()
    query = fill(dim, 23)
    scale = np.float32(1.0) / np.sqrt(np.float32(dim))
    got = cache.attention(query, 1, scale)
    expect = dense_attend(k_hat, v_hat, query, 1, 1, 1, seq, dim, scale)
    err = max_abs(got, expect)
    assert err < 1e-4, (bits, group, err)


def test_generic_kernel_matches_dequantized_attention(backend):
    """tests/attention.rs:62-66."""
    assert_matches_dequantized(backend, 2, 16, 32, 16, 40)
    assert_matches_dequantized(backend, 4, 32, 64, 32, 70)


def test_fast_2bit_group32_kernel_matches_dequantized_attention(backend):
    """tests/attention.rs:68-71."""
    assert_matches_dequantized(backend, 2, 32, 64, 64, 100)


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("seq", [1, 31, 32, 33, 127, 128, 129, 300, 1000])
def test_matches_dequantized_across_boundaries(backend, bits, seq):
    """Every packed/residual split (kq, vq, kres, vres) at D=128, G=32, R=128."""
    cfg = KiviConfig.try_new(backend, bits, 32, 128)
    cache = KiviCache(backend, cfg, 1, 2, 128)
    keys, values = fill(2 * seq * 128, 100 + seq), fill(2 * seq * 128, 200 + seq)
    cache.append(keys, values, seq)
    k_hat, v_hat = cache.dequantize()
    q = fill(2 * 4 * 128, 300 + seq)
    scale = np.float32(1.0) / np.sqrt(np.float32(128))
    got = cache.attention(q, 8, scale)
    expect = dense_attend(k_hat, v_hat, q, 1, 2, 8, seq, 128, scale)
    assert max_abs(got, expect) < 1e-4


def test_grouped_query_attention_repeats_kv_heads(backend):
    """tests/attention.rs:73-101."""
    dim, batch, kv, q_heads, seq = 32, 2, 2, 4, 48
    cfg = KiviConfig.try_new(backend, 2, 32, 64)
    cache = KiviCache(backend, cfg, batch, kv, dim)
    keys = fill(batch * kv * seq * dim, 31)
    values = fill(batch * kv * seq * dim, 32)
    cache.append(keys, values, seq)
    k_hat, v_hat = cache.dequantize()
    query = fill(batch * q_heads * dim, 33)
    got = cache.attention(query, q_heads, 0.125)
    expect = dense_attend(k_hat, v_hat, query, batch, kv, q_heads, seq, dim, 0.125)
    assert max_abs(got, expect) < 1e-4


def test_empty_cache_attention_is_zero(backend):
    """tests/attention.rs:103-108."""
    cache = KiviCache(backend, KiviConfig.default(), 1, 2, 128)
    y = cache.attention(np.full(2 * 128, 0.2, np.float32), 2, 1.0)
    assert (y == 0.0).all() and y.size == 256


def test_rejects_query_head_count_that_is_not_a_multiple(backend):
    """tests/attention.rs:110-114, with the check order of src/cache.rs:230-242."""
    cache = KiviCache(backend, KiviConfig.try_new(backend, 2, 16, 32), 1, 2, 16)
    with pytest.raises(KiviError) as e:
        cache.attention(np.zeros(3 * 16), 3, 1.0)
    assert e.value.variant == "QueryHeads"
    assert e.value.payload == {"num_q_heads": 3, "num_kv_heads": 2}
    assert e.value.message == "num_q_heads 3 must be a positive multiple of num_kv_heads 2"
    with pytest.raises(KiviError) as e:
        cache.attention(np.zeros(7), 3, 1.0)  # QueryHeads wins over Shape
    assert e.value.variant == "QueryHeads"
    with pytest.raises(KiviError) as e:
        cache.attention(np.zeros(7), 4, 1.0)
    assert e.value.variant == "Shape" and e.value.payload == {"expected": 64, "actual": 7}
    with pytest.raises(KiviError) as e:
        cache.attention(np.zeros(16), 0, 1.0)
    assert e.value.variant == "QueryHeads"


def golden_fixture(seq=64, dim=32):
    t = np.arange(seq)[:, None]
    d = np.arange(dim)[None, :]
    return ((t + d) % 4).astype(np.float32).reshape(-1)


def test_pytorch_golden_attention_is_exactly_one_and_a_half(backend):
    """examples/pytorch_golden.rs:48-65: uniform logits, mean of values = 1.5 exactly."""
    data = golden_fixture()
    cfg = KiviConfig.try_new(backend, 2, 32, 32)
    cache = KiviCache(backend, cfg, 1, 1, 32)
    cache.append(data, data, 64)
    scale = np.float32(1.0) / np.sqrt(np.float32(32))
    got = cache.attention(np.ones(32, np.float32), 1, scale)
    np.testing.assert_array_equal(got, np.full(32, 1.5, np.float32))
    assert cache.quantized_key_tokens() == 64
    assert cache.quantized_value_tokens() == 32


PASSKEY = [2, 7, 1, 8, 2, 8, 1]


def passkey_inputs():
    """examples/passkey_retrieval.rs:224-263."""
    dim, seq, needle = 128, 512, 256
    keys = np.zeros(seq * dim, np.float32)
    values = np.zeros(seq * dim, np.float32)
    s = 0x4B495649
    for t in range(seq):
        for d in range(dim):
            s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
            u = np.float32(s >> 8) / np.float32(1 << 24)
            noise = u * np.float32(0.1) - np.float32(0.05)
            keys[t * dim + d] = noise
            values[t * dim + d] = noise * np.float32(0.2)
        keys[t * dim] = np.clip(keys[t * dim], -0.2, 0.2)
    k = needle * dim
    keys[k:k + dim] = 0.0
    values[k:k + dim] = 0.0
    keys[k] = 8.0
    for i, digit in enumerate(PASSKEY):
        values[k + i * 10 + digit] = 1.0
    q = np.zeros(dim, np.float32)
    q[0] = 8.0
    return keys, values, q


@pytest.mark.parametrize("bits,residual", [(2, 32), (2, 128), (4, 32), (4, 128), (8, 32), (8, 128)])
def test_passkey_retrieval(backend, bits, residual):
    """examples/passkey_retrieval.rs:130-222: the needle is read back from packed KV."""
    keys, values, q = passkey_inputs()
    cfg = KiviConfig.try_new(backend, bits, 32, residual)
    cache = KiviCache(backend, cfg, 1, 1, 128)
    cache.append(keys, values, 512)
    assert 256 < cache.quantized_value_tokens()
    out = cache.attention(q, 1, np.float32(1.0) / np.sqrt(np.float32(128)))
    digits = [int(np.argmax(out[i * 10:(i + 1) * 10])) for i in range(7)]
    assert digits == PASSKEY


def test_runtime_decode_matches_direct_cache(backend):
    """tests/runtime.rs:13-52: decode == append(1) + attention, bit for bit."""
    cfg = KiviConfig.try_new(backend, 2, 32, 32)
    batch, kv, q_heads, dim, prompt, steps = 1, 2, 4, 32, 40, 3
    scale = np.float32(1.0) / np.sqrt(np.float32(dim))
    keys = fill(batch * kv * prompt * dim, 3)
    values = fill(batch * kv * prompt * dim, 4)
    runtime = RuntimeKv(backend, cfg, batch, kv, dim)
    cache = KiviCache(backend, cfg, batch, kv, dim)
    runtime.prefill(keys, values, prompt)
    cache.append(keys, values, prompt)
    previous = None
    for step in range(steps):
        key = fill(batch * kv * dim, 10 + step)
        value = fill(batch * kv * dim, 20 + step)
        query = fill(batch * q_heads * dim, 30 + step)
        got = runtime.decode(key, value, query, q_heads, scale)
        cache.append(key, value, 1)
        expect = cache.attention(query, q_heads, scale)
        np.testing.assert_array_equal(got, expect)
        if previous is not None:
            assert not np.array_equal(got, previous)
        previous = got
    assert runtime.cache().sequence_length() == prompt + steps
    assert runtime.cache().memory().compressed_bytes() == cache.memory().compressed_bytes()


def test_runtime_rejects_a_short_prefill(backend):
    """tests/runtime.rs:54-66."""
    runtime = RuntimeKv(backend, KiviConfig.try_new(backend, 2, 32, 32), 1, 1, 32)
    with pytest.raises(KiviError) as e:
        runtime.prefill(np.zeros(8), np.zeros(32), 1)
    assert e.value.payload == {"expected": 32, "actual": 8}


def test_runtime_bridge_hosts_agree(backend):
    """examples/runtime_bridge.rs:14-72: the same slices through RuntimeKv give one answer."""
    cfg = KiviConfig.try_new(backend, 2, 32, 32)
    kv, dim, prompt = 2, 32, 40
    pk, pv = fill(kv * prompt * dim, 3), fill(kv * prompt * dim, 4)
    results = []
    for copy in (lambda a: a.copy(), lambda a: np.frombuffer(a.tobytes(), np.float32), np.array):
        rt = RuntimeKv(backend, cfg, 1, kv, dim)
        rt.prefill(copy(pk), copy(pv), prompt)
        last = None
        for step in range(3):
            last = rt.decode(fill(kv * dim, 10 + step), fill(kv * dim, 20 + step),
                             fill(kv * dim, 30 + step), kv, np.float32(1) / np.sqrt(np.float32(dim)))
        results.append((last, rt.cache().memory().compressed_bytes(), rt.cache().sequence_length()))
    for r in results[1:]:
        np.testing.assert_array_equal(r[0], results[0][0])
        assert r[1:] == results[0][1:]
    assert results[0][2] == prompt + 3


def test_decode_attention_tracks_fp32(backend):
    """examples/decode_attention.rs:115-178: four decode steps stay close to fp32 attention."""
    cfg = KiviConfig.try_new(backend, 2, 32, 64)
    dim, heads, prompt, steps = 64, 4, 96, 4
    total = prompt + steps
    scale = np.float32(1.0) / np.sqrt(np.float32(dim))
    cache = KiviCache(backend, cfg, 1, heads, dim)
    keys, values = fill(heads * total * dim, 4), fill(heads * total * dim, 5)
    queries = fill(heads * steps * dim, 6)
    cache.append(slice_tokens(keys, 1, heads, total, dim, 0, prompt),
                 slice_tokens(values, 1, heads, total, dim, 0, prompt), prompt)
    for step in range(steps):
        t = prompt + step
        cache.append(slice_tokens(keys, 1, heads, total, dim, t, 1),
                     slice_tokens(values, 1, heads, total, dim, t, 1), 1)
        q = queries[step * heads * dim:(step + 1) * heads * dim]
        got = cache.attention(q, heads, scale)
        k_hat, v_hat = cache.dequantize()
        exact = dense_attend(k_hat, v_hat, q, 1, heads, heads, t + 1, dim, scale)
        assert max_abs(got, exact) < 1e-4
        fp32 = dense_attend(slice_tokens(keys, 1, heads, total, dim, 0, t + 1),
                            slice_tokens(values, 1, heads, total, dim, 0, t + 1),
                            q, 1, heads, heads, t + 1, dim, scale)
        cos = float(np.dot(got, fp32) / np.linalg.norm(got) / np.linalg.norm(fp32))
        assert cos > 0.9
