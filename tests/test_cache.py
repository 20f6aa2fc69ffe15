"""Streaming cache tests: reference tests/cache.rs, tests/trace.rs (state counters),
tests/budget.rs:68-91 (byte model), examples/rl_determinism.rs and the src/lib.rs:12-27
example. Run on the oracle and, with ``-m gpu``, on the HIP library."""

import numpy as np
import pytest

from kivi import KiviCache, KiviConfig, KiviError, quantize_per_channel, quantize_per_token
from helpers import fill, reference_minimum, signed_zero_rows, slice_tokens


def config(backend):
    """tests/cache.rs:3-5."""
    return KiviConfig.try_new(backend, 2, 16, 32)


def append_chunks(cache, keys, values, total, chunks):
    """tests/cache.rs:36-57."""
    b, h, d = cache.batch_size(), cache.num_kv_heads(), cache.head_dim()
    off = 0
    for n in chunks:
        cache.append(slice_tokens(keys, b, h, total, d, off, n),
                     slice_tokens(values, b, h, total, d, off, n), n)
        off += n


def test_streaming_boundaries_match_algorithm_1(backend):
    """tests/cache.rs:59-76."""
    dim = 16
    cache = KiviCache(backend, config(backend), 2, 3, dim)
    steps = [10, 20, 5, 100]
    total = sum(steps)
    n = 2 * 3 * total * dim
    keys, values = fill(n, 1), fill(n, 2)
    append_chunks(cache, keys, values, total, steps)
    r = 32
    assert cache.sequence_length() == total
    assert cache.key_residual_len() == total % r
    assert cache.value_residual_len() == min(r, total)
    assert cache.quantized_key_tokens() == total - total % r
    assert cache.quantized_value_tokens() == total - min(r, total)


def test_chunked_appends_match_token_by_token(backend):
    """tests/cache.rs:78-104: token-by-token == chunked == one-shot, bit for bit."""
    dim, batch, heads, total = 16, 2, 3, 70
    n = batch * heads * total * dim
    keys, values = fill(n, 7), fill(n, 9)
    streamed = KiviCache(backend, config(backend), batch, heads, dim)
    append_chunks(streamed, keys, values, total, [1] * total)
    chunked = KiviCache(backend, config(backend), batch, heads, dim)
    append_chunks(chunked, keys, values, total, [1, 50, 7, 12])
    once = KiviCache(backend, config(backend), batch, heads, dim)
    once.append(keys, values, total)
    sk, sv = streamed.dequantize()
    ck, cv = chunked.dequantize()
    ok, ov = once.dequantize()
    np.testing.assert_array_equal(sk, ck)
    np.testing.assert_array_equal(sv, cv)
    np.testing.assert_array_equal(sk, ok)
    np.testing.assert_array_equal(sv, ov)
    # the packed streams themselves agree too (stronger than the reference's check)
    for a, b in zip(streamed.export_streams(), once.export_streams()):
        np.testing.assert_array_equal(a, b)


def test_quantized_prefix_matches_one_shot_and_residual_is_exact(backend):
    """tests/cache.rs:106-130."""
    dim, total = 16, 80
    keys, values = fill(total * dim, 3), fill(total * dim, 4)
    cache = KiviCache(backend, config(backend), 1, 1, dim)
    cache.append(keys, values, total)
    kq, vq = cache.quantized_key_tokens(), cache.quantized_value_tokens()
    k_hat, v_hat = cache.dequantize()
    k_ref = quantize_per_channel(backend, keys[:kq * dim], 1, 1, kq, dim, 2, 16).dequantize()
    np.testing.assert_array_equal(k_hat[:kq * dim], k_ref)
    np.testing.assert_array_equal(k_hat[kq * dim:], keys[kq * dim:])
    v_ref = quantize_per_token(backend, values[:vq * dim], 1, 1, vq, dim, 2, 16).dequantize()
    np.testing.assert_array_equal(v_hat[:vq * dim], v_ref)
    np.testing.assert_array_equal(v_hat[vq * dim:], values[vq * dim:])


def test_empty_append_and_shape_errors(backend):
    """tests/cache.rs:132-145."""
    cache = KiviCache(backend, config(backend), 1, 1, 16)
    cache.append([], [], 0)
    assert cache.sequence_length() == 0
    with pytest.raises(KiviError) as e:
        cache.append(np.zeros(4), np.zeros(16), 1)
    assert e.value.variant == "Shape" and e.value.payload == {"expected": 16, "actual": 4}
    with pytest.raises(KiviError) as e:
        cache.append(np.zeros(16), np.zeros(15), 1)
    assert e.value.payload == {"expected": 16, "actual": 15}
    assert cache.sequence_length() == 0


def test_config_rejects_residual_that_is_not_a_group_multiple(backend):
    """tests/cache.rs:147-158 plus KiviCache::new's check order (src/cache.rs:93-104)."""
    with pytest.raises(KiviError) as e:
        KiviConfig.try_new(backend, 2, 32, 100)
    assert e.value.variant == "ResidualLength"
    assert e.value.message == "residual_length 100 must be a positive multiple of group_size 32"
    KiviCache(backend, KiviConfig.default(), 1, 1, 96)
    with pytest.raises(KiviError) as e:
        KiviCache(backend, KiviConfig.default(), 1, 1, 40)
    assert e.value.variant == "HeadDim"
    with pytest.raises(KiviError) as e:
        KiviCache(backend, KiviConfig.default(), 0, 0, 40)
    assert e.value.variant == "ZeroDimension" and e.value.payload["name"] == "batch"
    with pytest.raises(KiviError) as e:
        KiviCache(backend, KiviConfig.default(), 1, 0, 40)
    assert e.value.payload["name"] == "num_kv_heads"
    # The C ABI validates the config the reference trusts (kivi.h: kivi_cache_new).
    with pytest.raises(KiviError) as e:
        KiviCache(backend, KiviConfig(2, 32, 0), 1, 1, 32)
    assert e.value.variant == "ResidualLength"


def test_same_prompt_builds_the_same_cache_twice(backend):
    """tests/cache.rs:160-194 (and examples/rl_determinism.rs:12-73)."""
    cfg = KiviConfig.try_new(backend, 2, 32, 32)
    keys = fill(64 * 32, 4)
    values = fill(64 * 32, 5)
    keys[3], keys[4], keys[5] = 0.5, 1.5, 2.5
    qa, qb = fill(32, 8), fill(32, 9)
    scale = 0.25
    pk = quantize_per_channel(backend, keys, 1, 1, 64, 32, 2, 32)
    pk2 = quantize_per_channel(backend, keys, 1, 1, 64, 32, 2, 32)
    np.testing.assert_array_equal(pk.codes(), pk2.codes())
    np.testing.assert_array_equal(pk.scale_zero(), pk2.scale_zero())
    pv = quantize_per_token(backend, values, 1, 1, 64, 32, 2, 32)
    pv2 = quantize_per_token(backend, values, 1, 1, 64, 32, 2, 32)
    np.testing.assert_array_equal(pv.codes(), pv2.codes())
    first = KiviCache(backend, cfg, 1, 1, 32)
    second = KiviCache(backend, cfg, 1, 1, 32)
    first.append(keys, values, 64)
    second.append(keys, values, 64)
    for x, y in zip(first.dequantize(), second.dequantize()):
        np.testing.assert_array_equal(x, y)
    a = first.attention(qa, 1, scale)
    b = first.attention(qb, 1, scale)
    np.testing.assert_array_equal(a, second.attention(qa, 1, scale))
    np.testing.assert_array_equal(b, second.attention(qb, 1, scale))
    assert not np.array_equal(a, b)
    keys[0] = 50.0
    edited = KiviCache(backend, cfg, 1, 1, 32)
    edited.append(keys, values, 64)
    assert not np.array_equal(first.dequantize()[0], edited.dequantize()[0])


def rl_prompt(n, seed):
    """examples/rl_determinism.rs:81-95: LCG with planted half-ties every 17th element."""
    out = np.empty(n, np.float32)
    s = seed
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        unit = np.float32(s >> 8) / np.float32(1 << 24)
        out[i] = np.float32(i % 8) + np.float32(0.5) if i % 17 == 0 else unit * np.float32(2) - np.float32(1)
    return out


def test_rl_replay_is_bit_identical(backend):
    """examples/rl_determinism.rs:12-73: two builds of one prompt score identically."""
    cfg = KiviConfig.try_new(backend, 2, 32, 32)
    keys, values = rl_prompt(64 * 32, 4), rl_prompt(64 * 32, 5)
    pa, pb = rl_prompt(32, 8), rl_prompt(32, 9)
    scale = np.float32(1.0) / np.sqrt(np.float32(32))

    def store(k):
        c = KiviCache(backend, cfg, 1, 1, 32)
        c.append(k, values, 64)
        return c

    first, second = store(keys), store(keys)
    a1, a2 = first.attention(pa, 1, scale), second.attention(pa, 1, scale)
    b1, b2 = first.attention(pb, 1, scale), second.attention(pb, 1, scale)
    np.testing.assert_array_equal(a1, a2)
    np.testing.assert_array_equal(b1, b2)
    assert not np.array_equal(a1, b1)
    assert first.memory().compressed_bytes() == second.memory().compressed_bytes()
    edited = keys.copy()
    edited[0] = 50.0
    drifted = store(edited)
    assert np.float32(drifted.attention(pa, 1, scale).sum()) != np.float32(a1.sum())


def test_long_sequence_beats_fp16_footprint(backend):
    """tests/cache.rs:196-207."""
    cfg = KiviConfig.try_new(backend, 2, 32, 64)
    cache = KiviCache(backend, cfg, 1, 2, 64)
    seq = 512
    n = 2 * seq * 64
    cache.append(fill(n, 11), fill(n, 13), seq)
    report = cache.memory()
    assert report.compression_ratio_vs_fp16() > 2.0
    assert report.compressed_bytes() < report.fp16_baseline_bytes
    assert report.key_residual_bytes == 0


def layer_kv_bytes(bits, group, r, heads, dim, tokens):
    """Closed-form bytes of one layer (reference src/budget.rs:317-347)."""
    if tokens == 0:
        return 0
    key_res = tokens % r
    key_quant = tokens - key_res
    val_res = min(tokens, r)
    val_quant = max(tokens - r, 0)
    val_groups = (dim + group - 1) // group
    return (heads * key_quant * dim * bits // 8 + heads * (key_quant // group) * dim * 8
            + heads * val_quant * dim * bits // 8 + heads * val_quant * val_groups * 8
            + heads * dim * 4 * (key_res + val_res))


@pytest.mark.parametrize("seq", [1, 32, 127, 128, 129, 512, 2048])
def test_planner_bytes_match_live_cache(backend, seq):
    """tests/budget.rs:68-82: memory().compressed_bytes() equals the closed form."""
    cfg = KiviConfig.default()
    cache = KiviCache(backend, cfg, 1, 8, 128)
    n = 8 * seq * 128
    cache.append(np.full(n, 0.1, np.float32), np.full(n, 0.1, np.float32), seq)
    assert cache.memory().compressed_bytes() == layer_kv_bytes(2, 32, 128, 8, 128, seq)


def test_memory_report_fields(backend):
    """MemoryReport fields (src/cache.rs:362-380) on a mid-stream cache."""
    cfg = KiviConfig.try_new(backend, 4, 32, 64)
    cache = KiviCache(backend, cfg, 2, 3, 64)
    seq = 150
    n = 2 * 3 * seq * 64
    cache.append(fill(n, 1), fill(n, 2), seq)
    r = cache.memory()
    el = 2 * 3 * 64
    assert r.tokens == seq
    assert r.key_code_bytes == 6 * 128 * 64 * 4 // 8
    assert r.key_metadata_bytes == 6 * (128 // 32) * 64 * 8
    assert r.value_code_bytes == 6 * 86 * 64 * 4 // 8
    assert r.value_metadata_bytes == 6 * 86 * 2 * 8
    assert r.key_residual_bytes == 22 * el * 4
    assert r.value_residual_bytes == 64 * el * 4
    assert r.residual_capacity_bytes == 2 * 64 * el * 4
    assert r.fp16_baseline_bytes == 2 * seq * el * 2
    assert r.fp32_baseline_bytes == 2 * seq * el * 4
    assert cache.tokens_until_key_flush() == 64 - 22
    assert cache.value_residual_slots_remaining() == 0


def lib_example(backend):
    """src/lib.rs:12-27."""
    cache = KiviCache(backend, KiviConfig.default(), 1, 1, 128)
    seq = 160
    n = seq * 128
    keys = np.full(n, 0.25, np.float32)
    values = np.full(n, -1.5, np.float32)
    cache.append(keys, values, seq)
    return cache, keys, values


def test_lib_example(backend):
    cache, keys, values = lib_example(backend)
    assert cache.sequence_length() == 160
    assert cache.key_residual_len() == 32
    assert cache.value_residual_len() == 128
    k_hat, v_hat = cache.dequantize()
    np.testing.assert_array_equal(k_hat, keys)
    np.testing.assert_array_equal(v_hat, values)


# ---- trace counters: tests/trace.rs:14-118 restated on the getters CacheSnapshot copies
# (src/trace.rs:33-44): packed = [0, quantized), exact = [quantized, seq).

def _snap(c):
    return (c.sequence_length(), c.quantized_key_tokens(), c.quantized_value_tokens(),
            c.key_residual_len(), c.value_residual_len())


def _trace_cache(backend):
    return KiviCache(backend, KiviConfig.try_new(backend, 2, 32, 32), 1, 1, 32)


def _trace_append(c, n):
    c.append(np.full(n * 32, 0.25, np.float32), np.full(n * 32, -0.5, np.float32), n)


def test_trace_spans(backend):
    c = _trace_cache(backend)
    _trace_append(c, 40)
    seq, kq, vq, kr, vr = _snap(c)
    assert (kq, seq, vq) == (32, 40, 8) and (kr, vr) == (8, 32)
    c = _trace_cache(backend)
    _trace_append(c, 40)
    prev = _snap(c)
    key_spans, value_spans = [], []
    for _ in range(24):
        _trace_append(c, 1)
        now = _snap(c)
        if now[1] > prev[1]:
            key_spans.append((prev[1], now[1]))
        if now[2] > prev[2]:
            value_spans.append((prev[2], now[2]))
        prev = now
    assert key_spans == [(32, 64)]
    assert value_spans[0] == (8, 9) and value_spans[-1] == (31, 32) and len(value_spans) == 24


def test_no_config_can_loop_forever(backend):
    """Hazard fixed at the boundary: residual_length 0 never reaches append (kivi.h)."""
    for bad in (KiviConfig(2, 0, 32), KiviConfig(3, 32, 32), KiviConfig(2, 32, 0)):
        with pytest.raises(KiviError):
            KiviCache(backend, bad, 1, 1, 32)


ZERO_SCHEDULES = {"bulk": [300], "decode": [3] + [1] * 140, "mixed": [37, 1, 64, 1, 1, 130, 7, 1, 1, 60]}


@pytest.mark.parametrize("dim,group", [(128, 32), (128, 64), (256, 32), (64, 16), (96, 32)])
@pytest.mark.parametrize("schedule", list(ZERO_SCHEDULES))
def test_zero_minima_follow_the_first_zero_on_every_schedule(backend, dim, group, schedule):
    """Keys and values whose groups have zero minima with zeros of both signs, appended in
    bulk, token by token (window evictions) and in mixed chunks: every stored zero is the
    group's first zero in element order (src/quant.rs:303, 356), so the streams are the same
    bit for bit whatever the schedule (src/cache.rs:182-185). The shapes take each
    quantize path: lane-register reductions with 1, 2 or 4 channels per lane, 8 to 32 lanes
    per value group, and the LDS-staged kernels (head_dim 96)."""
    bits, residual = 2, 2 * group
    batch, heads = 1, 2
    chunks = ZERO_SCHEDULES[schedule]
    total = sum(chunks)
    rng = np.random.default_rng(dim + group)
    keys = signed_zero_rows(rng, (batch, heads, total, dim))
    keys[:, 1, :, 2::5] -= 1.0  # some channels with negative minima
    values = signed_zero_rows(rng, (batch, heads, total, dim))
    values[:, 0, ::7, 1] = -2.0  # some tokens with negative minima
    cache = KiviCache(backend, KiviConfig(bits, group, residual), batch, heads, dim)
    off = 0
    for n in chunks:
        cache.append(np.ascontiguousarray(keys[:, :, off:off + n]), np.ascontiguousarray(values[:, :, off:off + n]), n)
        off += n
    kq, vq = cache.quantized_key_tokens(), cache.quantized_value_tokens()
    assert kq > 0 and vq > 0
    _, kp, _, vp = cache.export_streams()
    units = batch * heads
    want_k = reference_minimum(keys.reshape(units, total, dim)[:, :kq].reshape(units, kq // group, group, dim), axis=2)
    got_k = kp.reshape(units, kq // group, dim, 2)[..., 1]
    np.testing.assert_array_equal(got_k.view(np.uint32), want_k.view(np.uint32))
    want_v = reference_minimum(values.reshape(units, total, dim)[:, :vq].reshape(units, vq, dim // group, group), axis=3)
    got_v = vp.reshape(units, vq, dim // group, 2)[..., 1]
    np.testing.assert_array_equal(got_v.view(np.uint32), want_v.view(np.uint32))
    for want in (want_k, want_v):
        signs = np.signbit(want[want == 0])
        assert signs.any() and not signs.all()
