"""Host-pointer calls on a cache or session right after a device-pointer append on another
stream.

The reference's calls are synchronous (src/cache.rs:186-279, src/prefix.rs:74-92): an append
has finished before the next call reads the cache. Here `append_device` only enqueues its work
on the caller's stream; a host-pointer call that follows on the cache's own stream must wait for
that work (kivi.h), even when the caller's stream does not synchronize with the default stream
(a non-blocking stream). Each case makes the host call at once, with no synchronization by the
caller, and checks the result against the oracle's synchronous cache.
"""
import ctypes as C

import numpy as np
import pytest

import kivi
from kivi import KiviCache, KiviConfig
from helpers import DeviceArrays
from test_parity import assert_close, assert_same_state, assert_streams_equal

pytestmark = pytest.mark.gpu

HIP_STREAM_NON_BLOCKING = 1


def non_blocking_stream(hip):
    s = C.c_void_p()
    assert hip.hipStreamCreateWithFlags(C.byref(s), HIP_STREAM_NON_BLOCKING) == 0
    return s


def prefill(rng, heads, seq, dim):
    k = rng.standard_normal(heads * seq * dim).astype(np.float32)
    v = rng.standard_normal(heads * seq * dim).astype(np.float32)
    k.reshape(heads, seq, dim)[:, :, 3] *= 10
    return k, v


def test_session_host_attention_after_device_append_on_another_stream(amd, oracle):
    """RagSession::append on device pointers (enqueued on a non-blocking stream) then the
    session's host-pointer attention and the batched host call, with no synchronization by the
    caller (src/prefix.rs:173-289)."""
    heads, dim, seq, qh, suffix = 8, 128, 4096, 32, 3000
    cfg = KiviConfig(2, 32, 128)
    rng = np.random.default_rng(620)
    k, v = prefill(rng, heads, seq, dim)
    a, o = KiviCache(amd, cfg, 1, heads, dim), KiviCache(oracle, cfg, 1, heads, dim)
    a.append(k, v, seq)
    o.append(k, v, seq)
    pa, po = a.share_prefix(), o.share_prefix()
    mem = DeviceArrays()
    hip = mem._hip
    s = non_blocking_stream(hip)
    try:
        ks, vs = prefill(rng, heads, suffix, dim)
        dk, dv = mem.upload(ks), mem.upload(vs)
        q = rng.standard_normal(qh * dim).astype(np.float32)
        scale = np.float32(1 / np.sqrt(dim))
        sa, so = pa.session(), po.session()
        so.append(ks, vs, suffix)
        sa.append_device(dk, ks.size, dv, vs.size, suffix, s.value)  # enqueued on s, not waited for
        assert_close(sa.attention(q, qh, scale), so.attention(q, qh, scale))
        sb = pa.session()
        sb.append_device(dk, ks.size, dv, vs.size, suffix, s.value)
        got = kivi.sessions_attention(amd, [sb], q, qh, scale)
        assert_close(got, so.attention(q, qh, scale))
        assert hip.hipStreamSynchronize(s) == 0
    finally:
        hip.hipStreamSynchronize(s)
        hip.hipStreamDestroy(s)
        mem.free()


def test_set_stream_waits_for_device_work_on_the_previous_stream(amd, oracle):
    """A device-pointer append on the cache's own stream (kivi_cache_set_stream) is ordered
    before later host-pointer calls by that stream alone. Switching the cache to another stream
    right after it must wait for it, so a host-pointer call on the new stream sees the tokens."""
    heads, dim, seq, qh = 8, 128, 16384, 32
    cfg = KiviConfig(2, 32, 128)
    rng = np.random.default_rng(640)
    k, v = prefill(rng, heads, seq, dim)
    mem = DeviceArrays()
    hip = mem._hip
    s1, s2 = non_blocking_stream(hip), non_blocking_stream(hip)
    try:
        o = KiviCache(oracle, cfg, 1, heads, dim)
        o.append(k, v, seq)
        a = KiviCache(amd, cfg, 1, heads, dim)
        a.set_stream(s1.value)
        dk, dv = mem.upload(k), mem.upload(v)
        a.append_device(dk, k.size, dv, v.size, seq, s1.value)  # on the cache's own stream
        a.set_stream(s2.value)
        q = rng.standard_normal(qh * dim).astype(np.float32)
        scale = np.float32(1 / np.sqrt(dim))
        assert_close(a.attention(q, qh, scale), o.attention(q, qh, scale))
        assert_streams_equal(a, o)
        a.set_stream(0)
        del a
    finally:
        for s in (s1, s2):
            hip.hipStreamSynchronize(s)
            hip.hipStreamDestroy(s)
        mem.free()


@pytest.mark.parametrize("bits", [2, 8])
@pytest.mark.parametrize("then", ["export", "attention", "share_prefix", "reserve_then_append", "free"])
def test_host_call_after_device_append_on_another_stream(amd, oracle, bits, then):
    heads, dim, seq, qh = 8, 128, 16384, 32
    cfg = KiviConfig(bits, 32, 128)
    rng = np.random.default_rng(610 + bits)
    k, v = prefill(rng, heads, seq, dim)
    mem = DeviceArrays()
    hip = mem._hip
    s = non_blocking_stream(hip)
    try:
        dk, dv = mem.upload(k), mem.upload(v)
        o = KiviCache(oracle, cfg, 1, heads, dim)
        o.append(k, v, seq)
        a = KiviCache(amd, cfg, 1, heads, dim)
        a.append_device(dk, k.size, dv, v.size, seq, s.value)  # enqueued on s, not waited for
        q = rng.standard_normal(qh * dim).astype(np.float32)
        scale = np.float32(1 / np.sqrt(dim))
        if then == "export":
            assert_streams_equal(a, o)
        elif then == "attention":
            assert_close(a.attention(q, qh, scale), o.attention(q, qh, scale))
        elif then == "share_prefix":
            pa, po = a.share_prefix(), o.share_prefix()
            del a
            sa, so = pa.session(), po.session()
            ks, vs = prefill(rng, heads, 40, dim)
            sa.append(ks, vs, 40)
            so.append(ks, vs, 40)
            assert_close(sa.attention(q, qh, scale), so.attention(q, qh, scale))
        elif then == "reserve_then_append":
            # the reserve regrows the arenas (copying them) after the device append's work
            a.reserve(seq + 5000)
            k2, v2 = prefill(rng, heads, 300, dim)
            a.append(k2, v2, 300)
            o.append(k2, v2, 300)
            assert_same_state(a, o)
            assert_streams_equal(a, o)
        else:
            del a  # freeing waits for the append's work before the arenas go
            assert hip.hipStreamSynchronize(s) == 0
        assert hip.hipStreamSynchronize(s) == 0
    finally:
        hip.hipStreamSynchronize(s)
        hip.hipStreamDestroy(s)
        mem.free()


@pytest.mark.parametrize("per_channel", [True, False])
def test_quantized_host_reads_after_device_quantize_on_another_stream(amd, oracle, per_channel):
    """quantize_per_channel / per_token on device input, enqueued on a non-blocking stream, then
    the QuantizedTensor's host reads at once (src/quant.rs:24-151): they wait for the quantize."""
    batch, heads, tokens, dim, bits, group = 4, 8, 8192, 128, 2, 32
    rng = np.random.default_rng(650 + per_channel)
    x = rng.standard_normal(batch * heads * tokens * dim).astype(np.float32)
    q = kivi.quantize_per_channel if per_channel else kivi.quantize_per_token
    want = q(oracle, x, batch, heads, tokens, dim, bits, group)
    mem = DeviceArrays()
    hip = mem._hip
    s = non_blocking_stream(hip)
    try:
        dx = mem.upload(x)
        got = kivi.quantize_device(amd, per_channel, dx, x.size, batch, heads, tokens, dim, bits, group, s.value)
        assert np.array_equal(got.codes(), want.codes())
        assert np.array_equal(got.scale_zero().view(np.uint32), want.scale_zero().view(np.uint32))
        assert np.array_equal(got.pytorch_codes(), want.pytorch_codes())
        assert np.array_equal(got.dequantize().view(np.uint32), want.dequantize().view(np.uint32))
        del got
    finally:
        hip.hipStreamSynchronize(s)
        hip.hipStreamDestroy(s)
        mem.free()
