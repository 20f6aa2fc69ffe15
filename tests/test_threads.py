"""Concurrent readers (``-m gpu``).

The reference's `KiviCache::attention` takes `&self`, so several threads may read one cache at
once (src/cache.rs:224), and `SharedPrefix` is `Send + Sync`, so the sessions of one prefix may
run on different threads (src/prefix.rs:29-35). Here the calls of one cache share its device
workspace: host-pointer calls are ordered by the cache's own stream, and device-pointer calls
on different streams by the workspace's event (kivi.h). Each case runs its calls from eight
threads at once (ctypes releases the GIL for the call) and checks every result against the
oracle's, computed one at a time beforehand.
"""
import ctypes as C
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import kivi
from kivi import KiviCache, KiviConfig
from helpers import DeviceArrays
from test_parity import assert_close

pytestmark = pytest.mark.gpu

THREADS = 8


def cache_pair(amd, oracle, bits, heads, dim, seq, seed):
    cfg = KiviConfig(bits, 32, 128)
    rng = np.random.default_rng(seed)
    k = rng.standard_normal(heads * seq * dim).astype(np.float32)
    k.reshape(heads, seq, dim)[:, :, 3] *= 10
    v = rng.standard_normal(heads * seq * dim).astype(np.float32)
    a, o = KiviCache(amd, cfg, 1, heads, dim), KiviCache(oracle, cfg, 1, heads, dim)
    a.append(k, v, seq)
    o.append(k, v, seq)
    return a, o, rng


@pytest.mark.parametrize("bits", [2, 8])
def test_host_attention_from_threads(amd, oracle, bits):
    heads, dim, seq, qh = 8, 128, 9000, 32
    a, o, rng = cache_pair(amd, oracle, bits, heads, dim, seq, 700 + bits)
    scale = np.float32(1 / np.sqrt(dim))
    qs = [rng.standard_normal(qh * dim).astype(np.float32) for _ in range(4 * THREADS)]
    want = [o.attention(q, qh, scale) for q in qs]
    with ThreadPoolExecutor(THREADS) as ex:
        got = list(ex.map(lambda q: a.attention(q, qh, scale), qs))
    for i, (g, w) in enumerate(zip(got, want)):
        assert_close(g, w, f"call {i}")


def test_device_attention_from_threads_on_their_own_streams(amd, oracle):
    """Each thread enqueues attention_device calls on its own non-blocking stream into its own
    output buffers; the cache's split-partial workspace is shared by all of them."""
    heads, dim, seq, qh = 8, 128, 12000, 64
    a, o, rng = cache_pair(amd, oracle, 2, heads, dim, seq, 720)
    scale = np.float32(1 / np.sqrt(dim))
    calls = 3
    qs = [rng.standard_normal(qh * dim).astype(np.float32) for _ in range(calls * THREADS)]
    want = [o.attention(q, qh, scale) for q in qs]
    mem = DeviceArrays()
    hip = mem._hip
    streams = []
    try:
        dq = [mem.upload(q) for q in qs]
        dout = [mem.alloc(qh * dim) for _ in qs]
        for _ in range(THREADS):
            s = C.c_void_p()
            assert hip.hipStreamCreateWithFlags(C.byref(s), 1) == 0
            streams.append(s)

        def worker(t):
            for j in range(calls):
                i = t * calls + j
                a.attention_device(dq[i], qh * dim, qh, scale, dout[i], qh * dim, streams[t].value)
            assert hip.hipStreamSynchronize(streams[t]) == 0

        with ThreadPoolExecutor(THREADS) as ex:
            list(ex.map(worker, range(THREADS)))
        for i in range(len(qs)):
            assert_close(mem.download(dout[i], qh * dim), want[i], f"call {i}")
    finally:
        for s in streams:
            hip.hipStreamSynchronize(s)
            hip.hipStreamDestroy(s)
        mem.free()


def test_sessions_of_one_prefix_on_threads(amd, oracle):
    """Every thread opens its own session of a shared prefix, appends its suffix and reads
    attention, alone and through the batched call over its session."""
    heads, dim, seq, qh = 8, 128, 6000, 32
    a, o, rng = cache_pair(amd, oracle, 2, heads, dim, seq, 740)
    pa, po = a.share_prefix(), o.share_prefix()
    scale = np.float32(1 / np.sqrt(dim))
    work = []
    for t in range(THREADS):
        n = 30 + 11 * t
        ks = rng.standard_normal(heads * n * dim).astype(np.float32)
        vs = rng.standard_normal(heads * n * dim).astype(np.float32)
        q = rng.standard_normal(qh * dim).astype(np.float32)
        so = po.session()
        so.append(ks, vs, n)
        work.append((ks, vs, n, q, so.attention(q, qh, scale)))

    def worker(t):
        ks, vs, n, q, want = work[t]
        s = pa.session()
        s.append(ks, vs, n)
        alone = s.attention(q, qh, scale)
        batched = kivi.sessions_attention(amd, [s], q, qh, scale)
        return alone, batched, want

    with ThreadPoolExecutor(THREADS) as ex:
        results = list(ex.map(worker, range(THREADS)))
    for t, (alone, batched, want) in enumerate(results):
        assert_close(alone, want, f"thread {t} session")
        assert_close(batched, want, f"thread {t} batched")
