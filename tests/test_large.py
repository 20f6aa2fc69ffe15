"""Caches whose arenas pass 4 GiB (``-m gpu``): unit offsets beyond byte 2^32 of an array.

A cache's packed arenas are [units][capacity] per stream (key codes, key params, value codes,
value params), and ``reserve`` sets the capacity. 64 units (batch 8 x 8 KV heads) at a large
reserved capacity place units 32-63 of every arena this test fills past byte offset 2^32 while
only 2800 tokens per unit are appended, so the inputs stay small (183 MB):

* 8-bit, capacity 2^20 tokens: 128 MiB of key codes and of value codes per unit (8 GiB each);
* 2-bit, capacity 2^22 tokens: 128 MiB per unit in all four arenas (32 GiB in all).

The same appends (host rows, then device rows) go to an oracle cache, and every unit is checked:
exported streams (host and device exports) bit-exact, the dense reconstruction bit-exact,
attention within the north-star tolerance at GQA 4 (the 4x4x4 kernel) and GQA 8 (the eight-head
kernel, host and device entry points), and a shared prefix cut from the large cache (its copy
reads the arenas at their full per-unit pitch) with four sessions through the batched GEMM form.
"""

import gc
import math

import numpy as np
import pytest

import kivi
from kivi import KiviCache, KiviConfig
from helpers import DeviceArrays
from test_parity import assert_close, assert_same_state, assert_streams_equal

pytestmark = pytest.mark.gpu

BATCH, HEADS, D = 8, 8, 128
UNITS = BATCH * HEADS
FIRST, SECOND = 1500, 1300
SCALE = np.float32(1.0 / math.sqrt(D))


def rows(rng, n):
    k = rng.standard_normal((BATCH, HEADS, n, D), dtype=np.float32)
    k[:, :, :, 5] *= np.float32(10.0)
    v = rng.standard_normal((BATCH, HEADS, n, D), dtype=np.float32)
    return k, v


@pytest.mark.parametrize("bits, capacity", [(8, 1 << 20), (2, 1 << 22)])
def test_arenas_beyond_4gib(amd, oracle, bits, capacity):
    cfg = KiviConfig(bits, 32, 128)
    a = KiviCache(amd, cfg, BATCH, HEADS, D)
    a.reserve(capacity)
    # the later units' arena offsets pass 2^32 bytes in the arenas this case fills
    per_unit = capacity * D * bits // 8  # key code bytes per unit
    assert per_unit * (UNITS - 1) >= 1 << 32
    print(f"[large] {bits}-bit capacity {capacity}: device bytes {a.device_bytes() / 2**30:.1f} GiB", flush=True)
    o = KiviCache(oracle, cfg, BATCH, HEADS, D)
    rng = np.random.default_rng(7000 + bits)
    k1, v1 = rows(rng, FIRST)
    a.append(k1, v1, FIRST)
    o.append(k1, v1, FIRST)
    k2, v2 = rows(rng, SECOND)
    mem = DeviceArrays()
    try:
        dk, dv = mem.upload(k2), mem.upload(v2)
        a.append_device(dk, k2.size, dv, v2.size, SECOND)
        o.append(k2, v2, SECOND)
        assert_same_state(a, o)
        assert_streams_equal(a, o)
        # device export of the same streams
        lens = a.stream_lengths()
        ptrs = [mem.alloc(n) for n in lens]
        a.export_streams_device(ptrs, lens)
        for got_p, n, want, name in zip(ptrs, lens, o.export_streams(),
                                        ("key codes", "key params", "value codes", "value params")):
            got = mem.download(got_p, n)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"device export: {name}"
        ka, va = a.dequantize()
        ko, vo = o.dequantize()
        assert np.array_equal(ka.view(np.uint32), ko.view(np.uint32)), "dequantized keys"
        assert np.array_equal(va.view(np.uint32), vo.view(np.uint32)), "dequantized values"
        for qh in (32, 64):
            q = rng.standard_normal((BATCH, qh, D), dtype=np.float32)
            want = o.attention(q, qh, SCALE)
            assert_close(a.attention(q, qh, SCALE), want, f"attention, {qh} query heads")
            dq, dout = mem.upload(q), mem.alloc(want.size)
            a.attention_device(dq, q.size, qh, SCALE, dout, want.size)
            assert_close(mem.download(dout, want.size), want, f"attention_device, {qh} query heads")
        # a prefix cut from the large cache, four sessions through the batched form
        pa, po = a.share_prefix(), o.share_prefix()
        sa, so = [pa.session() for _ in range(4)], [po.session() for _ in range(4)]
        for i, (x, y) in enumerate(zip(sa, so)):
            ks, vs = rows(rng, 20 + 7 * i)
            x.append(ks, vs, 20 + 7 * i)
            y.append(ks, vs, 20 + 7 * i)
        q = rng.standard_normal((4, BATCH, 32, D), dtype=np.float32)
        got = kivi.sessions_attention(amd, sa, q, 32, SCALE).reshape(4, -1)
        for i, y in enumerate(so):
            assert_close(got[i], y.attention(q[i], 32, SCALE), f"session {i}")
        del sa, so, pa, po
    finally:
        mem.free()
        del a
        gc.collect()
