"""Group sizes that do not divide the 64-token value block (``-m gpu``).

The reference accepts any group with group_size * bits % 32 == 0 (src/config.rs:40-55): 48 at
2 bits, 24 at 4 bits, 12 and 4 at 8 bits. A 64-token block then touches key groups that start
and end inside it, the capacity granule is lcm(64, G), and the kernels of this library take
their general forms (generic quantizers and attention, the decode step as an append then an
attention). Each case streams appends, then decode steps across flushes and evictions, and
checks against the oracle: counters and exported streams bit-exact (host and device exports),
the dense reconstruction bit-exact, attention within the north-star tolerance, and a batched
session call over a prefix cut from the cache.
"""

import numpy as np
import pytest

import kivi
from kivi import KiviCache, KiviConfig, RuntimeKv
from helpers import DeviceArrays
from test_parity import assert_close, assert_same_state, assert_streams_equal

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits,group,residual,dim", [
    (2, 48, 96, 96), (4, 24, 48, 96), (8, 12, 36, 96), (8, 4, 8, 32), (4, 8, 16, 64), (2, 48, 48, 192)])
def test_group_not_dividing_the_value_block(amd, oracle, bits, group, residual, dim):
    assert group * bits % 32 == 0 and 64 % group != 0 or group in (4, 8)
    batch, heads, qh = 2, 2, 4
    cfg = KiviConfig(bits, group, residual)
    rng = np.random.default_rng(9000 + 100 * bits + group)
    ra, ro = RuntimeKv(amd, cfg, batch, heads, dim), RuntimeKv(oracle, cfg, batch, heads, dim)
    a, o = ra.cache(), ro.cache()
    scale = np.float32(1 / np.sqrt(dim))
    for n in (1, 70, 5, 200, 3 * group + 1, 64):
        k = rng.standard_normal(batch * heads * n * dim).astype(np.float32)
        k.reshape(batch, heads, n, dim)[:, :, :, 1] *= 10
        v = rng.standard_normal(batch * heads * n * dim).astype(np.float32)
        a.append(k, v, n)
        o.append(k, v, n)
        assert_same_state(a, o)
    assert_streams_equal(a, o)
    for step in range(2 * residual + 3):
        kk = rng.standard_normal(batch * heads * dim).astype(np.float32)
        vv = rng.standard_normal(batch * heads * dim).astype(np.float32)
        q = rng.standard_normal(batch * qh * dim).astype(np.float32)
        assert_close(ra.decode(kk, vv, q, qh, scale), ro.decode(kk, vv, q, qh, scale), f"step {step}")
    assert_same_state(a, o)
    assert_streams_equal(a, o)
    ka, va = a.dequantize()
    ko, vo = o.dequantize()
    assert np.array_equal(ka.view(np.uint32), ko.view(np.uint32)), "dequantized keys"
    assert np.array_equal(va.view(np.uint32), vo.view(np.uint32)), "dequantized values"
    mem = DeviceArrays()
    try:
        lens = a.stream_lengths()
        ptrs = [mem.alloc(max(n, 1)) for n in lens]
        a.export_streams_device(ptrs, lens)
        for p, n, want, name in zip(ptrs, lens, o.export_streams(),
                                    ("key codes", "key params", "value codes", "value params")):
            got = mem.download(p, n)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"device export: {name}"
    finally:
        mem.free()
    pa, po = a.share_prefix(), o.share_prefix()
    sa, so = [pa.session() for _ in range(3)], [po.session() for _ in range(3)]
    for i, (x, y) in enumerate(zip(sa, so)):
        n = 10 + 17 * i
        ks = rng.standard_normal(batch * heads * n * dim).astype(np.float32)
        vs = rng.standard_normal(batch * heads * n * dim).astype(np.float32)
        x.append(ks, vs, n)
        y.append(ks, vs, n)
    q = rng.standard_normal((3, batch, qh, dim)).astype(np.float32)
    got = kivi.sessions_attention(amd, sa, q, qh, scale).reshape(3, -1)
    for i, y in enumerate(so):
        assert_close(got[i], y.attention(q[i], qh, scale), f"session {i}")
