"""kivi_cache_attention_device_noalloc: the attention entry point that allocates nothing (its
split partials live in the library's static per-device workspace) against
kivi_cache_attention_device, which allocates its workspace (``-m gpu``).

Both run the same kernels over the same cache, so the outputs must agree bit for bit. Two
calls in a row, the second over a smaller cache (the static workspace keeps the first call's
partials, which the second must not see), then a cache on the generic path (head_dim 64), an
empty cache (zeros from a fill kernel), and a call whose partials exceed the workspace
(KIVI_ERR_CAPACITY with the sizes, before any launch).
"""

import numpy as np
import pytest

import kivi
from kivi import KiviCache, KiviConfig, KiviError
from helpers import DeviceArrays

pytestmark = pytest.mark.gpu

STATIC_FLOATS = 2 << 20  # kStaticWorkspaceFloats


def filled_cache(amd, rng, bits, batch, heads, dim, seq):
    c = KiviCache(amd, KiviConfig(bits, 32, 128), batch, heads, dim)
    if seq:
        n = batch * heads * seq * dim
        k = rng.standard_normal(n).astype(np.float32)
        k.reshape(batch, heads, seq, dim)[:, :, :, 7] *= np.float32(10.0)
        c.append(k, rng.standard_normal(n).astype(np.float32), seq)
    return c


def both_paths(mem, cache, q, qh, scale):
    """(no-allocation output, allocating output) for query q on the null stream."""
    n = q.size
    dq, out_a, out_b = mem.upload(q), mem.empty(n), mem.empty(n)
    cache.attention_device_noalloc(dq, n, qh, scale, out_a, n)
    cache.attention_device(dq, n, qh, scale, out_b, n)
    return mem.download(out_a, n), mem.download(out_b, n)


def test_noalloc_attention_matches_the_allocating_entry_point(amd):
    rng = np.random.default_rng(2024)
    mem = DeviceArrays()
    scale = np.float32(1 / np.sqrt(128))
    cases = [
        # (bits, batch, kv heads, q heads, head_dim, tokens): large first, then smaller
        (2, 4, 8, 32, 128, 6000),
        (4, 1, 8, 64, 128, 1500),
        (8, 1, 2, 4, 64, 777),
        (2, 2, 4, 8, 128, 0),
    ]
    for bits, batch, heads, qh, dim, seq in cases:
        cache = filled_cache(amd, rng, bits, batch, heads, dim, seq)
        q = rng.standard_normal(batch * qh * dim).astype(np.float32)
        got, want = both_paths(mem, cache, q, qh, scale)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (bits, batch, heads, qh, dim, seq)
        if seq == 0:
            assert not got.any()
    mem.free()


def test_noalloc_attention_refuses_partials_beyond_the_workspace(amd):
    """head_dim 32, 64 query heads on 1 KV head, 8 units of 16384 tokens: 128 splits of 128
    tokens per unit, 8 * 128 * 64 * 34 = 2,228,224 floats of partials."""
    rng = np.random.default_rng(7)
    batch, heads, qh, dim, seq = 8, 1, 64, 32, 16384
    cache = filled_cache(amd, rng, 2, batch, heads, dim, seq)
    mem = DeviceArrays()
    n = batch * qh * dim
    dq, out = mem.upload(rng.standard_normal(n).astype(np.float32)), mem.empty(n)
    with pytest.raises(KiviError) as e:
        cache.attention_device_noalloc(dq, n, qh, np.float32(0.25), out, n)
    assert e.value.variant == "Capacity"
    assert (e.value.a, e.value.b) == (8 * 128 * 64 * 34, STATIC_FLOATS)
    assert "attention workspace floats" in str(e.value)
    # the allocating entry point takes the same call
    cache.attention_device(dq, n, qh, np.float32(0.25), out, n)
    assert np.isfinite(mem.download(out, n)).all()
    mem.free()
