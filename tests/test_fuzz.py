"""Seeded random sweep of the HIP library against the oracle (gpu).

Each case draws a configuration the API accepts (bits 2/4/8; G 16-128 with G*bits a multiple
of 32; R a multiple of G; head_dim 32-256 a multiple of G; 1-3 KV heads, batch 1-2, GQA 1-16)
and one of three workloads:
- a cache fed by 1-4 appends of random sizes (including empty ones), then attention: streams
  and state bit for bit (tests/cache.rs:78-130), attention within the parity tolerance
  (tests/attention.rs:47-101);
- the same cache shared as a prefix with up to 20 sessions of random suffixes, batched
  session attention against each session's oracle attention (src/prefix.rs:228-289), at the
  shapes the batched kernels take (head_dim 128, G 32);
- RuntimeKv prefill then up to 2R+2 decode steps, crossing key flushes and window
  evictions (src/runtime.rs:33-56, tests/runtime.rs:13-52); every other such case decodes on
  device pointers, where a step without a key flush is one attention launch carrying the
  append and the eviction.
One cache case in four also runs the allocation-free attention entry point and requires it
to equal the allocating one bit for bit (or to refuse with Capacity when the call's split
partials exceed its static workspace).
"""

import numpy as np
import pytest

import kivi
from kivi import KiviCache, KiviConfig, KiviError, RuntimeKv
from helpers import DeviceArrays
from test_parity import assert_close, assert_same_state, assert_streams_equal

pytestmark = pytest.mark.gpu


def draw(seed):
    rng = np.random.default_rng(91000 + seed)
    bits = int(rng.choice([2, 4, 8]))
    G = int(rng.choice([g for g in (16, 32, 64, 128) if g * bits % 32 == 0]))
    R = G * int(rng.integers(1, 5))
    D = int(rng.choice([d for d in (32, 64, 96, 128, 192, 256) if d % G == 0] or [G]))
    H, B = int(rng.integers(1, 4)), int(rng.integers(1, 3))
    gq = int(rng.choice([1, 2, 3, 4, 5, 6, 8, 12, 16]))
    n_app = int(rng.integers(1, 5))
    cap = max(2, min(600000 // (B * H * D), 2500) // n_app)
    sizes = [int(rng.integers(0, cap)) for _ in range(n_app)]
    kind = ("cache", "cache", "sessions", "runtime")[seed % 4]
    if kind == "sessions":
        D, G, R = 128, 32, 32 * int(rng.integers(1, 5))
    return rng, kind, KiviConfig(bits, G, R), B, H, D, gq, sizes


@pytest.mark.parametrize("seed", range(60))
def test_random_shapes_match_oracle(amd, oracle, seed):
    rng, kind, cfg, B, H, D, gq, sizes = draw(seed)
    scale = np.float32(1.0 / np.sqrt(D) * rng.uniform(0.5, 2.0))
    qh = H * gq
    if kind == "runtime":
        ra, ro = RuntimeKv(amd, cfg, B, H, D), RuntimeKv(oracle, cfg, B, H, D)
        n = sizes[0]
        k = rng.standard_normal(B * H * n * D).astype(np.float32)
        v = rng.standard_normal(B * H * n * D).astype(np.float32)
        ra.prefill(k, v, n)
        ro.prefill(k, v, n)
        on_device = seed % 8 == 7
        mem = DeviceArrays()
        n_kv, n_q = B * H * D, B * qh * D
        out = mem.empty(n_q)
        for s in range(int(rng.integers(1, 2 * cfg.residual_length + 3))):
            kk = rng.standard_normal(n_kv).astype(np.float32)
            vv = rng.standard_normal(n_kv).astype(np.float32)
            q = rng.standard_normal(n_q).astype(np.float32)
            if on_device:
                ra.decode_device(mem.upload(kk), n_kv, mem.upload(vv), n_kv, mem.upload(q), n_q, qh, scale, out, n_q)
                got = mem.download(out, n_q)
            else:
                got = ra.decode(kk, vv, q, qh, scale)
            assert_close(got, ro.decode(kk, vv, q, qh, scale), f"step {s}")
        mem.free()
        assert_same_state(ra.cache(), ro.cache())
        assert_streams_equal(ra.cache(), ro.cache())
        return
    ca, co = KiviCache(amd, cfg, B, H, D), KiviCache(oracle, cfg, B, H, D)
    for n in sizes:
        k = (rng.standard_normal(B * H * n * D) * rng.uniform(0.1, 5)).astype(np.float32)
        v = rng.standard_normal(B * H * n * D).astype(np.float32)
        if n and rng.random() < 0.3:
            k.reshape(B, H, n, D)[:, :, :, int(rng.integers(0, D))] *= 10
        ca.append(k, v, n)
        co.append(k, v, n)
    assert_same_state(ca, co)
    assert_streams_equal(ca, co)
    if kind == "cache":
        q = rng.standard_normal(B * qh * D).astype(np.float32)
        got = ca.attention(q, qh, scale)
        assert_close(got, co.attention(q, qh, scale))
        if seed % 8 == 1 and ca.sequence_length() > 0:
            mem = DeviceArrays()
            dq, out_a, out_b = mem.upload(q), mem.empty(q.size), mem.empty(q.size)
            ca.attention_device(dq, q.size, qh, scale, out_a, q.size)
            try:
                ca.attention_device_noalloc(dq, q.size, qh, scale, out_b, q.size)
                refused = False
            except KiviError as e:
                assert e.variant == "Capacity"
                refused = True
            a, b = mem.download(out_a, q.size), mem.download(out_b, q.size)
            mem.free()
            if not refused:
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
            assert np.array_equal(a.view(np.uint32), got.view(np.uint32))
        return
    pa, po = ca.share_prefix(), co.share_prefix()
    ns = int(rng.integers(1, 21))
    sa, so = [pa.session() for _ in range(ns)], [po.session() for _ in range(ns)]
    for a, o in zip(sa, so):
        n = int(rng.integers(0, 150))
        if n:
            sk = rng.standard_normal(B * H * n * D).astype(np.float32)
            sv = rng.standard_normal(B * H * n * D).astype(np.float32)
            a.append(sk, sv, n)
            o.append(sk, sv, n)
    per = B * qh * D
    qs = rng.standard_normal(ns * per).astype(np.float32)
    got = kivi.sessions_attention(amd, sa, qs, qh, scale)
    for i, o in enumerate(so):
        assert_close(got[i * per:(i + 1) * per], o.attention(qs[i * per:(i + 1) * per], qh, scale), f"session {i}")
