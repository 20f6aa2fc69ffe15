"""kivi_cache_attention_device_noalloc: the attention entry point that allocates nothing (its
split partials live in the library's static per-device workspace) against
kivi_cache_attention_device, which allocates its workspace (``-m gpu``).

Both run the same kernels over the same cache, so the outputs must agree bit for bit. Two
calls in a row, the second over a smaller cache (the static workspace keeps the first call's
partials, which the second must not see), then a cache on the generic path (head_dim 64), an
empty cache (zeros from a fill kernel), and a call whose partials exceed the workspace
(KIVI_ERR_CAPACITY with the sizes, before any launch).

The contract itself (no allocation, no memset, no host wait) is checked under global-mode
stream capture, where an allocation or a synchronization fails the capture: the captured graph
must instantiate, hold kernel nodes only, and replay the allocating call's output bit for bit,
for a filled cache and an empty one. Calls on two streams at once, which share the workspace,
are ordered by the library and must both match.
"""

import ctypes as C

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


HIP_GRAPH_NODE_KERNEL = 0  # hipGraphNodeTypeKernel
HIP_CAPTURE_GLOBAL = 0     # hipStreamCaptureModeGlobal


class Hip:
    """The HIP runtime calls the capture tests need (the runtime the library links)."""

    def __init__(self):
        self.lib = C.CDLL("libamdhip64.so.7")

    def __call__(self, name, *args):
        rc = getattr(self.lib, name)(*args)
        assert rc == 0, f"{name}: hipError {rc}"

    def stream(self):
        s = C.c_void_p()
        self("hipStreamCreate", C.byref(s))
        return s


def capture_noalloc(hip, stream, cache, dq, n, qh, scale, out):
    """The no-allocation call captured on `stream` in global mode -> (graph, exec)."""
    graph, exe = C.c_void_p(), C.c_void_p()
    hip("hipStreamBeginCapture", stream, HIP_CAPTURE_GLOBAL)
    try:
        cache.attention_device_noalloc(dq, n, qh, scale, out, n, stream.value)
    finally:
        rc = hip.lib.hipStreamEndCapture(stream, C.byref(graph))
    assert rc == 0, f"hipStreamEndCapture: hipError {rc} (the call allocated or waited under capture?)"
    count = C.c_size_t(0)
    hip("hipGraphGetNodes", graph, None, C.byref(count))
    nodes = (C.c_void_p * max(count.value, 1))()
    hip("hipGraphGetNodes", graph, nodes, C.byref(count))
    kinds = []
    for i in range(count.value):
        t = C.c_int(-1)
        hip("hipGraphNodeGetType", C.c_void_p(nodes[i]), C.byref(t))
        kinds.append(t.value)
    assert kinds and all(k == HIP_GRAPH_NODE_KERNEL for k in kinds), f"graph node types {kinds}"
    hip("hipGraphInstantiate", C.byref(exe), graph, None, None, C.c_size_t(0))
    return graph, exe


@pytest.mark.parametrize("seq", [6000, 0])
def test_noalloc_attention_under_graph_capture(amd, seq):
    """Global-mode capture of the no-allocation call succeeds (an allocation or a host wait
    inside it would fail the capture), the graph holds only kernel nodes (no memset), and
    three replays, with the program's own eager work and synchronizations between them, each
    give the allocating call's output bit for bit."""
    hip = Hip()
    rng = np.random.default_rng(55 + seq)
    batch, heads, qh, dim = 2, 8, 32, 128
    scale = np.float32(1 / np.sqrt(dim))
    cache = filled_cache(amd, rng, 2, batch, heads, dim, seq)
    mem = DeviceArrays()
    n = batch * qh * dim
    q = rng.standard_normal(n).astype(np.float32)
    dq, out_g, out_e = mem.upload(q), mem.empty(n), mem.empty(n)
    stream = hip.stream()
    cache.attention_device_noalloc(dq, n, qh, scale, out_g, n, stream.value)  # set-up, eager
    cache.attention_device(dq, n, qh, scale, out_e, n, stream.value)
    want = mem.download(out_e, n)
    assert np.array_equal(mem.download(out_g, n).view(np.uint32), want.view(np.uint32))
    graph, exe = capture_noalloc(hip, stream, cache, dq, n, qh, scale, out_g)
    other_q = mem.upload(rng.standard_normal(n).astype(np.float32))
    nan = np.full(n, np.nan, np.float32)
    for rep in range(3):
        hip("hipMemcpy", C.c_void_p(out_g), nan.ctypes.data_as(C.c_void_p), C.c_size_t(4 * n), 1)
        hip("hipGraphLaunch", exe, stream)
        hip("hipStreamSynchronize", stream)
        got = mem.download(out_g, n)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {rep}"
        # eager work between replays: the allocating and the no-allocation calls on another query
        cache.attention_device(other_q, n, qh, scale, out_e, n, stream.value)
        cache.attention_device_noalloc(other_q, n, qh, scale, out_e, n)
        hip("hipDeviceSynchronize")
    if seq == 0:
        assert not want.any()
    hip("hipGraphExecDestroy", exe)
    hip("hipGraphDestroy", graph)
    hip("hipStreamDestroy", stream)
    mem.free()


def test_noalloc_attention_on_two_streams(amd):
    """A long call on one stream and a short one on another, enqueued back to back: both share
    the device's workspace, the library orders the second after the first, and each matches
    the allocating entry point bit for bit."""
    hip = Hip()
    rng = np.random.default_rng(77)
    scale = np.float32(1 / np.sqrt(128))
    big = filled_cache(amd, rng, 2, 8, 8, 128, 12000)
    small = filled_cache(amd, rng, 4, 1, 8, 128, 700)
    mem = DeviceArrays()
    nb, ns = 8 * 32 * 128, 1 * 32 * 128
    qb = mem.upload(rng.standard_normal(nb).astype(np.float32))
    qs = mem.upload(rng.standard_normal(ns).astype(np.float32))
    want_b, want_s = mem.empty(nb), mem.empty(ns)
    big.attention_device(qb, nb, 32, scale, want_b, nb)
    small.attention_device(qs, ns, 32, scale, want_s, ns)
    wb, ws = mem.download(want_b, nb), mem.download(want_s, ns)
    s1, s2 = hip.stream(), hip.stream()
    for rep in range(4):
        first, second = (s1, s2) if rep % 2 == 0 else (s2, s1)
        ob, os_ = mem.empty(nb), mem.empty(ns)
        hip("hipDeviceSynchronize")
        big.attention_device_noalloc(qb, nb, 32, scale, ob, nb, first.value)
        small.attention_device_noalloc(qs, ns, 32, scale, os_, ns, second.value)
        hip("hipDeviceSynchronize")
        assert np.array_equal(mem.download(ob, nb).view(np.uint32), wb.view(np.uint32)), f"rep {rep}: long call"
        assert np.array_equal(mem.download(os_, ns).view(np.uint32), ws.view(np.uint32)), f"rep {rep}: short call"
    hip("hipStreamDestroy", s1)
    hip("hipStreamDestroy", s2)
    mem.free()
