"""Input generators and dense references shared by the tests.

The generators restate the reference tests' fixtures: the LCG ``fill`` (tests/attention.rs:3-11),
the closed-form ``document`` (tests/prefix.rs:7-18) and ``slice_tokens`` (tests/cache.rs:17-34).
Dense references follow tests/attention.rs:13-38 and tests/prefix.rs:20-68 (f32, as the Rust
tests compute them) and add an f64 brute force for stricter checks.
"""

import numpy as np

import kivi

fill = kivi.lcg_fill


def document(batch, heads, seq, dim):
    """tests/prefix.rs:7-18."""
    n = batch * heads * seq * dim
    i = np.arange(n, dtype=np.int64)
    keys = (((i * 17) % 23).astype(np.float32) / np.float32(11.0)) - np.float32(0.4)
    values = (((i * 13) % 19).astype(np.float32) / np.float32(9.0)) - np.float32(0.2)
    return keys.astype(np.float32), values.astype(np.float32)


def slice_tokens(full, batch, heads, total, dim, offset, count):
    """tests/cache.rs:17-34: tokens [offset, offset+count) of a [B,H,total,D] tensor."""
    a = np.asarray(full, dtype=np.float32).reshape(batch, heads, total, dim)
    return np.ascontiguousarray(a[:, :, offset:offset + count, :]).reshape(-1)


def concat_head_major(prefix, extra, batch, heads, prefix_len, extra_len, dim):
    """tests/prefix.rs:70-95."""
    a = np.asarray(prefix, np.float32).reshape(batch, heads, prefix_len, dim)
    b = np.asarray(extra, np.float32).reshape(batch, heads, extra_len, dim)
    return np.concatenate([a, b], axis=2).reshape(-1)


def dense_attend(keys, values, query, batch, kv_heads, q_heads, seq, dim, scale,
                 dtype=np.float64):
    """Dense softmax attention over [B,KV,seq,D] K/V for [B,QH,D] queries (GQA qh/(QH/KV)),
    computed in ``dtype`` (tests/prefix.rs:20-68 computes the same in f32)."""
    k = np.asarray(keys, dtype).reshape(batch, kv_heads, seq, dim)
    v = np.asarray(values, dtype).reshape(batch, kv_heads, seq, dim)
    q = np.asarray(query, dtype).reshape(batch, q_heads, dim)
    group = q_heads // kv_heads
    out = np.zeros((batch, q_heads, dim), dtype)
    for b in range(batch):
        for qh in range(q_heads):
            kvh = qh // group
            logits = (k[b, kvh] @ q[b, qh]) * dtype(scale)
            logits = logits - logits.max()
            w = np.exp(logits)
            w = w / w.sum()
            out[b, qh] = w @ v[b, kvh]
    return out.reshape(-1)


def max_abs(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b))) if a.size else 0.0


class DeviceArrays:
    """Device buffers for the ``*_device`` entry points, through the same HIP runtime the
    library links (/opt/rocm/lib/libamdhip64.so.7), so the test process holds one runtime."""

    def __init__(self):
        import ctypes as C
        self._C = C
        self._hip = C.CDLL("libamdhip64.so.7")
        self._ptrs = []

    def _ok(self, rc, what):
        assert rc == 0, f"{what}: hipError {rc}"

    def upload(self, host):
        C = self._C
        host = np.ascontiguousarray(host, dtype=np.float32)
        p = C.c_void_p()
        self._ok(self._hip.hipMalloc(C.byref(p), C.c_size_t(max(host.nbytes, 4))), "hipMalloc")
        self._ptrs.append(p)
        self._ok(self._hip.hipMemcpy(p, host.ctypes.data_as(C.c_void_p), C.c_size_t(host.nbytes), 1),
                 "hipMemcpy H2D")
        return p.value

    def empty(self, n):
        return self.upload(np.zeros(n, np.float32))

    def alloc(self, n):
        """Device buffer of n floats, contents undefined (no host copy)."""
        C = self._C
        p = C.c_void_p()
        self._ok(self._hip.hipMalloc(C.byref(p), C.c_size_t(max(4 * n, 4))), "hipMalloc")
        self._ptrs.append(p)
        return p.value

    def download(self, ptr, n):
        C = self._C
        out = np.empty(n, np.float32)
        self._ok(self._hip.hipDeviceSynchronize(), "hipDeviceSynchronize")
        self._ok(self._hip.hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), C.c_size_t(out.nbytes), 2),
                 "hipMemcpy D2H")
        return out

    def free(self):
        for p in self._ptrs:
            self._hip.hipFree(p)
        self._ptrs = []


def reference_minimum(x, axis):
    """Group minima as the reference's f32::min takes them in element order along ``axis``
    (src/quant.rs:303, 356): the minimum's value, and for a zero minimum the sign of the
    first zero (+0 and -0 compare equal, so the running minimum keeps the first)."""
    x = np.asarray(x, np.float32)
    mn = x.min(axis=axis)
    first = np.argmax(x == 0, axis=axis)
    fz = np.take_along_axis(x, np.expand_dims(first, axis), axis).squeeze(axis)
    return np.where(mn == 0, fz, mn).astype(np.float32)


def signed_zero_rows(rng, shape, p=0.25):
    """|N(0,1)| with zeros of random sign planted at rate p: nearly every group of 16+
    elements then has a zero minimum and zeros of both signs."""
    x = np.abs(rng.standard_normal(shape)).astype(np.float32)
    z = rng.random(shape) < p
    neg = rng.random(shape) < 0.5
    x[z & neg] = np.float32(-0.0)
    x[z & ~neg] = np.float32(0.0)
    return x


# ------------------------------------------------------------------ large-magnitude inputs
# The reference's quiet-channel fixture (tests/quant.rs:170-211, examples/streaming_cache.rs:
# 10-17): channel 0 of a 32-channel row is 100.0 and channel d >= 1 is d/32, the same for
# every token. The generators below tile that row across head_dim and add the magnitudes the
# KIVI observation is about (key channels x100 / x1000, value groups mixing 1e-3 and 1e2).


def quiet_channel_rows(tokens, dim, jitter=0.0, rng=None):
    """[tokens, dim] rows of the quiet-channel fixture tiled over head_dim (channels 0, 32,
    ... are 100.0; channel d is (d % 32)/32 otherwise). With ``jitter`` > 0, N(0, jitter)
    noise on the quiet channels and N(0, 1) on the loud ones, so group spans are non-zero."""
    d = np.arange(dim)
    row = np.where(d % 32 == 0, np.float32(100.0), (d % 32).astype(np.float32) / np.float32(32.0))
    x = np.broadcast_to(row.astype(np.float32), (tokens, dim)).copy()
    if jitter:
        noise = rng.standard_normal((tokens, dim)).astype(np.float32)
        x += np.where(d % 32 == 0, np.float32(1.0), np.float32(jitter)) * noise
    return x.astype(np.float32)


def loud_channel_keys(rng, shape, magnitude, per_head=2):
    """N(0,1) keys [.., heads, T, D] with ``per_head`` channels of every KV head scaled by
    ``magnitude`` (the same channels for every token)."""
    k = rng.standard_normal(shape).astype(np.float32)
    heads, dim = shape[-3], shape[-1]
    for h in range(heads):
        chans = rng.choice(dim, size=per_head, replace=False)
        k[..., h, :, chans] *= np.float32(magnitude)
    return k


def mixed_magnitude_values(rng, shape, group=32):
    """N(0,1) values [.., T, D] whose 32-channel groups take, per (token, group), one of:
    every channel ~1e-3; every channel ~1e2; channels alternating 1e-3 / 1e2; ~1."""
    v = rng.standard_normal(shape).astype(np.float32)
    lead, dim = shape[:-1], shape[-1]
    mode = rng.integers(0, 4, size=lead + (dim // group,))
    alt = np.where(np.arange(group) % 2 == 0, 1e-3, 1e2)
    table = np.stack([np.full(group, 1e-3), np.full(group, 1e2), alt, np.ones(group)])
    mag = table[mode].reshape(lead + (dim,)).astype(np.float32)
    return (v * mag).astype(np.float32)
