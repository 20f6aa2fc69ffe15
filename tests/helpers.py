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
