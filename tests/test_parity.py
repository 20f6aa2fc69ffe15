"""Parity of the HIP library with the oracle on identical seeded inputs (``-m gpu``).

* Packed codes and (scale, zero) values: bit-exact, compared in the reference's PackedStream
  order (kivi_cache_export_streams) after every append of a randomized append schedule.
* Dense reconstruction (dequantize): bit-exact.
* Attention: |got - oracle| <= ATOL + RTOL*|oracle| with the north-star tolerance
  (max-abs 1e-3, relative 1e-4 in f32), and within the reference's own 1e-4 of an f64
  dense brute force on the dequantized cache (tests/attention.rs:59).
"""

import numpy as np
import pytest

import kivi
from kivi import KiviCache, KiviConfig, RuntimeKv
from helpers import DeviceArrays, dense_attend, fill, max_abs, reference_minimum, signed_zero_rows

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-3, 1e-4


def assert_close(got, want, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bound = ATOL + RTOL * np.abs(want)
    bad = np.abs(got - want) > bound
    assert not bad.any(), f"{what}: {bad.sum()} elements beyond tolerance, max err {max_abs(got, want):.3g}"


def assert_same_state(a, o):
    assert a.sequence_length() == o.sequence_length()
    assert a.quantized_key_tokens() == o.quantized_key_tokens()
    assert a.quantized_value_tokens() == o.quantized_value_tokens()
    assert a.key_residual_len() == o.key_residual_len()
    assert a.value_residual_len() == o.value_residual_len()
    ma, mo = a.memory(), o.memory()
    for f, _ in kivi._MemoryReport._fields_:
        assert getattr(ma, f) == getattr(mo, f), f


def assert_streams_equal(a, o):
    for x, y, name in zip(a.export_streams(), o.export_streams(),
                          ("key codes", "key params", "value codes", "value params")):
        assert x.shape == y.shape, name
        if x.dtype == np.float32:
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), name
        else:
            assert np.array_equal(x, y), name


SCHEDULES = {
    "decode": [5] + [1] * 70,
    "chunks": [1, 50, 7, 12, 200, 3, 64, 1, 1, 130],
    "bulk": [333],
    "exact_r": [64, 64, 32, 32, 1],
}


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("group,residual,dim", [(32, 64, 128), (16, 32, 32), (32, 32, 64),
                                               (64, 128, 128)])
@pytest.mark.parametrize("schedule", list(SCHEDULES))
def test_streaming_cache_parity(amd, oracle, bits, group, residual, dim, schedule):
    if group * bits % 32:
        pytest.skip("invalid group for bits")
    chunks = SCHEDULES[schedule]
    batch, heads, qh = 2, 2, 4
    total = sum(chunks)
    rng = np.random.default_rng(1000 * bits + group + dim)
    keys = rng.standard_normal(batch * heads * total * dim).astype(np.float32)
    keys.reshape(batch, heads, total, dim)[:, :, :, 3] *= 10  # outlier channel
    values = rng.standard_normal(batch * heads * total * dim).astype(np.float32)
    cfg = KiviConfig(bits, group, residual)
    a = KiviCache(amd, cfg, batch, heads, dim)
    o = KiviCache(oracle, cfg, batch, heads, dim)
    off = 0
    for step, n in enumerate(chunks):
        k = keys.reshape(batch, heads, total, dim)[:, :, off:off + n].copy()
        v = values.reshape(batch, heads, total, dim)[:, :, off:off + n].copy()
        a.append(k, v, n)
        o.append(k, v, n)
        off += n
        assert_same_state(a, o)
        if step % 7 == 0 or step == len(chunks) - 1:
            assert_streams_equal(a, o)
            q = rng.standard_normal(batch * qh * dim).astype(np.float32)
            scale = np.float32(1.0) / np.sqrt(np.float32(dim))
            assert_close(a.attention(q, qh, scale), o.attention(q, qh, scale), f"step {step}")
    ka, va = a.dequantize()
    ko, vo = o.dequantize()
    assert np.array_equal(ka.view(np.uint32), ko.view(np.uint32))
    assert np.array_equal(va.view(np.uint32), vo.view(np.uint32))


@pytest.mark.parametrize("dim,group,gqa,bits", [
    (64, 32, 4, 2), (64, 64, 1, 4), (64, 32, 2, 8), (64, 64, 12, 2), (64, 32, 8, 8), (192, 64, 3, 2),
    (192, 32, 8, 8), (192, 64, 5, 4), (128, 32, 48, 2), (64, 64, 40, 4),
    (256, 32, 4, 4), (256, 128, 2, 8), (256, 64, 8, 8), (256, 32, 4, 2), (256, 64, 8, 2), (256, 128, 3, 2),
    (128, 64, 4, 2), (128, 32, 16, 2), (128, 128, 12, 4), (128, 128, 32, 2), (128, 64, 8, 8),
    (128, 64, 1, 4), (96, 32, 4, 2)])
def test_other_shapes_attention_parity(amd, oracle, dim, group, gqa, bits):
    """Shapes beyond head_dim 128 / G 32 / GQA <= 8. head_dim 64, 128, 192 and 256 stay on the
    matrix-core path: one key group per chunk half when G >= 64 (a 64-channel key set uses
    four of the eight broadcast blocks), query heads in groups of 8 (4 above head_dim 128)
    with a short last group, and at head_dims other than 128 only the fully packed chunks
    there, the rest on the generic splits in the same launch. head_dim 96 stays on the
    generic splits alone. Many splits, against the oracle and f64 dense attention on the
    dequantized cache."""
    batch, heads = 2, 2
    seq = 2500 + 13 * bits
    rng = np.random.default_rng(dim + group + gqa + bits)
    k = rng.standard_normal(batch * heads * seq * dim).astype(np.float32)
    k.reshape(batch, heads, seq, dim)[:, :, :, 2] *= np.float32(10.0)
    v = rng.standard_normal(batch * heads * seq * dim).astype(np.float32)
    cfg = KiviConfig(bits, group, 2 * group if group >= 64 else 128)
    a = KiviCache(amd, cfg, batch, heads, dim)
    o = KiviCache(oracle, cfg, batch, heads, dim)
    a.append(k, v, seq)
    o.append(k, v, seq)
    q = rng.standard_normal(batch * heads * gqa * dim).astype(np.float32)
    scale = np.float32(1 / np.sqrt(dim))
    got = a.attention(q, heads * gqa, scale)
    assert_close(got, o.attention(q, heads * gqa, scale))
    kh, vh = a.dequantize()
    assert max_abs(got, dense_attend(kh, vh, q, batch, heads, heads * gqa, seq, dim, scale)) < 1e-4


@pytest.mark.parametrize("bits,gqa,batch,heads,seq", [
    (2, 5, 1, 2, 200), (4, 6, 2, 1, 777), (8, 7, 1, 2, 2600), (4, 8, 1, 3, 4321), (2, 8, 2, 2, 9000),
    (8, 12, 1, 2, 5000), (4, 16, 1, 1, 3000), (2, 16, 2, 2, 9000), (8, 16, 1, 2, 5000), (4, 32, 1, 1, 6000),
    (2, 48, 1, 1, 2000), (4, 16, 1, 3, 70), (2, 16, 1, 1, 200)])
def test_eight_head_units_attention_parity(amd, oracle, bits, gqa, batch, heads, seq):
    """Units of five or more query heads at head_dim 128 and G = 32 take the 16x16x32
    kernels for their packed chunks: eight-head groups for GQA 5..8 and 12, sixteen-head groups
    for GQA 16, 32, 48. Padded heads (GQA 5..7), a short last head group (GQA 12), waves that
    own fewer chunks than they hold or none (seq 200: one packed chunk for four waves; seq 70:
    one packed chunk), the window chunks in the same launch (head groups of eight there), and
    many splits; against the oracle and f64 dense attention on the dequantized cache."""
    dim = 128
    rng = np.random.default_rng(4200 + 10 * gqa + bits)
    k = rng.standard_normal(batch * heads * seq * dim).astype(np.float32)
    k.reshape(batch, heads, seq, dim)[:, :, :, 7] *= np.float32(10.0)
    v = rng.standard_normal(batch * heads * seq * dim).astype(np.float32)
    cfg = KiviConfig(bits, 32, 128)
    a = KiviCache(amd, cfg, batch, heads, dim)
    o = KiviCache(oracle, cfg, batch, heads, dim)
    a.append(k, v, seq)
    o.append(k, v, seq)
    q = rng.standard_normal(batch * heads * gqa * dim).astype(np.float32)
    scale = np.float32(1 / np.sqrt(dim))
    got = a.attention(q, heads * gqa, scale)
    assert_close(got, o.attention(q, heads * gqa, scale))
    kh, vh = a.dequantize()
    assert max_abs(got, dense_attend(kh, vh, q, batch, heads, heads * gqa, seq, dim, scale)) < 1e-4


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("gqa", [1, 4, 8])
def test_attention_parity_long(amd, oracle, bits, gqa):
    """Several thousand tokens, many splits, every GQA grouping the configs use."""
    batch, heads, dim, seq = 1, 2, 128, 3000 + 17 * bits
    rng = np.random.default_rng(bits * 10 + gqa)
    k = rng.standard_normal(batch * heads * seq * dim).astype(np.float32)
    v = rng.standard_normal(batch * heads * seq * dim).astype(np.float32)
    cfg = KiviConfig(bits, 32, 128)
    a = KiviCache(amd, cfg, batch, heads, dim)
    o = KiviCache(oracle, cfg, batch, heads, dim)
    a.append(k, v, seq)
    o.append(k, v, seq)
    assert_streams_equal(a, o)
    q = rng.standard_normal(batch * heads * gqa * dim).astype(np.float32)
    scale = np.float32(1 / np.sqrt(128))
    got = a.attention(q, heads * gqa, scale)
    assert_close(got, o.attention(q, heads * gqa, scale))
    kh, vh = a.dequantize()
    assert max_abs(got, dense_attend(kh, vh, q, batch, heads, heads * gqa, seq, dim, scale)) < 1e-4


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_infinite_inputs_codes_parity(amd, oracle, bits):
    """Rows with +inf and -inf entries (the reference tests hold none): a group spanning an
    infinity gets scale inf and codes 0 (the quotient is 0 or NaN, and NaN casts to 0), the
    others quantize as usual. Packed streams bit-exact through bulk and decode appends, and
    the standalone quantize of both axes. NaN inputs are not covered: the reference's min/max
    skip a NaN, the kernels' compare-select reductions need not."""
    batch, heads, dim, total = 1, 2, 128, 300
    rng = np.random.default_rng(500 + bits)
    keys = rng.standard_normal((batch, heads, total, dim)).astype(np.float32)
    values = rng.standard_normal((batch, heads, total, dim)).astype(np.float32)
    for arr in (keys, values):
        flat = arr.reshape(-1)
        idx = rng.choice(flat.size, 24, replace=False)
        flat[idx[:12]] = np.inf
        flat[idx[12:]] = -np.inf
    cfg = KiviConfig(bits, 32, 128)
    a = KiviCache(amd, cfg, batch, heads, dim)
    o = KiviCache(oracle, cfg, batch, heads, dim)
    off = 0
    for n in [200, 1, 1, 98]:
        k = keys[:, :, off:off + n].copy()
        v = values[:, :, off:off + n].copy()
        a.append(k, v, n)
        o.append(k, v, n)
        off += n
    assert_streams_equal(a, o)
    k288 = np.ascontiguousarray(keys[:, :, :288])  # whole groups of tokens
    for fn, data, tokens in ((kivi.quantize_per_channel, k288, 288),
                             (kivi.quantize_per_token, values, total)):
        qa = fn(amd, data, batch, heads, tokens, dim, bits, 32)
        qo = fn(oracle, data, batch, heads, tokens, dim, bits, 32)
        assert np.array_equal(qa.codes(), qo.codes())
        assert np.array_equal(qa.scale_zero().view(np.uint32), qo.scale_zero().view(np.uint32))


@pytest.mark.parametrize("bits,gqa,batch,heads,seq", [(2, 4, 4, 8, 50000), (8, 8, 4, 8, 40000)])
def test_attention_parity_many_rounds(amd, oracle, bits, gqa, batch, heads, seq):
    """Caches whose packed splits need more workgroups than the chip holds at once (32 units
    of 40-50k tokens: 800 / 640 packed workgroups of 8 chunks per wave), so the launch runs in
    more than one round of workgroups."""
    dim = 128
    rng = np.random.default_rng(bits * 100 + gqa)
    n = batch * heads * seq * dim
    k = rng.standard_normal(n, dtype=np.float32)
    v = rng.standard_normal(n, dtype=np.float32)
    cfg = KiviConfig(bits, 32, 128)
    a = KiviCache(amd, cfg, batch, heads, dim)
    o = KiviCache(oracle, cfg, batch, heads, dim)
    a.append(k, v, seq)
    o.append(k, v, seq)
    del k, v
    q = rng.standard_normal(batch * heads * gqa * dim, dtype=np.float32)
    scale = np.float32(1 / np.sqrt(128))
    assert_close(a.attention(q, heads * gqa, scale), o.attention(q, heads * gqa, scale))


@pytest.mark.parametrize("bits,qh,seq", [(2, 8, 65536), (4, 2, 98304)])
def test_merge_several_rounds_parity(amd, oracle, bits, qh, seq):
    """head_dim 32 (generic splits only) over 65-98k tokens of one unit: hundreds of splits per
    output row, so each of the merge's four waves per row takes its splits in several rounds
    of its larger batch (src/attention.rs:18-105 over one long head)."""
    dim, heads = 32, 1
    rng = np.random.default_rng(bits * 7 + qh)
    n = heads * seq * dim
    k = rng.standard_normal(n, dtype=np.float32)
    k.reshape(heads, seq, dim)[:, :, 5] *= np.float32(10.0)
    v = rng.standard_normal(n, dtype=np.float32)
    cfg = KiviConfig(bits, 32, 128)
    a, o = KiviCache(amd, cfg, 1, heads, dim), KiviCache(oracle, cfg, 1, heads, dim)
    a.append(k, v, seq)
    o.append(k, v, seq)
    q = (rng.standard_normal(qh * dim) * 2).astype(np.float32)
    scale = np.float32(1 / np.sqrt(dim))
    assert_close(a.attention(q, qh, scale), o.attention(q, qh, scale))


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("dim,group", [(64, 16), (64, 64), (128, 16), (256, 16), (256, 32),
                                       (256, 64)])
def test_quantize_lane_layouts_parity(amd, oracle, bits, dim, group):
    """The quantize kernels' lane layouts (channels per lane 1/2/4, lanes per channel group
    4..64, lanes per code word) through bulk, odd-sized and single-token appends."""
    batch, heads, residual = 1, 3, 2 * group if group >= 64 else 64
    chunks = [200, 1, 37, 130, 1, 64]
    total = sum(chunks)
    rng = np.random.default_rng(dim * 10 + group + bits)
    keys = rng.standard_normal((batch, heads, total, dim)).astype(np.float32)
    keys[:, :, :, 1] *= 10
    values = rng.standard_normal((batch, heads, total, dim)).astype(np.float32)
    cfg = KiviConfig(bits, group, residual)
    a = KiviCache(amd, cfg, batch, heads, dim)
    o = KiviCache(oracle, cfg, batch, heads, dim)
    off = 0
    for n in chunks:
        k = keys[:, :, off:off + n].copy()
        v = values[:, :, off:off + n].copy()
        a.append(k, v, n)
        o.append(k, v, n)
        off += n
        assert_streams_equal(a, o)


def near_ties(levels, group, rows, cols, per_row, rng):
    """[rows][cols] f32 whose quotients (x - min) / scale sit within a few ulps of a
    half-integer: each group of `group` elements (along a row when per_row, down a column
    otherwise) holds its min m and m + levels*s, so scale = s, and the rest are
    m + (n + 0.5 + e)*s for random n < levels, with e = k*2^-21 (k in [-4, 4]) or, for half
    of them, e = +-(2^-12 + j*2^-17) (j in [0, 16]): just outside the band the kernels divide in."""
    m = rng.uniform(-3, 3, size=(rows, cols)).astype(np.float32)
    s = rng.uniform(0.01, 2, size=(rows, cols)).astype(np.float32)
    if per_row:  # one (m, s) per group of columns
        m = np.repeat(m[:, ::group], group, axis=1)[:, :cols]
        s = np.repeat(s[:, ::group], group, axis=1)[:, :cols]
    else:
        m = np.repeat(m[::group], group, axis=0)[:rows]
        s = np.repeat(s[::group], group, axis=0)[:rows]
    n = rng.integers(0, levels, size=(rows, cols)).astype(np.float64)
    e = rng.integers(-4, 5, size=(rows, cols)) * 2.0 ** -21
    edge = (2.0 ** -12 + rng.integers(0, 17, size=(rows, cols)) * 2.0 ** -17) * rng.choice([-1.0, 1.0], size=(rows, cols))
    e = np.where(rng.random((rows, cols)) < 0.5, e, edge)
    x = (m.astype(np.float64) + (n + 0.5 + e) * s.astype(np.float64)).astype(np.float32)
    lo = m
    hi = (m.astype(np.float64) + levels * s.astype(np.float64)).astype(np.float32)
    if per_row:
        x[:, 0::group], x[:, 1::group] = lo[:, 0::group], hi[:, 1::group]
    else:
        x[0::group], x[1::group] = lo[0::group], hi[1::group]
    return x


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_near_tie_codes_parity(amd, oracle, bits):
    """Codes whose quotients lie within a few ulps of a rounding boundary (the quantize
    kernels' reciprocal fast path hands those to an exact division): bit-exact streams through
    bulk appends, decode appends and value-window evictions."""
    batch, heads, dim, group, residual = 2, 2, 128, 32, 128
    chunks = [300, 1, 37, 64, 1, 1, 200]
    total = sum(chunks)
    levels = (1 << bits) - 1
    rng = np.random.default_rng(77 + bits)
    keys = near_ties(levels, group, batch * heads * total, dim, False, rng)  # groups of tokens
    values = near_ties(levels, group, batch * heads * total, dim, True, rng)  # groups of channels
    keys = keys.reshape(batch, heads, total, dim)
    values = values.reshape(batch, heads, total, dim)
    cfg = KiviConfig(bits, group, residual)
    a = KiviCache(amd, cfg, batch, heads, dim)
    o = KiviCache(oracle, cfg, batch, heads, dim)
    off = 0
    for n in chunks:
        k = keys[:, :, off:off + n].copy()
        v = values[:, :, off:off + n].copy()
        a.append(k, v, n)
        o.append(k, v, n)
        off += n
        assert_streams_equal(a, o)


@pytest.mark.parametrize("bits,group", [(2, 32), (4, 32), (8, 32), (2, 16), (4, 64), (8, 4)])
@pytest.mark.parametrize("dim", [32, 128])
def test_standalone_quantize_parity(amd, oracle, bits, group, dim):
    if dim % group:
        pytest.skip("head_dim not a multiple of group")
    batch, heads, tokens = 2, 3, 4 * group
    data = fill(batch * heads * tokens * dim, bits * 7 + group)
    data[::97] = 0.5  # half ties
    for fn in (kivi.quantize_per_channel, kivi.quantize_per_token):
        qa = fn(amd, data, batch, heads, tokens, dim, bits, group)
        qo = fn(oracle, data, batch, heads, tokens, dim, bits, group)
        assert np.array_equal(qa.codes(), qo.codes())
        assert np.array_equal(qa.scale_zero().view(np.uint32), qo.scale_zero().view(np.uint32))
        assert np.array_equal(qa.pytorch_codes(), qo.pytorch_codes())
        assert np.array_equal(qa.dequantize().view(np.uint32), qo.dequantize().view(np.uint32))
        assert (qa.code_bytes(), qa.metadata_bytes()) == (qo.code_bytes(), qo.metadata_bytes())


def test_session_parity(amd, oracle):
    """Prefix + private suffixes (src/prefix.rs:173-289) against the oracle."""
    batch, heads, dim, doc, qh = 2, 2, 64, 700, 8
    rng = np.random.default_rng(7)
    k = rng.standard_normal(batch * heads * doc * dim).astype(np.float32)
    v = rng.standard_normal(batch * heads * doc * dim).astype(np.float32)
    cfg = KiviConfig(2, 32, 128)
    ca, co = KiviCache(amd, cfg, batch, heads, dim), KiviCache(oracle, cfg, batch, heads, dim)
    ca.append(k, v, doc)
    co.append(k, v, doc)
    pa, po = ca.share_prefix(), co.share_prefix()
    assert pa.prefix_bytes() == po.prefix_bytes()
    sa, so = pa.session(), po.session()
    for n in (3, 1, 40):
        sk = rng.standard_normal(batch * heads * n * dim).astype(np.float32)
        sv = rng.standard_normal(batch * heads * n * dim).astype(np.float32)
        sa.append(sk, sv, n)
        so.append(sk, sv, n)
        q = rng.standard_normal(batch * qh * dim).astype(np.float32)
        assert_close(sa.attention(q, qh, 0.125), so.attention(q, qh, 0.125))
    # batched entry point == per-session calls
    sessions_a = [pa.session() for _ in range(5)]
    for i, s in enumerate(sessions_a):
        n = 1 + 7 * i
        s.append(rng.standard_normal(batch * heads * n * dim).astype(np.float32),
                 rng.standard_normal(batch * heads * n * dim).astype(np.float32), n)
    qs = rng.standard_normal(5 * batch * qh * dim).astype(np.float32)
    batched = kivi.sessions_attention(amd, sessions_a, qs, qh, 0.125)
    per = np.concatenate([s.attention(qs[i * batch * qh * dim:(i + 1) * batch * qh * dim], qh, 0.125)
                          for i, s in enumerate(sessions_a)])
    assert_close(batched, per)


@pytest.mark.parametrize("bits,batch,qh,n_sess,doc", [
    (2, 1, 32, 6, 1000), (2, 1, 64, 4, 1024), (4, 1, 32, 4, 777), (8, 1, 64, 3, 1000),
    (2, 1, 32, 70, 640), (4, 2, 32, 40, 300), (8, 1, 32, 2, 500)])
def test_batched_sessions_kernel_parity(amd, oracle, bits, batch, qh, n_sess, doc):
    """Batched RagSession attention on the packed-chunk path (head_dim 128, G=32): one launch
    per 64 sessions over the shared prefix (70 sessions = two launch groups), in the GEMM form
    (sessions x heads >= 16 rows) and the per-session form, suffixes of 0 to 130 tokens, every
    session against the oracle's RagSession::attention (src/prefix.rs:223-289)."""
    heads, dim = 8, 128
    rng = np.random.default_rng(bits * 1000 + n_sess)
    k = rng.standard_normal(batch * heads * doc * dim).astype(np.float32)
    k.reshape(batch, heads, doc, dim)[:, :, :, 3] *= np.float32(10.0)
    v = rng.standard_normal(batch * heads * doc * dim).astype(np.float32)
    cfg = KiviConfig(bits, 32, 128)
    ca, co = KiviCache(amd, cfg, batch, heads, dim), KiviCache(oracle, cfg, batch, heads, dim)
    ca.append(k, v, doc)
    co.append(k, v, doc)
    pa, po = ca.share_prefix(), co.share_prefix()
    sa = [pa.session() for _ in range(n_sess)]
    so = [po.session() for _ in range(n_sess)]
    lens = [(0, 1, 63, 64, 97, 130)[i % 6] for i in range(n_sess)]
    for a, o, n in zip(sa, so, lens):
        if n:
            sk = rng.standard_normal(batch * heads * n * dim).astype(np.float32)
            sv = rng.standard_normal(batch * heads * n * dim).astype(np.float32)
            a.append(sk, sv, n)
            o.append(sk, sv, n)
    per = batch * qh * dim
    qs = rng.standard_normal(n_sess * per).astype(np.float32)
    scale = np.float32(1 / np.sqrt(128))
    got = kivi.sessions_attention(amd, sa, qs, qh, scale)
    for i, o in enumerate(so):
        assert_close(got[i * per:(i + 1) * per], o.attention(qs[i * per:(i + 1) * per], qh, scale),
                     f"session {i} (suffix {lens[i]})")
    # the same call again (persistent workspace reused), then a smaller batch
    again = kivi.sessions_attention(amd, sa, qs, qh, scale)
    assert np.array_equal(again.view(np.uint32), got.view(np.uint32))
    few = kivi.sessions_attention(amd, sa[1:3], qs[per:3 * per], qh, scale)
    assert_close(few, got[per:3 * per], "sessions 1..2 alone")


def test_session_suffix_run_boundaries_parity(amd, oracle):
    """GEMM form (8 sessions x 4 heads = 32 rows) with suffixes on both sides of the
    128-token runs of the suffix kernel, grown by several appends so that each session's
    device capacity exceeds its length (src/prefix.rs:173-223, 228-289)."""
    batch, heads, qh, dim, doc = 1, 8, 32, 128, 700
    rng = np.random.default_rng(4242)
    k = rng.standard_normal(batch * heads * doc * dim).astype(np.float32)
    v = rng.standard_normal(batch * heads * doc * dim).astype(np.float32)
    cfg = KiviConfig(2, 32, 128)
    ca, co = KiviCache(amd, cfg, batch, heads, dim), KiviCache(oracle, cfg, batch, heads, dim)
    ca.append(k, v, doc)
    co.append(k, v, doc)
    pa, po = ca.share_prefix(), co.share_prefix()
    lens = (127, 128, 129, 255, 256, 257, 383, 2)
    sa, so = [pa.session() for _ in lens], [po.session() for _ in lens]
    for a, o, n in zip(sa, so, lens):
        done = 0
        for piece in (n // 3, n - n // 3 - 1, 1):
            if piece:
                sk = (rng.standard_normal(batch * heads * piece * dim) * 1.5).astype(np.float32)
                sv = rng.standard_normal(batch * heads * piece * dim).astype(np.float32)
                a.append(sk, sv, piece)
                o.append(sk, sv, piece)
                done += piece
        assert done == n
    per = batch * qh * dim
    qs = rng.standard_normal(len(lens) * per).astype(np.float32)
    scale = np.float32(1 / np.sqrt(dim))
    got = kivi.sessions_attention(amd, sa, qs, qh, scale)
    for i, o in enumerate(so):
        assert_close(got[i * per:(i + 1) * per], o.attention(qs[i * per:(i + 1) * per], qh, scale),
                     f"session {i} (suffix {lens[i]})")


@pytest.mark.parametrize("bits", [2, 8])
def test_shared_prefix_rising_logits_parity(amd, oracle, bits):
    """Batched sessions in the GEMM form over a prefix whose logits climb by ~2 (base 2) per
    64-token chunk in a 12-chunk sawtooth: each workgroup's ~10-chunk range sees its running
    maximum rise past the lazy-rescale slack several times, so the rescale of the accumulated
    rows runs repeatedly. Every session against the oracle's RagSession::attention
    (src/prefix.rs:223-289)."""
    heads, dim, qh, doc, n_sess = 8, 128, 32, 20480, 4
    rng = np.random.default_rng(4100 + bits)
    u = np.where(rng.random((heads, dim)) < 0.5, -1.0, 1.0).astype(np.float32)  # q.u = 128
    ramp = (0.1227 * ((np.arange(doc) // 64) % 12)).astype(np.float32)            # ~2 per chunk
    k = rng.standard_normal((1, heads, doc, dim)).astype(np.float32)
    k += ramp[None, None, :, None] * u[None, :, None, :]
    v = rng.standard_normal((1, heads, doc, dim)).astype(np.float32)
    cfg = KiviConfig(bits, 32, 128)
    ca, co = KiviCache(amd, cfg, 1, heads, dim), KiviCache(oracle, cfg, 1, heads, dim)
    ca.append(k.reshape(-1), v.reshape(-1), doc)
    co.append(k.reshape(-1), v.reshape(-1), doc)
    pa, po = ca.share_prefix(), co.share_prefix()
    sa = [pa.session() for _ in range(n_sess)]
    so = [po.session() for _ in range(n_sess)]
    lens = (0, 64, 97, 1)
    for a, o, n in zip(sa, so, lens):
        if n:
            sk = rng.standard_normal(heads * n * dim).astype(np.float32)
            sv = rng.standard_normal(heads * n * dim).astype(np.float32)
            a.append(sk, sv, n)
            o.append(sk, sv, n)
    # queries along each KV head's ramp direction, plus noise
    q = np.repeat(u, qh // heads, axis=0)[None] + 0.3 * rng.standard_normal((n_sess, qh, dim))
    qs = q.astype(np.float32).reshape(-1)
    per = qh * dim
    scale = np.float32(1 / np.sqrt(128))
    got = kivi.sessions_attention(amd, sa, qs, qh, scale)
    for i, o in enumerate(so):
        assert_close(got[i * per:(i + 1) * per], o.attention(qs[i * per:(i + 1) * per], qh, scale),
                     f"session {i} (suffix {lens[i]})")


def test_runtime_decode_parity(amd, oracle):
    """512-step streaming decode shape of config 1, scaled down: prefill, then decode steps
    crossing key flushes and window evictions, compared with the oracle each step."""
    heads, qh, dim, prefill, steps = 8, 32, 128, 640, 140
    cfg = KiviConfig(2, 32, 128)
    rng = np.random.default_rng(11)
    ra, ro = RuntimeKv(amd, cfg, 1, heads, dim), RuntimeKv(oracle, cfg, 1, heads, dim)
    k = rng.standard_normal(heads * prefill * dim).astype(np.float32)
    v = rng.standard_normal(heads * prefill * dim).astype(np.float32)
    ra.prefill(k, v, prefill)
    ro.prefill(k, v, prefill)
    scale = np.float32(1 / np.sqrt(128))
    for step in range(steps):
        kk = rng.standard_normal(heads * dim).astype(np.float32)
        vv = rng.standard_normal(heads * dim).astype(np.float32)
        q = rng.standard_normal(qh * dim).astype(np.float32)
        assert_close(ra.decode(kk, vv, q, qh, scale), ro.decode(kk, vv, q, qh, scale), f"step {step}")
    assert_streams_equal(ra.cache(), ro.cache())


@pytest.mark.parametrize("bits,residual,gqa,group,dim", [
    (2, 64, 4, 32, 128), (4, 64, 8, 32, 128), (8, 128, 4, 32, 128), (2, 128, 1, 32, 128), (2, 128, 4, 64, 128),
    (4, 128, 16, 128, 128), (4, 64, 4, 32, 64), (2, 128, 8, 64, 256), (2, 128, 8, 32, 128), (8, 64, 6, 32, 128),
    (2, 64, 5, 32, 128)])
def test_runtime_decode_device_parity(amd, oracle, bits, residual, gqa, group, dim):
    """RuntimeKv::decode on device pointers, which runs append + attention in one attention
    launch (the token the window evicts quantized inside it) for head_dim 128, G = 32 and GQA
    <= 8 (GQA 5-8 on the eight-head kernel) when no key flush is due, and as an append then an
    attention launch otherwise (GQA 16, G 64/128, head_dim 64/256 here): bit for bit equal to
    a cache taking append_device then attention_device (tests/runtime.rs:13-52), and within
    tolerance of the oracle's decode, streams bit-exact, across evictions and flushes."""
    heads, prefill, steps = 2, 3 * residual + 17, 2 * residual + 5
    qh = heads * gqa
    cfg = KiviConfig(bits, group, residual)
    rng = np.random.default_rng(300 + bits + residual + gqa + group + dim)
    k = rng.standard_normal(heads * prefill * dim).astype(np.float32)
    v = rng.standard_normal(heads * prefill * dim).astype(np.float32)
    k.reshape(heads, prefill, dim)[:, :, 5] *= 10
    ra, ro = RuntimeKv(amd, cfg, 1, heads, dim), RuntimeKv(oracle, cfg, 1, heads, dim)
    cb = KiviCache(amd, cfg, 1, heads, dim)
    for target in (ra.cache(), ro.cache(), cb):
        target.append(k, v, prefill)
    scale = np.float32(1 / np.sqrt(dim))
    mem = DeviceArrays()
    n_kv, n_q = heads * dim, qh * dim
    out_a, out_b = mem.empty(n_q), mem.empty(n_q)
    for step in range(steps):
        kk = rng.standard_normal(n_kv).astype(np.float32)
        vv = rng.standard_normal(n_kv).astype(np.float32)
        q = rng.standard_normal(n_q).astype(np.float32)
        dk, dv, dq = mem.upload(kk), mem.upload(vv), mem.upload(q)
        ra.decode_device(dk, n_kv, dv, n_kv, dq, n_q, qh, scale, out_a, n_q)
        cb.append_device(dk, n_kv, dv, n_kv, 1)
        cb.attention_device(dq, n_q, qh, scale, out_b, n_q)
        got = mem.download(out_a, n_q)
        assert np.array_equal(got.view(np.uint32), mem.download(out_b, n_q).view(np.uint32)), f"step {step}"
        assert_close(got, ro.decode(kk, vv, q, qh, scale), f"step {step}")
        if step % 16 == 0 or step == steps - 1:
            assert_same_state(ra.cache(), ro.cache())
            assert_streams_equal(ra.cache(), ro.cache())
            assert_streams_equal(cb, ro.cache())
    mem.free()


@pytest.mark.parametrize("bits,gqa", [(2, 4), (8, 4), (4, 8), (8, 7)])
def test_decode_device_zero_minima_parity(amd, oracle, bits, gqa):
    """RuntimeKv::decode on device pointers with window rows whose channel groups have zero
    minima and zeros of both signs: the token each step evicts is quantized inside the
    attention launch (the 4x4x4 kernel at GQA 4, the eight-head kernel at GQA 7-8), and its
    stored zeros must be each group's first zero, as the oracle's decode stores them
    (src/quant.rs:356)."""
    heads, dim, residual = 2, 128, 64
    prefill, steps = 3 * residual + 17, 2 * residual + 5
    qh = heads * gqa
    cfg = KiviConfig(bits, 32, residual)
    rng = np.random.default_rng(900 + bits)
    total = prefill + steps
    keys = rng.standard_normal((1, heads, total, dim)).astype(np.float32)
    values = signed_zero_rows(rng, (1, heads, total, dim))
    ra, ro = RuntimeKv(amd, cfg, 1, heads, dim), RuntimeKv(oracle, cfg, 1, heads, dim)
    for r in (ra, ro):
        r.prefill(np.ascontiguousarray(keys[:, :, :prefill]), np.ascontiguousarray(values[:, :, :prefill]), prefill)
    scale = np.float32(1 / np.sqrt(dim))
    mem = DeviceArrays()
    n_kv, n_q = heads * dim, qh * dim
    out = mem.empty(n_q)
    for step in range(steps):
        t = prefill + step
        kk = np.ascontiguousarray(keys[:, :, t]).reshape(-1)
        vv = np.ascontiguousarray(values[:, :, t]).reshape(-1)
        q = rng.standard_normal(n_q).astype(np.float32)
        ra.decode_device(mem.upload(kk), n_kv, mem.upload(vv), n_kv, mem.upload(q), n_q, qh, scale, out, n_q)
        assert_close(mem.download(out, n_q), ro.decode(kk, vv, q, qh, scale), f"step {step}")
    assert_streams_equal(ra.cache(), ro.cache())
    vq = ra.cache().quantized_value_tokens()
    want = reference_minimum(values.reshape(heads, total, dim)[:, :vq].reshape(heads, vq, dim // 32, 32), axis=3)
    got = ra.cache().export_streams()[3].reshape(heads, vq, dim // 32, 2)[..., 1]
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    mem.free()


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("dim,group", [(64, 16), (64, 32), (64, 64), (128, 16), (128, 64),
                                       (256, 16), (256, 32), (256, 64), (96, 32)])
def test_standalone_codec_lane_layouts_parity(amd, oracle, bits, dim, group):
    """quantize_per_channel / quantize_per_token on the wave forms (head_dim 64/128/256: 1, 2
    or 4 channels per lane) and the general kernels (head_dim 96, 4 channels per lane with
    G=64): several units, many groups, and for values a row count that leaves a partial
    16-row slab. Codes, (scale, zero), pytorch order and dequantize bit-exact."""
    if group * bits % 32:
        pytest.skip("invalid group for bits")
    rng = np.random.default_rng(dim * 7 + group + bits)
    batch, heads = 2, 3
    for fn, tokens in ((kivi.quantize_per_channel, 9 * group), (kivi.quantize_per_token, 37)):
        data = rng.standard_normal((batch, heads, tokens, dim)).astype(np.float32)
        data[:, :, :, 5] *= np.float32(10.0)
        flat = data.reshape(-1)
        qa = fn(amd, flat, batch, heads, tokens, dim, bits, group)
        qo = fn(oracle, flat, batch, heads, tokens, dim, bits, group)
        assert np.array_equal(qa.codes(), qo.codes()), fn.__name__
        assert np.array_equal(qa.scale_zero().view(np.uint32), qo.scale_zero().view(np.uint32)), fn.__name__
        assert np.array_equal(qa.pytorch_codes(), qo.pytorch_codes()), fn.__name__
        assert np.array_equal(qa.dequantize().view(np.uint32), qo.dequantize().view(np.uint32)), fn.__name__
