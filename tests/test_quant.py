"""Standalone codec tests: reference tests/quant.rs and examples/pytorch_golden.rs.

Run on the oracle (pins the C++ restatement to the reference's own expectations) and, with
``-m gpu``, on the HIP library through the C ABI (codes and params must be bit-exact).
"""

import numpy as np
import pytest

import kivi
from kivi import KiviError, quantize_per_channel, quantize_per_token
from helpers import fill, reference_minimum, signed_zero_rows


def pattern_token():
    """tests/quant.rs:3-11."""
    values = np.ones(16, dtype=np.float32)
    values[0:5] = [0.0, 0.5, 1.5, 2.5, 3.0]
    return values


def packed_word(start):
    """examples/pytorch_golden.rs:98-105: 16 2-bit codes (start+i)%4, first in the low bits."""
    w = 0
    for i in range(16):
        w |= ((start + i) % 4) << (2 * i)
    return w


def golden_fixture(seq=64, dim=32):
    """examples/pytorch_golden.rs:69-77: element [t, d] = (t + d) % 4."""
    t = np.arange(seq)[:, None]
    d = np.arange(dim)[None, :]
    return ((t + d) % 4).astype(np.float32).reshape(-1)


def test_pytorch_pack_matches_the_published_word_layout(backend):
    """tests/quant.rs:13-41 and the full golden vectors of examples/pytorch_golden.rs:79-96."""
    dim, seq = 32, 64
    data = golden_fixture(seq, dim)
    keys = quantize_per_channel(backend, data, 1, 1, seq, dim, 2, 32)
    values = quantize_per_token(backend, data, 1, 1, seq, dim, 2, 32)
    key_codes = keys.pytorch_codes()
    value_codes = values.pytorch_codes()
    assert key_codes.size == (seq // 16) * dim
    assert value_codes.size == seq * (dim // 16)
    rows = key_codes.reshape(-1, dim)
    assert (rows == rows[0]).all()
    assert key_codes[0] == 0xE4E4E4E4
    assert key_codes[1] == 0x39393939
    assert key_codes[2] == 0x4E4E4E4E
    assert key_codes[3] == 0x93939393
    assert value_codes[0] == 0xE4E4E4E4
    assert value_codes[1] == 0xE4E4E4E4
    assert value_codes[2] == 0x39393939
    # full golden vectors (pytorch_golden.rs:81-96)
    golden_k = np.tile(np.array([packed_word(d % 4) for d in range(dim)], np.uint32), seq // 16)
    golden_v = np.repeat(np.array([packed_word(t % 4) for t in range(seq)], np.uint32), 2)
    np.testing.assert_array_equal(key_codes, golden_k)
    np.testing.assert_array_equal(value_codes, golden_v)
    assert (keys.scale_zero().reshape(-1, 2) == [1.0, 0.0]).all()
    assert (values.scale_zero().reshape(-1, 2) == [1.0, 0.0]).all()
    np.testing.assert_array_equal(keys.dequantize(), data)
    np.testing.assert_array_equal(values.dequantize(), data)


def test_four_bit_half_ties_round_to_even(backend):
    """tests/quant.rs:43-66."""
    data = np.zeros(16, dtype=np.float32)
    data[[0, 1, 2, 3, 4, 5, 6, 15]] = [0.0, 0.5, 1.5, 2.5, 3.5, 1.2, 1.6, 15.0]
    out = quantize_per_token(backend, data, 1, 1, 1, 16, 4, 16).dequantize()
    assert list(out[[0, 1, 2, 3, 4, 5, 6, 15]]) == [0.0, 0.0, 2.0, 2.0, 4.0, 1.0, 2.0, 15.0]


def test_per_token_half_even_and_endpoints(backend):
    """tests/quant.rs:68-77."""
    out = quantize_per_token(backend, pattern_token(), 1, 1, 1, 16, 2, 16).dequantize()
    expect = [0.0, 0.0, 2.0, 2.0, 3.0] + [1.0] * 11
    np.testing.assert_array_equal(out, np.array(expect, np.float32))


def test_per_channel_half_even_on_one_channel(backend):
    """tests/quant.rs:79-97."""
    data = np.zeros(16 * 16, dtype=np.float32)
    data[0::16] = pattern_token()
    out = quantize_per_channel(backend, data, 1, 1, 16, 16, 2, 16).dequantize()
    expect_ch0 = [0.0, 0.0, 2.0, 2.0, 3.0] + [1.0] * 11
    o = out.reshape(16, 16)
    np.testing.assert_array_equal(o[:, 0], np.array(expect_ch0, np.float32))
    assert (o[:, 1:] == 0.0).all()


def test_negative_channel_endpoints_are_exact(backend):
    """tests/quant.rs:99-116."""
    data = np.zeros(16 * 16, dtype=np.float32)
    for t, v in enumerate([-2.0, -1.0, 0.0, 1.0]):
        data[t * 16] = v
    out = quantize_per_channel(backend, data, 1, 1, 16, 16, 2, 16).dequantize()
    assert (out[0], out[16], out[32], out[48]) == (-2.0, -1.0, 0.0, 1.0)
    assert all(out[t * 16] == 0.0 for t in range(4, 16))


def test_constant_group_reconstructs_exactly(backend):
    """tests/quant.rs:118-129."""
    data = np.full(2 * 3 * 32 * 16, 0.25, dtype=np.float32)
    out = quantize_per_channel(backend, data, 2, 3, 32, 16, 4, 16).dequantize()
    np.testing.assert_array_equal(out, data)
    out = quantize_per_token(backend, data, 2, 3, 32, 16, 4, 16).dequantize()
    np.testing.assert_array_equal(out, data)


def _lcg_range(n, seed, lo, width):
    out = np.empty(n, np.float32)
    s = seed
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(np.float32(s >> 8) / np.float32(1 << 24)) * np.float32(width) + np.float32(lo)
    return out


def test_reconstruction_error_is_bounded_by_half_scale(backend):
    """tests/quant.rs:131-168."""
    tokens, dim, bits, group = 32, 32, 2, 32
    data = _lcg_range(tokens * dim, 0x12345678, -3.0, 6.0)
    levels = (1 << bits) - 1
    out = quantize_per_channel(backend, data, 1, 1, tokens, dim, bits, group).dequantize()
    x = data.reshape(tokens, dim)
    o = out.reshape(tokens, dim)
    for d in range(dim):
        mn, mx = x[:, d].min(), x[:, d].max()
        scale = 0.0 if mx == mn else np.float32(mx - mn) / np.float32(levels)
        err = np.abs(o[:, d] - x[:, d])
        assert (err <= scale * 0.5 + 1e-4).all(), (d, err.max(), scale)


def test_per_channel_keys_keep_quiet_channels(backend):
    """tests/quant.rs:170-211."""
    tokens, dim = 32, 32
    data = np.zeros((tokens, dim), np.float32)
    data[:, 0] = 100.0
    data[:, 1:] = (np.arange(1, dim, dtype=np.float32) / np.float32(dim))[None, :]
    data = data.reshape(-1)
    pc = quantize_per_channel(backend, data, 1, 1, tokens, dim, 2, 32).dequantize()
    pt = quantize_per_token(backend, data, 1, 1, tokens, dim, 2, 32).dequantize()

    def mae(xs):
        a = xs.reshape(tokens, dim)[:, 1:]
        b = data.reshape(tokens, dim)[:, 1:]
        return float(np.abs(a - b).mean())

    assert mae(pc) < 1e-5
    assert mae(pt) > 0.2


def test_rejects_bad_shapes(backend):
    """tests/quant.rs:213-228, with the payloads and messages of src/error.rs:47-95."""
    data = np.zeros(8, np.float32)
    with pytest.raises(KiviError) as e:
        quantize_per_channel(backend, data, 1, 1, 8, 1, 3, 32)
    assert e.value.variant == "InvalidBits" and e.value.payload == {"bits": 3}
    assert e.value.message == "bit width 3 is not supported; use 2, 4, or 8"
    with pytest.raises(KiviError) as e:
        quantize_per_channel(backend, data, 1, 1, 7, 1, 2, 32)
    assert e.value.variant == "TokenGroup"
    assert e.value.message == ("token count 7 must be a positive multiple of group_size 32 "
                               "for per-channel quantization")
    with pytest.raises(KiviError) as e:
        quantize_per_token(backend, data, 1, 1, 4, 2, 2, 32)
    assert e.value.variant == "HeadDim"
    assert e.value.message == "head_dim 2 must be a positive multiple of group_size 32"


def test_check_quant_args_order(backend):
    """check_quant_args order (src/quant.rs:235-273): bits/group, batch, heads, head_dim,
    then the token/channel group rule, then the data length."""
    d = np.zeros(4, np.float32)
    with pytest.raises(KiviError) as e:
        quantize_per_channel(backend, d, 0, 0, 0, 0, 2, 24)
    assert e.value.variant == "MisalignedGroup"
    assert e.value.payload == {"group_size": 24, "bits": 2}
    assert e.value.message == "group_size 24 * bits 2 must be a multiple of 32"
    with pytest.raises(KiviError) as e:
        quantize_per_channel(backend, d, 0, 0, 0, 0, 2, 32)
    assert e.value.variant == "ZeroDimension" and e.value.payload["name"] == "batch"
    assert e.value.message == "batch must be greater than zero"
    with pytest.raises(KiviError) as e:
        quantize_per_token(backend, d, 1, 0, 0, 0, 2, 32)
    assert e.value.payload["name"] == "heads"
    with pytest.raises(KiviError) as e:
        quantize_per_token(backend, d, 1, 1, 0, 0, 2, 32)
    assert e.value.payload["name"] == "head_dim"
    with pytest.raises(KiviError) as e:
        quantize_per_channel(backend, d, 1, 1, 0, 32, 2, 32)
    assert e.value.variant == "TokenGroup" and e.value.payload == {"tokens": 0, "group_size": 32}
    with pytest.raises(KiviError) as e:
        quantize_per_channel(backend, d, 1, 1, 32, 32, 2, 32)
    assert e.value.variant == "Shape"
    assert e.value.payload == {"expected": 1024, "actual": 4}
    assert e.value.message == "expected 1024 elements, got 4"


def test_accessors_and_byte_counts(backend):
    """QuantizedTensor accessors (src/quant.rs:46-69) against the packing arithmetic."""
    for bits in (2, 4, 8):
        b, h, t, dim, g = 2, 3, 64, 32, 32
        data = fill(b * h * t * dim, 5 + bits)
        k = quantize_per_channel(backend, data, b, h, t, dim, bits, g)
        v = quantize_per_token(backend, data, b, h, t, dim, bits, g)
        assert k.axis() == kivi.PER_CHANNEL and v.axis() == kivi.PER_TOKEN
        assert k.bits() == bits and k.group_size() == g and k.num_tokens() == t
        assert k.code_bytes() == b * h * t * dim * bits // 8 == v.code_bytes()
        assert k.metadata_bytes() == b * h * (t // g) * dim * 8
        assert v.metadata_bytes() == b * h * t * (dim // g) * 8


def unpack_stream_keys(codes, params, tokens, dim, bits, group):
    """Decode one key PackedStream by its documented layout (src/quant.rs:307-323): word
    (g*D + d)*ipc + w holds tokens w*32/b.. of channel d, first token in the low bits."""
    ipc = group * bits // 32
    per = 32 // bits
    mask = (1 << bits) - 1
    out = np.zeros((tokens, dim), np.int64)
    for g in range(tokens // group):
        for d in range(dim):
            for w in range(ipc):
                word = int(codes[(g * dim + d) * ipc + w])
                for i in range(per):
                    out[g * group + w * per + i, d] = (word >> (bits * i)) & mask
    return out


def brute_force_codes_per_channel(data, tokens, dim, bits, group):
    """Codes from the definition (src/quant.rs:1-10): per channel and token group,
    scale = (max-min)/levels, code = round-half-even((x-min)/scale) clamped; f32 arithmetic."""
    levels = np.float32((1 << bits) - 1)
    x = data.reshape(tokens, dim)
    codes = np.zeros((tokens, dim), np.int64)
    params = []
    for g in range(tokens // group):
        blk = x[g * group:(g + 1) * group]
        mn = blk.min(axis=0)
        mx = blk.max(axis=0)
        span = (mx - mn).astype(np.float32)
        scale = np.where(span == 0, np.float32(0), span / levels).astype(np.float32)
        for d in range(dim):
            params += [scale[d], mn[d]]
            if scale[d] == 0:
                continue
            q = ((blk[:, d] - mn[d]) / scale[d]).astype(np.float32)
            codes[g * group:(g + 1) * group, d] = np.clip(np.rint(q), 0, levels).astype(np.int64)
    return codes, np.array(params, np.float32)


@pytest.mark.parametrize("bits,group", [(2, 32), (4, 32), (8, 32), (2, 16), (4, 8), (8, 4)])
def test_per_channel_codes_match_definition(backend, bits, group):
    """Keys: stream layout decoded independently and compared with a numpy brute force
    (np.rint is IEEE round-half-even, equal to src/quant.rs:475-485 on x >= 0)."""
    tokens, dim = 4 * group, 32
    data = fill(tokens * dim, 77 + bits)
    data[5] = np.float32(0.5)  # a few exact ties on an integer grid stay in the data
    q = quantize_per_channel(backend, data, 1, 1, tokens, dim, bits, group)
    got = unpack_stream_keys(q.codes(), q.scale_zero(), tokens, dim, bits, group)
    want, params = brute_force_codes_per_channel(data, tokens, dim, bits, group)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(q.scale_zero(), params)


@pytest.mark.parametrize("bits,group", [(2, 32), (4, 32), (8, 32), (2, 16), (4, 16), (8, 8)])
def test_per_token_codes_match_definition(backend, bits, group):
    """Values: word (t*(D/G) + cg)*ipg + w holds channels of token t (src/quant.rs:349-375)."""
    tokens, dim = 9, 64
    data = fill(tokens * dim, 91 + bits)
    q = quantize_per_token(backend, data, 1, 1, tokens, dim, bits, group)
    levels = np.float32((1 << bits) - 1)
    per = 32 // bits
    mask = (1 << bits) - 1
    ipg = group * bits // 32
    n_ch = dim // group
    codes = q.codes()
    sz = q.scale_zero()
    x = data.reshape(tokens, dim)
    for t in range(tokens):
        for cg in range(n_ch):
            grp = x[t, cg * group:(cg + 1) * group]
            mn, mx = grp.min(), grp.max()
            span = np.float32(mx - mn)
            scale = np.float32(0) if span == 0 else np.float32(span / levels)
            assert sz[2 * (t * n_ch + cg)] == scale and sz[2 * (t * n_ch + cg) + 1] == mn
            want = (np.zeros(group, np.int64) if scale == 0 else
                    np.clip(np.rint(((grp - mn) / scale).astype(np.float32)), 0, levels))
            for i in range(group):
                w = int(codes[(t * n_ch + cg) * ipg + i // per])
                assert (w >> (bits * (i % per))) & mask == int(want[i])


@pytest.mark.parametrize("bits,group,dim", [(2, 32, 128), (4, 16, 64), (8, 32, 96), (2, 64, 128)])
def test_zero_minimum_keeps_the_first_zeros_sign(backend, bits, group, dim):
    """Groups whose minimum is zero, with +0 and -0 both present: the stored zero is the
    group's first zero in element order, tokens for keys and channels for values (the
    reference's f32::min on x86-64 keeps the running minimum on ties). Compared bit for bit,
    so the sign of every zero counts; the codes still follow the definition."""
    rng = np.random.default_rng(bits * 100 + group + dim)
    batch, heads, tokens = 1, 2, 4 * group
    xk = signed_zero_rows(rng, (batch, heads, tokens, dim))
    xk[:, 1, :, 1::3] = -np.abs(xk[:, 1, :, 1::3]) - 0.5  # negative minima in some channels
    qk = quantize_per_channel(backend, xk.reshape(-1), batch, heads, tokens, dim, bits, group)
    keys = xk.reshape(batch * heads, tokens // group, group, dim)
    want = reference_minimum(keys, axis=2)  # [units][groups][D]
    got = qk.scale_zero().reshape(batch * heads, tokens // group, dim, 2)[..., 1]
    assert (want == 0).sum() > 0 and np.signbit(want[want == 0]).any() and not np.signbit(want[want == 0]).all()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    xv = signed_zero_rows(rng, (batch, heads, tokens, dim))
    xv[:, 1, ::5, 3] = -1.5  # negative minima in some tokens
    qv = quantize_per_token(backend, xv.reshape(-1), batch, heads, tokens, dim, bits, group)
    vals = xv.reshape(batch * heads, tokens, dim // group, group)
    want = reference_minimum(vals, axis=3)  # [units][tokens][D/G]
    got = qv.scale_zero().reshape(batch * heads, tokens, dim // group, 2)[..., 1]
    assert np.signbit(want[want == 0]).any() and not np.signbit(want[want == 0]).all()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
