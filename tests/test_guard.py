"""QualityGuard tests: reference tests/guard.rs (all six), run on the oracle and, with
``-m gpu``, on the HIP library; then pins of the oracle's guard pieces against closed forms and
a float64 brute force, and GPU-vs-oracle parity of whole guarded streams (same checks, same
upgrades, bit-identical rebuilt streams, cosines within 1e-5)."""

import ctypes as C

import numpy as np
import pytest

from kivi import KiviConfig, KiviError, QualityGuard, QualityPolicy, QualityUpgrade
from helpers import dense_attend, slice_tokens


def signal(seq, dim, seed):
    """tests/guard.rs:3-11: u32 LCG, top 24 bits mapped to [-1, 1)."""
    out = np.empty(seq * dim, dtype=np.float32)
    state = seed & 0xFFFFFFFF
    for i in range(seq * dim):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(np.float32(state >> 8) / np.float32(1 << 24)) * np.float32(2.0) - np.float32(1.0)
    return out


def guard(backend, policy, threshold, max_bits, max_residual):
    """tests/guard.rs:13-25."""
    return QualityGuard.try_new(backend, KiviConfig.try_new(backend, 2, 32, 32), 1, 1, 32,
                                threshold, policy, max_bits, max_residual)


# ------------------------------------------------------------------ tests/guard.rs


def test_no_flush_means_no_check(backend):
    """tests/guard.rs:27-37."""
    g = guard(backend, QualityPolicy.RaiseBits, 0.99, 8, 128)
    checks = g.append(signal(16, 32, 1), signal(16, 32, 2), 16, signal(1, 32, 3), 1, 0.5)
    assert checks == []
    assert g.config().bits == 2
    assert g.sequence_length() == 16


def test_passing_cosine_does_not_upgrade(backend):
    """tests/guard.rs:39-52."""
    g = guard(backend, QualityPolicy.RaiseBits, 0.0, 8, 128)
    checks = g.append(signal(32, 32, 4), signal(32, 32, 5), 32, signal(1, 32, 6), 1, 0.5)
    assert len(checks) == 1
    assert checks[0].upgrades == []
    assert checks[0].cosine_before == checks[0].cosine
    assert checks[0].sequence_tokens == 32
    assert g.config().bits == 2
    assert g.config().residual_length == 32


def test_raise_bits_stops_at_the_ceiling(backend):
    """tests/guard.rs:54-70."""
    g = guard(backend, QualityPolicy.RaiseBits, 1.1, 4, 128)
    checks = g.append(signal(32, 32, 7), signal(32, 32, 8), 32, signal(1, 32, 9), 1, 0.5)
    assert checks[0].upgrades == [QualityUpgrade.bits(2, 4)]
    assert g.config().bits == 4
    assert g.config().residual_length == 32
    assert g.cache().sequence_length() == 32
    assert checks[0].cosine < 1.1


def test_lengthen_residual_puts_the_flushed_block_back_in_fp32(backend):
    """tests/guard.rs:72-90."""
    g = guard(backend, QualityPolicy.LengthenResidual, 1.1, 8, 64)
    checks = g.append(signal(32, 32, 10), signal(32, 32, 11), 32, signal(1, 32, 12), 1, 0.25)
    assert checks[0].upgrades == [QualityUpgrade.residual(32, 64)]
    assert g.config().residual_length == 64
    assert g.config().bits == 2
    c = g.cache()
    assert c.quantized_key_tokens() == 0
    assert c.quantized_value_tokens() == 0
    assert c.key_residual_len() == 32
    assert c.value_residual_len() == 32
    assert checks[0].cosine > 0.999, checks[0].cosine


def test_one_append_checks_every_key_flush(backend):
    """tests/guard.rs:92-103."""
    g = guard(backend, QualityPolicy.RaiseBits, 0.0, 8, 128)
    checks = g.append(signal(64, 32, 13), signal(64, 32, 14), 64, signal(1, 32, 15), 1, 0.5)
    assert len(checks) == 2
    assert checks[0].sequence_tokens == 32
    assert checks[1].sequence_tokens == 64
    assert all(c.upgrades == [] for c in checks)


def test_four_bit_rebuild_beats_the_two_bit_flush(backend):
    """tests/guard.rs:105-124."""
    keys, values, query = signal(32, 32, 21), signal(32, 32, 22), signal(1, 32, 23)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(32.0)))
    loose = guard(backend, QualityPolicy.RaiseBits, 0.0, 8, 128)
    before = loose.append(keys, values, 32, query, 1, scale)[0].cosine_before
    g = guard(backend, QualityPolicy.RaiseBits, 0.995, 8, 128)
    checks = g.append(keys, values, 32, query, 1, scale)
    assert before < 0.995, f"2-bit cosine {before} did not miss 0.995"
    assert checks[0].upgrades == [QualityUpgrade.bits(2, 4)]
    assert checks[0].cosine > before
    assert checks[0].cosine >= 0.995, checks[0].cosine
    assert g.config().bits == 4


# ------------------------------------------------------------------ checks and errors


def test_append_checks_shapes_in_reference_order(backend):
    """src/guard.rs:99-128: keys, values, query heads, query length."""
    g = QualityGuard(backend, KiviConfig.try_new(backend, 2, 32, 32), 1, 2, 32, 0.5,
                     QualityPolicy.RaiseBits, 8, 128)
    k = signal(4, 64, 1)
    q = signal(2, 32, 2)
    with pytest.raises(KiviError) as e:
        g.append(k[:-1], k[:-1], 4, q[:1], 3, 0.5)
    assert (e.value.variant, e.value.payload) == ("Shape", {"expected": 256, "actual": 255})
    with pytest.raises(KiviError) as e:
        g.append(k, k[:-1], 4, q[:1], 3, 0.5)
    assert (e.value.variant, e.value.payload) == ("Shape", {"expected": 256, "actual": 255})
    with pytest.raises(KiviError) as e:
        g.append(k, k, 4, q[:1], 3, 0.5)
    assert (e.value.variant, e.value.payload) == ("QueryHeads", {"num_q_heads": 3, "num_kv_heads": 2})
    with pytest.raises(KiviError) as e:
        g.append(k, k, 4, q[:1], 2, 0.5)
    assert (e.value.variant, e.value.payload) == ("Shape", {"expected": 64, "actual": 1})
    assert g.sequence_length() == 0


def test_zero_token_append_makes_no_check(backend):
    g = guard(backend, QualityPolicy.RaiseBits, 1.1, 8, 128)
    assert g.append([], [], 0, signal(1, 32, 1), 1, 0.5) == []
    assert g.sequence_length() == 0 and g.config().bits == 2


# ------------------------------------------------------------------ oracle pins


def test_residual_ladder_saturates_at_the_ceiling(oracle):
    """next_residual (src/guard.rs:274-289): 32 -> 64 -> 96 when the ceiling is 96 (doubling
    would overshoot, the ceiling is a multiple of the group), then no further step; with a
    ceiling of 80 the capped step 64 -> 80 is not a multiple of 32 and is refused."""
    g = QualityGuard(oracle, KiviConfig.try_new(oracle, 2, 32, 32), 1, 1, 32, 1.1,
                     QualityPolicy.LengthenResidual, 8, 96)
    checks = g.append(signal(32, 32, 1), signal(32, 32, 2), 32, signal(1, 32, 3), 1, 0.5)
    assert checks[0].upgrades == [QualityUpgrade.residual(32, 64), QualityUpgrade.residual(64, 96)]
    assert g.config().residual_length == 96
    g = QualityGuard(oracle, KiviConfig.try_new(oracle, 2, 32, 32), 1, 1, 32, 1.1,
                     QualityPolicy.LengthenResidual, 8, 80)
    checks = g.append(signal(32, 32, 1), signal(32, 32, 2), 32, signal(1, 32, 3), 1, 0.5)
    assert checks[0].upgrades == [QualityUpgrade.residual(32, 64)]


def test_bit_ladder_walks_two_four_eight(oracle):
    """next_bits (src/guard.rs:261-272): 2 -> 4 -> 8 under an unreachable threshold, one
    rebuild per step, every later flush starts at 8 bits and proposes nothing."""
    g = guard(oracle, QualityPolicy.RaiseBits, 1.1, 8, 128)
    checks = g.append(signal(64, 32, 4), signal(64, 32, 5), 64, signal(1, 32, 6), 1, 0.5)
    assert checks[0].upgrades == [QualityUpgrade.bits(2, 4), QualityUpgrade.bits(4, 8)]
    assert checks[1].upgrades == []
    assert g.config().bits == 8
    assert checks[1].cosine_before == checks[1].cosine


def _fp32_attention(oracle, q, k, v, b, kv, qh, seq, d, scale):
    f = oracle.lib.kivi_oracle_fp32_attention
    f.restype = None
    fp = C.POINTER(C.c_float)
    f.argtypes = [fp, fp, fp] + [C.c_size_t] * 5 + [C.c_float, fp]
    out = np.zeros(b * qh * d, np.float32)
    f(q.ctypes.data_as(fp), k.ctypes.data_as(fp), v.ctypes.data_as(fp), b, kv, qh, seq, d,
      C.c_float(scale), out.ctypes.data_as(fp))
    return out


@pytest.mark.parametrize("b,kv,qh,seq,d", [(1, 1, 1, 1, 32), (2, 2, 4, 45, 32), (1, 2, 8, 130, 64)])
def test_oracle_fp32_attention_matches_float64(oracle, b, kv, qh, seq, d):
    """fp32_attention (src/guard.rs:344-385) against a float64 softmax brute force; with one
    token the output is that token's value row exactly."""
    rng = np.random.default_rng(seq)
    k = rng.standard_normal(b * kv * seq * d).astype(np.float32)
    v = rng.standard_normal(b * kv * seq * d).astype(np.float32)
    q = rng.standard_normal(b * qh * d).astype(np.float32)
    got = _fp32_attention(oracle, q, k, v, b, kv, qh, seq, d, 0.3)
    ref = dense_attend(k, v, q, b, kv, qh, seq, d, 0.3)
    assert np.max(np.abs(got - ref)) < 2e-5
    if seq == 1:
        group = qh // kv
        rows = v.reshape(b, kv, d)
        expect = np.stack([rows[:, h // group] for h in range(qh)], axis=1).reshape(-1)
        assert np.array_equal(got, expect)


def test_oracle_cosine_is_one_on_an_all_fp32_cache(oracle):
    """Cosine invariant: a rebuild into a residual window that covers the whole tape holds fp32
    rows only, so it scores cosine ~1 (the reference's own lengthen-residual test asserts
    > 0.999); a lower cosine marks a wrong term. The next flush of the 64-token window is at the
    ceiling: no proposal, cosine_before == cosine, and quantized rows score below 1."""
    g = QualityGuard(oracle, KiviConfig.try_new(oracle, 2, 32, 32), 1, 1, 32, 1.1,
                     QualityPolicy.LengthenResidual, 8, 64)
    checks = g.append(signal(64, 32, 7), signal(64, 32, 8), 64, signal(1, 32, 9), 1, 0.3)
    assert len(checks) == 2
    assert checks[0].upgrades == [QualityUpgrade.residual(32, 64)]
    assert checks[0].cosine > 0.99999
    assert checks[0].cosine_before < checks[0].cosine
    assert checks[1].sequence_tokens == 64
    assert checks[1].upgrades == []
    assert checks[1].cosine_before == checks[1].cosine < 0.9999


# ------------------------------------------------------------------ GPU parity


def _stream(backend, cfg, batch, heads, dim, qh, threshold, policy, max_bits, max_residual,
            appends, seed):
    g = QualityGuard(backend, KiviConfig.try_new(backend, *cfg), batch, heads, dim, threshold,
                     policy, max_bits, max_residual)
    total = sum(appends)
    rng = np.random.default_rng(seed)
    keys = (rng.standard_normal(batch * heads * total * dim) * 1.3).astype(np.float32)
    values = rng.standard_normal(batch * heads * total * dim).astype(np.float32)
    query = rng.standard_normal(batch * qh * dim).astype(np.float32)
    out, off = [], 0
    for n in appends:
        out.append(g.append(slice_tokens(keys, batch, heads, total, dim, off, n),
                            slice_tokens(values, batch, heads, total, dim, off, n), n, query, qh,
                            dim ** -0.5))
        off += n
    return g, out


GUARD_CASES = [
    # (bits, group, residual), batch, heads, dim, qh, threshold, policy, max_bits, max_residual, appends
    ((2, 32, 32), 2, 2, 128, 8, 0.9995, QualityPolicy.RaiseBits, 8, 128, [40, 200, 1, 23, 64]),
    ((2, 32, 32), 1, 2, 128, 4, 0.9999, QualityPolicy.LengthenResidual, 8, 256, [96, 33, 320]),
    ((4, 32, 64), 1, 1, 64, 2, 0.99999, QualityPolicy.RaiseBits, 8, 128, [64, 64, 7]),
    ((2, 16, 32), 2, 1, 32, 1, 0.0, QualityPolicy.RaiseBits, 8, 128, [330]),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(GUARD_CASES)))
def test_guard_parity_with_oracle(amd, oracle, case):
    """Whole guarded streams on the HIP library and the oracle: the same flush checks (token
    counts, upgrade lists), cosines within 1e-5 (the HIP fp32 attention sums in another order),
    and after the last append the same config and bit-identical packed streams."""
    args = GUARD_CASES[case]
    ga, ca = _stream(amd, *args, seed=100 + case)
    go, co = _stream(oracle, *args, seed=100 + case)
    assert [len(x) for x in ca] == [len(x) for x in co]
    for xa, xo in zip(ca, co):
        for a, o in zip(xa, xo):
            assert a.sequence_tokens == o.sequence_tokens
            assert a.upgrades == o.upgrades
            assert abs(a.cosine_before - o.cosine_before) < 1e-5
            assert abs(a.cosine - o.cosine) < 1e-5
    assert ga.config() == go.config()
    assert ga.sequence_length() == go.sequence_length()
    for x, y in zip(ga.cache().export_streams(), go.cache().export_streams()):
        assert np.array_equal(x, y)
