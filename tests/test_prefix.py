"""Shared prefix / RAG session tests: reference tests/prefix.rs and examples/shared_prefix.rs.
Run on the oracle and, with ``-m gpu``, on the HIP library."""

import numpy as np
import pytest

import kivi
from kivi import KiviCache, KiviConfig, KiviError
from helpers import concat_head_major, dense_attend, document, max_abs, slice_tokens


def cfg(backend):
    """tests/prefix.rs:3-5."""
    return KiviConfig.try_new(backend, 2, 32, 64)


def share(backend, config, batch, heads, dim, seq):
    """tests/prefix.rs:229-241."""
    keys, values = document(batch, heads, seq, dim)
    cache = KiviCache(backend, config, batch, heads, dim)
    cache.append(keys, values, seq)
    return cache, cache.share_prefix()


def test_sessions_share_one_prefix_allocation(backend):
    """tests/prefix.rs:97-110."""
    cache, prefix = share(backend, cfg(backend), 1, 2, 64, 160)
    again = prefix.clone()
    assert prefix.shares_allocation_with(again)
    assert prefix.prefix_tokens() == 160
    a, b = prefix.session(), prefix.session()
    assert a.prefix().shares_allocation_with(b.prefix())
    assert a.prefix().prefix_bytes() == prefix.prefix_bytes()
    other = cache.share_prefix()
    assert not other.shares_allocation_with(prefix)


def test_empty_question_matches_cache_attention(backend):
    """tests/prefix.rs:112-124: bit-exact."""
    cache, prefix = share(backend, cfg(backend), 1, 2, 64, 96)
    session = prefix.session()
    query = np.full(4 * 64, 0.3, np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(64))
    np.testing.assert_array_equal(session.attention(query, 4, scale),
                                  cache.attention(query, 4, scale))


def test_question_attention_matches_dense_prefix_plus_suffix(backend):
    """tests/prefix.rs:126-160."""
    batch, heads, dim, doc, qlen = 1, 2, 64, 96, 4
    cache, prefix = share(backend, cfg(backend), batch, heads, dim, doc)
    dk, dv = cache.dequantize()
    session = prefix.session()
    qk, qv = document(batch, heads, qlen, dim)
    session.append(qk, qv, qlen)
    full_k = concat_head_major(dk, qk, batch, heads, doc, qlen, dim)
    full_v = concat_head_major(dv, qv, batch, heads, doc, qlen, dim)
    query = np.full(batch * heads * dim, 0.15, np.float32)
    got = session.attention(query, heads, 0.25)
    expect = dense_attend(full_k, full_v, query, batch, heads, heads, doc + qlen, dim, 0.25)
    assert max_abs(got, expect) < 1e-4


def test_one_session_does_not_see_another_question(backend):
    """tests/prefix.rs:162-181."""
    cache, prefix = share(backend, cfg(backend), 1, 1, 64, 80)
    a, b = prefix.session(), prefix.session()
    ak, av = document(1, 1, 3, 64)
    a.append(ak, av, 3)
    assert b.question_tokens() == 0
    assert b.sequence_length() == 80
    query = np.full(64, 0.2, np.float32)
    only_prefix = prefix.session().attention(query, 1, 1.0)
    from_b = b.attention(query, 1, 1.0)
    np.testing.assert_array_equal(only_prefix, from_b)
    assert not np.array_equal(a.attention(query, 1, 1.0), from_b)


def test_shared_footprint_counts_the_document_once(backend):
    """tests/prefix.rs:183-199."""
    cache, prefix = share(backend, cfg(backend), 1, 2, 64, 256)
    foot = prefix.footprint(8, 8)
    assert foot.prefix_bytes == cache.memory().compressed_bytes()
    assert foot.shared_total_bytes < foot.fp16_all_users_bytes
    assert foot.savings_vs_fp16() > 1.0
    one, two = prefix.footprint(1, 8), prefix.footprint(2, 8)
    assert two.prefix_bytes == one.prefix_bytes
    assert two.question_bytes == 2 * one.question_bytes


def test_bad_question_shape_is_rejected(backend):
    """tests/prefix.rs:201-217."""
    cache = KiviCache(backend, cfg(backend), 1, 1, 64)
    cache.append(np.full(64, 0.1, np.float32), np.full(64, 0.2, np.float32), 1)
    session = cache.share_prefix().session()
    with pytest.raises(KiviError) as e:
        session.append(np.zeros(8), np.zeros(8), 1)
    assert e.value.variant == "Shape"
    with pytest.raises(KiviError) as e:
        session.append(np.zeros(64), np.zeros(8), 1)
    assert e.value.payload == {"expected": 64, "actual": 8}
    with pytest.raises(KiviError) as e:  # shapes are checked before the seq_len == 0 no-op
        session.append(np.zeros(3), np.zeros(0), 0)
    assert e.value.payload == {"expected": 0, "actual": 3}


def token_mean(values, batch, heads, seq, dim):
    """tests/prefix.rs:502-519."""
    v = np.asarray(values, np.float64).reshape(batch, heads, seq, dim)
    return v.mean(axis=2).reshape(-1)


def test_constant_keys_make_suffix_attention_the_value_mean(backend):
    """tests/prefix.rs:243-273."""
    batch, heads, dim, doc, qlen = 1, 2, 32, 96, 4
    config = KiviConfig.try_new(backend, 2, 32, 64)
    keys = np.zeros(batch * heads * doc * dim, np.float32)
    values = document(batch, heads, doc, dim)[1]
    cache = KiviCache(backend, config, batch, heads, dim)
    cache.append(keys, values, doc)
    assert cache.key_residual_len() == doc % 64
    assert cache.value_residual_len() == 64
    session = cache.share_prefix().session()
    qk = np.zeros(batch * heads * qlen * dim, np.float32)
    qv = document(batch, heads, qlen, dim)[1]
    session.append(qk, qv, qlen)
    dk, dv = cache.dequantize()
    assert (dk == 0.0).all()
    full_v = concat_head_major(dv, qv, batch, heads, doc, qlen, dim)
    expect = token_mean(full_v, batch, heads, doc + qlen, dim)
    got = session.attention(np.ones(batch * heads * dim, np.float32), heads, 3.5)
    assert max_abs(got, expect) < 1e-5


def test_four_bit_suffix_matches_dense_attention(backend):
    """tests/prefix.rs:275-307."""
    batch, heads, dim, doc, qlen = 1, 1, 64, 90, 6
    cache, prefix = share(backend, KiviConfig.try_new(backend, 4, 32, 64), batch, heads, dim, doc)
    assert cache.key_residual_len() == 26 and cache.value_residual_len() == 64
    dk, dv = cache.dequantize()
    session = prefix.session()
    qk, qv = document(batch, heads, qlen, dim)
    session.append(qk, qv, qlen)
    full_k = concat_head_major(dk, qk, batch, heads, doc, qlen, dim)
    full_v = concat_head_major(dv, qv, batch, heads, doc, qlen, dim)
    query = document(batch, heads, 1, dim)[0]
    scale = np.float32(1.0) / np.sqrt(np.float32(dim))
    got = session.attention(query, heads, scale)
    expect = dense_attend(full_k, full_v, query, batch, heads, heads, doc + qlen, dim, scale)
    assert max_abs(got, expect) < 1e-4


def test_grouped_query_batch_suffix_matches_dense_attention(backend):
    """tests/prefix.rs:309-340."""
    batch, kv, q_heads, dim, doc, qlen = 2, 2, 6, 32, 48, 3
    cache, prefix = share(backend, KiviConfig.try_new(backend, 2, 32, 32), batch, kv, dim, doc)
    dk, dv = cache.dequantize()
    session = prefix.session()
    qk, qv = document(batch, kv, qlen, dim)
    session.append(qk, qv, qlen)
    full_k = concat_head_major(dk, qk, batch, kv, doc, qlen, dim)
    full_v = concat_head_major(dv, qv, batch, kv, doc, qlen, dim)
    query = document(batch, q_heads, 1, dim)[0]
    got = session.attention(query, q_heads, 0.5)
    expect = dense_attend(full_k, full_v, query, batch, kv, q_heads, doc + qlen, dim, 0.5)
    assert max_abs(got, expect) < 1e-4


def test_chunked_question_append_matches_one_shot(backend):
    """tests/prefix.rs:342-366: bit-exact."""
    batch, heads, dim, doc = 2, 2, 32, 40
    _, prefix = share(backend, KiviConfig.try_new(backend, 2, 32, 32), batch, heads, dim, doc)
    qk, qv = document(batch, heads, 7, dim)
    chunked = prefix.session()
    chunked.append(slice_tokens(qk, batch, heads, 7, dim, 0, 2),
                   slice_tokens(qv, batch, heads, 7, dim, 0, 2), 2)
    chunked.append(slice_tokens(qk, batch, heads, 7, dim, 2, 5),
                   slice_tokens(qv, batch, heads, 7, dim, 2, 5), 5)
    once = prefix.session()
    once.append(qk, qv, 7)
    assert chunked.question_tokens() == 7
    assert chunked.sequence_length() == doc + 7
    query = np.full(batch * heads * dim, 0.4, np.float32)
    np.testing.assert_array_equal(chunked.attention(query, heads, 1.25),
                                  once.attention(query, heads, 1.25))


def test_matching_suffix_key_dominates_the_softmax(backend):
    """tests/prefix.rs:368-386."""
    dim, doc = 32, 40
    cache = KiviCache(backend, KiviConfig.try_new(backend, 2, 32, 32), 1, 1, dim)
    cache.append(np.full(doc * dim, 0.01, np.float32), np.zeros(doc * dim, np.float32), doc)
    session = cache.share_prefix().session()
    qv = np.full(dim, 5.0, np.float32)
    session.append(np.ones(dim, np.float32), qv, 1)
    got = session.attention(np.ones(dim, np.float32), 1, 20.0)
    assert max_abs(got, qv) < 1e-3


def test_question_only_session_matches_dense_attention(backend):
    """tests/prefix.rs:388-401."""
    cache = KiviCache(backend, cfg(backend), 1, 2, 64)
    prefix = cache.share_prefix()
    session = prefix.session()
    qk, qv = document(1, 2, 5, 64)
    session.append(qk, qv, 5)
    query = np.full(2 * 64, 0.2, np.float32)
    got = session.attention(query, 2, 0.7)
    expect = dense_attend(qk, qv, query, 1, 2, 2, 5, 64, 0.7)
    assert max_abs(got, expect) < 1e-5
    assert prefix.prefix_tokens() == 0 and prefix.prefix_bytes() == 0


def test_footprint_matches_the_byte_formula(backend):
    """tests/prefix.rs:403-428."""
    batch, heads, dim, doc, sessions, question = 2, 2, 32, 70, 3, 5
    cache, prefix = share(backend, KiviConfig.try_new(backend, 2, 32, 64), batch, heads, dim, doc)
    foot = prefix.footprint(sessions, question)
    elements = batch * heads * dim
    question_bytes = sessions * question * elements * 2 * 4
    fp16_per_user = 2 * (doc + question) * elements * 2
    assert foot.prefix_tokens == doc and foot.question_tokens == question
    assert foot.sessions == sessions
    assert foot.prefix_bytes == cache.memory().compressed_bytes()
    assert foot.question_bytes == question_bytes
    assert foot.shared_total_bytes == foot.prefix_bytes + question_bytes
    assert foot.fp16_per_user_bytes == fp16_per_user
    assert foot.fp16_all_users_bytes == sessions * fp16_per_user
    ratio = foot.fp16_all_users_bytes / foot.shared_total_bytes
    assert abs(foot.savings_vs_fp16() - ratio) < 1e-12


def test_empty_store_reports_unit_savings(backend):
    """tests/prefix.rs:430-439."""
    foot = KiviCache(backend, cfg(backend), 1, 1, 64).share_prefix().footprint(4, 0)
    assert (foot.prefix_bytes, foot.question_bytes, foot.shared_total_bytes,
            foot.fp16_all_users_bytes) == (0, 0, 0, 0)
    assert foot.savings_vs_fp16() == 1.0


def test_appending_a_question_leaves_the_prefix_unchanged(backend):
    """tests/prefix.rs:441-457."""
    cache, prefix = share(backend, cfg(backend), 1, 1, 64, 80)
    before_tokens, before_bytes = prefix.prefix_tokens(), prefix.prefix_bytes()
    query = np.full(64, 0.25, np.float32)
    before = prefix.session().attention(query, 1, 1.0)
    session = prefix.session()
    qk, qv = document(1, 1, 4, 64)
    session.append(qk, qv, 4)
    session.append([], [], 0)
    assert prefix.prefix_tokens() == before_tokens
    assert prefix.prefix_bytes() == before_bytes
    assert cache.sequence_length() == before_tokens
    np.testing.assert_array_equal(before, prefix.session().attention(query, 1, 1.0))


def test_prefix_is_a_frozen_copy(backend):
    """SharedPrefix::from_cache deep-copies (src/prefix.rs:74-92): later appends to the
    cache do not reach the prefix."""
    cache, prefix = share(backend, cfg(backend), 1, 1, 64, 80)
    query = np.full(64, 0.25, np.float32)
    before = prefix.session().attention(query, 1, 1.0)
    k, v = document(1, 1, 70, 64)
    cache.append(k, v, 70)
    np.testing.assert_array_equal(before, prefix.session().attention(query, 1, 1.0))
    assert prefix.prefix_tokens() == 80


def test_bad_query_shape_and_head_count_are_rejected(backend):
    """tests/prefix.rs:459-479."""
    _, prefix = share(backend, cfg(backend), 1, 2, 64, 32)
    session = prefix.session()
    with pytest.raises(KiviError) as e:
        session.attention(np.zeros(64), 3, 1.0)
    assert e.value.payload == {"num_q_heads": 3, "num_kv_heads": 2}
    with pytest.raises(KiviError) as e:
        session.attention(np.zeros(8), 2, 1.0)
    assert e.value.payload == {"expected": 128, "actual": 8}


def test_shared_prefix_example(backend):
    """examples/shared_prefix.rs:270-320: 16 users on one 512-token document."""
    dim, heads, doc_len, qlen, users = 64, 4, 512, 8, 16
    config = KiviConfig.try_new(backend, 2, 32, 128)
    cache = KiviCache(backend, config, 1, heads, dim)
    n = heads * doc_len * dim
    i = np.arange(n)
    keys = (((i * 17) % 29).astype(np.float32) / np.float32(14.0)) - np.float32(0.5)
    values = (((i * 11) % 23).astype(np.float32) / np.float32(12.0)) - np.float32(0.3)
    cache.append(keys, values, doc_len)
    prefix = cache.share_prefix()
    sessions = [prefix.session() for _ in range(users)]
    for user, s in enumerate(sessions):
        qn = heads * qlen * dim
        s.append(np.full(qn, np.float32(0.05) * np.float32(user + 1), np.float32),
                 np.full(qn, np.float32(-0.02) * np.float32(user + 1), np.float32), qlen)
    query = np.full(heads * dim, 0.1, np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(dim))
    first = sessions[0].attention(query, heads, scale)
    second = sessions[1].attention(query, heads, scale)
    assert sessions[0].prefix().shares_allocation_with(sessions[1].prefix())
    assert not np.array_equal(first, second)
    foot = prefix.footprint(users, qlen)
    assert foot.savings_vs_fp16() > 1.0
    # The batched entry equals the per-session calls (bit-exact on the oracle, which
    # defines it as that loop; the HIP library is checked to tolerance in its own tests).
    queries = np.tile(query, users)
    batched = kivi.sessions_attention(backend, sessions, queries, heads, scale)
    per = np.concatenate([s.attention(query, heads, scale) for s in sessions])
    assert max_abs(batched, per) < 1e-5
