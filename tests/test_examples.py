"""Acceptance checks of the reference's examples that exercise the hot path, run on the oracle
and, under ``-m gpu``, on the HIP library:

* examples/config_ablation.rs:17-70: one 560-token sequence stored 2-/4-bit with R = 32 and
  R = 128; the narrower window is smaller, its attention cosine against fp32 attention stays
  within 0.02 of the wider one's, and its reconstruction errors are not smaller.
* examples/quality_guard.rs:10-56: a 64-token sequence fed to a raise-bits guard and a
  lengthen-residual guard (threshold 0.995, start 2-bit R=32): the first upgrades are
  Bits{2->4} and Residual{32->64}, and every check ends at the threshold.

Inputs are the examples' LCG (tests/attention.rs:3-11). The examples' fp32 attention and cosine
are restated in f32 numpy (sequential sums are not needed at these tolerances).
"""

import numpy as np

from kivi import KiviCache, KiviConfig, QualityGuard, QualityPolicy, QualityUpgrade
from helpers import fill


def fp32_attention(query, keys, values, heads, seq, dim, scale):
    """examples/config_ablation.rs:133-168: per head, softmax(q.k * scale) @ v in f32."""
    q = query.reshape(heads, dim)
    k = keys.reshape(heads, seq, dim)
    v = values.reshape(heads, seq, dim)
    out = np.empty((heads, dim), np.float32)
    for h in range(heads):
        logits = (k[h] @ q[h]).astype(np.float32) * np.float32(scale)
        w = np.exp(logits - logits.max()).astype(np.float32)
        out[h] = (w / w.sum()) @ v[h]
    return out.reshape(-1)


def cosine(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(a @ b / np.sqrt(a @ a) / np.sqrt(b @ b))


def test_config_ablation_narrow_window_costs_little(backend):
    """examples/config_ablation.rs:17-70 (the GiB column is the layer's compressed bytes times
    its 32 layers, the same ordering as the layer bytes compared here)."""
    heads, dim, seq, group = 8, 128, 560, 32
    keys, values, query = fill(heads * seq * dim, 11), fill(heads * seq * dim, 12), fill(heads * dim, 13)
    scale = np.float32(1.0) / np.sqrt(np.float32(dim))
    ref = fp32_attention(query, keys, values, heads, seq, dim, scale)
    rows = {}
    for bits, residual in ((2, 32), (2, 128), (4, 32), (4, 128)):
        cache = KiviCache(backend, KiviConfig.try_new(backend, bits, group, residual), 1, heads, dim)
        cache.append(keys, values, seq)
        k_hat, v_hat = cache.dequantize()
        got = cache.attention(query, heads, scale)
        rows[(bits, residual)] = {
            "k_mae": float(np.mean(np.abs(keys.astype(np.float64) - k_hat))),
            "v_mae": float(np.mean(np.abs(values.astype(np.float64) - v_hat))),
            "cosine": cosine(got, ref),
            "bytes": cache.memory().compressed_bytes(),
        }
    narrow, wide = rows[(2, 32)], rows[(2, 128)]
    assert narrow["bytes"] < wide["bytes"]
    assert abs(narrow["cosine"] - wide["cosine"]) < 0.02
    assert narrow["k_mae"] + 1e-5 >= wide["k_mae"]
    assert narrow["v_mae"] + 1e-5 >= wide["v_mae"]
    # 4-bit reconstructs more closely than 2-bit at either window
    for residual in (32, 128):
        assert rows[(4, residual)]["k_mae"] < rows[(2, residual)]["k_mae"]
        assert rows[(4, residual)]["v_mae"] < rows[(2, residual)]["v_mae"]


def test_quality_guard_example_upgrades(backend):
    """examples/quality_guard.rs:10-56."""
    dim, seq, threshold = 32, 64, 0.995
    keys, values, query = fill(seq * dim, 21), fill(seq * dim, 22), fill(dim, 23)
    scale = np.float32(1.0) / np.sqrt(np.float32(dim))
    runs = {}
    for policy in (QualityPolicy.RaiseBits, QualityPolicy.LengthenResidual):
        g = QualityGuard.try_new(backend, KiviConfig.try_new(backend, 2, 32, 32), 1, 1, dim, threshold,
                                 policy, 8, 128)
        runs[policy] = g.append(keys, values, seq, query, 1, scale)
    assert any(c.upgrades[:1] == [QualityUpgrade.bits(2, 4)] for c in runs[QualityPolicy.RaiseBits])
    assert any(c.upgrades[:1] == [QualityUpgrade.residual(32, 64)] for c in runs[QualityPolicy.LengthenResidual])
    for checks in runs.values():
        assert checks
        for c in checks:
            assert c.cosine + 1e-5 >= threshold, f"cosine {c.cosine} stayed under {threshold}"
