#!/usr/bin/env python3
"""Writes the golden fixtures of tests/golden/ (run from the repository root after building the
oracle: ``make -C oracle && python tests/golden/make_golden.py``).

* pytorch_golden.json — the reference's own golden vectors for PyTorch KIVI packing
  (examples/pytorch_golden.rs:16-105): element [t, d] = (t + d) % 4 for a [1, 1, 64, 32]
  tensor, 2-bit G=32. Expected key/value code words in pytorch_codes order, every
  (scale, zero) = (1, 0), and cache attention (R=32, query of ones, scale 1/sqrt(32)) equal
  to 1.5 on every channel with 64 packed key and 32 packed value tokens. The words are
  written out by the rule the example states (pytorch_golden.rs:79-105).
* seeded_streams.npz — frozen outputs of the oracle (the C++ restatement of the reference
  CPU path) on small seeded streaming schedules: inputs from the reference tests' LCG
  (tests/attention.rs:3-11, regenerated from the seed by kivi.lcg_fill), packed streams in
  PackedStream order, cache counters and the attention output. The GPU tests compare the HIP
  library with these arrays (codes and params bit-exact, attention within tolerance), so the
  comparison does not depend on the oracle build of the machine that runs them.
"""

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "kivi-cache-rs_amd"))

import kivi  # noqa: E402

HERE = Path(__file__).resolve().parent

# name: (bits, G, R, batch, heads, q_heads, D, schedule, seed)
CASES = {
    "b2_g16_d32": (2, 16, 32, 1, 2, 4, 32, [70, 1, 1, 1, 1, 1, 40], 101),
    "b4_g16_d32": (4, 16, 32, 1, 2, 4, 32, [70, 1, 1, 1, 1, 1, 40], 102),
    "b8_g16_d32": (8, 16, 32, 1, 2, 4, 32, [70, 1, 1, 1, 1, 1, 40], 103),
    # head_dim 128, G=32: the shape of the packed-chunk MFMA kernel (several 64-token chunks)
    "b2_g32_d128": (2, 32, 128, 1, 1, 4, 128, [250, 1, 1, 1, 7], 104),
    "b4_g32_d128": (4, 32, 128, 1, 1, 8, 128, [200, 3, 7], 105),
    "b8_g32_d128": (8, 32, 128, 1, 1, 4, 128, [160, 40, 1], 106),
}


def packed_word(start):
    """pytorch_golden.rs:97-105: 16 2-bit codes (start + i) % 4, first in the low bits."""
    w = 0
    for i in range(16):
        w |= ((start + i) % 4) << (2 * i)
    return w


def pytorch_golden():
    seq, dim = 64, 32
    key_codes = [packed_word(d % 4) for d in range(dim)] * (seq // 16)
    value_codes = [packed_word(t % 4) for t in range(seq) for _ in range(2)]
    return {
        "source": "examples/pytorch_golden.rs:16-105",
        "shape": [1, 1, seq, dim],
        "bits": 2,
        "group_size": 32,
        "residual_length": 32,
        "element_rule": "(t + d) % 4",
        "key_pytorch_codes": key_codes,
        "value_pytorch_codes": value_codes,
        "scale_zero": [1.0, 0.0],
        "attention_query": "ones",
        "attention_scale": "1/sqrt(32)",
        "attention_expected": 1.5,
        "quantized_key_tokens": 64,
        "quantized_value_tokens": 32,
    }


def case_inputs(case):
    bits, G, R, batch, heads, qh, dim, schedule, seed = case
    total = sum(schedule)
    n = batch * heads * total * dim
    keys = kivi.lcg_fill(n, seed)
    values = kivi.lcg_fill(n, seed + 1000)
    # one outlier channel per head (x10), as in the workloads' key distributions
    keys.reshape(batch, heads, total, dim)[:, :, :, 1] *= np.float32(10.0)
    query = kivi.lcg_fill(batch * qh * dim, seed + 2000)
    return keys, values, query


def run_case(backend, case):
    """Append the schedule, then return streams, counters and attention."""
    bits, G, R, batch, heads, qh, dim, schedule, seed = case
    total = sum(schedule)
    keys, values, query = case_inputs(case)
    cache = kivi.KiviCache(backend, kivi.KiviConfig(bits, G, R), batch, heads, dim)
    off = 0
    for n in schedule:
        k = keys.reshape(batch, heads, total, dim)[:, :, off:off + n].copy()
        v = values.reshape(batch, heads, total, dim)[:, :, off:off + n].copy()
        cache.append(k, v, n)
        off += n
    scale = np.float32(1.0) / np.sqrt(np.float32(dim))
    out = cache.attention(query, qh, scale)
    kc, kp, vc, vp = cache.export_streams()
    counters = np.array([cache.sequence_length(), cache.quantized_key_tokens(),
                         cache.quantized_value_tokens(), cache.key_residual_len(),
                         cache.value_residual_len()], dtype=np.int64)
    return {"key_codes": kc, "key_params": kp, "value_codes": vc, "value_params": vp,
            "counters": counters, "attention": out.astype(np.float32)}


def main():
    oracle = kivi.Backend.load(ROOT / "oracle" / "libkivi_oracle.so", "kivi_oracle_", device=False)
    (HERE / "pytorch_golden.json").write_text(json.dumps(pytorch_golden(), indent=1) + "\n")
    arrays = {}
    for name, case in CASES.items():
        for field, arr in run_case(oracle, case).items():
            arrays[f"{name}/{field}"] = arr
    np.savez_compressed(HERE / "seeded_streams.npz", **arrays)
    size = (HERE / "seeded_streams.npz").stat().st_size
    print(f"wrote pytorch_golden.json and seeded_streams.npz ({size} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
