#!/usr/bin/env python3
"""Decode-attention benchmark of the MI355X KIVI path (one JSON line on stdout).

Workload (the north-star target): batch 16, 32 query / 8 KV heads,
head_dim 128, 32768 cached tokens per sequence, 2-bit G=32 R=128, K ~ N(0,1) with 1% of key
channels (2 per KV head) scaled x10, V ~ N(0,1), fp32 inputs. A step is one decode attention
over all 16 sequences (the cache and the queries already resident in HBM); value = decode
tokens/s = 16 * steps / time. The cache build (prefill quantization) is timed once and
reported as quantize GB/s; the device-side export formats (packed streams in the reference
order, dense reconstruction) are timed once each after it (`exports`: GB/s and fraction of
8 TB/s). The CPU baseline is the oracle (C++ restatement of the
reference CPU path, 1 core) on one of the 16 sequences. Before the prefill and before the W
warm-up steps the GPU runs ~0.3 s of untimed work (device copies, then the step's own
kernels) so that its clocks have ramped up; `clock_warmup_calls` counts the second part.
Workloads whose cache is smaller than three times the 256 MB Infinity Cache (C3, C4) rotate
over identical cache copies between steps (`cache_copies`), so each step reads its cache from
HBM rather than from the previous step's cache lines; C0 and C1 are too small for that and
report `cache_resident: true`.

The roofline object is for the dominant kernel (the packed-chunk attention kernel): its
algorithmic bytes per launch (packed codes + (scale, zero) of the chunks it covers, plus the
query) over its mean launch duration, both measured live by the library's HIP-event launch
timing (kivi_timing_*) on the launch stream during the timed region. `traffic` is the HBM
bytes per launch of that kernel from rocprofv3 FETCH_SIZE + WRITE_SIZE runs, calibrated on a
plain copy kernel (--copy-calibration), as recorded in profiles/traffic.json; null when no
record matches this kernel, workload and byte count.

Other workloads (a line each, same contract): --config c0 (the reference's CPU-runnable case),
c1 (streaming decode: a step is RuntimeKv::decode = append one token + attention, after an
8192-token prefill; warmup + 2*steps <= 512; its line also times one QualityGuard check,
`guard`), c3_4 / c3_8 (4-/8-bit at 131072 tokens, GQA 8),
c4 (64 RagSessions over one 65536-token prefix, one batched call per step).

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--config c2] [--no-cpu]
                       [--copy-calibration MIB]
"""

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "kivi-cache-rs_amd"
sys.path.insert(0, str(PKG))

METRIC = "decode-attn tokens/s + effective HBM GB/s (% of 8 TB/s); quantize GB/s"
HBM_PEAK_GBPS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense f16 matrix-core peak

CONFIGS = {
    # name: (batch, kv_heads, q_heads, head_dim, seq, bits, G, R, description)
    "c0": (1, 8, 8, 128, 4097, 2, 32, 128, "config 0: batch 1, 8q/8kv heads, seq 4097 (4096 prefill + 1), 2-bit"),
    "c1": (1, 8, 32, 128, 8192, 2, 32, 128,
           "config 1: streaming decode, batch 1, 32q/8kv heads, head_dim 128, 2-bit G=32 R=128, "
           "8192-token prefill then RuntimeKv::decode steps (append 1 token + attention)"),
    "c2": (16, 8, 32, 128, 32768, 2, 32, 128,
           "config 2: batch 16, 32q/8kv heads, head_dim 128, 32768 cached tokens, 2-bit G=32 R=128"),
    "c3_4": (1, 8, 64, 128, 131072, 4, 32, 128, "config 3: batch 1, 64q/8kv heads, 131072 tokens, 4-bit"),
    "c3_8": (1, 8, 64, 128, 131072, 8, 32, 128, "config 3: batch 1, 64q/8kv heads, 131072 tokens, 8-bit"),
    "c4": (1, 8, 32, 128, 65536, 2, 32, 128,
           "config 4: one 65536-token 2-bit G=32 R=128 prefix (8 KV heads, head_dim 128) shared by "
           "64 RagSessions with 96-token fp32 suffixes, 32 query heads, batched sessions attention"),
}
# batched-sessions workloads: name -> (sessions, suffix tokens per session)
SESSIONS = {"c4": (64, 96)}
# streaming-decode workloads: name -> decode steps the workload allows after the prefill
DECODE = {"c1": 512}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def outlier_channels(heads, dim, seed):
    """1% of channels per KV head (ceil(0.01*D)), fixed by the seed."""
    rng = np.random.default_rng(seed)
    k = max(1, math.ceil(0.01 * dim))
    return [sorted(rng.choice(dim, size=k, replace=False).tolist()) for _ in range(heads)]


def gpu_inputs(torch, batch, heads, qh, dim, seq, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    k = torch.randn((batch, heads, seq, dim), generator=g, device="cuda", dtype=torch.float32)
    for h, chans in enumerate(outlier_channels(heads, dim, seed)):
        k[:, h, :, chans] *= 10.0
    v = torch.randn((batch, heads, seq, dim), generator=g, device="cuda", dtype=torch.float32)
    q = torch.randn((batch, qh, dim), generator=g, device="cuda", dtype=torch.float32)
    return k, v, q


def cpu_baseline(kivi, cfg_tuple, target_s=12.0):
    """Oracle (CPU restatement of the reference, one thread) on one sequence of the workload."""
    _, heads, qh, dim, seq, bits, G, R, _ = cfg_tuple
    oracle = kivi.Backend.load(ROOT / "oracle" / "libkivi_oracle.so", "kivi_oracle_", device=False)
    rng = np.random.default_rng(7)
    k = rng.standard_normal((1, heads, seq, dim), dtype=np.float32)
    for h, chans in enumerate(outlier_channels(heads, dim, 7)):
        k[:, h, :, chans] *= 10.0
    v = rng.standard_normal((1, heads, seq, dim), dtype=np.float32)
    q = rng.standard_normal((1, qh, dim), dtype=np.float32)
    cache = kivi.KiviCache(oracle, kivi.KiviConfig(bits, G, R), 1, heads, dim)
    t0 = time.perf_counter()
    cache.append(k, v, seq)
    t_quant = time.perf_counter() - t0
    quant_bytes = 2 * k.nbytes + cache.memory().compressed_bytes()
    del k, v
    scale = 1.0 / math.sqrt(dim)
    reps, spent = 0, 0.0
    while spent < target_s and reps < 5:
        t0 = time.perf_counter()
        cache.attention(q, qh, scale)
        spent += time.perf_counter() - t0
        reps += 1
    per_step = spent / reps
    return {
        "value": 1.0 / per_step,
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": f"1 of the workload's sequences ({heads} KV / {qh} q heads, {seq} tokens): "
                  f"{reps} decode attention step(s) of the C++ restatement of the reference "
                  f"CPU path, single thread; prefill quantize {quant_bytes / t_quant / 1e9:.3f} GB/s",
        "quantize_gbps": quant_bytes / t_quant / 1e9,
        "ms_per_step": per_step * 1e3,
        "cpu": _cpu_model(),
    }


def cpu_baseline_sessions(kivi, cfg_tuple, n_sessions, suffix, target_s=12.0):
    """Oracle on the shared-prefix workload: the prefix once, then sessions one by one (the
    reference's RagSession::attention, src/prefix.rs:223-289), timed per session."""
    _, heads, qh, dim, seq, bits, G, R, _ = cfg_tuple
    oracle = kivi.Backend.load(ROOT / "oracle" / "libkivi_oracle.so", "kivi_oracle_", device=False)
    rng = np.random.default_rng(7)
    k = rng.standard_normal((1, heads, seq, dim), dtype=np.float32)
    for h, chans in enumerate(outlier_channels(heads, dim, 7)):
        k[:, h, :, chans] *= 10.0
    v = rng.standard_normal((1, heads, seq, dim), dtype=np.float32)
    cache = kivi.KiviCache(oracle, kivi.KiviConfig(bits, G, R), 1, heads, dim)
    cache.append(k, v, seq)
    del k, v
    prefix = cache.share_prefix()
    del cache
    scale = 1.0 / math.sqrt(dim)
    reps, spent = 0, 0.0
    while spent < target_s and reps < min(n_sessions, 5):
        sess = prefix.session()
        sk = rng.standard_normal((1, heads, suffix, dim), dtype=np.float32)
        sv = rng.standard_normal((1, heads, suffix, dim), dtype=np.float32)
        sess.append(sk, sv, suffix)
        q = rng.standard_normal((1, qh, dim), dtype=np.float32)
        t0 = time.perf_counter()
        sess.attention(q, qh, scale)
        spent += time.perf_counter() - t0
        reps += 1
    per_session = spent / reps
    return {
        "value": 1.0 / per_session,
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{reps} of the {n_sessions} sessions ({seq}-token prefix + {suffix}-token suffix, "
                  f"{heads} KV / {qh} q heads): one RagSession decode attention each, C++ "
                  f"restatement of the reference CPU path, single thread",
        "ms_per_step": per_session * 1e3,
        "cpu": _cpu_model(),
    }


def cpu_baseline_decode(kivi, cfg_tuple, target_s=10.0):
    """Oracle RuntimeKv (src/runtime.rs:12-57): the prefill, then decode steps (append one token
    and attend) timed one by one on one thread."""
    _, heads, qh, dim, seq, bits, G, R, _ = cfg_tuple
    oracle = kivi.Backend.load(ROOT / "oracle" / "libkivi_oracle.so", "kivi_oracle_", device=False)
    rng = np.random.default_rng(7)
    k = rng.standard_normal((1, heads, seq, dim), dtype=np.float32)
    for h, chans in enumerate(outlier_channels(heads, dim, 7)):
        k[:, h, :, chans] *= 10.0
    v = rng.standard_normal((1, heads, seq, dim), dtype=np.float32)
    rt = kivi.RuntimeKv(oracle, kivi.KiviConfig(bits, G, R), 1, heads, dim)
    rt.prefill(k, v, seq)
    del k, v
    scale = 1.0 / math.sqrt(dim)
    reps, spent = 0, 0.0
    while spent < target_s and reps < 200:
        kk = rng.standard_normal(heads * dim, dtype=np.float32)
        vv = rng.standard_normal(heads * dim, dtype=np.float32)
        q = rng.standard_normal(qh * dim, dtype=np.float32)
        t0 = time.perf_counter()
        rt.decode(kk, vv, q, qh, scale)
        spent += time.perf_counter() - t0
        reps += 1
    per_step = spent / reps
    return {
        "value": 1.0 / per_step,
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{reps} RuntimeKv::decode steps (append 1 token + attention, {heads} KV / {qh} q "
                  f"heads) after a {seq}-token prefill, C++ restatement of the reference CPU path, "
                  f"single thread",
        "ms_per_step": per_step * 1e3,
        "cpu": _cpu_model(),
    }


def guard_check(kivi, amd, cfg_tuple):
    """QualityGuard (src/guard.rs) on the streaming-decode shape: after a guarded prefill of
    the workload's tokens, one append of R tokens makes exactly one key flush and one check
    (cache attention and fp32 attention over the whole tape on the GPU, cosine on the host).
    Timed against the plain cache doing the same append and one attention. Host-pointer API:
    the times include the PCIe copies of the R new rows, the query and the outputs."""
    batch, heads, qh, dim, seq, bits, G, R, _ = cfg_tuple
    rng = np.random.default_rng(11)
    cfg = kivi.KiviConfig(bits, G, R)
    keys = rng.standard_normal((batch, heads, seq + 2 * R, dim), dtype=np.float32)
    values = rng.standard_normal((batch, heads, seq + 2 * R, dim), dtype=np.float32)
    query = rng.standard_normal((batch, qh, dim), dtype=np.float32)
    scale = 1.0 / math.sqrt(dim)
    pre_k, pre_v = np.ascontiguousarray(keys[:, :, :seq]), np.ascontiguousarray(values[:, :, :seq])
    mid_k, mid_v = np.ascontiguousarray(keys[:, :, seq:seq + R]), np.ascontiguousarray(values[:, :, seq:seq + R])
    new_k, new_v = np.ascontiguousarray(keys[:, :, seq + R:]), np.ascontiguousarray(values[:, :, seq + R:])
    guard = kivi.QualityGuard(amd, cfg, batch, heads, dim, 0.0, kivi.QualityPolicy.RaiseBits, 8, R)
    guard.append(pre_k, pre_v, seq, query, qh, scale)
    guard.append(mid_k, mid_v, R, query, qh, scale)  # untimed: the tape grows past seq here
    plain = kivi.KiviCache(amd, cfg, batch, heads, dim)
    plain.append(pre_k, pre_v, seq)
    plain.append(mid_k, mid_v, R)
    t0 = time.perf_counter()
    checks = guard.append(new_k, new_v, R, query, qh, scale)
    t_guard = time.perf_counter() - t0
    t0 = time.perf_counter()
    plain.append(new_k, new_v, R)
    plain.attention(query, qh, scale)
    t_plain = time.perf_counter() - t0
    log(f"[bench] guarded append of {R} tokens with {len(checks)} check(s): {t_guard * 1e3:.2f} ms "
        f"(plain append + attention {t_plain * 1e3:.2f} ms)")
    return {"append_tokens": R, "checks": len(checks), "tape_tokens": seq + 2 * R,
            "cosine": checks[0].cosine if checks else None,
            "guarded_ms": t_guard * 1e3, "plain_append_attention_ms": t_plain * 1e3,
            "note": "host-pointer API, PCIe copies included"}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def recorded_traffic(kernel, workload, bytes_per_launch):
    """HBM bytes per launch of `kernel` on `workload` from profiles/traffic.json, if that
    record was measured at the same algorithmic bytes per launch."""
    path = ROOT / "profiles" / "traffic.json"
    try:
        records = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    for r in records.get("records", []):
        if (r.get("kernel") == kernel and r.get("workload") == workload
                and abs(r.get("algorithmic_bytes_per_launch", -1) - bytes_per_launch) < 1.0):
            return r
    return None


CLOCK_WARMUP_S = 0.3
ROTATE_BYTES = 768 << 20  # three times the MI355X Infinity Cache
MAX_COPIES = 8


def clock_warmup(torch, stream, fn, seconds=CLOCK_WARMUP_S, batch=20):
    """Untimed GPU work before a measurement: the MI355X raises its clocks over tens of
    milliseconds of load, so a few warm-up steps alone leave the timed region on the ramp
    (C2: 137 us/step after 10 warm-up steps, 116 us after 200). Returns the calls made."""
    t0, n = time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        with torch.cuda.stream(stream):
            for _ in range(batch):
                fn()
        stream.synchronize()
        n += batch
    return n


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after the timed region, copy MIB MiB device-to-device 3 times (a plain "
                         "copy kernel of known size for calibrating rocprofv3 byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus "
              f"{args.gpus}); the (batch, kv_head) units would shard across GPUs with no "
              f"communication, each GPU running these kernels on its share",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import kivi

    amd = kivi.Backend.amd()
    assert amd["device_count"]() >= 1, "no HIP device"
    batch, heads, qh, dim, seq, bits, G, R, desc = CONFIGS[args.config]
    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream

    log(f"[bench] building inputs {desc}")
    k, v, q = gpu_inputs(torch, batch, heads, qh, dim, seq, 2001)
    out = torch.empty((batch, qh, dim), device="cuda", dtype=torch.float32)
    # warm-up: a small cache of the same shape loads the kernels' code objects before timing
    warm = kivi.KiviCache(amd, kivi.KiviConfig(bits, G, R), 1, heads, dim)
    wk = torch.randn((1, heads, 4 * R, dim), device="cuda", dtype=torch.float32)
    warm.append_device(wk.data_ptr(), wk.numel(), wk.data_ptr(), wk.numel(), 4 * R, sp)
    wq = torch.randn((1, qh, dim), device="cuda", dtype=torch.float32)
    wo = torch.empty_like(wq)
    warm.attention_device(wq.data_ptr(), wq.numel(), qh, 0.1, wo.data_ptr(), wo.numel(), sp)
    stream.synchronize()
    del warm, wk, wq, wo
    # clocks up before the prefill quantize is timed: device copies of the input's size
    scratch = torch.empty_like(k)
    clock_warmup(torch, stream, lambda: scratch.copy_(k), batch=4)
    del scratch
    torch.cuda.empty_cache()
    if DECODE.get(args.config):
        # RuntimeKv (src/runtime.rs:12-57): prefill through its cache, then decode steps
        runtime = kivi.RuntimeKv(amd, kivi.KiviConfig(bits, G, R), batch, heads, dim)
        cache = runtime.cache()
        cache.reserve(seq + DECODE[args.config])
    else:
        cache = kivi.KiviCache(amd, kivi.KiviConfig(bits, G, R), batch, heads, dim)
        cache.reserve(seq)
    torch.cuda.synchronize()
    # Prefill quantization, timed once on the library's stream (whole append, and per
    # quantize kernel with the library's launch timing).
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    kivi.timing_enable(amd, True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        cache.append_device(k.data_ptr(), k.numel(), v.data_ptr(), v.numel(), seq, sp)
        e1.record(stream)
    stream.synchronize()
    t_quant = e0.elapsed_time(e1) / 1e3
    quant_kernels = {}
    for fam in ("quant_keys", "quant_values"):
        n, ms, by = kivi.timing_read(amd, fam)
        if n:
            quant_kernels[fam] = {"launches": n, "ms": ms, "gbps": by / (ms / 1e3) / 1e9}
    kivi.timing_enable(amd, False)
    mem = cache.memory()
    quant_bytes = 2 * k.numel() * 4 + mem.compressed_bytes()
    log(f"[bench] prefill quantize {quant_bytes / t_quant / 1e9:.1f} GB/s ({t_quant * 1e3:.2f} ms)")

    # Export formats into device memory, each timed once after an untimed call: the packed
    # streams in the reference order (packed bytes read and written) and the dense
    # reconstruction (packed bytes read, fp32 keys and values written).
    exports = {}
    if not DECODE.get(args.config):
        lens = cache.stream_lengths()
        bufs = [torch.empty(max(n, 1), device="cuda", dtype=torch.float32) for n in lens]
        ptrs = [b.data_ptr() if n else 0 for b, n in zip(bufs, lens)]
        n_el = k.numel()
        dk, dv = torch.empty_like(k), torch.empty_like(v)
        jobs = (("export_streams", lambda: cache.export_streams_device(ptrs, lens, sp), 2 * 4 * sum(lens)),
                ("dequantize", lambda: cache.dequantize_device(dk.data_ptr(), n_el, dv.data_ptr(), n_el, sp),
                 mem.compressed_bytes() + 2 * n_el * 4))
        for name, fn, nbytes in jobs:
            fn()
            stream.synchronize()
            with torch.cuda.stream(stream):
                e0.record(stream)
                fn()
                e1.record(stream)
            stream.synchronize()
            t = e0.elapsed_time(e1) / 1e3
            exports[name] = {"ms": t * 1e3, "bytes": nbytes, "gbps": nbytes / t / 1e9,
                             "frac": nbytes / t / (HBM_PEAK_GBPS * 1e9)}
            log(f"[bench] {name} {nbytes / t / 1e9:.0f} GB/s ({t * 1e3:.3f} ms)")
        del bufs, dk, dv
        torch.cuda.empty_cache()

    # A step whose cache is smaller than the 256 MB Infinity Cache (MALL) could be served
    # from it by the previous step. Such workloads rotate over `copies` identical caches (the
    # same prefill), so consecutive steps touch >= ROTATE_BYTES of distinct data and each step
    # reads its cache from HBM. Decode steps (C1) and caches too small to rotate out of the
    # MALL within MAX_COPIES report `cache_resident`.
    decode_steps = DECODE.get(args.config)
    step_bytes = mem.compressed_bytes() + (SESSIONS[args.config][0] * batch * heads *
                                           SESSIONS[args.config][1] * dim * 8 if args.config in SESSIONS else 0)
    copies = 1
    if not decode_steps and step_bytes < ROTATE_BYTES:
        copies = min(MAX_COPIES, -(-ROTATE_BYTES // step_bytes))
    cache_resident = copies * step_bytes < ROTATE_BYTES
    caches = [cache]
    for _ in range(copies - 1):
        c2_ = kivi.KiviCache(amd, kivi.KiviConfig(bits, G, R), batch, heads, dim)
        c2_.reserve(seq)
        c2_.append_device(k.data_ptr(), k.numel(), v.data_ptr(), v.numel(), seq, sp)
        caches.append(c2_)
    stream.synchronize()
    if copies > 1:
        log(f"[bench] {copies} cache copies rotate between steps ({copies * step_bytes / 1e6:.0f} MB)")
    del k, v
    torch.cuda.empty_cache()

    scale = 1.0 / math.sqrt(dim)
    sessions_cfg = SESSIONS.get(args.config)
    if sessions_cfg:
        # shared prefix + RagSessions with private fp32 suffixes; a step is one batched
        # attention over all sessions (the prefix streamed once per step)
        n_sess, suffix = sessions_cfg
        gs = torch.Generator(device="cuda")
        gs.manual_seed(2002)
        sks = [torch.randn((batch, heads, suffix, dim), generator=gs, device="cuda") for _ in range(n_sess)]
        svs = [torch.randn((batch, heads, suffix, dim), generator=gs, device="cuda") for _ in range(n_sess)]
        prefixes, all_sessions, all_handles = [], [], []
        for cc in caches:
            prefix = cc.share_prefix()
            sessions = [prefix.session() for _ in range(n_sess)]
            for se, sk, sv in zip(sessions, sks, svs):
                se.append_device(sk.data_ptr(), sk.numel(), sv.data_ptr(), sv.numel(), suffix, sp)
            prefixes.append(prefix)
            all_sessions.append(sessions)
            all_handles.append(kivi.session_handles(sessions))
        del cache, caches, cc
        torch.cuda.empty_cache()
        stream.synchronize()
        q = torch.randn((n_sess, batch, qh, dim), generator=gs, device="cuda")
        out = torch.empty_like(q)
        qp, op, n_q = q.data_ptr(), out.data_ptr(), q.numel()
        tokens_per_step = n_sess * batch
        kv_bytes = prefixes[0].prefix_bytes() + n_sess * batch * heads * suffix * dim * 4 * 2
        turn = [0]

        def step():
            i = turn[0] % copies
            turn[0] += 1
            kivi.sessions_attention_device(amd, all_sessions[i], qp, n_q, qh, scale, op, n_q, sp,
                                           handles=all_handles[i])
    elif decode_steps:
        # one decode step = append one token (key residual, value window, flush every R) and
        # attend; the plain and the evented timed regions each run `steps` of them
        total = args.warmup + 2 * args.steps
        if total > decode_steps:
            sys.exit(f"c1 allows {decode_steps} decode steps after the prefill: warmup + 2 * steps = {total}")
        gd = torch.Generator(device="cuda")
        gd.manual_seed(2003)
        kd = torch.randn((total, batch, heads, 1, dim), generator=gd, device="cuda")
        for h, chans in enumerate(outlier_channels(heads, dim, 2001)):
            kd[:, :, h, :, chans] *= 10.0
        vd = torch.randn((total, batch, heads, 1, dim), generator=gd, device="cuda")
        qd = torch.randn((total, batch, qh, dim), generator=gd, device="cuda")
        n_kv, n_q = batch * heads * dim, batch * qh * dim
        op = out.data_ptr()
        counter = [0]
        tokens_per_step = batch
        kv_bytes = mem.compressed_bytes()

        def step():
            i = counter[0]
            counter[0] += 1
            runtime.decode_device(kd[i].data_ptr(), n_kv, vd[i].data_ptr(), n_kv, qd[i].data_ptr(),
                                  n_q, qh, scale, op, n_q, sp)
    else:
        qp, op, n_q = q.data_ptr(), out.data_ptr(), q.numel()
        tokens_per_step = batch
        kv_bytes = mem.compressed_bytes()
        turn = [0]

        def step():
            i = turn[0] % copies
            turn[0] += 1
            caches[i].attention_device(qp, n_q, qh, scale, op, n_q, sp)

    # clocks up on the step's own kernels (C1: attention over the cache, which leaves the
    # decode state alone), then the W warm-up steps
    extra_warmup = clock_warmup(torch, stream, step if not decode_steps else
                                (lambda: cache.attention_device(qd[0].data_ptr(), n_q, qh, scale, op, n_q, sp)))
    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            step()
    stream.synchronize()
    torch.cuda.synchronize()
    def timed_steps():
        t_start = torch.cuda.Event(enable_timing=True)
        t_end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            t_start.record(stream)
            for _ in range(args.steps):
                step()
            t_end.record(stream)
        stream.synchronize()
        torch.cuda.synchronize()
        return t_start.elapsed_time(t_end) / 1e3 / args.steps

    # Timed region 1: the K steps as they run in service (no per-launch events).
    per_step = timed_steps()
    # Timed region 2: the same K steps with the library's per-launch HIP events, for the
    # per-kernel durations (the event records add a few microseconds between launches).
    kivi.timing_enable(amd, True)
    per_step_evented = timed_steps()
    kernels = {}
    for fam in ("attn_packed", "attn_tail", "attn_merge"):
        n, ms, by = kivi.timing_read(amd, fam)
        if n:
            kernels[fam] = {"launches": n, "mean_us": ms * 1e3 / n, "bytes_per_launch": by / n,
                            "gbps": by / (ms / 1e3) / 1e9}
    kivi.timing_enable(amd, False)
    log(f"[bench] timed region with per-launch events: {per_step_evented * 1e6:.1f} us/step")
    for fam, r in kernels.items():
        log(f"[bench] {fam}: {r['mean_us']:.1f} us/launch, {r['bytes_per_launch'] / 1e6:.2f} MB, "
            f"{r['gbps']:.0f} GB/s")
    if args.copy_calibration > 0:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, device="cuda", dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: 3 x {args.copy_calibration} MiB device copies")
        del src, dst
    algo_bytes = kv_bytes + 2 * out.numel() * 4  # KV bytes + query + output
    eff_gbps = algo_bytes / per_step / 1e9
    tokens_per_s = tokens_per_step / per_step
    log(f"[bench] attention {per_step * 1e6:.1f} us/step, {eff_gbps:.0f} GB/s effective")

    dom = kernels.get("attn_packed") or kernels.get("attn_tail")
    # the sessions workload (64 sessions x 4 heads = 256 rows per unit) runs the GEMM form
    dom_name = ("k_attn_shared" if sessions_cfg else "k_attn_mfma") if "attn_packed" in kernels \
        else "k_attn_generic"
    achieved = dom["gbps"] if dom else eff_gbps
    rec = recorded_traffic(dom_name, args.config, dom["bytes_per_launch"]) if dom else None
    roofline = {
        "bound": "hbm",
        "achieved": achieved,
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": achieved / HBM_PEAK_GBPS,
        "traffic": rec["hbm_bytes_per_launch"] if rec else None,
        "kernel": dom_name,
        "algorithmic_bytes_per_launch": dom["bytes_per_launch"] if dom else algo_bytes,
        "mean_launch_us": dom["mean_us"] if dom else per_step * 1e6,
        "timing": "HIP events around each launch on its stream (kivi_timing_*), second timed "
                  "region of the same steps",
        "traffic_source": rec["source"] if rec else None,
    }
    if sessions_cfg and dom:
        # The batched-sessions GEMM form is bound by the matrix cores: algorithmic flops of the
        # launch (q.k and p.v over every session row and token, 4*D flops per row-token) over
        # its mean duration, against the dense f16 MFMA peak it runs on. Each product executes
        # as three f16 MFMA products (hi/lo operand splits), reported beside it.
        n_sess, suffix = sessions_cfg
        rows = n_sess * (qh // heads)
        flops = 4.0 * dim * rows * (seq + suffix) * batch * heads
        tflops = flops / (dom["mean_us"] * 1e-6) / 1e12
        roofline.update({
            "bound": "mfma", "achieved": tflops, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": tflops / MFMA_F16_PEAK_TFLOPS, "algorithmic_flops_per_launch": flops,
            "executed_f16_tflops": 3.0 * tflops,
            "hbm_gbps": dom["gbps"],
        })
    result = {
        "metric": METRIC,
        "value": tokens_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_warmup_calls": extra_warmup,
        "cache_copies": copies,
        "cache_resident": cache_resident,
        "ms_per_step": per_step * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": desc, "batch": batch, "kv_heads": heads, "q_heads": qh,
                   "head_dim": dim, "cached_tokens": seq, "bits": bits, "group_size": G,
                   "residual_length": R,
                   **({"sessions": sessions_cfg[0], "suffix_tokens": sessions_cfg[1]}
                      if sessions_cfg else {})},
        "effective_hbm_gbps": eff_gbps,
        "hbm_fraction": eff_gbps / HBM_PEAK_GBPS,
        "quantize_gbps": quant_bytes / t_quant / 1e9,
        "roofline": roofline,
        "kernels": kernels,
        "quantize_kernels": quant_kernels,
        "exports": exports,
    }
    if decode_steps:
        result["guard"] = guard_check(kivi, amd, CONFIGS[args.config])
    if not args.no_cpu:
        log("[bench] CPU baseline (oracle, 1 thread) ...")
        if sessions_cfg:
            result["cpu_baseline"] = cpu_baseline_sessions(kivi, CONFIGS[args.config], *sessions_cfg)
        elif decode_steps:
            result["cpu_baseline"] = cpu_baseline_decode(kivi, CONFIGS[args.config])
        else:
            result["cpu_baseline"] = cpu_baseline(kivi, CONFIGS[args.config])
        log(f"[bench] CPU {result['cpu_baseline']['value']:.3f} tokens/s")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
