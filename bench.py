#!/usr/bin/env python3
"""Decode-attention benchmark of the MI355X KIVI path (one JSON line on stdout).

Primary workload (the north-star target): batch 16, 32 query / 8 KV
heads, head_dim 128, 32768 cached tokens per sequence, 2-bit G=32 R=128, K ~ N(0,1) with 1% of
key channels (2 per KV head) scaled x10, V ~ N(0,1), fp32 inputs. A step is one decode attention
over all 16 sequences (the cache and the queries already resident in HBM); value = decode
tokens/s = 16 * steps / time.

The default run measures every BASELINE.json workload in the same process and puts the others
in `configs` as compact entries (step, throughput, HBM fraction, roofline, CPU baseline): c0
(the reference's CPU-runnable case), c1 (streaming decode: a step is RuntimeKv::decode = append
one token + attention after an 8192-token prefill), c3_4 / c3_8 (4-/8-bit at 131072 tokens,
GQA 8), c4 (64 RagSessions over one 65536-token prefix, one batched call per step). `--config
NAME` measures one workload and prints its line alone (the form the rocprof summaries use).
The printed line stays under LINE_LIMIT characters; the full result (per-kernel tables,
exports, codec, guard) is written to --full-json PATH when asked for.

Per workload: the cache build (prefill quantization) is timed once (`quantize_gbps`, and per
kernel); the timed region runs `steps` steps twice, plain (the step time) and with the library's
per-launch HIP events (kivi_timing_*, per-kernel durations and algorithmic bytes on the launch
stream). Before the prefill and before the warm-up steps the GPU runs ~0.3 s of untimed work so
its clocks have ramped up (`clock_warmup_calls`). Caches smaller than three times the 256 MB
Infinity Cache rotate over identical copies between steps (`cache_copies`), so each step reads
HBM; C0 and C1 are too small for that and report `cache_resident: true`.

`roofline` is for the dominant kernel: the packed-chunk attention kernel (k_attn_mfma, or
k_attn_wide for the eight-head units of c3, k_attn_wide16 for GQA 16; HBM bound: algorithmic
bytes per launch over its mean launch duration), or for c4 the shared-prefix GEMM kernel
(k_attn_shared, matrix-core
bound: 4*D flops per (session row, prefix token) over its mean duration, against the dense
f16 MFMA peak). `traffic` is that kernel's HBM bytes per
launch from rocprofv3 FETCH_SIZE + WRITE_SIZE runs calibrated on a plain copy kernel
(--copy-calibration), as recorded in profiles/traffic.json; null when no record matches the
kernel, workload and algorithmic bytes.

The primary line also carries the device exports (packed streams in the reference order, dense
reconstruction) and the standalone codec (quantize_per_channel / per_token of the C2 tensors),
and the c1 entry one QualityGuard check per R appended tokens (median over repetitions).
`cpu_baseline` is the oracle (C++ restatement of the reference CPU path, one thread) on a
bounded sample of each workload, on this host.

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--config NAME] [--no-cpu]
                       [--other-shapes] [--full-json PATH] [--copy-calibration MIB]
"""

import argparse
import json
import math
import os
import platform
import statistics
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
    # shapes beyond head_dim 128 / G 32 / GQA <= 8, timed on request only
    "g_d64": (16, 8, 32, 64, 32768, 2, 32, 128, "other shape: batch 16, 32q/8kv heads, head_dim 64, 32768 tokens, 2-bit"),
    "g_d256": (4, 8, 32, 256, 32768, 2, 32, 128, "other shape: batch 4, 32q/8kv heads, head_dim 256, 32768 tokens, 2-bit"),
    "g_gqa16": (4, 4, 64, 128, 32768, 2, 32, 128, "other shape: batch 4, 64q/4kv heads (GQA 16), head_dim 128, 32768 tokens, 2-bit"),
    "g_g64": (16, 8, 32, 128, 32768, 2, 64, 128, "other shape: batch 16, 32q/8kv heads, head_dim 128, 32768 tokens, 2-bit G=64"),
    "g_d256_b4": (4, 8, 32, 256, 32768, 4, 32, 128, "other shape: batch 4, 32q/8kv heads, head_dim 256, 32768 tokens, 4-bit"),
    "g_d256_b8": (4, 8, 32, 256, 32768, 8, 32, 128, "other shape: batch 4, 32q/8kv heads, head_dim 256, 32768 tokens, 8-bit"),
}
SECONDARY = ("c0", "c1", "c3_4", "c3_8", "c4")
# shapes beyond head_dim 128 / G 32 / GQA <= 8: measured with --other-shapes (stderr and
# --full-json only) or one at a time with --config
OTHER_SHAPES = ("g_d64", "g_d256", "g_d256_b4", "g_d256_b8", "g_g64", "g_gqa16")
# batched-sessions workloads: name -> (sessions, suffix tokens per session)
SESSIONS = {"c4": (64, 96)}
# streaming-decode workloads: name -> decode steps the workload allows after the prefill
DECODE = {"c1": 512}
# CPU-baseline time per workload (seconds of oracle work, beyond its prefill)
CPU_SECONDS = {"c2": 12.0, "c0": 3.0, "c1": 5.0, "c3_4": 4.0, "c3_8": 4.0, "c4": 5.0,
               "g_d64": 3.0, "g_d256": 3.0, "g_gqa16": 3.0, "g_g64": 3.0, "g_d256_b4": 3.0, "g_d256_b8": 3.0}


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


# ------------------------------------------------------------------ CPU baselines


def host_info():
    """CPU model and counts of this host (the CPU baselines run on one thread of it)."""
    info = {"cpu": "unknown", "nproc": os.cpu_count()}
    try:
        info["nproc_affinity"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        pass
    try:
        fields = {}
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                key, val = (x.strip() for x in line.split(":", 1))
                if key in ("model name", "cpu family", "model", "stepping", "vendor_id") and key not in fields:
                    fields[key] = val
            if not line.strip() and fields:
                break
        info["cpu"] = fields.get("model name", "unknown")
        info["cpu_id"] = (f"{fields.get('vendor_id', '?')} family {fields.get('cpu family', '?')} "
                          f"model {fields.get('model', '?')} stepping {fields.get('stepping', '?')}")
    except OSError:
        pass
    info["machine"] = platform.machine()
    return info


def oracle_backend(kivi):
    return kivi.Backend.load(ROOT / "oracle" / "libkivi_oracle.so", "kivi_oracle_", device=False)


def host_kv(heads, dim, seq, seed):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((1, heads, seq, dim), dtype=np.float32)
    for h, chans in enumerate(outlier_channels(heads, dim, seed)):
        k[:, h, :, chans] *= 10.0
    v = rng.standard_normal((1, heads, seq, dim), dtype=np.float32)
    return rng, k, v


def cpu_result(per_step, tokens_per_step, sample, **extra):
    r = {"value": tokens_per_step / per_step, "unit": "tokens/s", "cores": 1, "kind": "port",
         "sample": sample, "ms_per_step": per_step * 1e3}
    r.update(extra)
    r.update(host_info())
    return r


def cpu_baseline(kivi, name):
    """Oracle (CPU restatement of the reference, one thread) on one sequence of the workload:
    its prefill, then decode attention steps for about CPU_SECONDS[name]."""
    _, heads, qh, dim, seq, bits, G, R, _ = CONFIGS[name]
    rng, k, v = host_kv(heads, dim, seq, 7)
    cache = kivi.KiviCache(oracle_backend(kivi), kivi.KiviConfig(bits, G, R), 1, heads, dim)
    t0 = time.perf_counter()
    cache.append(k, v, seq)
    t_quant = time.perf_counter() - t0
    quant_bytes = 2 * k.nbytes + cache.memory().compressed_bytes()
    del k, v
    q = rng.standard_normal((1, qh, dim), dtype=np.float32)
    scale = 1.0 / math.sqrt(dim)
    reps, spent = 0, 0.0
    while spent < CPU_SECONDS[name] and reps < 5:
        t0 = time.perf_counter()
        cache.attention(q, qh, scale)
        spent += time.perf_counter() - t0
        reps += 1
    return cpu_result(spent / reps, 1,
                      f"1 of the workload's sequences ({heads} KV / {qh} q heads, {seq} tokens): "
                      f"{reps} decode attention step(s) of the C++ restatement of the reference CPU "
                      f"path, single thread; prefill quantize {quant_bytes / t_quant / 1e9:.3f} GB/s",
                      quantize_gbps=quant_bytes / t_quant / 1e9)


def cpu_baseline_sessions(kivi, name):
    """Oracle on the shared-prefix workload: the prefix once, then sessions one by one (the
    reference's RagSession::attention, src/prefix.rs:223-289), timed per session."""
    _, heads, qh, dim, seq, bits, G, R, _ = CONFIGS[name]
    n_sessions, suffix = SESSIONS[name]
    rng, k, v = host_kv(heads, dim, seq, 7)
    cache = kivi.KiviCache(oracle_backend(kivi), kivi.KiviConfig(bits, G, R), 1, heads, dim)
    cache.append(k, v, seq)
    del k, v
    prefix = cache.share_prefix()
    del cache
    scale = 1.0 / math.sqrt(dim)
    reps, spent = 0, 0.0
    while spent < CPU_SECONDS[name] and reps < min(n_sessions, 5):
        sess = prefix.session()
        sk = rng.standard_normal((1, heads, suffix, dim), dtype=np.float32)
        sv = rng.standard_normal((1, heads, suffix, dim), dtype=np.float32)
        sess.append(sk, sv, suffix)
        q = rng.standard_normal((1, qh, dim), dtype=np.float32)
        t0 = time.perf_counter()
        sess.attention(q, qh, scale)
        spent += time.perf_counter() - t0
        reps += 1
    return cpu_result(spent / reps, 1,
                      f"{reps} of the {n_sessions} sessions ({seq}-token prefix + {suffix}-token "
                      f"suffix, {heads} KV / {qh} q heads): one RagSession decode attention each, "
                      f"C++ restatement of the reference CPU path, single thread")


def cpu_baseline_decode(kivi, name):
    """Oracle RuntimeKv (src/runtime.rs:12-57): the prefill, then decode steps (append one token
    and attend) timed one by one on one thread."""
    _, heads, qh, dim, seq, bits, G, R, _ = CONFIGS[name]
    rng, k, v = host_kv(heads, dim, seq, 7)
    rt = kivi.RuntimeKv(oracle_backend(kivi), kivi.KiviConfig(bits, G, R), 1, heads, dim)
    rt.prefill(k, v, seq)
    del k, v
    scale = 1.0 / math.sqrt(dim)
    reps, spent = 0, 0.0
    while spent < CPU_SECONDS[name] and reps < 200:
        kk = rng.standard_normal(heads * dim, dtype=np.float32)
        vv = rng.standard_normal(heads * dim, dtype=np.float32)
        q = rng.standard_normal(qh * dim, dtype=np.float32)
        t0 = time.perf_counter()
        rt.decode(kk, vv, q, qh, scale)
        spent += time.perf_counter() - t0
        reps += 1
    return cpu_result(spent / reps, 1,
                      f"{reps} RuntimeKv::decode steps (append 1 token + attention, {heads} KV / "
                      f"{qh} q heads) after a {seq}-token prefill, C++ restatement of the reference "
                      f"CPU path, single thread")


def run_cpu_baseline(kivi, name):
    log(f"[bench] {name}: CPU baseline (oracle, 1 thread) ...")
    if name in SESSIONS:
        r = cpu_baseline_sessions(kivi, name)
    elif name in DECODE:
        r = cpu_baseline_decode(kivi, name)
    else:
        r = cpu_baseline(kivi, name)
    log(f"[bench] {name}: CPU {r['value']:.3f} tokens/s")
    return r


# ------------------------------------------------------------------ GPU measurement helpers


TRAFFIC_MATCH = 0.02  # relative difference of algorithmic bytes a traffic record still covers


def recorded_traffic(kernel, workload, bytes_per_launch):
    """HBM bytes per launch of `kernel` on `workload` from profiles/traffic.json, if that
    record was measured at the same algorithmic bytes per launch, within TRAFFIC_MATCH (a
    decode workload's mean bytes per launch move with the number of steps), scaled by the
    ratio of the two."""
    path = ROOT / "profiles" / "traffic.json"
    try:
        records = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    for r in records.get("records", []):
        algo = r.get("algorithmic_bytes_per_launch", -1)
        if (r.get("kernel") == kernel and r.get("workload") == workload and algo > 0
                and abs(algo - bytes_per_launch) <= TRAFFIC_MATCH * algo):
            return dict(r, hbm_bytes_per_launch=r["hbm_bytes_per_launch"] * bytes_per_launch / algo)
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


def timed_once(torch, stream, fn):
    """Seconds of one call of fn on `stream`, after an untimed call (HIP events)."""
    fn()
    stream.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        fn()
        e1.record(stream)
    stream.synchronize()
    return e0.elapsed_time(e1) / 1e3


def kernel_table(kivi, amd, families):
    out = {}
    for fam in families:
        n, ms, by = kivi.timing_read(amd, fam)
        if n:
            out[fam] = {"launches": n, "mean_us": ms * 1e3 / n, "bytes_per_launch": by / n,
                        "gbps": by / (ms / 1e3) / 1e9}
    return out


ATTN_FAMILIES = ("attn_packed", "attn_tail", "attn_merge", "attn_shared", "attn_sessions")


def measure(name, args, torch, kivi, amd, stream, with_cpu):
    """One workload: prefill, timed steps, roofline, CPU baseline. Returns its result dict."""
    batch, heads, qh, dim, seq, bits, G, R, desc = CONFIGS[name]
    sp = stream.cuda_stream
    cfg = kivi.KiviConfig(bits, G, R)
    log(f"[bench] {name}: building inputs ({desc})")
    k, v, q = gpu_inputs(torch, batch, heads, qh, dim, seq, 2001)
    out = torch.empty((batch, qh, dim), device="cuda", dtype=torch.float32)
    # warm-up: a small cache of the same shape loads the kernels' code objects before timing
    warm = kivi.KiviCache(amd, cfg, 1, heads, dim)
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
    decode_steps = DECODE.get(name)
    if decode_steps:
        # RuntimeKv (src/runtime.rs:12-57): prefill through its cache, then decode steps
        runtime = kivi.RuntimeKv(amd, cfg, batch, heads, dim)
        cache = runtime.cache()
        cache.reserve(seq + decode_steps)
    else:
        cache = kivi.KiviCache(amd, cfg, batch, heads, dim)
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
    for fam, r in kernel_table(kivi, amd, ("quant_keys", "quant_values")).items():
        quant_kernels[fam] = {"launches": r["launches"], "ms": r["mean_us"] * r["launches"] / 1e3,
                              "gbps": r["gbps"], "frac": r["gbps"] / HBM_PEAK_GBPS}
    kivi.timing_enable(amd, False)
    mem = cache.memory()
    quant_bytes = 2 * k.numel() * 4 + mem.compressed_bytes()
    log(f"[bench] {name}: prefill quantize {quant_bytes / t_quant / 1e9:.1f} GB/s ({t_quant * 1e3:.2f} ms)")

    extras = {}
    if name == "c2":
        extras.update(primary_extras(torch, kivi, amd, stream, cache, mem, k, v))

    # A step whose cache is smaller than the 256 MB Infinity Cache (MALL) could be served
    # from it by the previous step. Such workloads rotate over `copies` identical caches (the
    # same prefill), so consecutive steps touch >= ROTATE_BYTES of distinct data and each step
    # reads its cache from HBM. Decode steps (C1) and caches too small to rotate out of the
    # MALL within MAX_COPIES report `cache_resident`.
    sessions_cfg = SESSIONS.get(name)
    step_bytes = mem.compressed_bytes() + (sessions_cfg[0] * batch * heads * sessions_cfg[1] * dim * 8
                                           if sessions_cfg else 0)
    copies = 1
    if not decode_steps and step_bytes < ROTATE_BYTES:
        copies = min(MAX_COPIES, -(-ROTATE_BYTES // step_bytes))
    cache_resident = copies * step_bytes < ROTATE_BYTES
    caches = [cache]
    for _ in range(copies - 1):
        cc = kivi.KiviCache(amd, cfg, batch, heads, dim)
        cc.reserve(seq)
        cc.append_device(k.data_ptr(), k.numel(), v.data_ptr(), v.numel(), seq, sp)
        caches.append(cc)
    stream.synchronize()
    if copies > 1:
        log(f"[bench] {name}: {copies} cache copies rotate between steps ({copies * step_bytes / 1e6:.0f} MB)")
    del k, v
    torch.cuda.empty_cache()

    scale = 1.0 / math.sqrt(dim)
    keep = []  # device tensors and handles the steps use
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
        del cache, caches
        torch.cuda.empty_cache()
        stream.synchronize()
        q = torch.randn((n_sess, batch, qh, dim), generator=gs, device="cuda")
        out = torch.empty_like(q)
        keep += [sks, svs, prefixes, q, out]
        qp, op, n_q = q.data_ptr(), out.data_ptr(), q.numel()
        tokens_per_step = n_sess * batch
        kv_bytes = prefixes[0].prefix_bytes() + n_sess * batch * heads * suffix * dim * 4 * 2
        turn = [0]

        def step():
            i = turn[0] % copies
            turn[0] += 1
            kivi.sessions_attention_device(amd, all_sessions[i], qp, n_q, qh, scale, op, n_q, sp,
                                           handles=all_handles[i])
        warm_fn = step
    elif decode_steps:
        # one decode step = append one token (key residual, value window, flush every R) and
        # attend; the plain and the evented timed regions each run `steps` of them
        total = args.warmup + 2 * args.steps
        if total > decode_steps:
            sys.exit(f"{name} allows {decode_steps} decode steps after the prefill: warmup + 2 * steps = {total}")
        gd = torch.Generator(device="cuda")
        gd.manual_seed(2003)
        kd = torch.randn((total, batch, heads, 1, dim), generator=gd, device="cuda")
        for h, chans in enumerate(outlier_channels(heads, dim, 2001)):
            kd[:, :, h, :, chans] *= 10.0
        vd = torch.randn((total, batch, heads, 1, dim), generator=gd, device="cuda")
        qd = torch.randn((total, batch, qh, dim), generator=gd, device="cuda")
        keep += [kd, vd, qd, runtime]
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

        # clocks up on attention over the cache, which leaves the decode state alone
        def warm_fn():
            cache.attention_device(qd[0].data_ptr(), n_q, qh, scale, op, n_q, sp)
    else:
        qp, op, n_q = q.data_ptr(), out.data_ptr(), q.numel()
        tokens_per_step = batch
        kv_bytes = mem.compressed_bytes()
        turn = [0]

        def step():
            i = turn[0] % copies
            turn[0] += 1
            caches[i].attention_device(qp, n_q, qh, scale, op, n_q, sp)
        warm_fn = step

    extra_warmup = clock_warmup(torch, stream, warm_fn)
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
    kernels = kernel_table(kivi, amd, ATTN_FAMILIES)
    kivi.timing_enable(amd, False)
    log(f"[bench] {name}: timed region with per-launch events: {per_step_evented * 1e6:.1f} us/step")
    for fam, r in kernels.items():
        log(f"[bench] {name}: {fam}: {r['mean_us']:.1f} us/launch, {r['bytes_per_launch'] / 1e6:.2f} MB, "
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
    log(f"[bench] {name}: attention {per_step * 1e6:.1f} us/step, {eff_gbps:.0f} GB/s effective")

    if sessions_cfg and "attn_shared" in kernels:
        dom_fam, dom_name = "attn_shared", "k_attn_shared"
    elif "attn_packed" in kernels:
        # units of five or more heads at head_dim 128, G = 32 run their packed chunks on the
        # 16x16x32 kernels: sixteen-head groups for GQA a multiple of 16, eight-head otherwise
        gqa = qh // heads
        wide = dim == 128 and G == 32 and gqa > 4
        dom_name = ("k_attn_wide16" if gqa % 16 == 0 else "k_attn_wide") if wide else "k_attn_mfma"
        dom_fam = "attn_packed"
    elif "attn_sessions" in kernels:
        dom_fam, dom_name = "attn_sessions", "k_attn_sessions"
    else:
        dom_fam, dom_name = "attn_tail", "k_attn_generic"
    dom = kernels.get(dom_fam)
    rec = recorded_traffic(dom_name, name, dom["bytes_per_launch"]) if dom else None
    roofline = {
        "bound": "hbm",
        "achieved": dom["gbps"] if dom else eff_gbps,
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": (dom["gbps"] if dom else eff_gbps) / HBM_PEAK_GBPS,
        "traffic": rec["hbm_bytes_per_launch"] if rec else None,
        "kernel": dom_name,
        "algorithmic_bytes_per_launch": dom["bytes_per_launch"] if dom else algo_bytes,
        "mean_launch_us": dom["mean_us"] if dom else per_step * 1e6,
        "timing": "HIP events around each launch on its stream (kivi_timing_*), second timed "
                  "region of the same steps",
        "traffic_source": rec["source"] if rec else None,
    }
    if dom_fam == "attn_shared":
        # The shared-prefix GEMM form is bound by the matrix cores: algorithmic flops of the
        # launch (q.k and p.v over every session row and prefix token, 4*D flops per
        # row-token; the suffixes run in k_attn_suffix) over its mean duration,
        # against the dense f16 MFMA peak it runs on. Each product executes as three f16 MFMA
        # products (hi/lo operand splits), reported beside it.
        n_sess, _ = sessions_cfg
        rows = n_sess * (qh // heads)
        flops = 4.0 * dim * rows * seq * batch * heads
        tflops = flops / (dom["mean_us"] * 1e-6) / 1e12
        roofline.update({
            "bound": "mfma", "achieved": tflops, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": tflops / MFMA_F16_PEAK_TFLOPS, "algorithmic_flops_per_launch": flops,
            "executed_f16_tflops": 3.0 * tflops, "hbm_gbps": dom["gbps"],
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
        "ms_per_step_evented": per_step_evented * 1e3,
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
    }
    result.update(extras)
    del keep, step, warm_fn
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    if decode_steps:
        result["guard"] = guard_check(kivi, amd, CONFIGS[name])
    if with_cpu:
        result["cpu_baseline"] = run_cpu_baseline(kivi, name)
    return result


def primary_extras(torch, kivi, amd, stream, cache, mem, k, v):
    """Device exports of the primary cache and the standalone codec on its tensors."""
    sp = stream.cuda_stream
    _, heads, _, dim, seq, bits, G, _, _ = CONFIGS["c2"]
    batch = k.shape[0]
    exports = {}
    # Export formats into device memory, each timed once after an untimed call: the packed
    # streams in the reference order (packed bytes read and written) and the dense
    # reconstruction (packed bytes read, fp32 keys and values written).
    lens = cache.stream_lengths()
    bufs = [torch.empty(max(n, 1), device="cuda", dtype=torch.float32) for n in lens]
    ptrs = [b.data_ptr() if n else 0 for b, n in zip(bufs, lens)]
    n_el = k.numel()
    dk, dv = torch.empty_like(k), torch.empty_like(v)
    jobs = (("export_streams", lambda: cache.export_streams_device(ptrs, lens, sp), 2 * 4 * sum(lens)),
            ("dequantize", lambda: cache.dequantize_device(dk.data_ptr(), n_el, dv.data_ptr(), n_el, sp),
             mem.compressed_bytes() + 2 * n_el * 4))
    for name, fn, nbytes in jobs:
        t = timed_once(torch, stream, fn)
        exports[name] = {"ms": t * 1e3, "bytes": nbytes, "gbps": nbytes / t / 1e9,
                         "frac": nbytes / t / (HBM_PEAK_GBPS * 1e9)}
        log(f"[bench] {name} {nbytes / t / 1e9:.0f} GB/s ({t * 1e3:.3f} ms)")
    del bufs, dk, dv
    torch.cuda.empty_cache()
    # The standalone codec (quantize_per_channel / quantize_per_token, src/quant.rs:153-233) on
    # the C2 keys and values: device input, reference-order codes and (scale, zero) out. The
    # kernel is timed by the library's launch events (the call also allocates its outputs).
    codec = {}
    import ctypes as C
    for name, fam, t in (("quantize_per_channel", "codec_keys", k), ("quantize_per_token", "codec_values", v)):
        handles = []

        def call():
            h = C.c_void_p()
            amd.call(name + "_device", C.c_void_p(t.data_ptr()), t.numel(), batch, heads, seq, dim,
                     bits, G, C.c_void_p(sp), C.byref(h))
            handles.append(h)
        call()
        stream.synchronize()
        kivi.timing_enable(amd, True)
        call()
        r = kernel_table(kivi, amd, (fam,)).get(fam)
        kivi.timing_enable(amd, False)
        for h in handles:
            amd["quantized_free"](h)
        if r:
            codec[name] = {"kernel_us": r["mean_us"], "bytes": r["bytes_per_launch"], "gbps": r["gbps"],
                           "frac": r["gbps"] / HBM_PEAK_GBPS}
            log(f"[bench] {name}: {r['gbps']:.0f} GB/s ({r['mean_us']:.1f} us)")
    torch.cuda.empty_cache()
    return {"exports": exports, "codec": codec}


def guard_check(kivi, amd, cfg_tuple, reps=5):
    """QualityGuard (src/guard.rs) on the streaming-decode shape: after a guarded prefill of
    the workload's tokens, each append of R tokens makes exactly one key flush and one check
    (cache attention and fp32 attention over the whole tape on the GPU, cosine on the host).
    Timed against the plain cache doing the same append and one attention, alternating which
    runs first, after one untimed repetition; medians and ranges over `reps`. Host-pointer API:
    the times include the PCIe copies of the R new rows, the query and the outputs."""
    batch, heads, qh, dim, seq, bits, G, R, _ = cfg_tuple
    rng = np.random.default_rng(11)
    cfg = kivi.KiviConfig(bits, G, R)
    total = seq + (reps + 1) * R
    keys = rng.standard_normal((batch, heads, total, dim), dtype=np.float32)
    values = rng.standard_normal((batch, heads, total, dim), dtype=np.float32)
    query = rng.standard_normal((batch, qh, dim), dtype=np.float32)
    scale = 1.0 / math.sqrt(dim)
    pre_k, pre_v = np.ascontiguousarray(keys[:, :, :seq]), np.ascontiguousarray(values[:, :, :seq])
    guard = kivi.QualityGuard(amd, cfg, batch, heads, dim, 0.0, kivi.QualityPolicy.RaiseBits, 8, R)
    guard.append(pre_k, pre_v, seq, query, qh, scale)
    plain = kivi.KiviCache(amd, cfg, batch, heads, dim)
    plain.append(pre_k, pre_v, seq)
    t_guard, t_plain, checks = [], [], None
    for i in range(reps + 1):
        lo = seq + i * R
        nk, nv = np.ascontiguousarray(keys[:, :, lo:lo + R]), np.ascontiguousarray(values[:, :, lo:lo + R])

        def guarded():
            t0 = time.perf_counter()
            c = guard.append(nk, nv, R, query, qh, scale)
            return time.perf_counter() - t0, c

        def unguarded():
            t0 = time.perf_counter()
            plain.append(nk, nv, R)
            plain.attention(query, qh, scale)
            return time.perf_counter() - t0

        if i % 2 == 0:
            tg, checks = guarded()
            tp = unguarded()
        else:
            tp = unguarded()
            tg, checks = guarded()
        if i > 0:
            t_guard.append(tg)
            t_plain.append(tp)
    g_ms = [x * 1e3 for x in t_guard]
    p_ms = [x * 1e3 for x in t_plain]
    log(f"[bench] guarded append of {R} tokens with {len(checks)} check(s): median "
        f"{statistics.median(g_ms):.2f} ms (plain append + attention {statistics.median(p_ms):.2f} ms)")
    return {"append_tokens": R, "checks_per_append": len(checks), "repetitions": reps,
            "tape_tokens_first": seq + R, "tape_tokens_last": total,
            "cosine": checks[0].cosine if checks else None,
            "guarded_ms_median": statistics.median(g_ms), "guarded_ms_range": [min(g_ms), max(g_ms)],
            "plain_append_attention_ms_median": statistics.median(p_ms),
            "plain_append_attention_ms_range": [min(p_ms), max(p_ms)],
            "note": "host-pointer API, PCIe copies included; one untimed repetition first, order "
                    "alternating"}


# The driver keeps the tail of stdout, so the line bench.py prints must stay short: the
# headline workload with its roofline and CPU baseline, and one compact entry per other
# workload. The full result (per-kernel tables, exports, codec, guard) goes to --full-json.
LINE_LIMIT = 6000
PRIMARY_KEYS = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config")
ROOFLINE_KEYS = ("bound", "achieved", "peak", "unit", "frac", "traffic", "kernel",
                 "mean_launch_us", "algorithmic_bytes_per_launch", "algorithmic_flops_per_launch")


def rnd(x, digits=4):
    """x rounded to `digits` significant digits (ints, None and strings unchanged)."""
    if isinstance(x, float) and math.isfinite(x) and x != 0.0:
        return round(x, digits - 1 - int(math.floor(math.log10(abs(x)))))
    return x


def compact_roofline(r, full=True):
    keys = ROOFLINE_KEYS if full else ROOFLINE_KEYS[:7]
    counts = ("traffic", "algorithmic_bytes_per_launch", "algorithmic_flops_per_launch")
    return {k: (int(round(r[k])) if k in counts and r[k] is not None else rnd(r[k]))
            for k in keys if k in r}


def compact_cpu(c, full=True):
    if c is None:
        return None
    out = {"value": rnd(c["value"]), "unit": c["unit"], "ms_per_step": rnd(c["ms_per_step"]),
           "cores": c["cores"], "kind": c["kind"]}
    if full:
        out.update({"sample": c["sample"], "cpu": c.get("cpu"), "nproc": c.get("nproc")})
        if "quantize_gbps" in c:
            out["quantize_gbps"] = rnd(c["quantize_gbps"])
    return out


def compact(result, primary):
    """The short form of one workload's result: the primary line's fields, or a `configs`
    entry (throughput, step, HBM fraction, roofline and CPU baseline)."""
    out = {}
    if primary:
        out.update({k: rnd(result[k]) for k in PRIMARY_KEYS})
    else:
        out.update({"value": rnd(result["value"]), "ms_per_step": rnd(result["ms_per_step"])})
    out["hbm_fraction"] = rnd(result["hbm_fraction"])
    out["quantize_gbps"] = rnd(result["quantize_gbps"])
    if result.get("cache_resident"):
        out["cache_resident"] = True
    out["roofline"] = compact_roofline(result["roofline"], primary)
    out["kernels_us"] = {fam: rnd(r["mean_us"]) for fam, r in result["kernels"].items()}
    if primary:
        out["effective_hbm_gbps"] = rnd(result["effective_hbm_gbps"])
        out["cache_copies"] = result["cache_copies"]
        if "codec" in result:
            out["codec_gbps"] = {k: rnd(v["gbps"]) for k, v in result["codec"].items()}
        if "exports" in result:
            out["exports_gbps"] = {k: rnd(v["gbps"]) for k, v in result["exports"].items()}
    if "guard" in result:
        g = result["guard"]
        out["guard_ms"] = {"guarded": rnd(g["guarded_ms_median"]),
                           "plain": rnd(g["plain_append_attention_ms_median"])}
    out["cpu_baseline"] = compact_cpu(result.get("cpu_baseline"), primary)
    return out


def emit(line_obj, full_obj, path):
    """Print the one JSON line (refusing one over LINE_LIMIT characters) and write the full
    result to `path` when given."""
    if path:
        Path(path).parent.mkdir(parents=True, exist_ok=True)
        Path(path).write_text(json.dumps(full_obj, indent=1))
        log(f"[bench] full result written to {path}")
    line = json.dumps(line_obj, separators=(",", ":"))
    if len(line) > LINE_LIMIT:
        sys.exit(f"bench.py: the result line is {len(line)} characters, over the {LINE_LIMIT} "
                 f"the driver keeps; shorten compact()")
    print(line, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default=None, choices=sorted(CONFIGS),
                    help="measure only this workload (default: c2 as the primary line, the others "
                         "in `configs`)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--other-shapes", action="store_true",
                    help="also measure the shapes outside head_dim 128 / G 32 / GQA <= 8 (logged "
                         "to stderr and --full-json, not in the result line)")
    ap.add_argument("--full-json", default=None, metavar="PATH",
                    help="write the full result (per-kernel tables, exports, codec, guard) here")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after each timed region, copy MIB MiB device-to-device 3 times (a plain "
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
    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()
    with_cpu = not args.no_cpu
    if args.config is not None:
        result = measure(args.config, args, torch, kivi, amd, stream, with_cpu)
        emit(compact(result, True), result, args.full_json)
        return
    result = measure("c2", args, torch, kivi, amd, stream, with_cpu)
    line = compact(result, True)
    line["configs"], result["configs"] = {}, {}
    for name in SECONDARY + (OTHER_SHAPES if args.other_shapes else ()):
        sub = measure(name, args, torch, kivi, amd, stream, with_cpu)
        result["configs"][name] = sub
        if name in SECONDARY:
            line["configs"][name] = compact(sub, False)
        else:
            c = compact(sub, False)
            log(f"[bench] {name}: " + json.dumps(c, separators=(",", ":")))
    emit(line, result, args.full_json)


if __name__ == "__main__":
    main()
