#!/usr/bin/env python3
"""Benchmark of hako's quantized-matmul hot path on one MI355X.

Headline: the Q4_K x q8 matmul (q8_32 activation quantization fused with the
GEMV, one launch) at the Qwen2.5-3B ffn_up shape, 11008 x 2048, batch 1.
A step is one such matmul on a weight matrix already resident in HBM; the
timed region replays K steps captured in a HIP graph, cycling through enough
weight copies (>= 512 MB) that every step streams its weights from HBM rather
than the 256 MB last-level cache.

`value` is whole-job throughput in algorithmic GB/s: each weight byte, the
fp32 activation and the fp32 output once per step (12,733,440 B), times K,
over the timed region. Extra shapes (7B Q4_K, the Q6_K GEMVs) are reported
alongside. The reference's own CPU matmul (oracle/_ref, its AVX2 pthread
path) is timed on the host cores on a bounded sample of the same workload.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

from hako_amd import synth  # noqa: E402

METRIC = "Q4_K×q8 GEMV GB/s (% HBM peak) + decode tok/s, 3B/7B shapes, batch 1"
HBM_PEAK_GBPS = 8000.0            # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0           # MI355X dense int8 matrix cores
FP16_PEAK_TFLOPS = 2500.0         # MI355X dense fp16 matrix cores
ROTATION_BYTES = 512 << 20        # > 256 MB Infinity Cache
TRAFFIC_FILE = os.path.join(REPO, "profiles", "matmul_traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algo_bytes(qtype: int, n_out: int, n_in: int) -> int:
    """Compulsory traffic of one matmul: weights once, fp32 x once, fp32 y once."""
    return synth.row_nbytes(qtype, n_in) * n_out + 4 * n_in + 4 * n_out


def bench_gemv(g, qtype: int, n_out: int, n_in: int, steps: int, warmup: int, seed: int,
               eager: bool = False) -> dict:
    rng = np.random.default_rng(seed)
    w = synth.weight(rng, qtype, n_out, n_in)
    x = synth.activation(rng, n_in)
    copies = max(2, math.ceil(ROTATION_BYTES / w.nbytes))
    dws = [g.upload(w) for _ in range(copies)]
    dx, dout = g.upload(x), g.alloc(4 * n_out)

    def launch(k):
        g.matmul(dout, dx, qtype, dws[k % copies], None, n_out, n_in)

    res = _time_launches(g, launch, steps, warmup, eager)
    for b in dws + [dx, dout]:
        b.free()
    nbytes = algo_bytes(qtype, n_out, n_in)
    res.update({"n_out": n_out, "n_in": n_in, "qtype": qtype, "weight_copies": copies, "algo_bytes": nbytes,
                "gbps": nbytes / (res["us_per_launch"] * 1e-6) / 1e9})
    return res


def bench_copy(g, nbytes: int, steps: int, warmup: int, eager: bool) -> dict:
    """A plain 16-byte-per-lane copy of known size (the byte-counter calibration)."""
    copies = max(2, math.ceil(ROTATION_BYTES / nbytes))
    srcs = [g.alloc(nbytes) for _ in range(copies)]
    dst = g.alloc(nbytes)

    def launch(k):
        g.check(g.lib.hako_gpu_memcpy_d2d(dst.ptr, srcs[k % copies].ptr, nbytes), "d2d")

    res = _time_launches(g, launch, steps, warmup, eager)
    for b in srcs + [dst]:
        b.free()
    res.update({"algo_bytes": 2 * nbytes, "gbps": 2 * nbytes / (res["us_per_launch"] * 1e-6) / 1e9})
    return res


def _time_launches(g, launch, steps: int, warmup: int, eager: bool, spread_reps: int = 8) -> dict:
    """K launches: replayed from a captured HIP graph between two device
    wall-clock marks inside the graph, or (eager) issued one by one from
    Python between two events, as profilers' per-dispatch counter collection
    needs. Also the median single-launch latency and (graph) the p10 / p50 /
    p90 of the per-launch time over the first replay and `spread_reps` more."""
    e0, e1 = g.event(), g.event()
    if eager:
        for k in range(warmup):
            launch(k)
        g.sync()
        g.record(e0)
        for k in range(warmup, warmup + steps):
            launch(k)
        g.record(e1)
        ms = g.elapsed_ms(e0, e1)
    else:
        def capture(k0, n):
            g.capture_begin()
            for k in range(k0, k0 + n):
                launch(k)
            return g.capture_end()
        # the warm-up graph holds at least 64 launches, so the host queues its
        # replays faster than the GPU runs them
        nwarm = max(warmup, 64)
        warm = capture(0, nwarm)
        # The timed graph: nwarm lead-in launches, wall-clock mark t0, the K
        # timed launches, marks t1 and t2. The marks are one-wave kernels that
        # are nodes of the graph, so the timed region holds neither the
        # start-up of a graph launch (~14 us on an idle queue) nor anything of
        # the host; t1 - t0 spans the t0 mark's own slot and the K launches,
        # t2 - t1 one mark's slot, which is subtracted. The timed launches
        # start on the weight copy after the lead-in's last, so none of them
        # finds its weights left in the last-level cache.
        stamps = g.alloc(64)
        g.capture_begin()
        for k in range(nwarm, 2 * nwarm):
            launch(k)
        g.timestamp(stamps.offset(0))
        for k in range(2 * nwarm, 2 * nwarm + steps):
            launch(k)
        g.timestamp(stamps.offset(8))
        g.timestamp(stamps.offset(16))
        timed = g.capture_end()
        # the warm-up graph replayed for at least 30 ms: a GPU idle during the
        # host-side set-up runs its first milliseconds at lower clocks
        g.record(e0)
        g.graph_launch(warm)
        g.record(e1)
        reps = int(math.ceil(30.0 / max(g.elapsed_ms(e0, e1), 1e-3)))
        for _ in range(min(reps, 1000)):
            g.graph_launch(warm)
        g.record(e0)
        g.graph_launch(timed)
        g.record(e1)
        graph_ms = g.elapsed_ms(e0, e1)

        def region_ms():
            t = g.download(stamps, np.uint64, (3,)).astype(np.int64)
            ticks = int(t[2] - t[1])
            return (int(t[1] - t[0]) - ticks) / g.timestamp_hz() * 1e3, ticks

        ms, mark_ticks = region_ms()
        # The spread: the same timed graph replayed `spread_reps` more times (each
        # replay starts with its own lead-in launches); `ms` stays the first
        # replay's, the K launches the caller asked for.
        rep_ms = [ms]
        for _ in range(spread_reps):
            g.graph_launch(timed)
            rep_ms.append(region_ms()[0])
        stamps.free()
        g.graph_destroy(warm)
        g.graph_destroy(timed)
    single = []
    for k in range(51):
        g.record(e0)
        launch(k)
        g.record(e1)
        single.append(g.elapsed_ms(e0, e1))
    res = {"ms_total": ms, "us_per_launch": ms * 1e3 / steps, "single_launch_us": float(np.median(single)) * 1e3,
           "single_launch_us_p10_p90": [float(np.percentile(single, q)) * 1e3 for q in (10, 90)]}
    if not eager:
        res["graph_ms_with_lead_in"] = graph_ms
        res["mark_slot_us"] = mark_ticks / g.timestamp_hz() * 1e6
        per = np.array(rep_ms) * 1e3 / steps
        res["us_per_launch_p10_p50_p90"] = [float(np.percentile(per, q)) for q in (10, 50, 90)]
        res["timed_replays"] = len(rep_ms)
    return res


def host_info() -> dict:
    """The host the CPU baselines ran on, and how the reference was compiled."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    compiler = flags = ""
    try:
        with open(os.path.join(REPO, "oracle", "_ref", "build_info.txt")) as f:
            lines = f.read().splitlines()
        compiler, flags = (lines + ["", ""])[:2]
    except OSError:
        pass
    return {"cpu_model": model, "nproc": avail, "cpu_count": os.cpu_count(), "compiler": compiler,
            "flags": flags}


MAX_THREADS = 16                  # the reference caps its pool at 16 (src/nn.c:61,104)
_REF = {}


def ref_lib(threads: int):
    """The reference's own C path (oracle/_ref, compiled unmodified from its
    sources) with a pool of `threads` threads. Its thread count is read once
    per loaded copy, at the first matmul (src/nn.c:99-107), so every count gets
    its own copy of the library, and that first matmul happens here, with
    n_out >= threads (a smaller first call starts the pool without workers and
    later calls deadlock, src/nn.c:182-184)."""
    if threads not in _REF:
        import shutil
        import tempfile
        from oracle.hako_oracle import REF_LIB, RefLib
        path = os.path.join(tempfile.mkdtemp(prefix="hakm_ref_"), f"libhakm_ref_t{threads}.so")
        shutil.copy(REF_LIB, path)
        ref = RefLib(path, threads=threads)
        rng = np.random.default_rng(0)
        ref.matmul(synth.TYPE_Q4_K, synth.q4k_weight(rng, 1024, 256), synth.activation(rng, 256), 1024, 256)
        _REF[threads] = ref
    return _REF[threads]


def cpu_threads() -> int:
    return min(host_info()["nproc"], MAX_THREADS)


def time_ref_matmul(ref, qtype: int, ws: list, x: np.ndarray, n_out: int, n_in: int, seconds: float,
                    min_calls: int) -> tuple[float, int]:
    """Median wall time of the reference matmul (src/nn.c:179-210) over
    rotating weight copies, for `seconds` and at least `min_calls` calls."""
    ref.matmul(qtype, ws[0], x, n_out, n_in)
    times, t_end, k = [], time.perf_counter() + seconds, 0
    while time.perf_counter() < t_end or len(times) < min_calls:
        t0 = time.perf_counter()
        ref.matmul(qtype, ws[k % len(ws)], x, n_out, n_in)
        times.append(time.perf_counter() - t0)
        k += 1
    return float(np.median(times)), len(times)


def cpu_gemv_baseline(qtype: int, n_out: int, n_in: int, seconds: float, seed: int, copies: int = 8) -> dict:
    """The reference's matmul on one GEMV shape at T = min(nproc, 16) threads
    and at T = 1, rotating weight copies."""
    rng = np.random.default_rng(seed)
    ws = [synth.weight(rng, qtype, n_out, n_in) for _ in range(copies)]
    x = synth.activation(rng, n_in)
    nbytes = algo_bytes(qtype, n_out, n_in)
    T = cpu_threads()
    med, calls = time_ref_matmul(ref_lib(T), qtype, ws, x, n_out, n_in, seconds, 20)
    med1, calls1 = time_ref_matmul(ref_lib(1), qtype, ws, x, n_out, n_in, seconds / 4, 3)
    name = "Q4_K" if qtype == synth.TYPE_Q4_K else "Q6_K"
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": T, "kind": "reference",
            "t1_value": round(nbytes / med1 / 1e9, 3),
            "sample": f"{calls} calls (T={T}) and {calls1} calls (T=1) of the reference matmul on {name} "
                      f"{n_out}x{n_in} ({copies} rotating weight copies); median {med * 1e3:.3f} ms/call at "
                      f"T={T}, {med1 * 1e3:.3f} ms/call at T=1",
            "host": host_info()}


def cpu_baseline(seconds: float, seed: int) -> dict:
    """The reference's matmul (src/nn.c:179-210, compiled unmodified with its
    Makefile flags) on the headline shape."""
    return cpu_gemv_baseline(synth.TYPE_Q4_K, 11008, 2048, seconds, seed)


def cpu_prefill_baseline(qtype: int, m: int, n_out: int, n_in: int, seed: int) -> dict:
    """The reference has no multi-token matmul: a prompt is one matmul call
    per token (cli/main.c:56-60). Times m sequential calls at T = min(nproc,
    16) over the m activation rows."""
    rng = np.random.default_rng(seed)
    w = synth.weight(rng, qtype, n_out, n_in)
    xs = rng.standard_normal((m, n_in)).astype(np.float32)
    T = cpu_threads()
    ref = ref_lib(T)
    ref.matmul(qtype, w, xs[0], n_out, n_in)
    t0 = time.perf_counter()
    for t in range(m):
        ref.matmul(qtype, w, xs[t], n_out, n_in)
    sec = time.perf_counter() - t0
    ops = 2.0 * m * n_out * n_in
    return {"value": round(ops / sec / 1e12, 4), "unit": "TOPS" if qtype == synth.TYPE_Q4_K else "TFLOP/s",
            "cores": T, "kind": "reference", "tok_per_s": round(m / sec, 1),
            "sample": f"{m} sequential calls of the reference matmul ({'Q4_K' if qtype == synth.TYPE_Q4_K else 'Q6_K'}"
                      f" {n_out}x{n_in}), one per activation row, T={T}: {sec * 1e3:.1f} ms",
            "host": host_info()}


def bench_decode(g, steps: int, cpu_steps: int, seed: int = 30, shape: str = "3b") -> dict:
    """Batch-1 greedy decode with the KV cache prefilled to 1024 positions of
    seeded N(0,1) keys and values: shape "3b" is the Qwen2.5-3B shape (36
    layers, Q4_K_M mix, tied Q6_K embedding), "7b" the Qwen2-7B shape (28
    layers, Q4_K attn/gate/up, Q6_K down and untied output), random weights.
    `steps` graph-replayed device steps; the reference's own hakm_forward on
    the same file and cache timed for `cpu_steps` tokens on the host cores."""
    import tempfile
    from hako_amd import mlf2
    from hako_amd.decoder import Decoder
    cfg, pos = (mlf2.QWEN2_3B if shape == "3b" else mlf2.QWEN2_7B), 1024
    max_seq = pos + steps + 8
    kvd = cfg.n_kv_heads * cfg.head_dim
    fd, path = tempfile.mkstemp(suffix=".mlf2")
    os.close(fd)
    try:
        info = mlf2.write_qwen2(path, cfg, seed)
        kv = np.random.default_rng(seed + 1).standard_normal((2, cfg.n_layers, pos, kvd)).astype(np.float32)
        dec = Decoder(g, path, n_seq=1, max_seq=max_seq)
        try:
            k, v = dec.kv()
            for l in range(cfg.n_layers):
                g.h2d(k + dec.kv_offset(0, l, 0), kv[0, l])
                g.h2d(v + dec.kv_offset(0, l, 0), kv[1, l])
            dec.set_pos(pos)
            dec.generate(9, 4)          # capture and warm
            g.sync()
            dec.set_pos(pos)
            e0, e1 = g.event(), g.event()
            g.record(e0)
            dec.replay(steps)
            g.record(e1)
            ms = g.elapsed_ms(e0, e1)
        finally:
            dec.close()
        # an untied embedding contributes one row per token, not its matrix
        weight_bytes = sum(e[4] for name, e in info.items() if cfg.tied or name != "token_embd.weight")
        kv_bytes = cfg.n_layers * 2 * kvd * 4 * (pos + 1 + steps // 2)
        per_tok = weight_bytes + kv_bytes
        us = ms * 1e3 / steps
        res = {"workload": ("Qwen2.5-3B-shaped greedy decode (36 layers, Q4_K attn/gate/up, Q6_K down and tied "
                            "embedding), batch 1, KV cache from position 1024") if shape == "3b" else
                           ("Qwen2-7B-shaped greedy decode (28 layers, Q4_K attn/gate/up, Q6_K down and untied "
                            "output), batch 1, KV cache from position 1024"),
               "steps": steps, "us_per_token": round(us, 2), "tok_per_s": round(1e6 / us, 1),
               "bytes_per_token": per_tok, "gbps": round(per_tok / (us * 1e-6) / 1e9, 1),
               "hbm_frac": round(per_tok / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
               "timing": "HIP graph of one step replayed K times between two HIP events"}
        if cpu_steps > 0:
            from oracle.hako_oracle import prefilled_greedy
            threads = cpu_threads()
            times, times1 = [], []
            prefilled_greedy(ref_lib(threads).lib, path, kv, pos, 9, cpu_steps + 1, cfg.vocab, max_seq, times)
            prefilled_greedy(ref_lib(1).lib, path, kv, pos, 9, 2, cfg.vocab, max_seq, times1)
            med = float(np.median(times[1:]))
            res["cpu_baseline"] = {"value": round(1.0 / med, 3), "unit": "tok/s", "cores": threads,
                                   "kind": "reference", "t1_value": round(1.0 / times1[1], 3),
                                   "sample": f"{cpu_steps} hakm_forward steps (after one warm-up) of the reference "
                                             f"on the same model file and cache, {threads} threads, median "
                                             f"{med * 1e3:.1f} ms/token; one step at T=1: "
                                             f"{times1[1] * 1e3:.1f} ms",
                                   "host": host_info()}
        return res
    finally:
        os.unlink(path)


def bench_decode_batched(g, steps: int, cpu_steps: int, seed: int = 40, n_seq: int = 16) -> dict:
    """Greedy decode of 16 sequences of a Qwen2-7B-shaped model (28 layers,
    Q4_K attn/gate/up and embedding, Q6_K down and untied output, random
    weights), every sequence's KV cache prefilled with 4095 positions of seeded
    N(0,1) keys and values, so that the first step writes position 4096:
    `steps` graph-replayed steps, each advancing all 16 sequences. The
    reference steps one hakm_ctx per sequence; its hakm_forward on the same
    file and a cache of the same length is timed for `cpu_steps` tokens."""
    import tempfile
    from hako_amd import mlf2
    from hako_amd.decoder import Decoder
    cfg, pos = mlf2.QWEN2_7B, 4095
    max_seq = pos + steps + 8
    kvd = cfg.n_kv_heads * cfg.head_dim
    fd, path = tempfile.mkstemp(suffix=".mlf2")
    os.close(fd)
    try:
        info = mlf2.write_qwen2(path, cfg, seed)
        # one seeded N(0,1) cache, copied to every sequence's own (distinct) slots
        kv = np.random.default_rng(seed + 1).standard_normal((2, cfg.n_layers, pos, kvd)).astype(np.float32)
        starts = (np.arange(n_seq, dtype=np.int32) * 9973 + 11) % cfg.vocab
        dec = Decoder(g, path, n_seq=n_seq, max_seq=max_seq)
        try:
            k, v = dec.kv()
            for s in range(n_seq):
                for l in range(cfg.n_layers):
                    g.h2d(k + dec.kv_offset(s, l, 0), kv[0, l])
                    g.h2d(v + dec.kv_offset(s, l, 0), kv[1, l])
            dec.set_pos(pos)
            dec.generate(starts, 4)     # capture and warm
            g.sync()
            dec.set_pos(pos)
            e0, e1 = g.event(), g.event()
            g.record(e0)
            dec.replay(steps)
            g.record(e1)
            ms = g.elapsed_ms(e0, e1)
        finally:
            dec.close()
        # the untied embedding contributes one row per sequence, not its matrix
        weight_bytes = sum(e[4] for name, e in info.items() if name != "token_embd.weight")
        kv_bytes = n_seq * cfg.n_layers * 2 * kvd * 4 * (pos + 1 + (steps - 1) / 2)
        per_step = weight_bytes + kv_bytes
        us = ms * 1e3 / steps
        res = {"workload": "Qwen2-7B-shaped greedy decode (28 layers, Q4_K attn/gate/up, Q6_K down and untied "
                           "output), 16 sequences per step, each KV cache from position 4095",
               "n_seq": n_seq, "steps": steps, "us_per_step": round(us, 2),
               "tok_per_s": round(n_seq * 1e6 / us, 1), "bytes_per_step": int(per_step),
               "gbps": round(per_step / (us * 1e-6) / 1e9, 1),
               "hbm_frac": round(per_step / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
               "timing": "HIP graph of one 16-sequence step replayed K times between two HIP events"}
        if cpu_steps > 0:
            from oracle.hako_oracle import prefilled_greedy
            threads = cpu_threads()
            times = []
            prefilled_greedy(ref_lib(threads).lib, path, kv, pos, int(starts[0]), cpu_steps + 1, cfg.vocab,
                             pos + cpu_steps + 2, times)
            med = float(np.median(times[1:]))
            res["cpu_baseline"] = {"value": round(1.0 / med, 3), "unit": "tok/s", "cores": threads,
                                   "kind": "reference",
                                   "sample": f"{cpu_steps} hakm_forward steps (after one warm-up) of the reference "
                                             f"on the same model file, one sequence with its cache at position "
                                             f"4095, {threads} threads, median {med * 1e3:.1f} ms/token (the "
                                             f"reference steps its 16 contexts one after another)",
                                   "host": host_info()}
        return res
    finally:
        os.unlink(path)


def bench_prompt(g, n_prompt: int, cpu_tokens: int, seed: int = 50) -> dict:
    """A 512-token prompt fed to a Qwen2-7B-shaped model (28 layers, Q4_K
    attn/gate/up, Q6_K down and untied output, random weights) from position
    0: hako_gpu_decoder_prefill, 512 tokens per pass through the multi-token
    matmuls. The reference feeds a prompt one hakm_forward per token
    (src/hakm_api.c:105-111); its rate is timed on `cpu_tokens` tokens."""
    import tempfile
    from hako_amd import mlf2
    from hako_amd.decoder import Decoder
    cfg = mlf2.QWEN2_7B
    fd, path = tempfile.mkstemp(suffix=".mlf2")
    os.close(fd)
    try:
        info = mlf2.write_qwen2(path, cfg, seed)
        prompt = np.random.default_rng(seed).integers(0, cfg.vocab, n_prompt).astype(np.int32)
        dec = Decoder(g, path, n_seq=1, max_seq=n_prompt + 8)
        try:
            # warm: workspaces, first-touch, and the clocks of a GPU that sat
            # idle through the model's set-up (one warm call left the first
            # timed calls ~8% slower)
            for _ in range(3):
                dec.set_pos(0)
                dec.prefill(prompt)
            times = []
            for _ in range(5):
                dec.set_pos(0)
                t0 = time.perf_counter()
                dec.prefill(prompt)     # synchronous
                times.append(time.perf_counter() - t0)
        finally:
            dec.close()
        sec = float(np.median(times))
        weight_bytes = sum(e[4] for name, e in info.items() if name != "token_embd.weight")
        res = {"workload": f"Qwen2-7B-shaped prompt prefill, {n_prompt} tokens from position 0 (28 layers, Q4_K "
                           "attn/gate/up, Q6_K down and untied output)",
               "tokens": n_prompt, "ms": round(sec * 1e3, 2), "tok_per_s": round(n_prompt / sec, 1),
               "weight_passes": (n_prompt + 511) // 512,
               "weight_gbps": round(weight_bytes * ((n_prompt + 511) // 512) / sec / 1e9, 1),
               "timing": "host wall clock around the synchronous call, median of 5 after three warm-up calls"}
        if cpu_tokens > 0:
            threads = cpu_threads()
            lib = ref_lib(threads).lib
            ctx = lib.hakm_ctx_new(path.encode(), n_prompt + 8)
            assert ctx
            try:
                tt = []
                for t in prompt[:cpu_tokens + 1]:
                    t0 = time.perf_counter()
                    lib.hakm_forward(ctx, int(t))
                    tt.append(time.perf_counter() - t0)
            finally:
                lib.hakm_ctx_free(ctx)
            med = float(np.median(tt[1:]))
            res["cpu_baseline"] = {"value": round(1.0 / med, 3), "unit": "tok/s", "cores": threads,
                                   "kind": "reference",
                                   "sample": f"the first {cpu_tokens} prompt tokens (after one warm-up) fed with the "
                                             f"reference's hakm_forward on the same model file, {threads} threads, "
                                             f"median {med * 1e3:.1f} ms/token (its feed is one forward per token)",
                                   "host": host_info()}
        return res
    finally:
        os.unlink(path)


def bench_prefill(g, launches: int, eager: bool = False, cpu: bool = False) -> dict:
    """The 7B prefill matmuls: Q4_K 18944x3584 x 512 tokens (q8_32 quantize +
    int8-MFMA GEMM) and Q6_K 3584x18944 x 512 tokens (fp16-MFMA GEMM).
    `eager` launches from Python (per-dispatch counter collection)."""
    out = {}
    for name, qt, m, n_out, n_in in (("q4k_7b_ffn_up_512x18944x3584", synth.TYPE_Q4_K, 512, 18944, 3584),
                                     ("q6k_7b_ffn_down_512x3584x18944", synth.TYPE_Q6_K, 512, 3584, 18944)):
        rng = np.random.default_rng(n_out)
        w = synth.weight(rng, qt, n_out, n_in)
        x = rng.standard_normal((m, n_in)).astype(np.float32)
        dw, dx, dy = g.upload(w), g.upload(x), g.alloc(m * n_out * 4)
        g.matmul_batch(dy, dx, qt, dw, None, m, n_out, n_in)   # sizes the workspace outside the capture
        g.sync()
        r = _time_launches(g, lambda k: g.matmul_batch(dy, dx, qt, dw, None, m, n_out, n_in), launches, 3, eager)
        for b in (dw, dx, dy):
            b.free()
        ops = 2.0 * m * n_out * n_in
        tops = ops / (r["us_per_launch"] * 1e-6) / 1e12
        peak = INT8_PEAK_TOPS if qt == synth.TYPE_Q4_K else FP16_PEAK_TFLOPS
        traffic, ratio = read_traffic(("q4k_gemm_7b_ffn_up_512x18944x3584" if qt == synth.TYPE_Q4_K
                                       else "q6k_gemm_7b_ffn_down_512x3584x18944"))
        out[name] = {"us_per_launch": round(r["us_per_launch"], 2), "tops": round(tops, 1),
                     "peak": peak, "frac": round(tops / peak, 4),
                     "unit": "TOPS (int8)" if qt == synth.TYPE_Q4_K else "TFLOP/s (fp16 matrix cores)",
                     "traffic": traffic, "traffic_over_algorithmic": ratio}
        if cpu:
            out[name]["cpu_baseline"] = cpu_prefill_baseline(qt, m, n_out, n_in, n_out)
    return out


def read_traffic(name: str):
    """HBM bytes per launch (fetched + written) of workload `name` from the
    calibrated rocprofv3 counter summary, and their ratio to the algorithmic
    bytes; (None, None) when the summary has no entry."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)["workloads"][name]
        total = float(t["fetch_bytes_per_launch"]) + float(t["write_bytes_per_launch"])
        return total, round(total / float(t["algorithmic_bytes_per_launch"]), 3)
    except (OSError, KeyError, ValueError):
        return None, None


# name -> (type, n_out, n_in, default steps); the first is the headline.
WORKLOADS = {
    "q4k_3b_ffn_up_11008x2048": (synth.TYPE_Q4_K, 11008, 2048, None),
    "q4k_7b_ffn_up_18944x3584": (synth.TYPE_Q4_K, 18944, 3584, 1000),
    "q6k_3b_ffn_down_2048x11008": (synth.TYPE_Q6_K, 2048, 11008, 1000),
    "q6k_3b_vocab_151936x2048": (synth.TYPE_Q6_K, 151936, 2048, 200),
    "q6k_7b_ffn_down_3584x18944": (synth.TYPE_Q6_K, 3584, 18944, 500),
}
HEADLINE = "q4k_3b_ffn_up_11008x2048"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--only", choices=sorted(WORKLOADS) + ["copy", "decode", "decode7b", "decode16", "prompt",
                                                          "prefill"],
                    help="run one workload and print its timing only (profiling runs)")
    ap.add_argument("--eager", action="store_true", help="launch from Python instead of a HIP graph")
    ap.add_argument("--decode-steps", type=int, default=100)
    ap.add_argument("--cpu-decode-steps", type=int, default=3)
    ap.add_argument("--batched-steps", type=int, default=30)
    ap.add_argument("--prompt-tokens", type=int, default=512)
    ap.add_argument("--cpu-prompt-tokens", type=int, default=4)
    ap.add_argument("--cpu-batched-steps", type=int, default=2)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              f"(the GEMV shards by rows; this build runs and measures one GPU)", file=sys.stderr)
        sys.exit(2)

    from hako_amd.gpu import Gpu
    g = Gpu(0)
    info = g.info()
    log(f"device {info.name.decode()} CUs={info.compute_units} HBM={info.hbm_bytes / 2**30:.0f} GiB")

    if args.only in ("decode", "decode7b", "decode16", "prompt", "prefill"):
        if args.only == "decode":
            r = bench_decode(g, args.decode_steps, 0)
        elif args.only == "decode7b":
            r = bench_decode(g, args.decode_steps, 0, seed=35, shape="7b")
        elif args.only == "decode16":
            r = bench_decode_batched(g, args.batched_steps, 0)
        elif args.only == "prompt":
            r = bench_prompt(g, args.prompt_tokens, 0)
        else:
            r = bench_prefill(g, 30, args.eager)
        print(json.dumps(r), flush=True)
        return
    if args.only:
        if args.only == "copy":
            r = bench_copy(g, 64 << 20, args.steps, args.warmup, args.eager)
        else:
            qt, n_out, n_in, _ = WORKLOADS[args.only]
            r = bench_gemv(g, qt, n_out, n_in, args.steps, args.warmup, seed=n_out, eager=args.eager)
        r["workload"] = args.only
        print(json.dumps(r), flush=True)
        return

    qt, n_out, n_in, _ = WORKLOADS[HEADLINE]
    head = bench_gemv(g, qt, n_out, n_in, args.steps, args.warmup, seed=1)
    log(f"{HEADLINE}: {head['us_per_launch']:.2f} us/launch, {head['gbps']:.0f} GB/s")
    extra = {}
    if not args.no_extra:
        for name, (qt, n_out, n_in, steps) in WORKLOADS.items():
            if name == HEADLINE:
                continue
            r = bench_gemv(g, qt, n_out, n_in, steps, 20, seed=n_out)
            log(f"{name}: {r['us_per_launch']:.2f} us/launch, {r['gbps']:.0f} GB/s")
            traffic, ratio = read_traffic(name)
            extra[name] = {"us_per_launch": round(r["us_per_launch"], 3), "gbps": round(r["gbps"], 1),
                           "hbm_frac": round(r["gbps"] / HBM_PEAK_GBPS, 4),
                           "us_per_launch_p10_p50_p90": [round(v, 3) for v in r["us_per_launch_p10_p50_p90"]],
                           "single_launch_us": round(r["single_launch_us"], 3),
                           "single_launch_us_p10_p90": [round(v, 3) for v in r["single_launch_us_p10_p90"]],
                           "traffic": traffic, "traffic_over_algorithmic": ratio}
            if not args.no_cpu:
                # copies kept to about 1.3 GB of host memory for the vocab shape
                extra[name]["cpu_baseline"] = cpu_gemv_baseline(qt, n_out, n_in, args.cpu_seconds / 4, seed=n_out,
                                                                copies=8 if n_out < 100000 else 4)
                log(f"  cpu: {extra[name]['cpu_baseline']['value']:.2f} GB/s")
    decode = None
    if not args.no_decode:
        decode = bench_decode(g, args.decode_steps, 0 if args.no_cpu else args.cpu_decode_steps)
        log(f"decode: {decode['us_per_token']:.1f} us/token, {decode['tok_per_s']:.1f} tok/s, "
            f"{decode['gbps']:.0f} GB/s" + (f"; cpu {decode['cpu_baseline']['value']:.2f} tok/s"
                                          if 'cpu_baseline' in decode else ""))
    decode7 = None
    if not args.no_decode:
        decode7 = bench_decode(g, args.decode_steps, 0 if args.no_cpu else args.cpu_decode_steps, seed=35,
                               shape="7b")
        log(f"decode 7B: {decode7['us_per_token']:.1f} us/token, {decode7['tok_per_s']:.1f} tok/s, "
            f"{decode7['gbps']:.0f} GB/s" + (f"; cpu {decode7['cpu_baseline']['value']:.2f} tok/s"
                                           if 'cpu_baseline' in decode7 else ""))
    batched = None
    if not args.no_decode:
        batched = bench_decode_batched(g, args.batched_steps, 0 if args.no_cpu else args.cpu_batched_steps)
        log(f"decode x16: {batched['us_per_step']:.1f} us/step, {batched['tok_per_s']:.1f} tok/s, "
            f"{batched['gbps']:.0f} GB/s" + (f"; cpu {batched['cpu_baseline']['value']:.3f} tok/s"
                                           if 'cpu_baseline' in batched else ""))
    prompt = None
    if not args.no_prefill:
        prompt = bench_prompt(g, args.prompt_tokens, 0 if args.no_cpu else args.cpu_prompt_tokens)
        log(f"prompt: {prompt['tokens']} tokens in {prompt['ms']:.1f} ms, {prompt['tok_per_s']:.0f} tok/s"
            + (f"; cpu {prompt['cpu_baseline']['value']:.2f} tok/s" if 'cpu_baseline' in prompt else ""))
    prefill = None
    if not args.no_prefill:
        prefill = bench_prefill(g, 30, cpu=not args.no_cpu)
        for k, v in prefill.items():
            log(f"{k}: {v['us_per_launch']:.1f} us, {v['tops']:.1f} {v['unit']}")
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_seconds, seed=2)
        log(f"cpu baseline: {cpu['value']:.2f} GB/s ({cpu['sample']})")

    value = head["gbps"]
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": head["us_per_launch"] / 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded Q4_K blocks and N(0,1) activations)",
        "config": {"workload": "Q4_K x q8 matmul (q8_32 quantize + GEMV, one launch), Qwen2.5-3B ffn_up "
                               "11008x2048, batch 1", "n_out": 11008, "n_in": 2048,
                   "weight_copies": head["weight_copies"], "algo_bytes_per_step": head["algo_bytes"],
                   "timing": "K launches in a HIP graph after 64 lead-in launches, between two device wall-clock "
                             "marks in the graph (one mark's own slot subtracted)"},
        "hbm_frac": round(value / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "achieved": round(head["gbps"], 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(head["gbps"] / HBM_PEAK_GBPS, 4), "traffic": read_traffic(HEADLINE)[0]},
        "cpu_baseline": cpu,
        "single_launch_us": round(head["single_launch_us"], 3),
        "single_launch_us_p10_p90": [round(v, 3) for v in head["single_launch_us_p10_p90"]],
        "us_per_launch_p10_p50_p90": [round(v, 3) for v in head["us_per_launch_p10_p50_p90"]],
        "timed_replays": head["timed_replays"],
        "extra": extra,
        "decode": decode,
        "decode_7b": decode7,
        "decode_batched": batched,
        "prompt_prefill": prompt,
        "prefill": prefill,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
