"""Benchmarks of the paged KV path on one MI355X.

With no --workload the run covers every configuration of the path, one JSON
line each, the headline last:

  c1     SmolLM2-135M decode: 1 sequence x 512 tokens, 9/3 heads, d=64, f32;
  t176   the reference's T176 cache case: 1 sequence x 1,025 tokens, 4/2
         heads, d=32, f32 (latency beside the reference's published figure);
  c3     KV-management stress: 256 sequences forked from a 1,024-token
         prefix, 22 layers x 8 x 64 f32, one appended token per sequence a
         step (c3cow: a 1,025-token prefix, so the first step copies 256
         shared tail blocks);
  c4     chunked prefill: 8 x (2,048 cached + 512-token causal chunk), 32/8
         heads, d=64, bf16 MFMA;
  c5     Llama-3-8B decode: 16 x 32,768 tokens, 32/8 heads, d=128, Q8_0;
  prefix the prefix cache: the reference's radix benchmark (10,000 lookups
         with a KV restore, 75% hits), ns per request beside its published
         933 ns;
  llama1b  a Llama-3.2-1B-shaped model with random Q8_0 weights through the
         model-level C ABI: 64 sequences a step, and one sequence alone;
  c2     (headline, printed last) Llama-3.2-1B decode: 64 sequences, 32/8
         heads, d=64, f32 KV, contexts uniform in [128, 4096], 16-token blocks
         scattered over a 65,536-block pool.

A decode step is one batched paged decode attention launch (decode kernel
plus the split merge) with every input resident in HBM before the timed
region; value = algorithmic bytes per step / step time.  The roofline is the
dominant kernel's algorithmic bytes (or flops) over its own duration, from
HIP events the library records around its launches in a second pass of the
same steps.  Each line carries the reference's own CPU path (oracle/_ref,
built from its sources) timed on this host: one warm-up, then the median of
nine runs, on one thread and on every host thread the box grants, with the
host's CPU model, core count, compiler, flags, AVX2 use and a STREAM-style
triad bandwidth.

Other shapes, one line each with --workload: c4d128, c4q8 and c4f32 (the
chunks at head_dim 128, over Q8_0 blocks, and in f32 through the decode
kernels), c4x3 / c4x3d128 / c4q8x3 (the three-product tiles at f32
accuracy), gqa8 / gqa8q8 (Llama-3-70B, eight query
heads per KV head), gqa16 / gqa16q8 (Llama-3.1-405B, sixteen, run as two
slices), tiny / tinyq8 (TinyLlama-1.1B), gemma2 (head_dim 256), phi3
(head_dim 96).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
MFMA_BF16_PEAK_TFS = 2500.0  # MI355X dense bf16
METRIC = "paged decode attn: achieved HBM GB/s (% of peak) + decode tokens/s, 1 MI355X"
MODEL_LAYERS = {"llama-3.2-1b-decode-64x[128,4096]": 16, "smollm2-135m-decode-1x512": 30,
                "llama-3-8b-q8_0-decode-16x32768": 32}
DEFAULT_RUN = ["c1", "t176", "c3", "c3cow", "c4", "c5", "prefix", "conv", "llama1b", "c2"]
REF_FLAGS = "g++ -O2 -std=c++20 -fPIC (oracle/Makefile, target ref; the reference's recorded flags)"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ----------------------------------------------------------- CPU baseline

def host_threads():
    """Host threads the CPU baseline uses: what the process may run on,
    capped at 16 (the host threads a machine grants one GPU's job)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


_HOST = None


def host_info():
    """The host the CPU baseline ran on (recorded once per run)."""
    global _HOST
    if _HOST is None:
        from oracle import pyoracle

        model = "unknown"
        try:
            for line in Path("/proc/cpuinfo").read_text().splitlines():
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
        try:
            gxx = subprocess.run(["g++", "-dumpfullversion"], capture_output=True, text=True).stdout.strip()
        except OSError:
            gxx = "unknown"
        t = host_threads()
        doubles = 1 << 24  # 128 MiB per array
        _HOST = {"cpu": model, "nproc": os.cpu_count(), "threads_used": t, "compiler": f"g++ {gxx}",
                 "flags": REF_FLAGS, "avx2_dot": pyoracle.ref_uses_avx2(),
                 "triad_GBps_1thread": round(pyoracle.host_triad_gbs(doubles, 1), 2),
                 f"triad_GBps_{t}threads": round(pyoracle.host_triad_gbs(doubles, t), 2)}
        log("host:", json.dumps(_HOST))
    return _HOST


def median_of_9(run):
    """One warm-up run, then the median of nine (tests/core/prefill_support.hpp:13-16)."""
    run()
    times = []
    for _ in range(9):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_result(unit, one, alln, threads, sample, work_per_run_one, work_per_run_all, extra=None):
    """A cpu_baseline object: value and cores from the all-thread run (on
    `threads` threads), the one-thread run beside it."""
    t = threads
    out = {"value": round(work_per_run_all / alln, 6), "unit": unit, "cores": t, "kind": "reference",
           "sample": sample, "protocol": "1 warm-up, median of 9 runs",
           "one_thread": {"value": round(work_per_run_one / one, 6), "unit": unit, "cores": 1,
                          "ms_per_run": round(one * 1e3, 3)},
           "all_threads": {"value": round(work_per_run_all / alln, 6), "unit": unit, "cores": t,
                           "ms_per_run": round(alln * 1e3, 3)},
           "host": host_info()}
    if extra:
        out.update(extra)
    return out


# Where the default run parks the host baselines: every GPU measurement runs
# first, back to back, so no configuration's timed steps follow seconds of an
# idle GPU; the baselines then run and fill in their lines.
DEFERRED = None


def baseline(result, job):
    """Fill result["cpu_baseline"] with job(), now or after the GPU runs."""
    if DEFERRED is not None:
        DEFERRED.append((result, job))
    else:
        result["cpu_baseline"] = job()


def ref_ready(args):
    if args.no_cpu_baseline:
        return False
    from oracle import pyoracle

    if not pyoracle.ref_available():
        log("cpu baseline skipped: oracle/_ref is not built")
        return False
    return True


# ------------------------------------------------------------- GPU timing

def timed_steps(call, steps):
    """ms per step over `steps` back-to-back calls, bracketed by device
    synchronisation and HIP events on the library's stream (the null stream)."""
    from tvara_amd import hip

    start, stop = hip.Event(), hip.Event()
    hip.synchronize()
    start.record()
    for _ in range(steps):
        call()
    stop.record()
    hip.synchronize()
    return start.elapsed_ms(stop) / steps


def kernel_times(call, steps, names):
    """Average duration of each named kernel over `steps` more calls, from the
    HIP event pair the library records around its own launches (kept out of
    the throughput region: the extra event packets add gaps between launches)."""
    from tvara_amd import attention, hip

    attention.profile_reset()
    attention.profile_enable(True)
    hip.synchronize()
    for _ in range(steps):
        call()
    hip.synchronize()
    attention.profile_enable(False)
    out = {}
    for n in names:
        ms, k = attention.profile_read(n)
        out[n] = (ms / max(k, 1), k)
    return out


TRAFFIC_FILE = "profiles/hbm_traffic.json"


def _traffic_entries():
    f = ROOT / TRAFFIC_FILE
    return json.loads(f.read_text()) if f.exists() else {}


def hbm_traffic(workload, kernel):
    """The roofline's traffic fields: HBM bytes per launch of `kernel` on
    `workload` as counted by two rocprofv3 --pmc runs (FETCH_SIZE, then
    WRITE_SIZE, scaled by the copy-kernel calibration) and recorded in
    profiles/hbm_traffic.json; read from that file, not measured in this run."""
    entry = _traffic_entries().get(f"{workload}/{kernel}")
    if entry is None:
        return {"traffic": None, "traffic_source": f"no {TRAFFIC_FILE} entry for {workload}/{kernel}"}
    return {"traffic": int(entry["bytes_per_launch"]),
            "traffic_source": f"{TRAFFIC_FILE} {workload}/{entry.get('kernel', kernel)}: FETCH_SIZE + WRITE_SIZE "
                              "per dispatch from rocprofv3 --pmc runs, not this run"}


def kv_traffic(workload, steps):
    """C3's traffic per append step: the append kernel's bytes per launch
    plus the zero-fill / copy kernel's bytes per launch times its launches
    per pass over the pass's steps (profiles/hbm_traffic.json)."""
    e = _traffic_entries()
    ap, bi = e.get(f"{workload}/kv_append"), e.get(f"{workload}/kv_block_init")
    if ap is None or bi is None:
        return {"traffic": None, "traffic_source": f"no {TRAFFIC_FILE} entries for {workload}"}
    per_step = ap["bytes_per_launch"] + bi["bytes_per_launch"] * bi["launches_per_pass"] / steps
    return {"traffic": int(round(per_step)),
            "traffic_source": f"{TRAFFIC_FILE} {workload}: FETCH_SIZE + WRITE_SIZE of {ap['kernel']} per launch "
                              f"plus {bi['kernel']} x {bi['launches_per_pass']} launches per {steps}-step pass, "
                              "from rocprofv3 --pmc runs, not this run"}


# ----------------------------------------------------------------- decode

# CPU samples per decode workload: sequences for the one-thread run, for the
# all-thread run, and reference calls per run (a single short row repeats)
CPU_DECODE_SAMPLE = {"c1": (1, 1, 50), "c2": (64, 64, 1), "c5": (1, 16, 1), "t176": (1, 1, 50)}
# the reference's own published figure for the T176 cache case: one
# fused_paged_attention call, median of 9 (bench/results/prefill/T176.json)
T176_PUBLISHED_US = 523.7


def cpu_rows(w, k, v):
    """The rows the reference's cache holds for the CPU baseline: Q8_0
    workloads take their dequantised values (the reference has no quantised
    KV; Q8_0 dequantisation is quant.hpp:40-49)."""
    if not w.q8:
        return k, v
    from oracle import pyoracle

    return (pyoracle.dequantize_q8_0(pyoracle.quantize_q8_0(k)).reshape(k.shape),
            pyoracle.dequantize_q8_0(pyoracle.quantize_q8_0(v)).reshape(v.shape))


def cpu_decode(key, w, ref, rseqs, qh):
    """The reference's fused_paged_attention over a sample of the batch: one
    thread, then every host thread over sequences (std::thread in the shim)."""
    n1, nall, calls = CPU_DECODE_SAMPLE.get(key, (1, min(w.sequences, host_threads()), 1))
    threads = min(host_threads(), nall)

    def run(n, th):
        def go():
            for _ in range(calls):
                ref.fused_batch(rseqs[:n], qh[:n], 0, w.heads, w.context, th)
        return go

    one = median_of_9(run(n1, 1))
    alln = median_of_9(run(nall, threads))
    per_token = w.kv_bytes() / w.total_tokens
    tokens = lambda n: sum(w.lengths[:n])  # noqa: E731
    sample = (f"the reference's fused_paged_attention over {n1} (1 thread) and {nall} ({threads} threads) of "
              f"the {w.sequences} sequences" + (f", {calls} calls a run" if calls > 1 else "") +
              (", on the dequantised Q8_0 values (the reference has no quantised KV)" if w.q8 else "") +
              "; GB/s counts the workload's algorithmic bytes of the rows processed")
    return cpu_result("GB/s", one, alln, threads, sample, calls * tokens(n1) * per_token / 1e9,
                      calls * tokens(nall) * per_token / 1e9,
                      {"decode_tokens_per_s": round(calls * nall / alln, 2),
                       "ms_per_step_one_thread": round(one / calls * w.sequences / n1 * 1e3, 3)})


def bench_decode(args, key, w):
    import numpy as np

    from tvara_amd import attention, hip, kv, workloads

    log(f"workload {w.name}: {w.sequences} sequences, {w.total_tokens} tokens")
    g = (w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks)
    cache = kv.PagedCache(*g, fmt=kv.Q8_0 if w.q8 else kv.F32)
    # the reference's cache takes the same rows (Q8_0 workloads: their
    # dequantised values, as the reference has no quantised KV) in the same
    # fill, so the inputs are generated once
    ref, rseqs = None, []
    if ref_ready(args):
        from oracle import pyoracle

        blocks = sum((n + w.tokens_per_block - 1) // w.tokens_per_block for n in w.lengths) + 8
        ref = pyoracle.RefCache(w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, blocks)
    t0 = time.perf_counter()
    workloads.place_blocks(cache, w.placement())
    seqs = []
    for i in range(w.sequences):
        k, v = w.keys(i), w.values(i)
        s = cache.create_sequence()
        cache.append_many(s, k, v)
        seqs.append(s)
        if ref is not None:
            r = ref.create_sequence()
            ref.append_many(r, *cpu_rows(w, k, v))
            rseqs.append(r)
    cache.synchronize()
    log(f"filled in {time.perf_counter() - t0:.1f}s")
    qh = w.queries()
    q = hip.DeviceArray.from_numpy(qh)
    out = hip.DeviceArray(q.shape)
    plan = attention.DecodePlan(cache, seqs, w.heads, w.context)
    log(f"plan: split {plan.split_tokens} tokens, {plan.items} work items")
    for _ in range(args.warmup):
        plan.launch(0, q.ptr, out.ptr)
    plan.check()
    hip.synchronize()

    # the timed region: K launches on the cache's stream (the null stream)
    step = lambda: plan.launch(0, q.ptr, out.ptr)  # noqa: E731
    ms_per_step = timed_steps(step, args.steps)
    plan.check()
    kt = kernel_times(step, args.steps, ["paged_decode", "paged_decode_merge"])
    kernel_avg_ms, launches = kt["paged_decode"]
    merge_ms, merges = kt["paged_decode_merge"]
    kernel_source = "start/stop events the runtime stamps on each launch, a second pass of the same steps"
    if not merges and kernel_avg_ms > ms_per_step:
        # a one-launch step (the split merge runs in the kernel): the events'
        # own packets can lengthen a launch of a few microseconds past the
        # step that contains it, so the step time bounds the kernel
        kernel_avg_ms = ms_per_step
        kernel_source = "the step time: the step is this one launch (its event-bracketed duration was longer)"
    log(f"step {ms_per_step * 1e3:.1f} us; decode kernel {kernel_avg_ms * 1e3:.1f} us x{launches}; "
        f"merge {merge_ms * 1e3:.1f} us x{merges}")
    assert np.isfinite(out.numpy()).all()
    # the same batch through the host-buffer entry point (queries in and
    # outputs out over PCIe): reported beside the value, never as it
    attention.decode_batch(cache, qh, seqs, 0, w.heads, w.context)
    reps = 20
    t0 = time.perf_counter()
    for _ in range(reps):
        attention.decode_batch(cache, qh, seqs, 0, w.heads, w.context)
    host_ms = (time.perf_counter() - t0) / reps * 1e3

    kv_bytes = w.kv_bytes()
    step_bytes = kv_bytes + w.qo_bytes() + w.table_bytes()
    gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    kernel_bytes = kv_bytes + w.qo_bytes() // 2 + w.table_bytes()
    kernel_gbs = kernel_bytes / (kernel_avg_ms * 1e-3) / 1e9
    tokens_per_s = w.sequences / (ms_per_step * 1e-3)
    layers = MODEL_LAYERS.get(w.name, 1)
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0" if w.q8 else "f32",
        "data": "synthetic: K/V/q ~ N(0,1) from a seeded splitmix64 stream, blocks at a seeded permutation",
        "config": {"workload": w.name, "sequences": w.sequences, "heads": w.heads, "kv_heads": w.kv_heads,
                   "head_dim": w.head_dim, "tokens_per_block": w.tokens_per_block, "total_tokens": w.total_tokens,
                   "pool_blocks": w.pool_blocks, "split_tokens": plan.split_tokens, "work_items": plan.items},
        "pct_of_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "latency_us": round(ms_per_step * 1e3, 2),
        "decode_tokens_per_s": round(tokens_per_s, 1),
        "model_decode_tokens_per_s": round(tokens_per_s / layers, 1),
        "model_layers": layers,
        "host_buffers_ms_per_step": round(host_ms, 4),
        "roofline": {"bound": "hbm", "achieved": round(kernel_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kernel_gbs / HBM_PEAK_GBS, 4), **hbm_traffic(w.name, "paged_decode"),
                     "kernel": "paged_decode", "kernel_avg_us": round(kernel_avg_ms * 1e3, 3),
                     "kernel_time_source": kernel_source,
                     "merge_avg_us": round(merge_ms * 1e3, 3) if merges else 0.0,
                     "algorithmic_bytes": kernel_bytes},
        "cpu_baseline": None,
    }
    if key == "t176":
        result["reference_published"] = {
            "us_per_call": T176_PUBLISHED_US,
            "source": "bench/results/prefill/T176.json cache_plain_us (the reference's own run: g++ 15.2 -O2, "
                      "Windows, median of 9)"}
    del plan, cache, q, out
    if ref is not None:
        def job():
            t0 = time.perf_counter()
            c = cpu_decode(key, w, ref, rseqs, qh)
            log(f"{w.name}: cpu baseline in {time.perf_counter() - t0:.1f}s")
            return c

        baseline(result, job)
    return result


# ---------------------------------------------------------------- prefill

def chunk_flops(w, first, count):
    """Causal chunk rows first .. first+count-1 of one sequence: 4·d flops per
    (row, head, visible key)."""
    keys = sum(w.prefix + i + 1 for i in range(first, first + count))
    return 4 * w.head_dim * w.heads * keys


def cpu_prefill(w):
    """The reference's fused_prompt_attention (FP64, row by row) over the first
    chunk: its first 64 rows on one thread, all its rows in runs of 16 on
    every host thread."""
    from oracle import pyoracle
    from tvara_amd import workloads

    ref = pyoracle.RefCache(1, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks())
    rs = workloads.fill_prefill(ref, w)[0]
    qs = w.chunk_queries(0)
    threads = host_threads()
    n1 = 64
    one = median_of_9(lambda: ref.prompt_batch(qs[:n1], rs, 0, w.prefix, n1, w.heads, w.context, n1, 1))
    alln = median_of_9(lambda: ref.prompt_batch(qs, rs, 0, w.prefix, w.chunk, w.heads, w.context, 16, threads))
    return cpu_result("TFLOP/s", one, alln, threads,
                      f"the reference's fused_prompt_attention on chunk 0: rows 0-{n1 - 1} on 1 thread, all "
                      f"{w.chunk} rows in runs of 16 on {threads} threads",
                      chunk_flops(w, 0, n1) / 1e12, chunk_flops(w, 0, w.chunk) / 1e12)


FP32_PEAK_TFS = 157.3  # MI355X dense fp32 (matrix)


def bench_prefill(args, w, precision="bf16"):
    """Chunked prefill: TFLOP/s over the algorithmic flops of the causal
    chunks.  bf16: the MFMA kernel.  f32 (the reference's arithmetic, within
    1e-4): every chunk row runs as a decode row whose visible length stops at
    its own position (attention.hpp:85-89), through the decode kernels and the
    split merge; its dominant kernel is priced against the fp32 peak.  f32x3
    (within the same 1e-4): the MFMA tiles with every operand split into two
    16-bit parts and three products per product, priced against a third of
    the 16-bit MFMA peak (the matrix rate left for the algorithmic flops)."""
    import numpy as np

    from tvara_amd import attention, hip, kv, workloads

    cache = kv.PagedCache(1, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks(),
                          fmt=kv.Q8_0 if w.q8 else kv.F32)
    seqs = workloads.fill_prefill(cache, w)
    q = hip.DeviceArray.from_numpy(np.concatenate([w.chunk_queries(i) for i in range(w.sequences)]))
    out = hip.DeviceArray(q.shape)
    # one plan per prompt chunk (as an executor keeps it for every layer); a
    # step is one launch of it
    plan = attention.PrefillPlan(cache, seqs, [w.prefix] * w.sequences, [w.chunk] * w.sequences, w.heads, w.context,
                                 precision)
    call = lambda: plan.launch(0, q.ptr, out.ptr)  # noqa: E731
    for _ in range(args.warmup):
        call()
    plan.check()
    steps = args.steps if precision != "f32" else max(1, min(args.steps, 20))
    ms_per_step = timed_steps(call, steps)
    kernel = {"bf16": "paged_prefill_bf16", "f32x3": "paged_prefill_x3"}.get(precision, "paged_decode")
    kt = kernel_times(call, steps, [kernel, "paged_decode_merge"])
    kernel_ms, _ = kt[kernel]
    merge_ms, merges = kt["paged_decode_merge"]
    plan.check()
    assert np.isfinite(out.numpy()).all()
    tfs = w.flops() / (kernel_ms * 1e-3) / 1e12
    log(f"prefill ({precision}) kernel {kernel_ms * 1e3:.1f} us, call {ms_per_step * 1e3:.1f} us, {tfs:.1f} TFLOP/s")
    del plan, cache, q, out
    peak = {"bf16": MFMA_BF16_PEAK_TFS, "f32x3": round(MFMA_BF16_PEAK_TFS / 3, 1)}.get(precision, FP32_PEAK_TFS)
    name = w.name if precision == "bf16" else w.name + "-" + precision
    metric = {
        "bf16": "paged chunked prefill attn: achieved TFLOP/s (MFMA utilisation), 1 MI355X",
        "f32x3": "paged chunked prefill attn, f32-accurate (three-product tiles): achieved TFLOP/s, 1 MI355X",
    }.get(precision, "paged chunked prefill attn, f32 (reference arithmetic): achieved TFLOP/s, 1 MI355X")
    result = {
        "metric": metric,
        "value": round(w.flops() / (ms_per_step * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": precision, "data": "synthetic: K/V/q ~ N(0,1)",
        "config": {"workload": name, "sequences": w.sequences, "prefix": w.prefix, "chunk": w.chunk,
                   "heads": w.heads, "kv_heads": w.kv_heads, "head_dim": w.head_dim,
                   "kv": "q8_0" if w.q8 else "f32", "precision": precision},
        "roofline": {"bound": "fp32" if precision == "f32" else "mfma", "achieved": round(tfs, 2), "peak": peak,
                     "unit": "TFLOP/s", "frac": round(tfs / peak, 4), **hbm_traffic(name, kernel),
                     "kernel": kernel, "kernel_avg_us": round(kernel_ms * 1e3, 3),
                     "merge_avg_us": round(merge_ms * 1e3, 3) if merges else 0.0, "algorithmic_flops": w.flops()},
        "cpu_baseline": None,
    }
    if precision == "bf16":
        result["f32_accurate_x3"] = x3_beside(args, w)
    if ref_ready(args) and not w.q8:
        baseline(result, lambda: cpu_prefill(w))
    return result


def x3_beside(args, w):
    """The same chunks through the three-product tiles (TVARA_ATTN_F32X3,
    within the f32 bar), reported beside the bf16 line: kernel time from the
    library's HIP events, algorithmic TFLOP/s and their fraction of a third of
    the 16-bit MFMA peak (three products per product), over the same blocks
    (f32 or Q8_0)."""
    import numpy as np

    from tvara_amd import attention, hip, kv, workloads

    cache = kv.PagedCache(1, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks(),
                          fmt=kv.Q8_0 if w.q8 else kv.F32)
    seqs = workloads.fill_prefill(cache, w)
    q = hip.DeviceArray.from_numpy(np.concatenate([w.chunk_queries(i) for i in range(w.sequences)]))
    out = hip.DeviceArray(q.shape)
    plan = attention.PrefillPlan(cache, seqs, [w.prefix] * w.sequences, [w.chunk] * w.sequences, w.heads, w.context,
                                 "f32x3")
    call = lambda: plan.launch(0, q.ptr, out.ptr)  # noqa: E731
    for _ in range(max(1, args.warmup // 4)):
        call()
    plan.check()
    steps = max(1, args.steps // 4)
    kernel_ms, _ = kernel_times(call, steps, ["paged_prefill_x3"])["paged_prefill_x3"]
    plan.check()
    assert np.isfinite(out.numpy()).all()
    del plan, cache, q, out
    tfs = w.flops() / (kernel_ms * 1e-3) / 1e12
    peak = MFMA_BF16_PEAK_TFS / 3
    log(f"prefill (f32x3) kernel {kernel_ms * 1e3:.1f} us, {tfs:.1f} TFLOP/s")
    return {"kernel": "paged_prefill_x3", "kernel_avg_us": round(kernel_ms * 1e3, 3), "achieved": round(tfs, 2),
            "unit": "TFLOP/s", "peak": round(peak, 1), "frac": round(tfs / peak, 4), "steps": steps,
            "bar": "1e-4 * (1 + |ref|), the f32 path's"}


# -------------------------------------------------------------- KV stress

def cpu_kv(w, step_bytes):
    """The reference's PagedCache: a run is one fork of the prefix for every
    sequence and 32 append steps.  The cache is single-owner
    (docs/kv-cache.md), so one thread."""
    from oracle import pyoracle

    ref = pyoracle.RefCache(w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.max_blocks())
    src = ref.create_sequence()
    ref.append_many(src, w.tokens("prefix-k", w.prefix), w.tokens("prefix-v", w.prefix))
    hk = [w.tokens(f"step{i}-k", w.sequences) for i in range(4)]
    hv = [w.tokens(f"step{i}-v", w.sequences) for i in range(4)]
    n_cpu = 32

    def run():
        rseqs = [ref.fork(src) for _ in range(w.sequences)]
        for i in range(n_cpu):
            ref.append_batch(rseqs, hk[i % 4], hv[i % 4])
        for s in rseqs:
            ref.drop(s)

    per_run = median_of_9(run)
    cpu_bytes = sum(step_bytes(i) for i in range(n_cpu))
    return {"value": round(cpu_bytes / per_run / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "reference",
            "sample": f"one fork of the prefix for {w.sequences} sequences and {n_cpu} append steps a run; "
                      "the reference cache is single-owner, so one thread",
            "protocol": "1 warm-up, median of 9 runs", "ms_per_step": round(per_run / n_cpu * 1e3, 4),
            "host": host_info()}


def kv_step_bytes(w):
    """Algorithmic bytes of append step i: every token's K and V rows read from
    the batch and written to their blocks, a zero fill per new block, a read
    and a write per copy-on-write block."""
    width = w.layers * w.kv_heads * w.head_dim
    block_bytes = w.tokens_per_block * width * 2 * 4
    row_bytes = 2 * width * 2 * 4  # read + write of the K and V rows

    def step_bytes(i):
        length = w.prefix + i
        slot = length % w.tokens_per_block
        if slot == 0:
            extra = w.sequences * block_bytes  # new tail blocks, zero-filled
        elif i == 0:
            extra = (w.sequences - 1) * 2 * block_bytes  # shared tail copied for all but the last appender
        else:
            extra = 0
        return w.sequences * row_bytes + extra

    return step_bytes


def bench_kv(args, cow):
    """KV-management stress: 256 sequences forked from a shared 1,024-token
    (or 1,025-token, copy-on-write) prefix, 22 layers x 8 x 64 f32; a step is
    one batched append of one token to every sequence (host bookkeeping, the
    zero-fill / copy-on-write launch and the row-copy launch).  K/V rows are
    resident in HBM.  Bytes per step: the rows read and written, plus a
    block's zero fill for every new block and a read and a write of a block
    for every copy-on-write."""
    import numpy as np

    from tvara_amd import hip, kv, workloads

    w = workloads.kv_c3(unaligned=cow)
    cache = kv.PagedCache(w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.max_blocks())
    step_bytes = kv_step_bytes(w)
    # four distinct step batches, used in turn (the contents do not change the work)
    batches = [(hip.DeviceArray.from_numpy(w.tokens(f"step{i}-k", w.sequences)),
                hip.DeviceArray.from_numpy(w.tokens(f"step{i}-v", w.sequences))) for i in range(4)]
    steps_k = [batches[i % 4][0] for i in range(w.steps)]
    steps_v = [batches[i % 4][1] for i in range(w.steps)]
    pk, pv = w.tokens("prefix-k", w.prefix), w.tokens("prefix-v", w.prefix)

    def setup():
        src = cache.create_sequence()
        cache.append_many(src, pk, pv)
        seqs = [cache.fork(src) for _ in range(w.sequences)]
        cache.drop(src)
        cache.synchronize()
        return seqs

    # the seeded rollback: every sequence back by 0-64 tokens from the
    # length a pass leaves (the scheduler knows its sequences' lengths)
    kept = np.asarray([w.prefix + w.steps - r for r in w.rollback()], np.uintp)

    def run_pass(seqs):
        """One whole pass: the 128 append steps, then the seeded 0-64 token
        speculative rollback of every sequence (metadata only, one batched
        truncation), between two events on the cache's stream.  The stop
        event is recorded once the host has issued every append and the
        rollback, so the interval covers the host's work where it outlasts
        the GPU's."""
        batch = np.asarray(seqs, np.uint64)  # the batch as a scheduler holds it
        start, stop = hip.Event(), hip.Event()
        hip.synchronize()
        start.record()
        for i in range(w.steps):
            cache.append_batch_device(batch, steps_k[i].ptr, steps_v[i].ptr)
        cache.truncate_batch(batch, kept)
        stop.record()
        hip.synchronize()
        return start.elapsed_ms(stop)

    # warm-up: whole passes, untimed
    for _ in range(max(1, args.warmup // w.steps)):
        seqs = setup()
        run_pass(seqs)
        for s in seqs:
            cache.drop(s)
    # timed: whole passes only, as many as --steps asks for (at least one)
    passes = max(1, -(-args.steps // w.steps))
    total_ms = 0.0
    for _ in range(passes):
        seqs = setup()
        total_ms += run_pass(seqs)
        cache.audit()
        for s in seqs:
            cache.drop(s)
    done = passes * w.steps
    nbytes = passes * sum(step_bytes(i) for i in range(w.steps))
    ms_per_step = total_ms / done
    gbs = nbytes / (total_ms * 1e-3) / 1e9
    log(f"{w.name}: {ms_per_step * 1e3:.1f} us per step, {gbs:.1f} GB/s")
    del cache, batches, steps_k, steps_v
    result = {
        "metric": "paged KV management stress: us per append step + GB/s, 1 MI355X", "value": round(gbs, 2),
        "unit": "GB/s", "n_gpus": 1, "steps": done, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: K/V rows from a seeded splitmix64 stream (floats in [1, 2))",
        "config": {"workload": w.name, "sequences": w.sequences, "prefix": w.prefix, "steps_per_pass": w.steps,
                   "passes": passes, "rollback": "seeded 0-64 tokens per sequence, inside the timed pass",
                   "layers": w.layers, "kv_heads": w.kv_heads, "head_dim": w.head_dim,
                   "tokens_per_block": w.tokens_per_block},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "kernel": "kv_append (step)",
                     "algorithmic_bytes_per_step": round(nbytes / done), **kv_traffic(w.name, w.steps)},
        "cpu_baseline": None,
    }
    if ref_ready(args):
        baseline(result, lambda: cpu_kv(w, step_bytes))
    return result


# ----------------------------------------------------------- prefix cache

PREFIX_PUBLISHED_NS = 933.08  # bench/results/radix-prefix.json: 9,330,800 ns for 10,000 requests


def prefix_driver():
    """bench_prefix.cpp built into build/release (by build() or here, when
    missing or older than its source)."""
    src = ROOT / "bench_prefix.cpp"
    exe = ROOT / "build" / "release" / "bench_prefix"
    if not exe.exists() or exe.stat().st_mtime < src.stat().st_mtime:
        exe.parent.mkdir(parents=True, exist_ok=True)
        subprocess.run(["g++", "-O2", "-std=c++17", "-o", str(exe), str(src), "-ldl"], check=True)
    return exe


def run_prefix_driver(kind, library, runs=9):
    res = subprocess.run([str(prefix_driver()), kind, str(library), str(runs)], capture_output=True, text=True,
                         timeout=300)
    if res.returncode != 0:
        raise RuntimeError(f"bench_prefix {kind} failed ({res.returncode}): {res.stderr[-2000:]}")
    return json.loads(res.stdout)


def bench_prefix(args):
    """The prefix cache: the reference's radix benchmark (bench/radix_prefix.cpp:
    10,000 lookups with a KV restore of an 8-token prefix, 75% hits) through
    this library's C ABI, timed in C++ as the reference times it.  Host
    metadata only (the prefix tree and the block ledger): no kernel runs."""
    from tvara_amd import _capi

    mine = run_prefix_driver("tvara", _capi.find_library())
    ns = statistics.median(mine["runs_ns"]) / mine["requests"]
    log(f"prefix cache: {ns:.1f} ns per request (median of {len(mine['runs_ns'])} runs of 10,000)")
    result = {
        "metric": "prefix cache lookup + KV restore: ns per request (10,000 requests, 75% hits), 1 MI355X host",
        "value": round(ns, 2), "unit": "ns/request", "n_gpus": 1, "steps": mine["requests"],
        "warmup": mine["requests"], "ms_per_step": round(ns * 1e-6, 8), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "int32 tokens",
        "data": "the reference's fixture: an 8-token prefix in 4-token blocks; every fourth request misses",
        "config": {"workload": "radix-prefix-10000x8-75pct", "requests": mine["requests"], "hits": mine["hits"],
                   "saved_prefill_tokens": mine["saved_prefill_tokens"], "runs": len(mine["runs_ns"]),
                   "runs_ns": mine["runs_ns"]},
        "reference_published": {"ns_per_request": PREFIX_PUBLISHED_NS,
                                "source": "bench/results/radix-prefix.json (host A: Intel Family 6 Model 61, "
                                          "Windows 11, one run)"},
        "roofline": {"bound": "host", "achieved": None, "peak": None, "unit": "ns/request", "frac": None,
                     "traffic": None, "traffic_source": "none: no device memory is touched",
                     "kernel": "none: host metadata (prefix tree and block ledger)"},
        "cpu_baseline": None,
    }
    if ref_ready(args):
        def job():
            from oracle import pyoracle

            ref = run_prefix_driver("ref", pyoracle.REF_PATH)
            rns = statistics.median(ref["runs_ns"]) / ref["requests"]
            assert (ref["hits"], ref["saved_prefill_tokens"]) == (mine["hits"], mine["saved_prefill_tokens"])
            return {"value": round(rns, 2), "unit": "ns/request", "cores": 1, "kind": "reference",
                    "sample": "the same 10,000 requests through the reference's RadixCache and PagedCache built "
                              "from its headers (oracle/_ref), timed by the same driver",
                    "protocol": "1 warm-up run, median of 9 runs", "runs_ns": ref["runs_ns"], "host": host_info()}

        baseline(result, job)
    return result


# ---------------------------------------------------------- conversations

CONV_PUBLISHED = {"prefill_speedup": 3.554, "reused_token_fraction": 0.7524, "prompt_tokens": 3675,
                  "reused_prompt_tokens": 2765, "turn_hits": 16,
                  "source": "bench/results/prefix-cache-traces.json (the reference's CPU executor on its tiny-random "
                            "Llama fixture; Intel Family 6 Model 61, Windows 11; median of 3)"}
CONV_ISOLATION = "tiny-random-llama/synthetic-ids/tenant-a"


def conversation_runs(model, traces, repeats, modes, tree_for=None):
    """Median prefill seconds, counts and outputs of each mode over `repeats`
    runs, the order alternating per repetition as the reference's tool does
    (tools/run_prefix_cache_traces.py:105-118)."""
    from tvara_amd import workloads

    runs = {mode: [] for mode in modes}
    for rep in range(repeats):
        for mode in (modes if rep % 2 == 0 else modes[::-1]):
            tree = tree_for() if mode == "radix" else None
            try:
                runs[mode].append(workloads.replay_conversations(model, traces, mode, tree=tree))
            finally:
                if tree is not None:
                    tree.close()
    return runs


def conversation_summary(runs):
    import numpy as np

    out = {}
    first = None
    equal = True
    for mode, reps in runs.items():
        turns = [t for trace in reps[0] for t in trace]
        seconds = [sum(t["prefill_seconds"] for trace in rep for t in trace) for rep in reps]
        out[mode] = {"prompt_tokens": sum(t["prompt_tokens"] for t in turns),
                     "reused_prompt_tokens": sum(t["reused_tokens"] for t in turns),
                     "turn_hits": sum(t["reused_tokens"] > 0 for t in turns),
                     "prefill_seconds_median": round(statistics.median(seconds), 6),
                     "prefill_seconds": [round(x, 6) for x in seconds]}
        out[mode]["reused_token_fraction"] = round(out[mode]["reused_prompt_tokens"] / out[mode]["prompt_tokens"], 4)
        for rep in reps:
            flat = [t for trace in rep for t in trace]
            if first is None:
                first = flat
            equal = equal and all(a["reply"] == b["reply"] and np.array_equal(a["logits"], b["logits"])
                                  for a, b in zip(first, flat))
    off = out["off"]["prefill_seconds_median"]
    for mode in out:
        out[mode]["prefill_speedup"] = round(off / out[mode]["prefill_seconds_median"], 3)
    return out, equal


def bench_conversations(args):
    """Prefix reuse on the reference's conversation traces (docs/prefix-cache.md:
    13-23; tools/run_prefix_cache_traces.py): four seeded conversations of five
    turns (a 64-token shared system prompt, 16-48-token user turns, 12-token
    greedy replies) through the model-level C ABI on a model of the reference
    fixture's shape (tiny-random Llama: hidden 16, two layers, vocabulary
    32,000; random f32 weights).  Modes off and on are the reference's; radix
    also restores the system prompt across conversations from a prefix tree
    over the model's cache (tvara_model_cache + tvara_radix_*), which the
    reference's ABI cannot.  Three repetitions, the order alternating; the
    value is the median prefill speedup of on over off."""
    import shutil
    import tempfile

    from tvara_amd import gguf_writer, native, radix, workloads

    spec = gguf_writer.tiny_random_llama()
    tmp = Path(tempfile.mkdtemp(prefix="tvara-conv-"))
    try:
        path = spec.write(tmp / "tiny-random-llama.gguf")
        m = native.NativeModel(path, max_blocks=256, block_tokens=16)
        traces = workloads.conversation_traces(vocab=m.vocab_size)
        cache = m.cache()
        tree_for = lambda: radix.RadixCache(cache, CONV_ISOLATION)  # noqa: E731
        conversation_runs(m, traces, 1, ("off", "on", "radix"), tree_for)  # warm-up
        summary, equal = conversation_summary(conversation_runs(m, traces, 3, ("off", "on", "radix"), tree_for))
        m.close()
        on = summary["on"]
        log(f"conversations: off {summary['off']['prefill_seconds_median'] * 1e3:.1f} ms, on "
            f"{on['prefill_seconds_median'] * 1e3:.1f} ms ({on['prefill_speedup']}x), radix "
            f"{summary['radix']['prefill_seconds_median'] * 1e3:.1f} ms ({summary['radix']['prefill_speedup']}x); "
            f"outputs equal {equal}")
        result = {
            "metric": "prefix reuse on the reference's conversation traces: prefill speedup, cache on vs off, "
                      "1 MI355X",
            "value": on["prefill_speedup"], "unit": "x", "n_gpus": 1, "steps": 3, "warmup": 1,
            "ms_per_step": round(on["prefill_seconds_median"] * 1e3, 3), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "the reference's seeded traces (numpy PCG64, seed 262); random f32 weights of the fixture's "
                    "shape",
            "config": {"workload": "conversations-4x5-tiny-random-llama", "conversations": 4, "turns": 5,
                       "reply_tokens": 12, "layers": spec.layers, "hidden": spec.hidden, "heads": spec.heads,
                       "kv_heads": spec.kv_heads, "vocab": spec.vocab},
            "modes": summary, "outputs_equal": equal,
            "reference_published": CONV_PUBLISHED,
            "roofline": {"bound": "latency", "achieved": None, "peak": None, "unit": "s", "frac": None,
                         "traffic": None, "traffic_source": "none: a 16-wide model is launch-bound",
                         "kernel": "whole prefill calls (hidden 16: token by token)"},
            "cpu_baseline": None,
        }
        if ref_ready(args) and (ROOT / "oracle" / "_ref" / "libtvara_ref_capi.so").exists():
            refso = ROOT / "oracle" / "_ref" / "libtvara_ref_capi.so"

            def job():  # may run after this function returned: a file of its own
                jtmp = Path(tempfile.mkdtemp(prefix="tvara-conv-ref-"))
                try:
                    r = native.NativeModel(spec.write(jtmp / "tiny-random-llama.gguf"), library=str(refso),
                                           max_blocks=256, block_tokens=16)
                    ref, ref_equal = conversation_summary(conversation_runs(r, traces, 3, ("off", "on")))
                    r.close()
                finally:
                    shutil.rmtree(jtmp, ignore_errors=True)
                assert ref["on"]["reused_prompt_tokens"] == on["reused_prompt_tokens"]
                return {"value": ref["on"]["prefill_speedup"], "unit": "x", "cores": 1, "kind": "reference",
                        "sample": "the same traces through the reference's C ABI and CPU executor (oracle/_ref), "
                                  "modes off and on, 3 repetitions",
                        "modes": ref, "outputs_equal": ref_equal, "host": host_info()}

            baseline(result, job)
        return result
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


# ------------------------------------------------------------------ model

PREFILL_PROMPT = 2048


def bench_model(args):
    """Decode through the model-level C ABI on a Llama-3.2-1B-shaped GGUF file
    with random Q8_0 weights (tied embedding): one sequence token by token
    (tvara_sequence_decode), and 64 sequences stepping together
    (tvara_sequences_decode) after a 128-token prompt each.  A step is one
    decode of every sequence in the batch."""
    import shutil
    import tempfile

    import numpy as np

    from tvara_amd import gguf_writer, native

    spec = gguf_writer.llama32_1b()
    tmp = Path(tempfile.mkdtemp(prefix="tvara-model-"))
    try:
        t0 = time.perf_counter()
        path = spec.write(tmp / "llama32-1b-q8_0.gguf")
        log(f"wrote {path.stat().st_size / 1e9:.2f} GB GGUF in {time.perf_counter() - t0:.1f}s")
        nseq, prompt = 64, 128
        t0 = time.perf_counter()
        m = native.NativeModel(path, max_blocks=nseq * ((prompt + args.steps + args.warmup + 64) // 16 + 1) +
                               PREFILL_PROMPT // 16 + 64, block_tokens=16)
        log(f"loaded in {time.perf_counter() - t0:.1f}s")
        rng = np.random.default_rng(3)
        # one 2,048-token prompt through tvara_sequence_prefill (passes of 512
        # tokens), rolled back between repetitions
        sp = m.new_sequence()
        ptoks = rng.integers(0, spec.vocab, PREFILL_PROMPT)
        m.prefill(sp, ptoks[:600])
        m.truncate(sp, 0)
        prefill_runs = []
        for _ in range(5):
            t0 = time.perf_counter()
            last = m.prefill(sp, ptoks)
            prefill_runs.append(time.perf_counter() - t0)
            m.truncate(sp, 0)
        assert np.isfinite(last).all()
        m.drop_sequence(sp)
        prefill_s = statistics.median(prefill_runs)
        # one sequence, token by token
        s1 = m.new_sequence()
        for t in rng.integers(0, spec.vocab, 8):
            m.logits(s1, int(t))
        single_steps = min(args.steps, 64)
        toks = rng.integers(0, spec.vocab, single_steps)
        t0 = time.perf_counter()
        for t in toks:
            m.logits(s1, int(t))
        single_s = (time.perf_counter() - t0) / single_steps
        m.drop_sequence(s1)
        # a batch of sequences
        seqs = [m.new_sequence() for _ in range(nseq)]
        for _ in range(prompt):
            m.decode_sequences(seqs, rng.integers(0, spec.vocab, nseq))
        for _ in range(args.warmup):
            m.decode_sequences(seqs, rng.integers(0, spec.vocab, nseq))
        steps = [rng.integers(0, spec.vocab, nseq) for _ in range(args.steps)]
        t0 = time.perf_counter()
        for st in steps:
            logits = m.decode_sequences(seqs, st)
        batch_s = (time.perf_counter() - t0) / args.steps
        assert np.isfinite(logits).all()
        m.close()
        weights = spec.vocab * spec.hidden + spec.layers * (
            spec.hidden * (spec.hidden * 2 + 2 * spec.hidden // spec.heads * spec.kv_heads) +
            3 * spec.hidden * spec.intermediate)
        # per step: every weight once, as the kernels read it (Q8_0 kept
        # quantised: 34 B per 32), plus each sequence's cached K/V in every
        # layer at the mean position of the timed steps
        kv_width = spec.hidden // spec.heads * spec.kv_heads
        mean_pos = prompt + args.warmup + args.steps / 2
        weight_bytes = weights * 34 // 32
        kv_bytes = int(nseq * mean_pos * spec.layers * kv_width * 2 * 4)
        step_bytes = weight_bytes + kv_bytes
        tps = nseq / batch_s
        log(f"single sequence {single_s * 1e3:.2f} ms/token; {nseq} sequences {batch_s * 1e3:.2f} ms/step, "
            f"{tps:.0f} tokens/s; a {PREFILL_PROMPT}-token prompt in {prefill_s * 1e3:.2f} ms "
            f"({PREFILL_PROMPT / prefill_s:.0f} tokens/s)")
        cpu = None
        if ref_ready(args):
            refso = ROOT / "oracle" / "_ref" / "libtvara_ref_capi.so"
            t0 = time.perf_counter()
            r = native.NativeModel(path, library=str(refso), max_blocks=16, block_tokens=16)
            log(f"reference loaded in {time.perf_counter() - t0:.1f}s")
            rs = r.new_sequence()
            r.logits(rs, 1)
            t0 = time.perf_counter()
            for t in (2, 3, 4):
                r.logits(rs, t)
            cpu_s = (time.perf_counter() - t0) / 3
            r.close()
            cpu = {"value": round(1 / cpu_s, 4), "unit": "tokens/s", "cores": 1, "kind": "reference",
                   "sample": f"3 tokens of one sequence through the reference's tvara_sequence_decode (its "
                             f"f32 executor on the calling thread); {cpu_s:.2f} s per token",
                   "s_per_token": round(cpu_s, 4)}
        return {
            "metric": "llama-3.2-1b-shaped decode through the model-level C ABI: tokens/s, 1 MI355X",
            "value": round(tps, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(batch_s * 1e3, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32",
            "data": "synthetic: random Q8_0 weights (numpy PCG64), random token ids",
            "config": {"workload": "llama-3.2-1b-q8_0-decode-64seq", "sequences": nseq, "prompt": prompt,
                       "layers": spec.layers, "hidden": spec.hidden, "heads": spec.heads,
                       "kv_heads": spec.kv_heads, "intermediate": spec.intermediate, "vocab": spec.vocab},
            "single_sequence_ms_per_token": round(single_s * 1e3, 4),
            "prompt_prefill": {"tokens": PREFILL_PROMPT, "ms": round(prefill_s * 1e3, 3),
                               "tokens_per_s": round(PREFILL_PROMPT / prefill_s, 1),
                               "call": "tvara_sequence_prefill, passes of 512 tokens, median of 5",
                               "token_loop_tokens_per_s": round(1 / single_s, 1)},
            "single_sequence_weight_GBps": round(weight_bytes / single_s / 1e9, 1),
            "roofline": {"bound": "hbm", "achieved": round(step_bytes / batch_s / 1e9, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(step_bytes / batch_s / 1e9 / HBM_PEAK_GBS, 4),
                         "traffic": None, "traffic_source": "not counted: a step is about 180 launches of 20 kernels",
                         "kernel": "whole decode step (Q8_0 weights once + cached K/V)",
                         "algorithmic_bytes": step_bytes, "weight_bytes": weight_bytes, "kv_bytes": kv_bytes},
            "cpu_baseline": cpu,
        }
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


# ------------------------------------------------------------------- main

def compact(r):
    """The fields of a configuration line that precede the headline."""
    cpu = r.get("cpu_baseline")
    out = {"metric": r["metric"], "value": r["value"], "unit": r["unit"], "ms_per_step": r["ms_per_step"],
           "steps": r["steps"], "warmup": r["warmup"], "dtype": r["dtype"],
           "config": {"workload": r["config"]["workload"]},
           "roofline": {k: r["roofline"][k] for k in ("bound", "achieved", "peak", "unit", "frac", "traffic")},
           "cpu_baseline": None}
    for k in ("kernel", "kernel_avg_us", "merge_avg_us", "kernel_time_source", "traffic_source"):
        if k in r["roofline"]:
            out["roofline"][k] = r["roofline"][k]
    for k in ("latency_us", "reference_published", "decode_tokens_per_s", "model_decode_tokens_per_s",
              "prompt_prefill", "f32_accurate_x3"):
        if k in r:
            out[k] = r[k]
    if cpu:
        out["cpu_baseline"] = {"value": cpu["value"], "unit": cpu["unit"], "cores": cpu["cores"], "kind": cpu["kind"]}
        if "one_thread" in cpu:
            out["cpu_baseline"]["one_thread"] = cpu["one_thread"]["value"]
    return out


def run_one(args, key):
    from tvara_amd import workloads

    if key in ("c4", "c4d128", "c4q8", "c4f32", "c4x3", "c4x3d128", "c4q8x3"):
        make = {"c4": workloads.prefill_c4, "c4d128": workloads.prefill_8b, "c4q8": workloads.prefill_c4_q8,
                "c4f32": workloads.prefill_c4, "c4x3": workloads.prefill_c4, "c4x3d128": workloads.prefill_8b,
                "c4q8x3": workloads.prefill_c4_q8}
        precision = {"c4f32": "f32", "c4x3": "f32x3", "c4x3d128": "f32x3", "c4q8x3": "f32x3"}.get(key, "bf16")
        return bench_prefill(args, make[key](), precision)
    if key in ("c3", "c3cow"):
        return bench_kv(args, key == "c3cow")
    if key == "llama1b":
        return bench_model(args)
    if key == "prefix":
        return bench_prefix(args)
    if key == "conv":
        return bench_conversations(args)
    w = {"c1": workloads.decode_c1, "c2": workloads.decode_c2, "c5": workloads.decode_c5,
         "gqa8": workloads.decode_gqa8, "gqa8q8": lambda: workloads.decode_gqa8(q8=True),
         "gqa16": workloads.decode_gqa16, "gqa16q8": lambda: workloads.decode_gqa16(q8=True),
         "gemma2": workloads.decode_gemma2, "phi3": workloads.decode_phi3,
         "tiny": workloads.decode_tinyllama, "tinyq8": lambda: workloads.decode_tinyllama(q8=True),
         "t176": workloads.decode_t176}[key]()
    return bench_decode(args, key, w)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--workload", default="all",
                    choices=["all", "c1", "c2", "c3", "c3cow", "c4", "c4d128", "c4q8", "c4f32", "c4x3", "c4x3d128", "c4q8x3", "c5", "gqa8", "gqa8q8", "gqa16", "gqa16q8", "gemma2", "phi3",
                             "tiny", "tinyq8", "t176", "llama1b", "prefix", "conv"],
                    help="one configuration; `all` (the default) runs c1, t176, c3, c3cow, c4, c5, prefix and llama1b, "
                         "one JSON line each, then the c2 headline line last")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--split-tokens", type=int, default=0)
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="first run 3 device-to-device copies of this many MiB (a known-size kernel that "
                         "calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the path shards by sequence or KV head with no exchange; see the design notes)", file=sys.stderr)
        sys.exit(2)
    if args.split_tokens:
        os.environ["TVARA_SPLIT_TOKENS"] = str(args.split_tokens)

    from tvara_amd import hip

    if args.copy_mib:
        a, b = hip.DeviceArray((args.copy_mib << 18,)), hip.DeviceArray((args.copy_mib << 18,))
        for _ in range(3):
            hip.copy(b.ptr, a.ptr, a.nbytes)
        hip.synchronize()
        log(f"copied {args.copy_mib} MiB x3")
        del a, b
    if args.workload != "all":
        print(json.dumps(run_one(args, args.workload)), flush=True)
        return
    global DEFERRED
    DEFERRED = []
    results = []
    for key in DEFAULT_RUN:
        t0 = time.perf_counter()
        # the lines before the headline warm up for at least 100 steps: the
        # GPU clock ramps over the first few dozen launches after a fill (the
        # headline keeps exactly --warmup, right after the others' GPU runs)
        run_args = args if key == "c2" else argparse.Namespace(**{**vars(args), "warmup": max(args.warmup, 100)})
        results.append((key, run_one(run_args, key)))
        log(f"{key} done in {time.perf_counter() - t0:.1f}s")
    jobs, DEFERRED = DEFERRED, None
    for r, job in jobs:
        r["cpu_baseline"] = job()
    for key, r in results:
        print(json.dumps(r if key == "c2" else compact(r)), flush=True)


if __name__ == "__main__":
    main()
