"""Paged decode attention benchmark on one MI355X.

A step is one batched paged decode attention launch (decode kernel plus the
split merge) over the Llama-3.2-1B attention shape: 64 sequences, 32 query /
8 KV heads, head_dim 64, f32 KV, contexts uniform in [128, 4096], 16-token
blocks scattered over a 65,536-block pool.  Inputs (K/V blocks, block tables,
queries) are resident in HBM before the timed region.

Prints one JSON line: value = algorithmic bytes moved per step / step time
(GB/s), plus decode tokens/s, the roofline of the decode kernel from HIP events
around its own launches (a second pass of the same steps, so the event packets
stay out of the throughput region), and the reference CPU path timed on this
host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
METRIC = "paged decode attn: achieved HBM GB/s (% of peak) + decode tokens/s, 1 MI355X"
MODEL_LAYERS = {"llama-3.2-1b-decode-64x[128,4096]": 16, "smollm2-135m-decode-1x512": 30,
                "llama-3-8b-q8_0-decode-16x32768": 32}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(w, seconds_cap=30.0):
    """The reference's fused_paged_attention (oracle/_ref, built from the
    reference headers) on one host thread over the same workload; the C
    restatement of the oracle when _ref was not built."""
    import numpy as np

    from oracle import pyoracle
    from tvara_amd import workloads

    kind = "reference" if pyoracle.ref_available() else "port"
    make = pyoracle.RefCache if kind == "reference" else pyoracle.Cache
    g = (w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks)
    cache = make(*g)
    seqs = workloads.fill_decode(cache, w)
    q = w.queries()
    times, done_seqs = [], 0
    t_all = time.perf_counter()
    for rep in range(3):
        t0 = time.perf_counter()
        n = 0
        for i, s in enumerate(seqs):
            cache.fused_paged_attention(q[i], s, 0, w.heads, w.context)
            n += 1
            if time.perf_counter() - t_all > seconds_cap:
                break
        times.append((time.perf_counter() - t0, n))
        if time.perf_counter() - t_all > seconds_cap:
            break
    # median per-sequence-batch time scaled to the whole batch
    per_pass = sorted(t * len(seqs) / n for t, n in times)[len(times) // 2]
    done_seqs = times[-1][1]
    value = w.kv_bytes() / per_pass / 1e9
    del cache
    return {
        "value": round(value, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": kind,
        "sample": f"{len(times)} pass(es) of fused_paged_attention over {done_seqs} of {len(seqs)} sequences, "
                  f"1 thread, median scaled to the batch; {per_pass * 1e3:.1f} ms per batch, "
                  f"{len(seqs) / per_pass:.1f} decode tokens/s",
        "ms_per_step": round(per_pass * 1e3, 3),
    }


MFMA_BF16_PEAK_TFS = 2500.0  # MI355X dense bf16


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


def hbm_traffic(workload, kernel):
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
    (profiles/hbm_traffic.json, written from those runs), or None."""
    f = ROOT / "profiles" / "hbm_traffic.json"
    if not f.exists():
        return None
    entry = json.loads(f.read_text()).get(f"{workload}/{kernel}")
    return None if entry is None else int(entry["bytes_per_launch"])


def bench_prefill(args, w):
    """Chunked prefill, 8 x (2,048 cached + 512 causal chunk), 32/8 heads, d=64
    (or d=128): the bf16 MFMA kernel's TFLOP/s over the algorithmic 77.3 (154.6)
    GFLOP."""
    import numpy as np

    from tvara_amd import attention, hip, kv, workloads
    cache = kv.PagedCache(1, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks(), fmt=kv.Q8_0 if w.q8 else kv.F32)
    seqs = workloads.fill_prefill(cache, w)
    q = hip.DeviceArray.from_numpy(np.concatenate([w.chunk_queries(i) for i in range(w.sequences)]))
    out = hip.DeviceArray(q.shape)
    # one plan per prompt chunk (as an executor keeps it for every layer); a
    # step is one launch of it
    plan = attention.PrefillPlan(cache, seqs, [w.prefix] * w.sequences, [w.chunk] * w.sequences, w.heads, w.context,
                                 "bf16")
    call = lambda: plan.launch(0, q.ptr, out.ptr)  # noqa: E731
    for _ in range(args.warmup):
        call()
    plan.check()
    ms_per_step = timed_steps(call, args.steps)
    kernel_ms, _ = kernel_times(call, args.steps, ["paged_prefill_bf16"])["paged_prefill_bf16"]
    plan.check()
    assert np.isfinite(out.numpy()).all()
    tfs = w.flops() / (kernel_ms * 1e-3) / 1e12
    log(f"prefill kernel {kernel_ms * 1e3:.1f} us, call {ms_per_step * 1e3:.1f} us, {tfs:.1f} TFLOP/s")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import pyoracle

        if pyoracle.ref_available():
            # the reference's fused_prompt_attention (its FP64 loop, one
            # thread), sequence by sequence over about 80 GFLOP of the workload
            ns = max(1, min(w.sequences, int(80e9 * w.sequences / w.flops())))
            ref = pyoracle.RefCache(1, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks())
            rseqs = workloads.fill_prefill(ref, w)[:ns]
            t0 = time.perf_counter()
            for i, rs in enumerate(rseqs):
                ref.fused_prompt_attention(w.chunk_queries(i), rs, 0, w.prefix, w.chunk, w.heads, w.context)
            cpu_s = time.perf_counter() - t0
            cpu = {"value": round(w.flops() * ns / w.sequences / cpu_s / 1e12, 6), "unit": "TFLOP/s", "cores": 1,
                   "kind": "reference",
                   "sample": f"{ns} of the {w.sequences} chunks ({w.chunk} rows, {w.heads} heads each) through "
                             f"the reference's fused_prompt_attention, 1 thread: {cpu_s:.2f} s",
                   "seconds": round(cpu_s, 3)}
    print(json.dumps({
        "metric": "paged chunked prefill attn: achieved TFLOP/s (MFMA utilisation), 1 MI355X",
        "value": round(w.flops() / (ms_per_step * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic: K/V/q ~ N(0,1)",
        "config": {"workload": w.name, "sequences": w.sequences, "prefix": w.prefix, "chunk": w.chunk,
                   "heads": w.heads, "kv_heads": w.kv_heads, "head_dim": w.head_dim},
        "roofline": {"bound": "mfma", "achieved": round(tfs, 2), "peak": MFMA_BF16_PEAK_TFS, "unit": "TFLOP/s",
                     "frac": round(tfs / MFMA_BF16_PEAK_TFS, 4),
                     "traffic": hbm_traffic(w.name, "paged_prefill_bf16"), "kernel": "paged_prefill_bf16",
                     "kernel_avg_us": round(kernel_ms * 1e3, 3), "algorithmic_flops": w.flops()},
        "cpu_baseline": cpu,
    }), flush=True)


def bench_kv(args, cow):
    """KV-management stress: 256 sequences forked from a shared 1,024-token
    (or 1,025-token, copy-on-write) prefix, 22 layers x 8 x 64 f32; a step is
    one batched append of one token to every sequence (host bookkeeping, the
    zero-fill / copy-on-write launch and the row-copy launch).  K/V rows are
    resident in HBM.  Bytes per step: the rows written, plus a block's zero
    fill for every new block and a read and a write of a block for every
    copy-on-write."""
    import numpy as np

    from tvara_amd import hip, kv, workloads

    w = workloads.kv_c3(unaligned=cow)
    cache = kv.PagedCache(w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.max_blocks())
    width = w.layers * w.kv_heads * w.head_dim
    block_bytes = w.tokens_per_block * width * 2 * 4
    row_bytes = width * 2 * 4
    # four distinct step batches, used in turn (the contents do not change the work)
    batches = [(hip.DeviceArray.from_numpy(w.tokens(f"step{i}-k", w.sequences)),
                hip.DeviceArray.from_numpy(w.tokens(f"step{i}-v", w.sequences))) for i in range(4)]
    steps_k = [batches[i % 4][0] for i in range(w.steps)]
    steps_v = [batches[i % 4][1] for i in range(w.steps)]
    pk, pv = w.tokens("prefix-k", w.prefix), w.tokens("prefix-v", w.prefix)

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

    def setup():
        src = cache.create_sequence()
        cache.append_many(src, pk, pv)
        seqs = [cache.fork(src) for _ in range(w.sequences)]
        cache.drop(src)
        cache.synchronize()
        return seqs

    def run_pass(seqs, first, count, timed):
        start, stop = hip.Event(), hip.Event()
        hip.synchronize()
        start.record()
        for i in range(first, first + count):
            cache.append_batch_device(seqs, steps_k[i].ptr, steps_v[i].ptr)
        stop.record()
        hip.synchronize()
        return start.elapsed_ms(stop)

    # warm-up: whole passes, untimed
    for _ in range(max(1, args.warmup // w.steps)):
        seqs = setup()
        run_pass(seqs, 0, w.steps, False)
        for s in seqs:
            cache.drop(s)
    total_ms, done, nbytes = 0.0, 0, 0
    while done < args.steps:
        seqs = setup()
        n = min(w.steps, args.steps - done)
        total_ms += run_pass(seqs, 0, n, True)
        nbytes += sum(step_bytes(i) for i in range(n))
        done += n
        for s, r in zip(seqs, w.rollback()):  # speculative rollback (metadata only)
            cache.truncate(s, cache.length(s) - r)
        cache.audit()
        for s in seqs:
            cache.drop(s)
    ms_per_step = total_ms / done
    gbs = nbytes / (total_ms * 1e-3) / 1e9
    log(f"{w.name}: {ms_per_step * 1e3:.1f} us per step, {gbs:.1f} GB/s")
    cpu = None
    if not args.no_cpu_baseline:
        # the reference's PagedCache (oracle/_ref) on one host thread: one fork
        # of the prefix and the first 32 append steps
        from oracle import pyoracle

        kind = "reference" if pyoracle.ref_available() else "port"
        ref = (pyoracle.RefCache if kind == "reference" else pyoracle.Cache)(
            w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.max_blocks())
        src = ref.create_sequence()
        ref.append_many(src, pk, pv)
        rseqs = [ref.fork(src) for _ in range(w.sequences)]
        ref.drop(src)
        hk = [w.tokens(f"step{i}-k", w.sequences) for i in range(4)]
        hv = [w.tokens(f"step{i}-v", w.sequences) for i in range(4)]
        n_cpu = 32
        t0 = time.perf_counter()
        for i in range(n_cpu):
            ref.append_batch(rseqs, hk[i % 4], hv[i % 4])
        cpu_s = (time.perf_counter() - t0) / n_cpu
        cpu_bytes = sum(step_bytes(i) for i in range(n_cpu)) / n_cpu
        cpu = {"value": round(cpu_bytes / cpu_s / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind,
               "sample": f"{n_cpu} append steps of 256 tokens after one fork of the prefix, 1 thread; "
                         f"{cpu_s * 1e3:.2f} ms per step", "ms_per_step": round(cpu_s * 1e3, 4)}
        del ref
    print(json.dumps({
        "metric": "paged KV management stress: us per append step + GB/s, 1 MI355X", "value": round(gbs, 2),
        "unit": "GB/s", "n_gpus": 1, "steps": done, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: K/V rows from a seeded splitmix64 stream (floats in [1, 2))",
        "config": {"workload": w.name, "sequences": w.sequences, "prefix": w.prefix, "steps_per_pass": w.steps,
                   "layers": w.layers, "kv_heads": w.kv_heads, "head_dim": w.head_dim,
                   "tokens_per_block": w.tokens_per_block},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "kv_append (step)",
                     "algorithmic_bytes_per_step": round(nbytes / done)},
        "cpu_baseline": cpu,
    }), flush=True)


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
        m = native.NativeModel(path, max_blocks=nseq * ((prompt + args.steps + args.warmup + 64) // 16 + 1) + 64,
                               block_tokens=16)
        log(f"loaded in {time.perf_counter() - t0:.1f}s")
        rng = np.random.default_rng(3)
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
            f"{tps:.0f} tokens/s")
        cpu = None
        if not args.no_cpu_baseline:
            from oracle import pyoracle

            if pyoracle.ref_available():
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
        print(json.dumps({
            "metric": "llama-3.2-1b-shaped decode through the model-level C ABI: tokens/s, 1 MI355X",
            "value": round(tps, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(batch_s * 1e3, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32",
            "data": "synthetic: random Q8_0 weights (numpy PCG64), random token ids",
            "config": {"workload": "llama-3.2-1b-q8_0-decode-64seq", "sequences": nseq, "prompt": prompt,
                       "layers": spec.layers, "hidden": spec.hidden, "heads": spec.heads,
                       "kv_heads": spec.kv_heads, "intermediate": spec.intermediate, "vocab": spec.vocab},
            "single_sequence_ms_per_token": round(single_s * 1e3, 4),
            "single_sequence_weight_GBps": round(weight_bytes / single_s / 1e9, 1),
            "roofline": {"bound": "hbm", "achieved": round(step_bytes / batch_s / 1e9, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(step_bytes / batch_s / 1e9 / HBM_PEAK_GBS, 4),
                         "traffic": None, "kernel": "whole decode step (Q8_0 weights once + cached K/V)",
                         "algorithmic_bytes": step_bytes, "weight_bytes": weight_bytes, "kv_bytes": kv_bytes},
            "cpu_baseline": cpu,
        }), flush=True)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--workload", default="c2", choices=["c1", "c2", "c3", "c3cow", "c4", "c4d128", "c4q8", "c5", "gqa8", "gqa8q8", "tiny",
                             "tinyq8", "llama1b"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--split-tokens", type=int, default=0)
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="first run 3 device-to-device copies of this many MiB (a known-size kernel that "
                         "calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the path shards by sequence or KV head with no exchange; see the design notes)", file=sys.stderr)
        sys.exit(2)
    if args.split_tokens:
        os.environ["TVARA_SPLIT_TOKENS"] = str(args.split_tokens)

    import numpy as np

    from tvara_amd import attention, hip, kv, workloads

    if args.copy_mib:
        a, b = hip.DeviceArray((args.copy_mib << 18,)), hip.DeviceArray((args.copy_mib << 18,))
        for _ in range(3):
            hip.copy(b.ptr, a.ptr, a.nbytes)
        hip.synchronize()
        log(f"copied {args.copy_mib} MiB x3")
        del a, b
    if args.workload in ("c4", "c4d128", "c4q8"):
        make = {"c4": workloads.prefill_c4, "c4d128": workloads.prefill_8b, "c4q8": workloads.prefill_c4_q8}
        return bench_prefill(args, make[args.workload]())
    if args.workload in ("c3", "c3cow"):
        return bench_kv(args, args.workload == "c3cow")
    if args.workload == "llama1b":
        return bench_model(args)
    w = {"c1": workloads.decode_c1, "c2": workloads.decode_c2, "c5": workloads.decode_c5,
         "gqa8": workloads.decode_gqa8, "gqa8q8": lambda: workloads.decode_gqa8(q8=True),
         "tiny": workloads.decode_tinyllama, "tinyq8": lambda: workloads.decode_tinyllama(q8=True)}[args.workload]()
    log(f"workload {w.name}: {w.sequences} sequences, {w.total_tokens} tokens")
    g = (w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks)
    cache = kv.PagedCache(*g, fmt=kv.Q8_0 if w.q8 else kv.F32)
    t0 = time.perf_counter()
    seqs = workloads.fill_decode(cache, w)
    cache.synchronize()
    log(f"filled in {time.perf_counter() - t0:.1f}s")
    q = hip.DeviceArray.from_numpy(w.queries())
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
    log(f"step {ms_per_step * 1e3:.1f} us; decode kernel {kernel_avg_ms * 1e3:.1f} us x{launches}; "
        f"merge {merge_ms * 1e3:.1f} us x{merges}")
    assert np.isfinite(out.numpy()).all()
    # the same batch through the host-buffer entry point (queries in and
    # outputs out over PCIe, block tables uploaded per call): reported beside
    # the value, never as it
    qh = w.queries()
    attention.decode_batch(cache, qh, seqs, 0, w.heads, w.context)
    t0 = time.perf_counter()
    for _ in range(20):
        attention.decode_batch(cache, qh, seqs, 0, w.heads, w.context)
    host_ms = (time.perf_counter() - t0) / 20 * 1e3

    kv_bytes = w.kv_bytes()
    step_bytes = kv_bytes + w.qo_bytes() + w.table_bytes()
    gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    kernel_gbs = (kv_bytes + w.qo_bytes() // 2 + w.table_bytes()) / (kernel_avg_ms * 1e-3) / 1e9
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
        "decode_tokens_per_s": round(tokens_per_s, 1),
        "model_decode_tokens_per_s": round(tokens_per_s / layers, 1),
        "model_layers": layers,
        "host_buffers_ms_per_step": round(host_ms, 4),
        "roofline": {"bound": "hbm", "achieved": round(kernel_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kernel_gbs / HBM_PEAK_GBS, 4), "traffic": hbm_traffic(w.name, "paged_decode"),
                     "kernel": "paged_decode", "kernel_avg_us": round(kernel_avg_ms * 1e3, 3),
                     "algorithmic_bytes": kv_bytes + w.qo_bytes() // 2 + w.table_bytes()},
    }
    del plan, cache, q, out
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        result["cpu_baseline"] = cpu_baseline(w)
        log(f"cpu baseline in {time.perf_counter() - t0:.1f}s")
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
