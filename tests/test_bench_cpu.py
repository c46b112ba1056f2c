"""bench.py's CPU-baseline leg on the CPU: the reference's fused_paged_attention
run through the threaded shim runner gives the reference's own single-call
outputs, and a baseline record carries the protocol and host fields."""

import numpy as np

import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
import bench  # noqa: E402
from tvara_amd import workloads


def test_threaded_runner_matches_single_calls(ref):
    w = workloads.decode_c1()
    cache = ref.RefCache(1, w.kv_heads, w.head_dim, 16, 64)
    s = cache.create_sequence()
    cache.append_many(s, w.keys(0), w.values(0))
    q = w.queries()
    one = cache.fused_paged_attention(q[0], s, 0, w.heads, w.context)
    assert np.array_equal(cache.fused_batch([s, s, s], np.repeat(q, 3, 0), 0, w.heads, w.context, 3)[2], one)


def test_decode_baseline_record(ref):
    w = workloads.decode_c1()
    cache = ref.RefCache(1, w.kv_heads, w.head_dim, 16, 64)
    s = cache.create_sequence()
    cache.append_many(s, *bench.cpu_rows(w, w.keys(0), w.values(0)))
    r = bench.cpu_decode("c1", w, cache, [s], w.queries())
    assert r["kind"] == "reference" and r["protocol"] == "1 warm-up, median of 9 runs"
    assert r["value"] > 0 and r["one_thread"]["cores"] == 1 and r["cores"] == 1  # one sequence: one thread
    host = r["host"]
    assert host["nproc"] >= 1 and host["compiler"].startswith("g++") and isinstance(host["avx2_dot"], bool)
    assert host["triad_GBps_1thread"] > 0


def test_prefix_driver_replays_the_reference_workload(ref):
    """bench_prefix.cpp through the library's own ledger and prefix tree (the
    HIP-free host build) and through the reference's RadixCache: both give
    the counts the reference's benchmark records (bench/results/
    radix-prefix.json: 7,500 hits, 60,000 saved of 80,000 requested tokens)."""
    import shutil
    import subprocess

    import pytest

    if not shutil.which("g++") or not shutil.which("make"):
        pytest.skip("g++ / make not available")
    native = Path(__file__).resolve().parents[0] / "native"
    res = subprocess.run(["make", "-C", str(native)], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    from oracle import pyoracle

    for kind, lib in (("tvara", native / "_build" / "libtvara_host.so"), ("ref", pyoracle.REF_PATH)):
        r = bench.run_prefix_driver(kind, lib, runs=2)
        assert (r["requests"], r["hits"], r["saved_prefill_tokens"], r["requested_tokens"]) == (10000, 7500, 60000,
                                                                                                 80000), (kind, r)
        assert len(r["runs_ns"]) == 2 and min(r["runs_ns"]) > 0


def test_conversation_traces_are_the_references(ref, tmp_path):
    """The conversation traces replayed through the reference's own C ABI and
    CPU executor (oracle/_ref) on a model of its fixture's shape give the
    counts its tool recorded (bench/results/prefix-cache-traces.json: 3,675
    prompt tokens, 2,765 reused, 16 of 20 turns), and cache on/off give the
    same replies and logits, as that tool checks."""
    from tvara_amd import gguf_writer, native

    refso = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libtvara_ref_capi.so"
    m = native.NativeModel(gguf_writer.tiny_random_llama().write(tmp_path / "tiny.gguf"), library=str(refso),
                           max_blocks=256, block_tokens=16)
    traces = workloads.conversation_traces(vocab=m.vocab_size)
    summary, equal = bench.conversation_summary(bench.conversation_runs(m, traces, 1, ("off", "on")))
    m.close()
    assert equal
    assert (summary["on"]["prompt_tokens"], summary["on"]["reused_prompt_tokens"], summary["on"]["turn_hits"]) == \
        (3675, 2765, 16)
    assert (summary["off"]["prompt_tokens"], summary["off"]["reused_prompt_tokens"]) == (3675, 0)
