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
