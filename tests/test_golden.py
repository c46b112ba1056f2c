"""The oracle against fixtures the reference's own code wrote
(tests/golden/make_golden.py, oracle/_ref).  CPU only."""

import hashlib

import numpy as np
import pytest

import golden_data
import refmath
from tvara_amd import synth, workloads

TIGHT = 1e-6  # FP64 restatement of an FP64 reference: only the f32 rounding differs


def test_reference_test_outputs(oracle):
    g = golden_data.load("reference_tests")
    c = oracle.Cache(1, 2, 8, 7, 32)
    s = c.create_sequence()
    c.append_many(s, synth.signal(53 * 16), synth.signal(53 * 16, 2))
    assert refmath.close(c.fused_paged_attention(synth.signal(32, 3), s, 0, 4, 128), g["t171"], TIGHT)
    assert refmath.close(c.fused_paged_attention(synth.signal(32, 3), s, 0, 4, 128, synth.signal(16, 4),
                                                 synth.signal(16, 5)), g["t171_tail"], TIGHT)
    for kv in (1, 2, 4, 8):
        c = oracle.Cache(1, kv, 8, 16, 8)
        s = c.create_sequence()
        c.append_many(s, synth.signal(67 * kv * 8), synth.signal(67 * kv * 8, 2))
        assert refmath.close(c.fused_paged_attention(synth.signal(64, 3), s, 0, 8, 128), g[f"t172_kv{kv}"], TIGHT)
    c = oracle.Cache(1, 1, 8, 7, 20)
    s = c.create_sequence()
    c.append_many(s, synth.signal(39 * 8), synth.signal(39 * 8, 2))
    assert refmath.close(c.fused_prompt_attention(synth.signal(13 * 32, 3), s, 0, 11, 13, 4, 128), g["t173"], TIGHT)
    for length in (1, 127, 1024, 4097, 8192):
        c = oracle.Cache(1, 2, 16, 16, 512)
        s = c.create_sequence()
        c.append_many(s, synth.signal(length * 32, 8), synth.signal(length * 32, 2))
        assert refmath.close(c.fused_paged_attention(synth.signal(64, 6), s, 0, 4, 8192), g[f"t177_{length}"], TIGHT)


def test_encoder_vectors(oracle):
    g = golden_data.load("q8_encoder")
    for x, enc in zip(g["x"], g["encoded"]):
        assert np.array_equal(oracle.quantize_q8_0(x), enc)


@pytest.mark.parametrize("name,make,count", [("c1_decode", workloads.decode_c1, None),
                                             ("c2_decode_first4", workloads.decode_c2, 4)])
def test_decode_fixtures(oracle, name, make, count):
    g = golden_data.load(name)
    w = make()
    count = count or w.sequences
    c = oracle.Cache(w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks)
    workloads.place_blocks(c, w.placement())
    q = w.queries()
    ids = []
    for i in range(count):
        s = c.create_sequence()
        c.append_many(s, w.keys(i), w.values(i))
        ids += [b[0] for b in c.blocks(s)]
        assert refmath.close(c.fused_paged_attention(q[i], s, 0, w.heads, w.context), g["out"][i], TIGHT)
    assert np.array_equal(np.array(ids), g["table_ids"])


def test_prefill_rows(oracle):
    g = golden_data.load("c4_rows")
    w = workloads.prefill_c4()
    c = oracle.Cache(1, 8, 64, 16, 200)
    s = c.create_sequence()
    c.append_many(s, w.keys(0), w.values(0))
    q = w.chunk_queries(0)
    for r, want in zip(g["rows"], g["out"]):
        got = c.fused_prompt_attention(q[r], s, 0, w.prefix + int(r), 1, w.heads, w.context)
        assert refmath.close(got, want, TIGHT)


def test_q8_decode_fixture(oracle):
    g = golden_data.load("c5_q8")
    w = workloads.decode_c5(sequences=1, length=1024)
    k, v = w.keys(0), w.values(0)
    qk, qv = oracle.quantize_q8_0(k), oracle.quantize_q8_0(v)
    assert hashlib.sha256(qk.tobytes() + qv.tobytes()).digest() == bytes(g["sha256"])
    c = oracle.Cache(1, 8, 128, 16, 70)
    s = c.create_sequence()
    c.append_many(s, oracle.dequantize_q8_0(qk).reshape(k.shape), oracle.dequantize_q8_0(qv).reshape(v.shape))
    assert refmath.close(c.fused_paged_attention(w.queries()[0], s, 0, 32, w.context), g["out"], TIGHT)


@pytest.mark.parametrize("unaligned", [False, True], ids=["aligned-1024", "cow-1025"])
def test_kv_stress_traces(oracle, unaligned):
    w = workloads.kv_c3(unaligned=unaligned)
    c = oracle.Cache(w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.max_blocks())
    golden_data.check_stress(c, unaligned, lambda cache, live: [oracle.checksum_words(cache.block_data(h))
                                                                 for h in live])
