"""Write the golden fixtures of tests/golden/ from the reference's own code.

Run where the reference tree is present, after `make -C oracle ref`:

    python tests/golden/make_golden.py

Every expected value comes from core/include/tvara/{kv,attention,quant}.hpp
compiled into oracle/_ref/libtvara_ref.so (see oracle/ref_shim.cpp).  Inputs
are regenerated from tvara_amd.synth seeds (or the reference tests' signal()),
so the fixtures hold only seeds, shapes and outputs; the Q8_0 encoder vectors
hold the numpy evaluation of tools/make_api_fixture.py:131-137.
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import pyoracle as po  # noqa: E402
from tvara_amd import synth, workloads  # noqa: E402

OUT = Path(__file__).resolve().parent


def save(name, **arrays):
    np.savez_compressed(OUT / f"{name}.npz", **arrays)
    print(name, {k: v.shape for k, v in arrays.items()})


def decode_fixture(name, w, count=None):
    """fused_paged_attention outputs for the first `count` sequences of w."""
    count = count or w.sequences
    c = po.RefCache(w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks)
    workloads.place_blocks(c, w.placement())
    q = w.queries()
    out, tables = [], []
    for i in range(count):
        s = c.create_sequence()
        c.append_many(s, w.keys(i), w.values(i))
        out.append(c.fused_paged_attention(q[i], s, 0, w.heads, w.context))
        tables.append(np.array([b[0] for b in c.blocks(s)], np.int64))
    save(name, out=np.stack(out), lengths=np.array(w.lengths[:count]), first_table=tables[0],
         table_sizes=np.array([t.size for t in tables]), table_ids=np.concatenate(tables))


def reference_tests():
    """Outputs of the reference's own attention tests (tests/core/prefill_t171..t177.cpp
    inputs: signal(n, scale) = scale*sin(i*0.173f))."""
    arrays = {}
    # T171: 53 positions, 7-token blocks, 4 q / 2 kv heads, d=8; with and without a tail
    c = po.RefCache(1, 2, 8, 7, 32)
    s = c.create_sequence()
    k, v, q = synth.signal(53 * 16), synth.signal(53 * 16, 2), synth.signal(32, 3)
    c.append_many(s, k, v)
    arrays["t171"] = c.fused_paged_attention(q, s, 0, 4, 128)
    arrays["t171_tail"] = c.fused_paged_attention(q, s, 0, 4, 128, synth.signal(16, 4), synth.signal(16, 5))
    # T172: GQA ratios 8/4/2/1, 67 positions, d=8
    for kv in (1, 2, 4, 8):
        c = po.RefCache(1, kv, 8, 16, 8)
        s = c.create_sequence()
        w = kv * 8
        c.append_many(s, synth.signal(67 * w), synth.signal(67 * w, 2))
        arrays[f"t172_kv{kv}"] = c.fused_paged_attention(synth.signal(64, 3), s, 0, 8, 128)
    # T173: causal chunk rows 11..23 of 39 positions, 7-token blocks, 4 q / 1 kv, d=8
    c = po.RefCache(1, 1, 8, 7, 20)
    s = c.create_sequence()
    c.append_many(s, synth.signal(39 * 8), synth.signal(39 * 8, 2))
    arrays["t173"] = c.fused_prompt_attention(synth.signal(13 * 32, 3), s, 0, 11, 13, 4, 128)
    # T177: long contexts, 4 q / 2 kv heads, d=16
    for length in (1, 127, 1024, 4097, 8192):
        c = po.RefCache(1, 2, 16, 16, 512)
        s = c.create_sequence()
        c.append_many(s, synth.signal(length * 32, 8), synth.signal(length * 32, 2))
        arrays[f"t177_{length}"] = c.fused_paged_attention(synth.signal(64, 6), s, 0, 4, 8192)
    save("reference_tests", **arrays)


def prefill_fixture():
    """fused_prompt_attention rows of the 8 x (2048 + 512) chunked-prefill shape
    (32 q / 8 kv heads, d=64): sequence 0, chunk rows 0, 1, 255, 256, 510, 511."""
    w = workloads.prefill_c4()
    c = po.RefCache(1, 8, 64, 16, 200)
    s = c.create_sequence()
    k, v = w.keys(0), w.values(0)
    c.append_many(s, k, v)
    q = w.chunk_queries(0)
    rows = np.array([0, 1, 255, 256, 510, 511])
    out = np.stack([c.fused_prompt_attention(q[r], s, 0, w.prefix + r, 1, w.heads, w.context) for r in rows])
    save("c4_rows", rows=rows, out=out)


def q8_fixture():
    """Q8_0 decode: one Llama-3-8B-shaped sequence of 1,024 tokens (32/8 heads,
    d=128) quantised by the encoder expression; the reference dequantises with
    dequantize_q8_0 (quant.hpp:40-49) and runs fused_paged_attention in f32."""
    w = workloads.decode_c5(sequences=1, length=1024)
    k, v = w.keys(0), w.values(0)
    qk, qv = po.quantize_q8_0(k), po.quantize_q8_0(v)
    dk = po.ref_dequantize_q8_0(qk).reshape(k.shape)
    dv = po.ref_dequantize_q8_0(qv).reshape(v.shape)
    c = po.RefCache(1, 8, 128, 16, 70)
    s = c.create_sequence()
    c.append_many(s, dk, dv)
    out = c.fused_paged_attention(w.queries()[0], s, 0, 32, w.context)
    digest = hashlib.sha256(qk.tobytes() + qv.tobytes()).hexdigest()
    save("c5_q8", out=out, sha256=np.frombuffer(bytes.fromhex(digest), np.uint8))


def encoder_vectors():
    """The encoder of tools/make_api_fixture.py:131-137 evaluated by numpy on
    N(0,1) groups, exact .5 ties, a zero group and a subnormal-scale group."""
    groups = [synth.normal(9, "enc", 32 * 56).reshape(56, 32)]
    ties = np.linspace(-127, 127, 32, dtype=np.float32) / np.float32(127) * np.float32(3)
    half = (np.arange(32, dtype=np.float32) - 15.5) * np.float32(0.25)
    groups.append(np.stack([ties, half, np.zeros(32, np.float32), np.full(32, -1e-30, np.float32),
                            np.linspace(-1e4, 1e4, 32, dtype=np.float32), np.float32(1e-3) * half,
                            np.eye(32, dtype=np.float32)[3] * np.float32(-7), np.full(32, 0.5, np.float32)]))
    x = np.concatenate(groups).astype(np.float32)
    enc = []
    for block in x:
        scale = float(np.max(np.abs(block))) / 127
        quant = (np.zeros(32, dtype=np.int8) if scale == 0
                 else np.clip(np.round(block / scale), -127, 127).astype(np.int8))
        enc.append(np.frombuffer(np.asarray(scale, dtype="<f2").tobytes() + quant.tobytes(), np.uint8))
    save("q8_encoder", x=x, encoded=np.stack(enc))


def kv_stress_fixture(unaligned, **kw):
    """Block tables, reference counts, generations and free list after each
    phase of the shared-prefix stress, plus checksums of every live block."""
    w = workloads.kv_c3(unaligned=unaligned, **kw)
    c = po.RefCache(w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.max_blocks())
    phases = {}
    keep = {"fork", "step0", f"step{w.steps - 1}", "rollback"}

    def record(name, seqs):
        if name in keep:
            phases[name] = c.state(max_generation=16)

    seqs = workloads.run_kv_stress(c, w, record)
    arrays = {}
    for name, st in phases.items():
        arrays[f"{name}_refs"] = np.array(st["refs"], np.uint32)
        arrays[f"{name}_generations"] = np.array(st["generations"], np.uint32)
        arrays[f"{name}_free"] = np.array(st["free"], np.uint32)
        ids = sorted(st["tables"])
        arrays[f"{name}_seq_ids"] = np.array(ids, np.uint64)
        arrays[f"{name}_lengths"] = np.array([st["tables"][s][0] for s in ids], np.uint32)
        arrays[f"{name}_sizes"] = np.array([len(st["tables"][s][1]) for s in ids], np.uint32)
        arrays[f"{name}_blocks"] = np.array([b for s in ids for b in st["tables"][s][1]], np.uint32).reshape(-1, 2)
    live = sorted({h for s in seqs for h in c.blocks(s)})
    arrays["live"] = np.array(live, np.uint32).reshape(-1, 2)
    arrays["checksums"] = np.array([po.checksum_words(c.block_data(h)) for h in live], np.uint64)
    save(w.name.replace("(", "").replace(")", "").replace("+", "_"), **arrays)


if __name__ == "__main__":
    if not po.ref_available():
        sys.exit("build oracle/_ref first: make -C oracle ref")
    reference_tests()
    encoder_vectors()
    decode_fixture("c1_decode", workloads.decode_c1())
    decode_fixture("c2_decode_first4", workloads.decode_c2(), count=4)
    prefill_fixture()
    q8_fixture()
    kv_stress_fixture(False)
    kv_stress_fixture(True)
