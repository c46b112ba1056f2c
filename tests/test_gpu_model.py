"""The model-level exports on the GPU against the reference's own C ABI
(core/src/c_api.cpp + its CPU executor, built into oracle/_ref) on the same
synthetic GGUF files: logits of every decoded token, metadata JSON, and the
sequence semantics of decode_batch (rollback), truncate, drop and the error
paths (c_api.cpp:35-78, paged_model.hpp:12-28).

Logit bar: |gpu - ref| <= 1e-4 * (1 + |ref|) per element.  Derivation: the
matvecs and RMSNorm accumulate in double and round once as the reference
does, RoPE uses the host's cos/sin exactly as rotary() computes them, and
weights dequantise to the reference's floats; what differs is the attention
(f32 online softmax against the reference's FP64, within 1e-6 relative,
tests/test_gpu_decode.py) and expf in the SwiGLU gate (within 2 ulp).  Those
relative errors of ~1e-6 per layer pass through the remaining matvecs with a
gain of order one for these 1/sqrt(fan-in)-scaled weights, so a few layers
stay near 1e-5 of the logit scale -- a tenth of the bar.
"""

import sys
from pathlib import Path

import numpy as np
import pytest

from tvara_amd import gguf_writer as gf
from tvara_amd import native

pytestmark = pytest.mark.gpu
TOL = 1e-4
REF = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libtvara_ref_capi.so"


def say(*a):
    print(*a, flush=True, file=sys.stderr)


@pytest.fixture(scope="module")
def ref_capi():
    if not REF.exists():
        pytest.skip("reference C ABI not built (make -C oracle ref)")
    return str(REF)


def close(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return bool(np.all(np.abs(got - want) <= TOL * (1 + np.abs(want)))), float(
        np.max(np.abs(got - want) / (1 + np.abs(want))))


SPECS = {
    "f32-gqa": dict(),
    "f16-split-tied": dict(matrix_type=gf.T_F16, embed_type=gf.T_F16, norm_type=gf.T_F16, rope_layout="split",
                           output=False),
    "q8_0-gqa4": dict(matrix_type=gf.T_Q8_0, heads=8, kv_heads=2, hidden=128, intermediate=256),
    "q4_0-mha": dict(matrix_type=gf.T_Q4_0, heads=4, kv_heads=4, rope_layout="interleaved"),
    "q4_k-256": dict(matrix_type=gf.T_Q4_K, hidden=256, intermediate=512, heads=4, kv_heads=1, layers=3),
    # Q8_0 kept quantised in HBM, the tied embedding too: a vocabulary and
    # widths that leave partial 16-row tiles and group counts not divisible
    # by four
    "q8_0-tied-ragged": dict(matrix_type=gf.T_Q8_0, embed_type=gf.T_Q8_0, output=False, vocab=100, hidden=96,
                             intermediate=160, heads=3, kv_heads=1),
    # Q8_0 with the split RoPE layout (rotation outside the product epilogue)
    "q8_0-split-rope": dict(matrix_type=gf.T_Q8_0, rope_layout="split", hidden=128, intermediate=256, heads=4,
                            kv_heads=2),
}


@pytest.mark.parametrize("name", list(SPECS))
def test_logits_match_reference(tmp_path, ref_capi, name):
    spec = gf.LlamaSpec(**SPECS[name])
    path = spec.write(tmp_path / f"{name}.gguf")
    say("model", name)
    mine = native.NativeModel(path, max_blocks=32, block_tokens=4)
    ref = native.NativeModel(path, library=ref_capi, max_blocks=32, block_tokens=4)
    assert (mine.vocab_size, mine.context_size) == (ref.vocab_size, ref.context_size)
    assert mine.metadata_json() == ref.metadata_json()
    sm, sr = mine.new_sequence(), ref.new_sequence()
    assert sm == sr
    tokens = [int(t) for t in np.random.default_rng(1).integers(0, spec.vocab, 40)]
    worst = 0.0
    for t in tokens[:13]:  # token by token, across block boundaries (4-token blocks)
        ok, err = close(mine.logits(sm, t), ref.logits(sr, t))
        worst = max(worst, err)
        assert ok, (name, t, err)
    got, want = mine.decode_batch(sm, tokens[13:20]), ref.decode_batch(sr, tokens[13:20])
    ok, err = close(got, want)
    assert ok, err
    worst = max(worst, err)
    # speculative rollback: truncate and continue with other tokens
    mine.truncate(sm, 15)
    ref.truncate(sr, 15)
    got, want = mine.decode_batch(sm, tokens[20:28]), ref.decode_batch(sr, tokens[20:28])
    ok, err = close(got, want)
    assert ok, err
    worst = max(worst, err)
    # a second sequence interleaved with the first
    s2m, s2r = mine.new_sequence(), ref.new_sequence()
    for t in tokens[28:34]:
        ok, err = close(mine.logits(s2m, t), ref.logits(s2r, t))
        assert ok, err
        ok, err = close(mine.logits(sm, t), ref.logits(sr, t))
        assert ok, err
    mine.drop_sequence(s2m)
    ref.drop_sequence(s2r)
    say(name, "worst relative logit error", worst)
    mine.close()
    ref.close()


def errors(model, fn, *args):
    try:
        fn(*args)
    except RuntimeError as e:
        return str(e)
    return None


def test_sequence_semantics_match_reference(tmp_path, ref_capi):
    spec = gf.LlamaSpec(context=24)
    path = spec.write(tmp_path / "m.gguf")
    # a 5-block pool of 4-token blocks: 20 tokens fit
    mine = native.NativeModel(path, max_blocks=5, block_tokens=4)
    ref = native.NativeModel(path, library=ref_capi, max_blocks=5, block_tokens=4)
    sm, sr = mine.new_sequence(), ref.new_sequence()
    first = list(range(1, 11))
    ok, err = close(mine.decode_batch(sm, first), ref.decode_batch(sr, first))
    assert ok, err
    # a batch that exhausts the pool midway fails and leaves the sequence at its entry length
    more = list(range(20, 32))
    em, er = errors(mine, mine.decode_batch, sm, more), errors(ref, ref.decode_batch, sr, more)
    assert em == er and em is not None, (em, er)
    ok, err = close(mine.logits(sm, 5), ref.logits(sr, 5))  # continues from length 10
    assert ok, err
    # a token outside the vocabulary anywhere in a batch: nothing is decoded
    bad = [1, 2, spec.vocab]
    assert errors(mine, mine.decode_batch, sm, bad) == errors(ref, ref.decode_batch, sr, bad) == "invalid batch token"
    ok, err = close(mine.logits(sm, 6), ref.logits(sr, 6))
    assert ok, err
    # context: 12 cached + 13 > 24
    long = [3] * 13
    assert errors(mine, mine.decode_batch, sm, long) == errors(ref, ref.decode_batch, sr, long) == \
        "batch exceeds context"
    # unknown sequence, truncate past the end, drop twice
    for fn_m, fn_r, args in [(mine.logits, ref.logits, (999, 1)), (mine.truncate, ref.truncate, (sm, 100)),
                             (mine.drop_sequence, ref.drop_sequence, (999,))]:
        a, b = errors(mine, fn_m, *args), errors(ref, fn_r, *args)
        assert a == b and a is not None, (a, b)
    mine.drop_sequence(sm)
    ref.drop_sequence(sr)
    assert errors(mine, mine.logits, sm, 1) == errors(ref, ref.logits, sr, 1)


def test_context_limit_and_geometry(tmp_path, ref_capi):
    spec = gf.LlamaSpec(context=6)
    path = spec.write(tmp_path / "m.gguf")
    mine = native.NativeModel(path, max_blocks=8, block_tokens=2)
    ref = native.NativeModel(path, library=ref_capi, max_blocks=8, block_tokens=2)
    sm, sr = mine.new_sequence(), ref.new_sequence()
    mine.decode_batch(sm, [1, 2, 3, 4, 5, 6])
    ref.decode_batch(sr, [1, 2, 3, 4, 5, 6])
    assert errors(mine, mine.logits, sm, 1) == errors(ref, ref.logits, sr, 1) == \
        "paged decode exceeds token/context limits"
    # cache geometry the reference rejects (kv.hpp:24-27)
    for blocks, tokens in [(0, 16), (2000000, 16), (8, 0)]:
        lm, lr = native._capi.lib(), native._capi.model_lib(ref_capi)
        assert not lm.tvara_model_open(str(path).encode(), blocks, tokens)
        assert not lr.tvara_model_open(str(path).encode(), blocks, tokens)
        assert lm.tvara_last_error() == lr.tvara_last_error(), (blocks, tokens)


def test_nonfinite_weight_rejected(tmp_path, ref_capi):
    spec = gf.LlamaSpec()
    tensors = spec.tensors()
    name, dims, ttype, payload = tensors[3]
    w = np.frombuffer(payload, "<f4").copy()
    w[7] = np.inf
    tensors[3] = (name, dims, ttype, w.tobytes())
    path = tmp_path / "inf.gguf"
    gf.write_gguf(path, spec.metadata(), tensors)
    a = errors(None, native.NativeModel, path)
    b = errors(None, native.NativeModel, path, ref_capi)
    assert a == b == "nonfinite model weight"


@pytest.mark.parametrize("scale", [0x7C00, 0x7E00])  # fp16 inf, NaN
def test_nonfinite_q8_0_scale_rejected(tmp_path, ref_capi, scale):
    # a Q8_0 matrix kept quantised: a non-finite group scale makes its values
    # non-finite, which the reference rejects at load (model.hpp:138)
    spec = gf.LlamaSpec(matrix_type=gf.T_Q8_0)
    tensors = spec.tensors()
    i = next(k for k, t in enumerate(tensors) if t[0] == "blk.1.ffn_up.weight")
    name, dims, ttype, payload = tensors[i]
    raw = bytearray(payload() if isinstance(payload, gf.Lazy) else payload)
    raw[34 * 5:34 * 5 + 2] = scale.to_bytes(2, "little")
    tensors[i] = (name, dims, ttype, bytes(raw))
    path = tmp_path / "bad.gguf"
    gf.write_gguf(path, spec.metadata(), tensors)
    a = errors(None, native.NativeModel, path)
    b = errors(None, native.NativeModel, path, ref_capi)
    assert a == b == "nonfinite model weight"


@pytest.mark.parametrize("nseq,embed,vocab", [(3, gf.T_F32, 96), (20, gf.T_F32, 96), (41, gf.T_Q8_0, 96),
                                               (70, gf.T_Q8_0, 96), (64, gf.T_Q8_0, 16390),
                                               (64, gf.T_Q8_0, 32800), (20, gf.T_Q8_0, 131072)])
def test_sequences_decode_matches_serial_reference(tmp_path, ref_capi, nseq, embed, vocab):
    # one pass for many sequences (tvara_sequences_decode) against the
    # reference decoding each sequence on its own; 41 and 70 sequences take
    # partial and multiple 64-vector passes of the batched Q8_0 products.  The
    # 16,390-row tied logits matrix (1,025 row tiles, the last one partial)
    # takes the four-tile workgroups that the model's largest products use;
    # at 32,800 rows (8.4 MB of logits for 64 sequences) and 131,072 rows
    # (10.5 MB for 20 sequences, two-wave workgroups) the logits are computed
    # and copied to the host in four bands of row tiles.
    spec = gf.LlamaSpec(matrix_type=gf.T_Q8_0, embed_type=embed, output=embed == gf.T_F32, hidden=128,
                        intermediate=256, heads=8, kv_heads=2, vocab=vocab)
    path = spec.write(tmp_path / "m.gguf")
    mine = native.NativeModel(path, max_blocks=512, block_tokens=4)
    ref = native.NativeModel(path, library=ref_capi, max_blocks=512, block_tokens=4)
    rng = np.random.default_rng(nseq)
    sm = [mine.new_sequence() for _ in range(nseq)]
    sr = [ref.new_sequence() for _ in range(nseq)]
    for a, b in zip(sm, sr):  # ragged prompts, 1..9 tokens
        prompt = [int(t) for t in rng.integers(0, spec.vocab, int(rng.integers(1, 10)))]
        ok, err = close(mine.decode_batch(a, prompt), ref.decode_batch(b, prompt))
        assert ok, err
    worst = 0.0
    for step in range(4):
        toks = [int(t) for t in rng.integers(0, spec.vocab, nseq)]
        got = mine.decode_sequences(sm, toks)
        for i, (b, t) in enumerate(zip(sr, toks)):
            ok, err = close(got[i], ref.logits(b, t))
            worst = max(worst, err)
            assert ok, (step, i, err)
    say("sequences_decode", nseq, "worst relative logit error", worst)


def test_sequences_decode_all_or_nothing(tmp_path, ref_capi):
    spec = gf.LlamaSpec(context=12)
    path = spec.write(tmp_path / "m.gguf")
    mine = native.NativeModel(path, max_blocks=6, block_tokens=4)
    ref = native.NativeModel(path, library=ref_capi, max_blocks=6, block_tokens=4)
    a, b, c = mine.new_sequence(), mine.new_sequence(), mine.new_sequence()
    ra, rb, rc = ref.new_sequence(), ref.new_sequence(), ref.new_sequence()
    for s, r, n in [(a, ra, 4), (b, rb, 8), (c, rc, 11)]:
        ok, err = close(mine.decode_batch(s, list(range(1, n + 1))), ref.decode_batch(r, list(range(1, n + 1))))
        assert ok, err
    assert mine.decode_sequences([], []).shape == (0, spec.vocab)
    # duplicate sequence, a token past the vocabulary, a full context (c at 11 -> 12 ok, then 12 -> fail)
    assert errors(mine, mine.decode_sequences, [a, a], [1, 2]) == "duplicate sequence in decode batch"
    assert errors(mine, mine.decode_sequences, [a, b], [1, spec.vocab]) == "paged decode exceeds token/context limits"
    # the pool: a (4 tokens, 1 block) + b (8, 2) + c (11, 3) = all 6 blocks.  In the
    # order [c, b, a], c's row fits its tail block and is appended, then b needs a
    # new block: the pool is exhausted, and c must be rolled back
    e = errors(mine, mine.decode_sequences, [c, b, a], [5, 6, 7])
    assert e == errors(ref, ref.logits, rb, 6), e
    ok, err = close(mine.decode_sequences([c], [5]), ref.logits(rc, 5)[None])  # c continues at 11
    assert ok, err
    mine.drop_sequence(a)
    ref.drop_sequence(ra)
    ok, err = close(mine.decode_sequences([b], [6]), ref.logits(rb, 6)[None])  # b continues at 8
    assert ok, err
    assert errors(mine, mine.decode_sequences, [c, b], [1, 2]) == "paged decode exceeds token/context limits"


def test_sequences_decode_odd_width_falls_back(tmp_path, ref_capi):
    # hidden 40 is not a multiple of the batched kernels' 32-column tiles: the
    # batch runs sequence by sequence with the same all-or-nothing contract
    spec = gf.LlamaSpec(hidden=40, intermediate=72, heads=4, kv_heads=2)
    path = spec.write(tmp_path / "odd.gguf")
    mine = native.NativeModel(path, max_blocks=32, block_tokens=4)
    ref = native.NativeModel(path, library=ref_capi, max_blocks=32, block_tokens=4)
    sm = [mine.new_sequence() for _ in range(3)]
    sr = [ref.new_sequence() for _ in range(3)]
    for step in range(3):
        toks = [step + 1, step + 5, step + 9]
        got = mine.decode_sequences(sm, toks)
        ok, err = close(got, np.stack([ref.logits(r, t) for r, t in zip(sr, toks)]))
        assert ok, err
    # decode_batch and prefill decode such a model token by token
    ok, err = close(mine.decode_batch(sm[0], [4, 5, 6]), ref.decode_batch(sr[0], [4, 5, 6]))
    assert ok, err
    ok, err = close(mine.prefill(sm[1], [7, 8, 9]), ref.decode_batch(sr[1], [7, 8, 9])[-1])
    assert ok, err


CHUNK_SPECS = {
    "f32": dict(context=1200),
    "q8_0-gqa4": dict(matrix_type=gf.T_Q8_0, heads=8, kv_heads=2, hidden=128, intermediate=256, context=1200),
    "q8_0-tied-ragged": dict(matrix_type=gf.T_Q8_0, embed_type=gf.T_Q8_0, output=False, vocab=100, hidden=96,
                             intermediate=160, heads=3, kv_heads=1, context=1200),
    "f16-split": dict(matrix_type=gf.T_F16, rope_layout="split", context=1200),
    # head_dim 64 and 128: with blocks of 16 tokens the passes' attention runs
    # on the three-product MFMA tiles, with blocks of 4 on the f32 rows
    "q8_0-d64": dict(matrix_type=gf.T_Q8_0, hidden=256, intermediate=512, heads=4, kv_heads=2, context=1200),
    "f32-d128": dict(hidden=256, intermediate=256, heads=2, kv_heads=1, context=1200),
    # sixteen query heads per KV head: the tiles run as two slices of eight
    "q8_0-d64-g16": dict(matrix_type=gf.T_Q8_0, hidden=1024, intermediate=512, heads=16, kv_heads=1, context=1200),
}


@pytest.mark.parametrize("name", list(CHUNK_SPECS))
@pytest.mark.parametrize("block_tokens", [4, 16])
def test_decode_batch_chunks_match_reference(tmp_path, ref_capi, name, block_tokens):
    # tvara_sequence_decode_batch runs a chunk of tokens as one pass (batched
    # products, each layer's K/V written into the cache, causal attention over
    # it) where the reference decodes token by token: a batch starting
    # mid-block, one of 1,100 tokens (passes of 512, 512 and 76 rows), a
    # rollback into the middle of it and a continuation, every logit row
    # against the reference's
    spec = gf.LlamaSpec(**CHUNK_SPECS[name])
    path = spec.write(tmp_path / f"{name}.gguf")
    mine = native.NativeModel(path, max_blocks=1200 // block_tokens + 8, block_tokens=block_tokens)
    ref = native.NativeModel(path, library=ref_capi, max_blocks=1200 // block_tokens + 8, block_tokens=block_tokens)
    sm, sr = mine.new_sequence(), ref.new_sequence()
    rng = np.random.default_rng(3)
    tokens = [int(t) for t in rng.integers(0, spec.vocab, 1200)]
    worst = 0.0
    for t in tokens[:3]:
        ok, err = close(mine.logits(sm, t), ref.logits(sr, t))
        assert ok, err
    for lo, hi in [(3, 9), (9, 1109)]:
        say(name, block_tokens, "batch", lo, hi)
        got, want = mine.decode_batch(sm, tokens[lo:hi]), ref.decode_batch(sr, tokens[lo:hi])
        ok, err = close(got, want)
        worst = max(worst, err)
        assert ok, (lo, hi, err, int(np.argmax(np.max(np.abs(got - want), axis=1))))
    mine.truncate(sm, 600)
    ref.truncate(sr, 600)
    got, want = mine.decode_batch(sm, tokens[1109:1150]), ref.decode_batch(sr, tokens[1109:1150])
    ok, err = close(got, want)
    worst = max(worst, err)
    assert ok, err
    ok, err = close(mine.logits(sm, 7), ref.logits(sr, 7))
    assert ok, err
    say(name, block_tokens, "worst relative logit error", worst)


def test_chunk_attention_rows_switch(tmp_path, ref_capi, monkeypatch):
    # TVARA_CHUNK_ATTENTION=rows: the chunked pass attends through the f32 rows
    # (the reference's arithmetic) where the three-product tiles would run;
    # both stay within the bar, and the rows come closer
    spec = gf.LlamaSpec(**CHUNK_SPECS["q8_0-d64"])
    path = spec.write(tmp_path / "m.gguf")
    ref = native.NativeModel(path, library=ref_capi, max_blocks=1200 // 16 + 8, block_tokens=16)
    tokens = [int(t) for t in np.random.default_rng(5).integers(0, spec.vocab, 600)]
    sr = ref.new_sequence()
    want = ref.decode_batch(sr, tokens)
    errs = {}
    for choice in ("tiles", "rows"):
        monkeypatch.setenv("TVARA_CHUNK_ATTENTION", choice)
        mine = native.NativeModel(path, max_blocks=1200 // 16 + 8, block_tokens=16)
        got = mine.decode_batch(mine.new_sequence(), tokens)
        ok, err = close(got, want)
        assert ok, (choice, err)
        errs[choice] = err
        mine.close()
    say("chunk attention worst relative logit error", errs)
    assert errs["rows"] < errs["tiles"]


def test_chunk_tiles_beyond_fp16_take_the_rows(tmp_path, monkeypatch):
    # attention norms of 2e5 put queries and keys past the fp16 range (65,504)
    # that the three-product tiles carry them in: the tiles flag the pass and it
    # runs again on the f32 rows, whose logits these are, bit for bit
    spec = gf.LlamaSpec(**CHUNK_SPECS["f32-d128"], attn_norm_scale=2e5)
    path = spec.write(tmp_path / "m.gguf")
    tokens = [int(t) for t in np.random.default_rng(8).integers(0, spec.vocab, 300)]
    got = {}
    for choice in ("tiles", "rows"):
        monkeypatch.setenv("TVARA_CHUNK_ATTENTION", choice)
        mine = native.NativeModel(path, max_blocks=1200 // 16 + 8, block_tokens=16)
        sm = mine.new_sequence()
        got[choice] = mine.decode_batch(sm, tokens)
        assert mine.cache().length(sm) == len(tokens)
        mine.close()
    assert np.isfinite(got["rows"]).all()
    assert np.array_equal(got["tiles"], got["rows"])


def test_prefill_matches_reference_last_logits(tmp_path, ref_capi):
    # tvara_sequence_prefill: the last token's logits of a chunked pass, with
    # decode_batch's checks, messages and rollback
    spec = gf.LlamaSpec(matrix_type=gf.T_Q8_0, heads=8, kv_heads=2, hidden=128, intermediate=256, context=64)
    path = spec.write(tmp_path / "m.gguf")
    mine = native.NativeModel(path, max_blocks=10, block_tokens=4)  # 40 tokens fit
    ref = native.NativeModel(path, library=ref_capi, max_blocks=10, block_tokens=4)
    sm, sr = mine.new_sequence(), ref.new_sequence()
    ok, err = close(mine.prefill(sm, [5]), ref.decode_batch(sr, [5])[-1])
    assert ok, err
    prompt = [int(t) for t in np.random.default_rng(9).integers(0, spec.vocab, 25)]
    ok, err = close(mine.prefill(sm, prompt), ref.decode_batch(sr, prompt)[-1])
    assert ok, err
    cache = mine.cache()
    assert cache.length(sm) == 26
    with pytest.raises(ValueError, match="empty prompt"):
        mine.prefill(sm, [])
    assert errors(mine, mine.prefill, sm, [1, 2, spec.vocab]) == "invalid batch token"
    assert cache.length(sm) == 26
    # 26 + 20 > 40 pool tokens: the pool runs out partway; nothing stays appended
    more = list(range(1, 21))
    em, er = errors(mine, mine.prefill, sm, more), errors(ref, ref.decode_batch, sr, more)
    assert em == er and em is not None, (em, er)
    assert cache.length(sm) == 26
    ok, err = close(mine.logits(sm, 3), ref.logits(sr, 3))
    assert ok, err
    # 27 cached + 38 > 64: the context check, as decode_batch's
    long = [2] * 38
    assert errors(mine, mine.prefill, sm, long) == errors(ref, ref.decode_batch, sr, long) == "batch exceeds context"


def test_decode_batch_on_a_fork_copies_on_write(tmp_path, ref_capi):
    # a chunk appended to a fork whose last block is shared and partly full:
    # the block is copied on write before the chunk's rows land, and the
    # forked-from sequence still decodes as before
    spec = gf.LlamaSpec(matrix_type=gf.T_Q8_0, heads=8, kv_heads=2, hidden=128, intermediate=256, context=128)
    path = spec.write(tmp_path / "m.gguf")
    mine = native.NativeModel(path, max_blocks=64, block_tokens=4)
    ref = native.NativeModel(path, library=ref_capi, max_blocks=64, block_tokens=4)
    rng = np.random.default_rng(4)
    prefix = [int(t) for t in rng.integers(0, spec.vocab, 10)]
    tail = [int(t) for t in rng.integers(0, spec.vocab, 30)]
    other = [int(t) for t in rng.integers(0, spec.vocab, 7)]
    a, ra, rf = mine.new_sequence(), ref.new_sequence(), ref.new_sequence()
    mine.decode_batch(a, prefix)
    ref.decode_batch(ra, prefix)
    ref.decode_batch(rf, prefix)
    cache = mine.cache()
    f = cache.fork(a)
    shared = cache.blocks(a)[-1]
    ok, err = close(mine.decode_batch(f, tail), ref.decode_batch(rf, tail))
    assert ok, err
    assert cache.blocks(a)[-1] == shared and cache.blocks(f)[-1] != shared
    ok, err = close(mine.decode_batch(a, other), ref.decode_batch(ra, other))
    assert ok, err


def test_conversation_replay_reuses_prefixes(tmp_path, ref_capi):
    # the reference's conversation traces (tools/run_prefix_cache_traces.py)
    # on a model of its fixture's shape (hidden 16: token by token): modes
    # off, on and radix give the same replies and bit-identical prompt logits;
    # on reuses the reference's 2,765 of 3,675 prompt tokens, radix also the
    # 64-token system prompt of the three later conversations; the first
    # prompt's logits are within the bar of the reference executor's
    from tvara_amd import radix, workloads

    spec = gf.tiny_random_llama()
    path = spec.write(tmp_path / "tiny.gguf")
    mine = native.NativeModel(path, max_blocks=256, block_tokens=16)
    traces = workloads.conversation_traces(vocab=mine.vocab_size)
    cache = mine.cache()
    out = {}
    for mode in ("off", "on", "radix"):
        say("conversations", mode)
        tree = radix.RadixCache(cache, "tiny/test") if mode == "radix" else None
        out[mode] = [t for trace in workloads.replay_conversations(mine, traces, mode, tree=tree) for t in trace]
        if tree is not None:
            tree.close()
        assert cache.sequence_ids() == []
    for mode, reused in (("off", 0), ("on", 2765), ("radix", 2765 + 3 * 64)):
        assert sum(t["prompt_tokens"] for t in out[mode]) == 3675
        assert sum(t["reused_tokens"] for t in out[mode]) == reused, mode
    for a, b, c in zip(out["off"], out["on"], out["radix"]):
        assert a["reply"] == b["reply"] == c["reply"]
        assert np.array_equal(a["logits"], b["logits"]) and np.array_equal(a["logits"], c["logits"])
    ref = native.NativeModel(path, library=ref_capi, max_blocks=256, block_tokens=16)
    s = ref.new_sequence()
    ok, err = close(out["off"][0]["logits"], ref.decode_batch(s, traces[0]["system"] + traces[0]["users"][0])[-1])
    assert ok, err
    ref.close()
    mine.close()


class _SerialBackend:
    """The reference's NativeSchedulerBackend loop (scheduler.py:201-210),
    over any NativeModel (here the reference's own library)."""

    def __init__(self, model):
        self.model, self.sequences, self.pending = model, {}, {}

    def create(self, key):
        self.sequences[key] = self.model._new_sequence()

    def prefill(self, key, tokens):
        for token in tokens:
            self.pending[key] = self.model.logits(self.sequences[key], token)

    def decode_batch(self, keys):
        result = []
        for key in keys:
            logits = self.pending[key]
            if not np.isfinite(logits).all():
                raise ValueError("Nonfinite model logits")
            token = int(logits.argmax())
            result.append(token)
            self.pending[key] = self.model.logits(self.sequences[key], token)
        return result


def test_scheduler_backend_batches_like_serial_reference(tmp_path, ref_capi):
    # the batched backend against the reference's serial loop: the same
    # greedy tokens and pending logits within the bar, including a key listed
    # twice in one iteration and a key dropped midway
    from tvara_amd.scheduler import NativeSchedulerBackend

    spec = gf.LlamaSpec(matrix_type=gf.T_Q8_0, hidden=128, intermediate=256, heads=8, kv_heads=2, vocab=64)
    path = spec.write(tmp_path / "m.gguf")
    mine = NativeSchedulerBackend(native.NativeModel(path, max_blocks=256, block_tokens=4))
    ref = _SerialBackend(native.NativeModel(path, library=ref_capi, max_blocks=256, block_tokens=4))
    keys = [f"r{i}" for i in range(9)]
    rng = np.random.default_rng(5)
    for k in keys:
        prompt = [int(t) for t in rng.integers(0, spec.vocab, int(rng.integers(1, 6)))]
        for b in (mine, ref):
            b.create(k)
            b.prefill(k, prompt)
    for step in range(5):
        batch = keys + ([keys[2]] if step == 1 else [])
        # greedy choices can only differ where two logits tie within the bar
        margins = [np.sort(ref.pending[k])[-2:] for k in batch]
        got, want = mine.decode_batch(batch), ref.decode_batch(batch)
        for k, g, w, m in zip(batch, got, want, margins):
            assert g == w or abs(m[1] - m[0]) < 1e-3, (step, k, g, w)
        if got != want:
            pytest.skip("a greedy choice tied within the bar; the sequences diverge from here")
        for k in keys:
            ok, err = close(mine.pending[k], ref.pending[k])
            assert ok, (step, k, err)
        if step == 2:
            mine.drop(keys[0])
            ref.model._drop_sequence(ref.sequences.pop(keys[0]))
            keys = keys[1:]
    bad = keys[3]
    for b in (mine, ref):
        b.pending[bad] = np.full(spec.vocab, np.nan, np.float32)
    cache = mine.model.cache()
    before = {k: cache.length(mine.sequences[k]) for k in keys}
    for b in (mine, ref):
        with pytest.raises(ValueError, match="Nonfinite model logits"):
            b.decode_batch(keys)
    # the keys before the bad one were decoded, the rest were not
    after = {k: cache.length(mine.sequences[k]) for k in keys}
    assert [after[k] - before[k] for k in keys] == [1, 1, 1] + [0] * (len(keys) - 3)
    for k in keys[:3]:
        ok, err = close(mine.pending[k], ref.pending[k])
        assert ok, (k, err)
