"""Synthetic workloads of the paged KV path, shared by the parity tests and
bench.py.  Inputs come from tvara_amd.synth (counter-based splitmix64), so a
test can rebuild exactly the bench's data on any backend that has the
PagedCache method surface.

decode_c1  1 sequence, SmolLM2-135M attention: 9 q / 3 kv heads, d=64, 512
           cached tokens in 16-token blocks at a seeded permutation of ids.
decode_c2  64 sequences, Llama-3.2-1B attention: 32 q / 8 kv heads, d=64,
           contexts uniform in [128, 4096], blocks scattered over a
           65,536-block pool.
kv_c3      KV-management stress: 256 sequences share a 1,024-token prefix
           (22 layers x 8 kv heads x 64), 128 steps of one appended token per
           sequence, then a seeded 0-64 token rollback per sequence; the
           unaligned-prefix variant (1,025 tokens) makes step 1 copy-on-write.
prefill_c4 8 sequences x (2,048 cached + 512-token causal chunk), 32/8 heads, d=64.
decode_c5  16 sequences x 32,768 tokens, Llama-3-8B attention: 32/8 heads,
           d=128, Q8_0 blocks.
conversations  the reference's seeded multi-turn conversation traces replayed
           through a model, with and without prefix reuse.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import numpy as np

from . import synth


@dataclass
class DecodeWorkload:
    name: str
    heads: int
    kv_heads: int
    head_dim: int
    lengths: list
    pool_blocks: int
    seed: int
    tokens_per_block: int = 16
    layers: int = 1
    q8: bool = False
    context: int = 1 << 20
    meta: dict = field(default_factory=dict)

    @property
    def kv_width(self):
        return self.kv_heads * self.head_dim

    @property
    def sequences(self):
        return len(self.lengths)

    @property
    def total_tokens(self):
        return int(sum(self.lengths))

    def kv_bytes(self):
        """Algorithmic K+V bytes one decode launch reads."""
        per_element = 34 / 32 if self.q8 else 4
        return int(self.total_tokens * self.kv_width * 2 * per_element)

    def qo_bytes(self):
        return self.sequences * self.heads * self.head_dim * 4 * 2

    def table_bytes(self):
        return sum((n + self.tokens_per_block - 1) // self.tokens_per_block for n in self.lengths) * 4

    def keys(self, i):
        n = self.lengths[i]
        return synth.normal(self.seed, f"k{i}", n * self.kv_width).reshape(n, self.kv_width)

    def values(self, i):
        n = self.lengths[i]
        return synth.normal(self.seed, f"v{i}", n * self.kv_width).reshape(n, self.kv_width)

    def queries(self):
        return synth.normal(self.seed, "q", self.sequences * self.heads * self.head_dim).reshape(
            self.sequences, self.heads * self.head_dim)

    def placement(self):
        return synth.permutation(self.seed, "blocks", self.pool_blocks)


def decode_c1():
    return DecodeWorkload("smollm2-135m-decode-1x512", 9, 3, 64, [512], 64, seed=1, context=2048)


def decode_c2(sequences=64):
    lengths = synth.integers(2, "ctx", 64, 128, 4096)[:sequences].tolist()
    return DecodeWorkload("llama-3.2-1b-decode-64x[128,4096]", 32, 8, 64, lengths, 65536, seed=2, context=8192)


def decode_c5(sequences=16, length=32768):
    blocks = sequences * length // 16
    return DecodeWorkload("llama-3-8b-q8_0-decode-16x32768", 32, 8, 128, [length] * sequences, blocks + 64, seed=5,
                          q8=True, context=1 << 17)


def decode_gqa8(q8=False, sequences=16, length=4096):
    """Llama-3-70B's attention shape (64 query heads over 8 KV heads, d=128):
    eight query heads per KV head."""
    blocks = sequences * length // 16
    name = "llama-3-70b-attn-decode-16x4096" + ("-q8_0" if q8 else "")
    return DecodeWorkload(name, 64, 8, 128, [length] * sequences, blocks + 64, seed=6, q8=q8, context=1 << 17)


def decode_gqa16(q8=False, sequences=16, length=4096):
    """Llama-3.1-405B's attention shape (128 query heads over 8 KV heads,
    d=128): sixteen query heads per KV head, run as two slices of eight."""
    blocks = sequences * length // 16
    name = "llama-3.1-405b-attn-decode-16x4096" + ("-q8_0" if q8 else "")
    return DecodeWorkload(name, 128, 8, 128, [length] * sequences, blocks + 64, seed=9, q8=q8, context=1 << 17)


def decode_gemma2(sequences=16, length=4096):
    """Gemma-2-9B's attention shape (16 query heads over 8 KV heads, d=256):
    a token's 256 columns take a 16-lane row."""
    blocks = sequences * length // 16
    return DecodeWorkload("gemma-2-9b-attn-decode-16x4096", 16, 8, 256, [length] * sequences, blocks + 64, seed=10,
                          context=1 << 17)


def decode_phi3(sequences=16, length=4096):
    """Phi-3-mini's attention shape (32 query and 32 KV heads, d=96)."""
    blocks = sequences * length // 16
    return DecodeWorkload("phi-3-mini-attn-decode-16x4096", 32, 32, 96, [length] * sequences, blocks + 64, seed=11,
                          context=1 << 17)


def decode_tinyllama(q8=False, sequences=64, length=2048):
    """TinyLlama-1.1B's attention shape (32 query heads over 4 KV heads, d=64):
    eight query heads per KV head at head_dim 64."""
    blocks = sequences * length // 16
    name = "tinyllama-1.1b-attn-decode-64x2048" + ("-q8_0" if q8 else "")
    return DecodeWorkload(name, 32, 4, 64, [length] * sequences, blocks + 64, seed=7, q8=q8, context=1 << 17)


def decode_t176():
    """The reference's T176 cache case (tests/core/prefill_t176.cpp): one
    sequence of 1,025 tokens, 4 query heads over 2 KV heads, head_dim 32,
    16-token blocks, a 128-block cache."""
    return DecodeWorkload("t176-decode-1x1025-d32", 4, 2, 32, [1025], 128, seed=8, context=2048)


def place_blocks(cache, order):
    """Make the pool hand out block ids in `order`: allocate every block, then
    release them in reverse (the LIFO free list pops the last release first)."""
    handles = {}
    for _ in range(cache.max_blocks):
        h = cache.allocate()
        handles[h[0]] = h
    for i in reversed(list(order)):
        cache.release(handles[int(i)])


def fill_decode(cache, w: DecodeWorkload, progress=None):
    """Create one sequence per length and append its K/V; returns the ids."""
    place_blocks(cache, w.placement())
    seqs = []
    for i in range(w.sequences):
        s = cache.create_sequence()
        cache.append_many(s, w.keys(i), w.values(i))
        seqs.append(s)
        if progress:
            progress(i)
    return seqs


# ------------------------------------------------------------------- prefill

@dataclass
class PrefillWorkload:
    """Chunked prefill: each sequence holds `prefix` cached tokens plus a
    `chunk`-token causal chunk whose K/V are appended first; chunk row i sees
    positions 0 .. prefix+i."""
    name: str
    sequences: int = 8
    prefix: int = 2048
    chunk: int = 512
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 64
    tokens_per_block: int = 16
    seed: int = 4
    context: int = 8192
    q8: bool = False  # Q8_0 blocks

    @property
    def kv_width(self):
        return self.kv_heads * self.head_dim

    @property
    def total(self):
        return self.prefix + self.chunk

    def pool_blocks(self):
        return self.sequences * ((self.total + self.tokens_per_block - 1) // self.tokens_per_block) + 8

    def keys(self, i):
        return synth.normal(self.seed, f"k{i}", self.total * self.kv_width).reshape(self.total, self.kv_width)

    def values(self, i):
        return synth.normal(self.seed, f"v{i}", self.total * self.kv_width).reshape(self.total, self.kv_width)

    def chunk_queries(self, i):
        n = self.chunk * self.heads * self.head_dim
        return synth.normal(self.seed, f"q{i}", n).reshape(self.chunk, self.heads * self.head_dim)

    def flops(self):
        """QK^T and PV multiply-adds over the causal chunk, 2 flops each."""
        pairs = self.chunk * self.prefix + self.chunk * (self.chunk + 1) // 2
        return 4 * self.head_dim * pairs * self.heads * self.sequences

    def bytes(self):
        qo = 2 * self.sequences * self.chunk * self.heads * self.head_dim * 4
        return qo + int(self.sequences * self.total * self.kv_width * 2 * (34 / 32 if self.q8 else 4))


def prefill_c4(**kw):
    return PrefillWorkload("llama-3.2-1b-chunked-prefill-8x(2048+512)", **kw)


def prefill_c4_q8(**kw):
    """The Llama-3.2-1B chunks over Q8_0 blocks."""
    return PrefillWorkload("llama-3.2-1b-chunked-prefill-8x(2048+512)-q8_0", q8=True, **kw)


def prefill_8b(**kw):
    """The same chunks at Llama-3-8B's attention shape (32/8 heads, d=128)."""
    return PrefillWorkload("llama-3-8b-chunked-prefill-8x(2048+512)", head_dim=128, **kw)


def fill_prefill(cache, w: PrefillWorkload):
    seqs = []
    for i in range(w.sequences):
        s = cache.create_sequence()
        cache.append_many(s, w.keys(i), w.values(i))
        seqs.append(s)
    return seqs


# ------------------------------------------------------------------- KV stress

@dataclass
class KVStress:
    name: str
    sequences: int = 256
    prefix: int = 1024
    steps: int = 128
    max_rollback: int = 64
    layers: int = 22
    kv_heads: int = 8
    head_dim: int = 64
    tokens_per_block: int = 16
    seed: int = 3

    @property
    def width(self):
        return self.layers * self.kv_heads * self.head_dim

    def max_blocks(self):
        tpb = self.tokens_per_block
        prefix_blocks = (self.prefix + tpb - 1) // tpb
        own = (self.prefix + self.steps + tpb - 1) // tpb - self.prefix // tpb
        return prefix_blocks + self.sequences * own + 8

    def tokens(self, tag, n):
        """n rows of `width` floats in [1, 2) (bit patterns from the stream)."""
        bits = synth.bits(self.seed, tag, (n * self.width + 1) // 2)
        words = np.empty(2 * bits.size, np.uint32)
        words[0::2] = (bits & np.uint64(0xFFFFFFFF)).astype(np.uint32)
        words[1::2] = (bits >> np.uint64(32)).astype(np.uint32)
        words = (words[: n * self.width] >> np.uint32(9)) | np.uint32(0x3F800000)
        return words.view(np.float32).reshape(n, self.width)

    def rollback(self):
        return synth.integers(self.seed, "rollback", self.sequences, 0, self.max_rollback).tolist()


def kv_c3(unaligned=False, **kw):
    if unaligned:
        kw.setdefault("prefix", 1025)
    return KVStress("kv-stress-256x(1024+128)-22l" + ("-cow" if unaligned else ""), **kw)


def run_kv_stress(cache, w: KVStress, on_phase=None):
    """The stress on one cache; on_phase(name, seqs) is called after each phase."""
    src = cache.create_sequence()
    k = w.tokens("prefix-k", w.prefix)
    v = w.tokens("prefix-v", w.prefix)
    cache.append_many(src, k, v)
    seqs = [cache.fork(src) for _ in range(w.sequences)]
    cache.drop(src)
    if on_phase:
        on_phase("fork", seqs)
    for step in range(w.steps):
        k = w.tokens(f"step{step}-k", w.sequences)
        v = w.tokens(f"step{step}-v", w.sequences)
        cache.append_batch(seqs, k, v)
        if on_phase:
            on_phase(f"step{step}", seqs)
    for s, r in zip(seqs, w.rollback()):
        cache.truncate(s, cache.length(s) - r)
    if on_phase:
        on_phase("rollback", seqs)
    return seqs


# ------------------------------------------------------------ conversations

def conversation_traces(seed=262, conversations=4, turns=5, vocab=32000):
    """The reference's conversation traces (tools/run_prefix_cache_traces.py:22-33,
    defaults :93-98): a 64-token system prompt shared by every conversation,
    then `turns` user turns of 16-48 random token ids.  The ids come from the
    same numpy generator calls in the same order, so the traces are the
    reference's own."""
    rng = np.random.default_rng(seed)
    system = rng.integers(1, vocab, 64).tolist()
    traces = []
    for _ in range(conversations):
        users = []
        for _ in range(turns):
            length = int(rng.integers(16, 49))
            users.append(rng.integers(1, vocab, length).tolist())
        traces.append({"system": system, "users": users})
    return traces


def replay_conversations(model, traces, mode, reply_tokens=12, tree=None, clock=None):
    """Replays the traces through `model` (a tvara_amd.native.NativeModel) as
    run_trace does (tools/run_prefix_cache_traces.py:53-91): per turn the
    prompt (the history plus the user turn) is prefilled and reply_tokens
    greedy tokens follow, all but the last fed back.  Modes:

    off    every turn prefills its whole prompt in a fresh sequence;
    on     a conversation keeps its live sequence between turns, so only the
           new suffix is prefilled (the reference's cache-on mode);
    radix  as on, and a conversation's first turn restores the shared system
           prompt from `tree` (a tvara_amd.radix.RadixCache over the model's
           cache), the first conversation inserting it.

    Prefills go through NativeModel.prefill (one chunked pass per 512 tokens
    on this library).  Returns per trace the list of turns: prompt and
    reused token counts, prefill seconds, the prompt's last logits and the
    reply."""
    clock = clock or time.perf_counter
    if mode not in ("off", "on", "radix") or (mode == "radix" and tree is None):
        raise ValueError("mode is off, on or radix (with a tree)")
    results = []
    for trace in traces:
        system = list(trace["system"])
        history, turns, sequence, fed = list(system), [], None, []
        try:
            for user in trace["users"]:
                history += user
                seconds = 0.0
                if mode != "off" and sequence is not None and history[: len(fed)] == fed:
                    suffix, reused = history[len(fed):], len(fed)
                else:
                    if sequence is not None:
                        model.drop_sequence(sequence)
                    sequence, fed, reused = None, [], 0
                    if mode == "radix":
                        start = clock()
                        node, matched = tree.lookup(system)
                        if matched == len(system) and tree.node(node)["kv_length"] is not None:
                            sequence, reused = tree.reuse(system)
                            fed = system[:reused]
                        else:
                            sequence = model.new_sequence()
                            model.prefill(sequence, system)
                            tree.attach(tree.insert(system), sequence)
                            fed = list(system)
                        seconds += clock() - start
                    else:
                        sequence = model.new_sequence()
                    suffix = history[len(fed):]
                start = clock()
                logits = model.prefill(sequence, suffix)
                seconds += clock() - start
                fed += suffix
                reply = []
                for index in range(reply_tokens):
                    token = int(np.asarray(logits if index == 0 else step).argmax())
                    reply.append(token)
                    if index + 1 < reply_tokens:
                        step = model.logits(sequence, token)
                fed += reply[:-1]
                history += reply
                turns.append({"prompt_tokens": len(history) - len(reply), "reused_tokens": reused,
                              "prefill_seconds": seconds, "logits": logits, "reply": reply})
                if mode == "off":
                    model.drop_sequence(sequence)
                    sequence, fed = None, []
        finally:
            if sequence is not None:
                model.drop_sequence(sequence)
        results.append(turns)
    return results
