"""KV block management on the GPU, bit-exact against the oracle: the
reference's known-answer checks, random operation sequences compared state by
state, and the 256-sequence shared-prefix stress with and without
copy-on-write."""

import sys

import numpy as np
import pytest

import kv_cases
from tvara_amd import workloads

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


@pytest.mark.parametrize("case", kv_cases.CASES, ids=lambda f: f.__name__)
def test_known_answers_on_device(device, case):
    say("kv case", case.__name__)
    case(lambda *g: device.PagedCache(*g), (device.InvalidArgument, device.CacheExhausted))


@pytest.mark.parametrize("geometry,seed", [((2, 2, 4, 4, 12), 1), ((1, 1, 2, 3, 9), 2), ((3, 1, 4, 5, 20), 3),
                                           ((1, 8, 64, 16, 10), 4), ((2, 2, 64, 16, 8), 5)])
def test_random_ops_match_oracle(device, oracle, geometry, seed):
    say("random ops", geometry, seed)
    layers, kv_heads, dim, tpb, _ = geometry
    kv_cases.random_ops(oracle.Cache(*geometry), device.PagedCache(*geometry), 250, seed, layers * kv_heads * dim, tpb)


def test_batch_append_matches_sequential(device, oracle):
    # one batched call equals the loop of PagedCache::append, including shared
    # tails (copy-on-write), fresh blocks and a repeated sequence
    g = (2, 2, 8, 4, 64)
    a, b = oracle.Cache(*g), device.PagedCache(*g)
    w = 2 * 16
    rng = np.random.default_rng(0)
    for c in (a, b):
        s = c.create_sequence()
        c.append_many(s, np.ones((6, w)), np.ones((6, w)))
        for _ in range(3):
            c.fork(s)
    seqs = [1, 2, 3, 4, 2, 2, 3]
    for _ in range(5):
        k = rng.standard_normal((len(seqs), w)).astype(np.float32)
        v = rng.standard_normal((len(seqs), w)).astype(np.float32)
        a.append_batch(seqs, k, v)
        b.append_batch(seqs, k, v)
        assert a.state() == b.state()
    for s in a.sequence_ids():
        for h in a.blocks(s):
            assert np.array_equal(a.block_data(h), b.block_data(h))


def test_batch_append_op_count_limits(device, oracle):
    # batches of 400 appends pass their block ops in the kernel arguments, 401
    # upload them; with one token per block every append also starts a block
    g = (2, 2, 8, 1, 1700)
    a, b = oracle.Cache(*g), device.PagedCache(*g)
    w = 2 * 16
    rng = np.random.default_rng(7)
    for c in (a, b):
        for _ in range(3):
            c.create_sequence()
    for n in (400, 401, 399, 401):
        say("batch of", n)
        seqs = [1 + i % 3 for i in range(n)]
        k = rng.standard_normal((n, w)).astype(np.float32)
        v = rng.standard_normal((n, w)).astype(np.float32)
        a.append_batch(seqs, k, v)
        b.append_batch(seqs, k, v)
        assert a.state() == b.state()
    for s in a.sequence_ids():
        for layer in (0, 1):
            assert np.array_equal(a.read_all(s, layer), b.read_all(s, layer))
            assert np.array_equal(a.read_all(s, layer, True), b.read_all(s, layer, True))


def test_batch_exhaustion_applies_prefix(device, oracle):
    # a batch that runs out of blocks keeps the appends before the failure, as
    # a loop over PagedCache::append would, and the failed one changes nothing
    g = (1, 1, 4, 2, 3)
    a, b = oracle.Cache(*g), device.PagedCache(*g)
    for c in (a, b):
        s = c.create_sequence()
        t = c.create_sequence()
        c.append(s, np.ones(4), np.ones(4))
        c.append(t, np.ones(4), np.ones(4))
    k = np.arange(5 * 4, dtype=np.float32).reshape(5, 4)
    seqs = [1, 2, 1, 2, 1]
    applied = 0
    with pytest.raises(oracle.CacheExhausted):
        for i in range(5):
            a.append(seqs[i], k[i], k[i])
            applied += 1
    with pytest.raises(device.CacheExhausted):
        b.append_batch(seqs, k, k)
    assert b.last_applied == applied == 3
    assert a.state() == b.state()
    for s in (1, 2):
        assert np.array_equal(a.read_all(s, 0), b.read_all(s, 0))
        assert np.array_equal(a.read_all(s, 0, True), b.read_all(s, 0, True))


@pytest.mark.parametrize("unaligned", [False, True], ids=["aligned-1024", "cow-1025"])
def test_kv_stress_bit_exact(device, oracle, unaligned):
    w = workloads.kv_c3(unaligned=unaligned)
    say("kv stress", w.name)
    g = (w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.max_blocks())
    a, b = oracle.Cache(*g), device.PagedCache(*g)
    states = {}

    def record(cache, key):
        def phase(name, seqs):
            if name in ("fork", "step0", "step1", "step15", "step16", "step127", "rollback"):
                states.setdefault(name, []).append(cache.state())
        return phase

    workloads.run_kv_stress(a, w, record(a, "oracle"))
    seqs = workloads.run_kv_stress(b, w, record(b, "device"))
    for name, pair in states.items():
        assert pair[0] == pair[1], name
    # every live block's bytes: device checksums against the oracle's
    handles = sorted({h for s in seqs for h in b.blocks(s)})
    got = b.checksums(handles)
    want = [oracle.checksum_words(a.block_data(h)) for h in handles]
    assert got == want
    # a direct byte comparison of a sample, including a copied-on-write tail
    for h in handles[:: max(1, len(handles) // 16)]:
        assert np.array_equal(a.block_data(h), b.block_data(h))
    if unaligned:
        # step 0 copies the shared one-token tail for every sequence but the last
        # to append, which finds it at refcount 1 and writes in place (kv.hpp:97)
        tails = {t[1][w.prefix // 16] for t in states["step0"][1]["tables"].values()}
        shared = {t[1][w.prefix // 16] for t in states["fork"][1]["tables"].values()}
        assert len(shared) == 1 and len(tails) == w.sequences and len(tails & shared) == 1


def test_q8_append_matches_encoder(device, oracle):
    # quantise-on-append produces the encoder's exact bytes (fixture.py:131-137)
    from tvara_amd import synth

    g = (2, 2, 64, 16, 8)
    c = device.PagedCache(*g, fmt=device.Q8_0)
    s = c.create_sequence()
    n, w = 21, 2 * 2 * 64
    k = synth.normal(8, "k", n * w).reshape(n, w)
    v = synth.normal(8, "v", n * w).reshape(n, w)
    k[3, :32] = 0.0  # an all-zero group
    c.append_many(s, k, v)
    f = oracle.Cache(*g)
    fs = f.create_sequence()
    f.append_many(fs, k, v)
    for blk_index, h in enumerate(c.blocks(s)):
        want = oracle.quantize_q8_0(f.block_data(f.blocks(fs)[blk_index]))
        got = c.block_data(h)
        live = min(16, n - 16 * blk_index)
        # compare the written slots group by group (unwritten slots are zero in both)
        elems = np.zeros(f.elements_per_block, bool)
        for layer in range(2):
            for kind in range(2):
                for slot in range(live):
                    o = f.kv_offset(layer, kind, slot)
                    elems[o : o + 128] = True
        groups = elems.reshape(-1, 32).all(axis=1)
        assert np.array_equal(got.reshape(-1, 34)[groups], want.reshape(-1, 34)[groups])
        assert not got.reshape(-1, 34)[~groups].any()
    # reading back dequantises exactly like dequantize_q8_0 (quant.hpp:40-49)
    got = c.read_all(s, 1, True)
    want = oracle.dequantize_q8_0(oracle.quantize_q8_0(v[:, 128:]))
    assert np.array_equal(got, want)
