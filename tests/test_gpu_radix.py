"""Prefix cache (RadixCache, core/include/tvara/radix.hpp) over the device KV
pool: the known-answer checks of tests/core/test_radix.cpp, random operation
sequences compared node by node and pool state by pool state with the oracle's
restatement (oracle/radix.py) and, where built, the reference's own class,
and the model fixture of test_radix.cpp through the model exports: decoding
after a reused prefix gives logits bit-identical to a cold decode of the
whole prompt."""

import sys

import numpy as np
import pytest

import radix_cases
from tvara_amd import gguf_writer as gf
from tvara_amd import native
from tvara_amd.radix import RadixCache

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def _oracle_tree(oracle):
    from oracle.radix import Radix

    return lambda cache, iso: Radix(cache, iso, (oracle.InvalidArgument, oracle.LogicError, oracle.OracleError))


def test_known_answers_on_device(device):
    say("radix known answers")
    radix_cases.known_answers(device.PagedCache(1, 1, 1, 4, 64), RadixCache)


@pytest.mark.parametrize("geometry,seed,alphabet", [((1, 1, 2, 4, 24), 1, 3), ((2, 1, 2, 3, 40), 2, 4),
                                                    ((1, 2, 2, 2, 16), 3, 2), ((2, 2, 64, 16, 48), 5, 5)])
def test_random_ops_match_oracle(device, oracle, geometry, seed, alphabet):
    say("radix random ops", geometry, seed)
    layers, kv_heads, dim, _, _ = geometry
    dc, oc = device.PagedCache(*geometry), oracle.Cache(*geometry)
    pairs = [(oc, _oracle_tree(oracle)(oc, "model/tokenizer/tenant")), (dc, RadixCache(dc, "model/tokenizer/tenant"))]
    if oracle.ref_available():
        rc = oracle.RefCache(*geometry)
        pairs.append((rc, oracle.RefRadix(rc, "model/tokenizer/tenant")))
    assert radix_cases.random_ops(pairs, 300, seed, layers * kv_heads * dim, alphabet) > 10


def test_isolation_and_lifetime(device):
    # trees over one pool are independent; destroying a tree releases every
    # retained block (radix.hpp:82)
    cache = device.PagedCache(1, 1, 4, 4, 16)
    a, b = RadixCache(cache, "tenant-a"), RadixCache(cache, "tenant-b")
    s = cache.create_sequence()
    cache.append_many(s, np.ones((5, 4)), np.ones((5, 4)))
    a.attach(a.insert([1, 2, 3, 4, 5]), s)
    assert b.lookup([1, 2, 3, 4, 5]) == (0, 0)
    assert sum(a.external_references()) == 2
    cache.drop(s)
    assert cache.available() == 14
    a.close()
    assert cache.available() == 16
    cache.audit(b.external_references())


def test_model_prefix_reuse_is_bit_exact(tmp_path):
    # test_radix.cpp's model fixture: a 3-token stem decoded once, attached,
    # then reused for six requests; each cached decode equals, bit for bit,
    # the cold decode of the prompt through the same calls (the stem as one
    # decode_batch, then the tail), and the whole prompt as one chunked
    # decode_batch within the logit bar
    spec = gf.LlamaSpec(layers=2)
    m = native.NativeModel(spec.write(tmp_path / "m.gguf"), max_blocks=32, block_tokens=4)
    cache = m.cache()
    tree = RadixCache(cache, "model-fixture/tenant-a")
    stem = [1, 2, 3]
    source = m.new_sequence()
    m.decode_batch(source, stem)
    tree.attach(tree.insert(stem), source)
    for tail in range(4, 10):
        say("prefix reuse tail", tail)
        restored, length = tree.reuse(stem + [tail], True)
        assert length == 3 and cache.length(restored) == 3
        cached = m.logits(restored, tail)
        cold_seq = m.new_sequence()
        m.decode_batch(cold_seq, stem)
        cold = m.logits(cold_seq, tail)
        assert np.array_equal(cached.view(np.uint32), cold.view(np.uint32)), tail
        whole_seq = m.new_sequence()
        whole = m.decode_batch(whole_seq, stem + [tail])[-1]
        assert np.all(np.abs(whole - cold) <= 1e-4 * (1 + np.abs(cold))), tail
        m.drop_sequence(whole_seq)
        for layer in range(spec.layers):
            for value in (False, True):
                assert np.array_equal(cache.read_all(restored, layer, value), cache.read_all(cold_seq, layer, value))
        m.drop_sequence(cold_seq)
        cache.drop(restored)
    m.drop_sequence(source)
    cache.audit(tree.external_references())
    tree.reset()
    cache.audit()
    tree.close()
    cache.close()
    m.close()
