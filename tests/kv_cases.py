"""Known-answer checks of the paged KV cache, restated from the reference's
tests/core/test_kv.cpp:7-46 and the KV contract of tests/core/test_radix.cpp:8-21.

Each case takes ``make(layers, kv_heads, head_dim, tokens_per_block, max_blocks)``
returning a cache with the common Python surface (oracle.pyoracle.Cache,
oracle.pyoracle.RefCache or tvara_amd.kv.PagedCache) and the backend's
(InvalidArgument, CacheExhausted) exception classes, so the oracle, the
reference and the GPU library all run the same checks.
"""

import numpy as np


def rejects(errors, fn):
    invalid = errors[0]
    try:
        fn()
    except invalid:
        return True
    raise AssertionError("expected invalid_argument")


def geometry(make, errors):  # test_kv.cpp:7-8
    c = make(2, 2, 4, 4, 8)
    assert c.elements_per_block == 128 and c.kv_offset(1, 1, 3) == 120
    rejects(errors, lambda: make(2, 2, (1 << 64) - 1, 4, 8))


def allocator(make, errors):  # test_kv.cpp:9-10
    c = make(1, 1, 4, 4, 2)
    first = c.allocate()
    c.block_write(first, 0, [9.0])
    c.release(first)
    rejects(errors, lambda: c.block_data(first))
    second = c.allocate()
    assert second[0] == first[0] and second[1] != first[1] and c.block_data(second)[0] == 0
    c.release(second)
    assert c.available() == 2


def tables(make, errors):  # test_kv.cpp:12
    c = make(1, 1, 4, 4, 4)
    a, b = c.create_sequence(), c.create_sequence()
    assert a != b and c.length(a) == 0
    rejects(errors, lambda: c.physical_block(a, 0))


def append(make, errors):  # test_kv.cpp:14-16
    c = make(2, 1, 4, 2, 4)
    s = c.create_sequence()
    keys, values = np.full(8, 2, np.float32), np.full(8, 3, np.float32)
    for _ in range(3):
        c.append(s, keys, values)
    assert c.length(s) == 3 and len(c.blocks(s)) == 2 and c.available() == 2
    block = c.block_data(c.physical_block(s, 2))
    assert block[c.kv_offset(1, 1, 0)] == 3


def reads(make, errors):  # test_kv.cpp:18-19
    c = make(1, 1, 2, 2, 4)
    s = c.create_sequence()
    keys, values = np.array([1, 2], np.float32), np.array([3, 4], np.float32)
    for i in range(3):
        keys[0] = i
        c.append(s, keys, values)
    assert c.read(s, 0, 2)[0] == 2
    assert c.read_all(s, 0, True).tolist() == [3, 4, 3, 4, 3, 4]
    rejects(errors, lambda: c.read(s, 0, 3))


def refs(make, errors):  # test_kv.cpp:21
    c = make(1, 1, 2, 2, 2)
    block = c.allocate()
    c.retain(block)
    assert c.references(block) == 2
    c.release(block)
    assert c.available() == 1
    c.release(block)
    assert c.available() == 2
    rejects(errors, lambda: c.release(block))


def completion(make, errors):  # test_kv.cpp:23
    c = make(1, 1, 2, 2, 3)
    s = c.create_sequence()
    x = np.ones(2, np.float32)
    for _ in range(3):
        c.append(s, x, x)
    assert c.available() == 1
    c.drop(s)
    assert c.available() == 3
    rejects(errors, lambda: c.length(s))


def sharing(make, errors):  # test_kv.cpp:25-26
    c = make(1, 1, 2, 2, 3)
    s = c.create_sequence()
    x = np.ones(2, np.float32)
    c.append(s, x, x)
    branch = c.fork(s)
    assert c.references(c.physical_block(s, 0)) == 2 and c.read(branch, 0, 0).tolist() == x.tolist()
    c.drop(s)
    assert c.read(branch, 0, 0).tolist() == x.tolist()
    c.drop(branch)
    assert c.available() == 3


def copy_on_write(make, errors):  # test_kv.cpp:28-30
    c = make(1, 1, 2, 4, 4)
    source = c.create_sequence()
    x = np.ones(2, np.float32)
    c.append(source, x, x)
    branch = c.fork(source)
    x[0] = 9
    c.append(branch, x, x)
    x[0] = 5
    c.append(source, x, x)
    assert c.read(branch, 0, 1)[0] == 9 and c.read(source, 0, 1)[0] == 5
    assert c.physical_block(source, 0)[0] != c.physical_block(branch, 0)[0]
    c.drop(source)
    c.drop(branch)
    assert c.available() == 4


def tail_boundaries(make, errors):  # test_kv.cpp:32-35
    c = make(1, 1, 2, 2, 5)
    source = c.create_sequence()
    x = np.ones(2, np.float32)
    c.append(source, x, x)
    c.append(source, x, x)
    branch = c.fork(source)
    shared = c.physical_block(source, 0)
    x[0] = 7
    c.append(branch, x, x)
    assert c.references(shared) == 2 and len(c.blocks(branch)) == 2 and c.length(source) == 2
    c.drop(branch)
    c.drop(source)
    assert c.available() == 5


def rollback(make, errors):  # test_kv.cpp:37-39
    c = make(1, 1, 2, 2, 5)
    s = c.create_sequence()
    x = np.ones(2, np.float32)
    for _ in range(5):
        c.append(s, x, x)
    c.truncate(s, 3)
    assert len(c.blocks(s)) == 2 and c.available() == 3
    x[0] = 9
    c.append(s, x, x)
    assert c.read(s, 0, 3)[0] == 9
    c.truncate(s, 0)
    assert c.available() == 5
    c.drop(s)


def exhaustion(make, errors):  # test_kv.cpp:41-43
    c = make(1, 1, 2, 2, 1)
    s = c.create_sequence()
    x = np.ones(2, np.float32)
    c.append(s, x, x)
    branch = c.fork(s)
    try:
        c.append(branch, x, x)
        raise AssertionError("expected CacheExhausted")
    except errors[1]:
        pass
    assert c.length(branch) == 1 and c.references(c.physical_block(s, 0)) == 2
    c.drop(branch)
    c.append(s, x, x)
    assert c.length(s) == 2
    c.drop(s)
    assert c.available() == 1


def invariants(make, errors):  # test_kv.cpp:45-46
    c = make(1, 1, 2, 3, 8)
    s = c.create_sequence()
    x = np.ones(2, np.float32)
    for _ in range(7):
        c.append(s, x, x)
        c.audit()
    branch = c.fork(s)
    c.audit()
    c.append(branch, x, x)
    c.audit()
    c.truncate(branch, 2)
    c.audit()
    c.drop(branch)
    c.audit()
    c.drop(s)
    c.audit()


def radix_contract(make, errors):
    """The KV side of RadixCache (radix.hpp:72-96) as test_radix.cpp:8-21
    exercises it: a snapshot retains a sequence's blocks (attach), reuse imports
    a block-aligned or partial prefix, appending to a partial shared tail copies
    it, and audits count the snapshot's references as external."""
    c = make(1, 1, 1, 4, 64)
    seq = c.create_sequence()
    for i in range(6):
        f = np.array([i], np.float32)
        c.append(seq, f, f)
    snapshot = (c.length(seq), c.blocks(seq))
    for h in snapshot[1]:
        c.retain(h)  # attach (radix.hpp:77)
    external = np.zeros(64, np.uint64)
    for h in snapshot[1]:
        external[h[0]] += 1
    c.audit(external)
    full = c.import_sequence(snapshot[1], snapshot[0], 4)  # reuse, block-aligned (radix.hpp:94)
    assert c.length(full) == 4 and c.physical_block(full, 0)[0] == c.physical_block(seq, 0)[0]
    c.drop(full)
    partial = c.import_sequence(snapshot[1], snapshot[0], 6)  # reuse(partial=true)
    old = c.physical_block(seq, 5)
    nine = np.array([9], np.float32)
    c.append(partial, nine, nine)
    assert c.physical_block(partial, 5)[0] != old[0]  # copy-on-write of the partial tail
    assert c.read(seq, 0, 5)[0] == 5 and c.read(partial, 0, 6)[0] == 9
    c.drop(partial)
    c.audit(external)
    rejects(errors, lambda: c.import_sequence(snapshot[1], snapshot[0], 7))
    # churn (test_radix.cpp:21): snapshot, restore, read, drop, with audits
    snaps = []
    for rnd in range(60):
        s = c.create_sequence()
        for i in range(3):
            f = np.array([i + rnd], np.float32)
            c.append(s, f, f)
        blocks = c.blocks(s)
        for h in blocks:
            c.retain(h)
            external[h[0]] += 1
        snaps.append(blocks)
        restored = c.import_sequence(blocks, 3, 3)
        assert c.read(restored, 0, 2)[0] == 2 + rnd
        c.drop(restored)
        c.drop(s)
        c.audit(external)
        while len(snaps) > 12:  # evict the oldest snapshot (radix.hpp:113-116)
            for h in snaps.pop(0):
                c.release(h)
                external[h[0]] -= 1
        c.audit(external)
    for blocks in snaps:
        for h in blocks:
            c.release(h)
            external[h[0]] -= 1
    for h in snapshot[1]:
        c.release(h)
        external[h[0]] -= 1
    c.drop(seq)
    c.audit()
    assert c.available() == 64


CASES = [geometry, allocator, tables, append, reads, refs, completion, sharing, copy_on_write, tail_boundaries,
         rollback, exhaustion, invariants, radix_contract]


def random_ops(a, b, steps, seed, width, tokens_per_block=None):
    """Drive two caches through the same random operation sequence (appends,
    forks, truncations, drops, prefix imports, pool allocate/release) and
    compare their complete state -- tables, reference counts, generations and
    free-list order -- after every step, and every live block's bytes at the
    end.  Exceptions are compared by class name."""
    rng = np.random.default_rng(seed)
    seqs = []
    for step in range(steps):
        op = int(rng.integers(0, 10))
        s = seqs[int(rng.integers(len(seqs)))] if seqs else None
        k = rng.standard_normal(width).astype(np.float32)
        v = rng.standard_normal(width).astype(np.float32)
        t = int(rng.integers(0, 3 * (tokens_per_block or 4) + 1))
        results = []
        for cache in (a, b):
            try:
                if op == 0 or s is None:
                    r = ("create", cache.create_sequence())
                elif op in (1, 2, 3, 4):
                    cache.append(s, k, v)
                    r = ("append",)
                elif op == 5:
                    r = ("fork", cache.fork(s))
                elif op == 6:
                    cache.truncate(s, max(0, cache.length(s) - t))
                    r = ("truncate",)
                elif op == 7 and len(seqs) > 1:
                    cache.drop(s)
                    r = ("drop",)
                elif op == 8:
                    n = cache.length(s)
                    r = ("import", cache.import_sequence(cache.blocks(s), n, min(n, t)))
                else:
                    h = cache.allocate()
                    zero = not np.any(cache.block_data(h))
                    cache.release(h)
                    r = ("pool", h, zero)
            except Exception as e:  # noqa: BLE001 - the exception classes are compared
                r = ("error", type(e).__name__)
            results.append(r)
        assert results[0] == results[1], (step, op, results)
        r = results[0]
        if r[0] in ("create", "fork", "import"):
            seqs.append(r[1])
        elif r[0] == "drop":
            seqs.remove(s)
        sa, sb = a.state(), b.state()
        assert sa == sb, (step, op)
    for s in seqs:
        for h in a.blocks(s):
            assert np.array_equal(np.asarray(a.block_data(h)).view(np.uint8), np.asarray(b.block_data(h)).view(np.uint8)), (s, h)
    return len(seqs)
