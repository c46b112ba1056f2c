"""Prefix-cache checks shared by the oracle, reference and device tests.

``known_answers`` restates the checks of tests/core/test_radix.cpp (all but
the model fixture, which tests/test_gpu_radix.py covers through the model
exports) over any cache/tree pair with the PagedCache and RadixCache surface;
``random_ops`` drives several pairs through one random operation sequence
and compares every result, error, node and the complete pool state."""

import numpy as np


def category(e):
    """Exception class family and message, comparable across back ends."""
    for name in ("InvalidArgument", "CacheExhausted", "LogicError"):
        if any(c.__name__ == name for c in type(e).__mro__):
            return (name, str(e))
    return ("error", str(e))


def _expect(errors, family, f, *a):
    try:
        f(*a)
    except Exception as e:  # noqa: BLE001 - the family is checked
        assert category(e)[0] == family, (family, e)
        return
    raise AssertionError(f"expected {family}")


def known_answers(cache, make_tree):
    """cache: geometry (1, 1, 1, 4, 64); make_tree(cache, isolation)."""
    one = lambda x: np.array([x], np.float32)  # noqa: E731
    tree = make_tree(cache, "fixture-model/tokenizer/tenant-a")
    assert tree.size() == 0 and tree.node(0)["edge"] == []
    assert tree.lookup([1, 2])[1] == 0
    prompt = [1, 2, 3, 4, 5, 6]
    a = tree.insert(prompt)
    assert tree.insert(prompt) == a and tree.lookup(prompt)[1] == 6
    b = tree.insert([1, 2, 7])
    assert b != a and tree.lookup([1, 2, 8])[1] == 2 and tree.insert([1, 2]) != a
    seq = cache.create_sequence()
    for i in range(6):
        cache.append(seq, one(i), one(i))
    tree.attach(a, seq)
    cache.audit(tree.external_references())

    full = tree.reuse(prompt)
    assert full[1] == 4 and cache.physical_block(full[0], 0)[0] == cache.physical_block(seq, 0)[0]
    cache.drop(full[0])
    partial = tree.reuse(prompt, True)
    assert partial[1] == 6
    old = cache.physical_block(seq, 5)
    cache.append(partial[0], one(9), one(9))
    assert cache.physical_block(partial[0], 5)[0] != old[0]  # copy-on-write of the shared tail
    assert cache.read(seq, 0, 5)[0] == 5
    cache.drop(partial[0])
    cache.audit(tree.external_references())

    tree.pin(a)
    assert tree.node(a)["pins"] == 1
    shorter = tree.insert([1])
    assert tree.node(shorter)["pins"] == 1
    tree.unpin(a)
    assert tree.node(shorter)["pins"] == 0
    _expect(None, "InvalidArgument", tree.unpin, a)
    tree.touch(a)
    tree.touch(b)
    assert tree.node(a)["accessed"] < tree.node(b)["accessed"]
    assert tree.eviction_candidate() == a
    tree.pin(a)
    assert tree.eviction_candidate() == b
    tree.unpin(a)
    tree.pin(b)
    assert tree.evict_one()
    assert tree.node(b)["edge"]
    tree.unpin(b)
    cache.audit(tree.external_references())

    c = tree.insert(prompt)
    tree.attach(c, seq)
    survivor = tree.reuse(prompt, True)
    tree.touch(b)
    assert tree.evict_one()
    assert cache.length(survivor[0]) == 6
    cache.append(survivor[0], one(9), one(9))
    assert cache.read(seq, 0, 5)[0] == 5
    cache.drop(survivor[0])
    cache.audit(tree.external_references())

    for r in range(200):
        path = [10, 11, r % 7]
        node = tree.insert(path)
        s = cache.create_sequence()
        for i in range(3):
            cache.append(s, one(i), one(i))
        tree.attach(node, s)
        restored = tree.reuse(path, True)
        assert restored[1] == 3 and cache.read(restored[0], 0, 2)[0] == 2
        cache.drop(restored[0])
        cache.drop(s)
        cache.audit(tree.external_references())
        while tree.size() > 12:
            assert tree.evict_one()
    cache.drop(seq)
    cache.audit(tree.external_references())

    protected = tree.insert([123])
    tree.pin(protected)
    _expect(None, "LogicError", tree.reset)
    tree.unpin(protected)
    isolated = make_tree(cache, "fixture-model/tokenizer/tenant-b")
    assert isolated.lookup(prompt)[1] == 0
    tree.reset()
    assert tree.size() == 0
    cache.audit(tree.external_references())
    _expect(None, "InvalidArgument", make_tree, cache, "")
    _expect(None, "InvalidArgument", tree.insert, [])
    return tree


def random_ops(pairs, steps, seed, width, alphabet=4):
    """pairs: [(cache, tree)], all of one geometry, fresh.  Every step applies
    one operation to each pair and compares results (errors by family and
    message), then every node, the retained counts and the pool state."""
    rng = np.random.default_rng(seed)
    seqs, nodes, paths = [], [0], []
    for step in range(steps):
        op = int(rng.integers(0, 13))
        n = int(rng.integers(0, 7))
        tokens = [int(x) for x in rng.integers(0, alphabet, n)]
        node = nodes[int(rng.integers(len(nodes)))] + (1 if rng.random() < 0.05 else 0)
        if paths and rng.random() < 0.6:
            # an inserted path, sometimes extended: attach then mostly
            # succeeds and reuse finds KV to share
            node, tokens = paths[int(rng.integers(len(paths)))]
            tokens = tokens + [int(x) for x in rng.integers(0, alphabet, int(rng.integers(0, 3)))]
            if op in (3, 4):
                tokens = tokens[: len(tokens) - int(rng.random() < 0.2)]
            n = len(tokens)
        s = seqs[int(rng.integers(len(seqs)))] if seqs else None
        k = rng.standard_normal((max(1, n), width)).astype(np.float32)
        partial = bool(rng.integers(0, 2))
        coin = rng.random() < 0.5
        results = []
        for cache, tree in pairs:
            try:
                if op in (0, 1):
                    r = ("insert", tree.insert(tokens))
                elif op == 2:
                    r = ("lookup", tree.lookup(tokens))
                elif op in (3, 4):
                    # a sequence holding len(tokens) positions, attached to
                    # the node (a length mismatch is an error)
                    q = cache.create_sequence()
                    for i in range(n):
                        cache.append(q, k[i], -k[i])
                    r = ("attach", q)
                    try:
                        tree.attach(node, q)
                    finally:
                        cache.drop(q)
                elif op in (5, 6):
                    r = ("reuse", tree.reuse(tokens, partial))
                elif op == 7:
                    r = ("pin", tree.pin(node))
                elif op == 8:
                    r = ("unpin", tree.unpin(node))
                elif op == 9:
                    r = ("touch", tree.touch(node))
                elif op == 10:
                    r = ("evict", tree.eviction_candidate(), tree.evict_one())
                elif op == 11 and s is not None and coin:
                    cache.append(s, k[0], k[0])
                    r = ("append",)
                elif op == 11 and s is not None:
                    cache.drop(s)
                    r = ("drop", s)
                else:
                    r = ("reset", tree.reset())
            except Exception as e:  # noqa: BLE001 - the family and message are compared
                r = ("error",) + category(e)
            results.append(r)
        assert all(x == results[0] for x in results), (step, op, results)
        r = results[0]
        if r[0] == "insert":
            nodes.append(r[1])
            paths.append((r[1], tokens))
        elif r[0] == "reuse":
            seqs.append(r[1][0])
        elif r[0] == "drop":
            seqs.remove(r[1])
        states = []
        for cache, tree in pairs:
            ids = sorted(set(nodes) | set(range(0, max(nodes) + 2)))
            dump = {}
            for i in ids:
                try:
                    dump[i] = tree.node(i)
                except Exception:  # noqa: BLE001 - absent nodes are compared as absent
                    dump[i] = None
            states.append((tree.size(), dump, tree.external_references(), cache.state()))
        for st in states[1:]:
            assert st == states[0], (step, op)
    for s in seqs:
        ref = [pairs[0][0].read_all(s, 0), pairs[0][0].read_all(s, 0, True)]
        for cache, _ in pairs[1:]:
            assert np.array_equal(ref[0], cache.read_all(s, 0)) and np.array_equal(ref[1], cache.read_all(s, 0, True))
    return len(nodes)
