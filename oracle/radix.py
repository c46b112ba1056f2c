"""RadixCache restated in Python over an oracle cache: TEST INFRASTRUCTURE
ONLY (imported by tests/), the oracle for tvara_amd.radix.

Follows core/include/tvara/radix.hpp: constructor :19-22, lookup :29-42,
insert :44-69 (a split node takes the split child's pins), attach :72-81,
external_references :83-87, reuse :90-96, pin/unpin :99-100, touch :103,
eviction_candidate :106-110 (least recently touched unpinned leaf, lowest id
among equals), evict_one :113-116, reset :119-122 (node ids keep counting;
the clock restarts).  Works over any object with the PagedCache surface of
oracle.pyoracle.Cache (sequence tables, retain/release, import_sequence).
Errors carry the reference's messages; ``nodes_.at`` failures raise
LookupError the way std::out_of_range reaches a logic_error handler.

Pinned against the reference's own class (oracle/_ref, tests/test_oracle_vs_ref.py)
on test_radix.cpp's checks and on random operation sequences.
"""

from __future__ import annotations

U64_MAX = (1 << 64) - 1


class RadixError(Exception):
    pass


class _Node:
    __slots__ = ("id", "parent", "edge", "children", "kv", "pins", "accessed")

    def __init__(self, id=0, parent=0, edge=()):
        self.id, self.parent, self.edge = id, parent, list(edge)
        self.children = {}
        self.kv = None  # (length, [block handles])
        self.pins = 0
        self.accessed = 0


class Radix:
    def __init__(self, cache, isolation, errors):
        """errors: (InvalidArgument, LogicError, OverflowError-like) classes."""
        self.cache = cache
        self.invalid, self.logic, self.overflow = errors
        if not isolation:
            raise self.invalid("prefix isolation key is required")
        self.isolation = isolation
        self.nodes = {0: _Node()}
        self.next = 0
        self.clock = 0

    def _at(self, i):
        if i not in self.nodes:
            raise self.logic("map::at")
        return self.nodes[i]

    def size(self):
        return len(self.nodes) - 1

    def _common(self, edge, tokens, offset):
        k = 0
        while k < len(edge) and offset + k < len(tokens) and edge[k] == tokens[offset + k]:
            k += 1
        return k

    def lookup(self, tokens):
        tokens = [int(t) for t in tokens]
        current, offset, result = 0, 0, (0, 0)
        while offset < len(tokens):
            child_id = self.nodes[current].children.get(tokens[offset])
            if child_id is None:
                break
            child = self.nodes[child_id]
            k = self._common(child.edge, tokens, offset)
            offset += k
            result = (child.id, offset)
            if k != len(child.edge):
                break
            current = child.id
        return result

    def insert(self, tokens):
        tokens = [int(t) for t in tokens]
        if not tokens:
            raise self.invalid("cannot cache empty prefix")
        current, offset = 0, 0
        while offset < len(tokens):
            parent = self.nodes[current]
            found = parent.children.get(tokens[offset])
            if found is None:
                if self.next == U64_MAX:
                    raise self.overflow("radix ID exhausted")
                self.next += 1
                self.nodes[self.next] = _Node(self.next, current, tokens[offset:])
                parent.children[tokens[offset]] = self.next
                return self.next
            child = self.nodes[found]
            k = self._common(child.edge, tokens, offset)
            if k != len(child.edge):
                if self.next == U64_MAX:
                    raise self.overflow("radix ID exhausted")
                self.next += 1
                middle = _Node(self.next, current, child.edge[:k])
                middle.pins = child.pins
                child.edge = child.edge[k:]
                middle.children[child.edge[0]] = child.id
                child.parent = middle.id
                parent.children[tokens[offset]] = middle.id
                self.nodes[middle.id] = middle
                current, offset = middle.id, offset + k
                continue
            current, offset = child.id, offset + k
        return current

    def _release(self, node):
        if node.kv is not None:
            for b in node.kv[1]:
                self.cache.release(b)

    def attach(self, node_id, sequence):
        entry = self._at(node_id)
        length, blocks = self.cache.length(sequence), self.cache.blocks(sequence)
        depth, c = 0, node_id
        while c:
            depth += len(self._at(c).edge)
            c = self._at(c).parent
        if length != depth:
            raise self.invalid("token and KV prefix lengths differ")
        retained = 0
        try:
            for b in blocks:
                self.cache.retain(b)
                retained += 1
        except Exception:
            for b in blocks[:retained]:
                self.cache.release(b)
            raise
        self._release(entry)
        entry.kv = (length, list(blocks))

    def external_references(self):
        counts = [0] * self.cache.max_blocks
        for n in self.nodes.values():
            if n.kv is not None:
                for b in n.kv[1]:
                    counts[b[0]] += 1
        return counts

    def reuse(self, tokens, partial=False):
        node, matched = self.lookup(tokens)
        if not node or self.nodes[node].kv is None:
            return self.cache.create_sequence(), 0
        length = matched if partial else matched - matched % self.cache.tokens_per_block
        kv_length, blocks = self.nodes[node].kv
        return self.cache.import_sequence(blocks, kv_length, length), length

    def _path(self, node_id):
        out, c = [], node_id
        while c:
            out.append(self._at(c))
            c = out[-1].parent
        return out

    def pin(self, node_id):
        path = self._path(node_id)
        if any(n.pins == U64_MAX for n in path):
            raise self.overflow("prefix pin overflow")
        for n in path:
            n.pins += 1

    def unpin(self, node_id):
        path = self._path(node_id)
        if any(n.pins == 0 for n in path):
            raise self.invalid("prefix pin underflow")
        for n in path:
            n.pins -= 1

    def touch(self, node_id):
        entry = self._at(node_id)
        if self.clock == U64_MAX:
            raise self.overflow("prefix access clock exhausted")
        self.clock += 1
        entry.accessed = self.clock

    def eviction_candidate(self):
        best = None
        for i in sorted(self.nodes):
            n = self.nodes[i]
            if i and not n.children and not n.pins and (best is None or n.accessed < self.nodes[best].accessed):
                best = i
        return best

    def evict_one(self):
        c = self.eviction_candidate()
        if c is None:
            return False
        entry = self.nodes[c]
        self._release(entry)
        del self.nodes[entry.parent].children[entry.edge[0]]
        del self.nodes[c]
        return True

    def reset(self):
        if any(i and n.pins for i, n in self.nodes.items()):
            raise self.logic("cannot reset pinned prefix nodes")
        for n in self.nodes.values():
            self._release(n)
        self.nodes = {0: _Node()}
        self.clock = 0

    def node(self, node_id):
        n = self._at(node_id)
        return {"id": node_id, "parent": n.parent, "edge": list(n.edge), "pins": n.pins, "accessed": n.accessed,
                "kv_length": n.kv[0] if n.kv is not None else None,
                "kv_blocks": len(n.kv[1]) if n.kv is not None else None, "children": len(n.children)}
