"""RadixCache over the paged KV pool (core/include/tvara/radix.hpp:17-131),
through libtvara_capi's tvara_radix_* exports: the prefix tree lives in the
library (host metadata), its KV snapshots are retained blocks of the device
pool, and reuse imports a matched prefix as a new sequence sharing them.

Method names, arguments and errors follow the reference class; a node is
returned by ``node(id)`` as a dict.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _capi

_sz = C.c_size_t
_u64 = C.c_uint64


def _tokens(tokens):
    t = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
    return t, t.ctypes.data_as(C.POINTER(C.c_int32))


class RadixCache:
    def __init__(self, cache, isolation):
        """cache: a tvara_amd.kv.PagedCache (or one lent by a model)."""
        self.cache = cache
        self.lib = cache.lib
        self.h = self.lib.tvara_radix_create(cache.h, isolation.encode("utf-8"))
        if not self.h:
            _capi.raise_last(self.lib)
        self.isolation = isolation

    def close(self):
        if getattr(self, "h", None):
            self.lib.tvara_radix_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def _check(self, rc):
        _capi.check(rc, self.lib)

    def size(self):
        n = _sz()
        self._check(self.lib.tvara_radix_size(self.h, C.byref(n)))
        return n.value

    def lookup(self, tokens):
        """(node, tokens matched) (radix.hpp:29-42)."""
        t, p = _tokens(tokens)
        node, matched = _u64(), _sz()
        self._check(self.lib.tvara_radix_lookup(self.h, p, t.size, C.byref(node), C.byref(matched)))
        return node.value, matched.value

    def insert(self, tokens):
        t, p = _tokens(tokens)
        node = _u64()
        self._check(self.lib.tvara_radix_insert(self.h, p, t.size, C.byref(node)))
        return node.value

    def attach(self, node, sequence):
        self._check(self.lib.tvara_radix_attach(self.h, node, sequence))

    def reuse(self, tokens, partial=False):
        """(new sequence, prefix length) (radix.hpp:90-96)."""
        t, p = _tokens(tokens)
        seq, length = _u64(), _sz()
        self._check(self.lib.tvara_radix_reuse(self.h, p, t.size, int(partial), C.byref(seq), C.byref(length)))
        return seq.value, length.value

    def pin(self, node):
        self._check(self.lib.tvara_radix_pin(self.h, node))

    def unpin(self, node):
        self._check(self.lib.tvara_radix_unpin(self.h, node))

    def touch(self, node):
        self._check(self.lib.tvara_radix_touch(self.h, node))

    def eviction_candidate(self):
        node = _u64()
        self._check(self.lib.tvara_radix_eviction_candidate(self.h, C.byref(node)))
        return node.value or None

    def evict_one(self):
        e = C.c_int()
        self._check(self.lib.tvara_radix_evict_one(self.h, C.byref(e)))
        return bool(e.value)

    def reset(self):
        self._check(self.lib.tvara_radix_reset(self.h))

    def node(self, node_id):
        parent, elen, pins, acc, kvlen, kvb, ch = _u64(), _sz(), _sz(), _u64(), _sz(), _sz(), _sz()
        self._check(self.lib.tvara_radix_node(self.h, node_id, C.byref(parent), None, 0, C.byref(elen), C.byref(pins),
                                              C.byref(acc), C.byref(kvlen), C.byref(kvb), C.byref(ch)))
        edge = np.zeros(max(1, elen.value), np.int32)
        self._check(self.lib.tvara_radix_node(self.h, node_id, C.byref(parent), edge.ctypes.data_as(C.POINTER(C.c_int32)),
                                              elen.value, C.byref(elen), C.byref(pins), C.byref(acc), C.byref(kvlen),
                                              C.byref(kvb), C.byref(ch)))
        has_kv = kvb.value != (1 << 64) - 1
        return {"id": node_id, "parent": parent.value, "edge": [int(x) for x in edge[: elen.value]],
                "pins": pins.value, "accessed": acc.value, "kv_length": kvlen.value if has_kv else None,
                "kv_blocks": kvb.value if has_kv else None, "children": ch.value}

    def external_references(self):
        counts = np.zeros(self.cache.max_blocks, np.uint64)
        self._check(self.lib.tvara_radix_external_references(self.h, counts.ctypes.data_as(C.POINTER(_sz)),
                                                             counts.size))
        return [int(x) for x in counts]
