"""Python surface of the MI355X paged KV cache (libtvara_capi.so).

``PagedCache`` mirrors the reference's PagedCache and BlockPool
(core/include/tvara/kv.hpp:36-165) method for method; block bytes live in HBM
and every operation that touches them runs a gfx950 kernel.  Handles are
``(id, generation)`` tuples (BlockHandle, kv.hpp:35).  Errors raise
``InvalidArgument`` (std::invalid_argument), ``CacheExhausted``
(tvara::CacheExhausted) or ``LogicError`` (std::logic_error).

Attention over the cache (attention.hpp:57-89) is in ``tvara_amd.attention``.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _capi
from ._capi import CacheExhausted, Handle, InvalidArgument, LogicError, NativeError  # noqa: F401

F32 = _capi.KV_F32
Q8_0 = _capi.KV_Q8_0

_fp = C.POINTER(C.c_float)
_u64p = C.POINTER(C.c_uint64)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return a.ctypes.data_as(_fp) if a is not None else None


class PagedCache:
    """PagedCache(CacheGeometry{layers, kv_heads, head_dim, tokens_per_block,
    max_blocks}) (kv.hpp:80) on one GPU; ``fmt`` selects f32 or Q8_0 blocks."""

    def __init__(self, layers, kv_heads, head_dim, tokens_per_block, max_blocks, fmt=F32, lib=None):
        self.lib = lib or _capi.lib()
        self.geometry = (layers, kv_heads, head_dim, tokens_per_block, max_blocks)
        self.layers, self.kv_heads, self.head_dim, self.tokens_per_block, self.max_blocks = self.geometry
        self.format = fmt
        self.kv_width = kv_heads * head_dim
        self.h = self.lib.tvara_kv_cache_create(layers, kv_heads, head_dim, tokens_per_block, max_blocks, fmt)
        if not self.h:
            _capi.raise_last(self.lib)
        self.block_bytes = self.lib.tvara_kv_block_bytes(self.h)

    @classmethod
    def lent(cls, handle, layers, kv_heads, head_dim, tokens_per_block, max_blocks, owner=None, fmt=F32):
        """Wrap a cache handle another object owns (tvara_model_cache); closing
        it does not destroy the cache.  `owner` is kept alive with it."""
        self = cls.__new__(cls)
        self.lib = _capi.lib()
        self.geometry = (layers, kv_heads, head_dim, tokens_per_block, max_blocks)
        self.layers, self.kv_heads, self.head_dim, self.tokens_per_block, self.max_blocks = self.geometry
        self.format = fmt
        self.kv_width = kv_heads * head_dim
        self.h = handle
        self._owner = owner
        self.block_bytes = self.lib.tvara_kv_block_bytes(self.h)
        return self

    def close(self):
        if getattr(self, "h", None):
            if getattr(self, "_owner", None) is None:
                self.lib.tvara_kv_cache_destroy(self.h)
            self.h = None
            self._owner = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *args):
        self.close()

    def _check(self, rc):
        _capi.check(rc, self.lib)

    @property
    def elements_per_block(self):
        return self.layers * 2 * self.tokens_per_block * self.kv_width

    def kv_offset(self, layer, kind, slot):
        """kv_offset (kv.hpp:30-33)."""
        if layer >= self.layers or kind > 1 or slot >= self.tokens_per_block:
            raise InvalidArgument("KV position outside block")
        return ((layer * 2 + kind) * self.tokens_per_block + slot) * self.kv_width

    def synchronize(self):
        self._check(self.lib.tvara_kv_synchronize(self.h))

    def set_stream(self, stream):
        self._check(self.lib.tvara_kv_set_stream(self.h, stream))

    # ----------------------------------------------------------- BlockPool
    def allocate(self):
        h = Handle()
        self._check(self.lib.tvara_kv_pool_allocate(self.h, C.byref(h)))
        return (h.id, h.generation)

    def retain(self, handle):
        self._check(self.lib.tvara_kv_pool_retain(self.h, Handle(*handle)))

    def release(self, handle):
        self._check(self.lib.tvara_kv_pool_release(self.h, Handle(*handle)))

    free = release

    def references(self, handle):
        out = C.c_size_t()
        self._check(self.lib.tvara_kv_pool_references(self.h, Handle(*handle), C.byref(out)))
        return out.value

    def references_by_id(self, i):
        out = C.c_size_t()
        self._check(self.lib.tvara_kv_pool_references_by_id(self.h, i, C.byref(out)))
        return out.value

    def available(self):
        return self.lib.tvara_kv_pool_available(self.h)

    def pool_audit(self):
        self._check(self.lib.tvara_kv_pool_audit(self.h))

    def block_bytes_of(self, handle):
        """The block's canonical bytes (BlockPool::data, kv.hpp:52-53)."""
        out = np.empty(self.block_bytes, np.uint8)
        self._check(self.lib.tvara_kv_block_read(self.h, Handle(*handle), out.ctypes.data, out.size))
        return out

    def block_data(self, handle):
        """f32 blocks: the block's floats; Q8_0 blocks: its 34-byte groups."""
        raw = self.block_bytes_of(handle)
        return raw.view(np.float32).copy() if self.format == F32 else raw

    def block_write(self, handle, offset, values):
        """Write f32 values at element ``offset`` (f32 blocks) or raw bytes at
        byte ``offset`` (Q8_0 blocks)."""
        if self.format == F32:
            v = _f32(values).reshape(-1)
            self._check(self.lib.tvara_kv_block_write(self.h, Handle(*handle), offset * 4, v.ctypes.data, v.nbytes))
        else:
            v = np.ascontiguousarray(values, dtype=np.uint8).reshape(-1)
            self._check(self.lib.tvara_kv_block_write(self.h, Handle(*handle), offset, v.ctypes.data, v.nbytes))

    def checksums(self, handles):
        n = len(handles)
        arr = (Handle * max(1, n))(*[Handle(*h) for h in handles])
        out = np.zeros(max(1, n), np.uint64)
        self._check(self.lib.tvara_kv_block_checksums(self.h, arr, n, out.ctypes.data_as(C.POINTER(C.c_uint64))))
        return [int(x) for x in out[:n]]

    # ---------------------------------------------------------- PagedCache
    def create_sequence(self):
        s = self.lib.tvara_kv_sequence_create(self.h)
        if not s:
            _capi.raise_last(self.lib)
        return s

    def _sequence(self, seq):
        length, count = C.c_size_t(), C.c_size_t()
        self._check(self.lib.tvara_kv_sequence(self.h, seq, C.byref(length), None, 0, C.byref(count)))
        arr = (Handle * max(1, count.value))()
        self._check(self.lib.tvara_kv_sequence(self.h, seq, C.byref(length), arr, count.value, C.byref(count)))
        return length.value, [(arr[i].id, arr[i].generation) for i in range(count.value)]

    def sequence(self, seq):
        """PagedCache::sequence (kv.hpp:82-84): (length, block handles)."""
        return self._sequence(seq)

    def length(self, seq):
        return self._sequence(seq)[0]

    def blocks(self, seq):
        return self._sequence(seq)[1]

    def sequence_ids(self):
        count = C.c_size_t()
        self._check(self.lib.tvara_kv_sequence_ids(self.h, None, 0, C.byref(count)))
        arr = np.zeros(max(1, count.value), np.uint64)
        self._check(self.lib.tvara_kv_sequence_ids(self.h, arr.ctypes.data_as(C.POINTER(C.c_uint64)), count.value,
                                                   C.byref(count)))
        return [int(x) for x in arr[: count.value]]

    def physical_block(self, seq, position):
        h = Handle()
        self._check(self.lib.tvara_kv_physical_block(self.h, seq, position, C.byref(h)))
        return (h.id, h.generation)

    def append(self, seq, keys, values):
        """PagedCache::append (kv.hpp:91-108)."""
        k, v = _f32(keys).reshape(-1), _f32(values).reshape(-1)
        if k.size != self.layers * self.kv_width or v.size != k.size:
            raise InvalidArgument("invalid paged KV append dimensions")
        self._check(self.lib.tvara_kv_append(self.h, seq, _ptr(k), _ptr(v)))

    def append_batch(self, seqs, keys, values):
        """One append per listed sequence, in order; returns the number applied
        when all succeed, raises (after applying the prefix) otherwise."""
        seqs = np.ascontiguousarray(seqs, dtype=np.uint64)
        w = self.layers * self.kv_width
        k = _f32(keys).reshape(-1, w)
        v = _f32(values).reshape(-1, w)
        if k.shape[0] != seqs.size or v.shape != k.shape:
            raise InvalidArgument("invalid paged KV append dimensions")
        applied = C.c_size_t()
        rc = self.lib.tvara_kv_append_batch(self.h, seqs.ctypes.data_as(C.POINTER(C.c_uint64)), seqs.size, _ptr(k),
                                            _ptr(v), 0, C.byref(applied))
        self.last_applied = applied.value
        self._check(rc)
        return applied.value

    def append_batch_device(self, seqs, keys_ptr, values_ptr):
        """As append_batch with K/V already in HBM ([n][layers*kv_width] f32).
        A scheduler that keeps its batch as a contiguous uint64 array saves the
        per-call list conversion (about 10 us for 256 sequences), and the call
        reuses that array's address while it passes the same array: the
        binding's own work is then about a microsecond of the step."""
        fast = self.__dict__.get("_append_dev")
        if fast is None:
            # the same export bound with plain addresses: no pointer casts or
            # fresh ctypes objects per call
            fast = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p, C.c_int,
                               C.c_void_p)(("tvara_kv_append_batch", self.lib))
            self._append_dev = fast
            self._applied = C.c_size_t()
            self._applied_at = C.addressof(self._applied)
            self._batch = (None, 0)
        if seqs is not self._batch[0]:
            if not (isinstance(seqs, np.ndarray) and seqs.dtype == np.uint64 and seqs.flags.c_contiguous):
                seqs = np.ascontiguousarray(seqs, dtype=np.uint64)
            self._batch = (seqs, seqs.ctypes.data)
        rc = fast(self.h, self._batch[1], seqs.size, keys_ptr, values_ptr, 1, self._applied_at)
        self.last_applied = self._applied.value
        if rc:
            self._check(rc)
        return self.last_applied

    def append_many(self, seq, keys, values):
        """len(keys) consecutive appends to one sequence."""
        w = self.layers * self.kv_width
        k = _f32(keys).reshape(-1, w)
        v = _f32(values).reshape(-1, w)
        if v.shape != k.shape:
            raise InvalidArgument("invalid paged KV append dimensions")
        applied = C.c_size_t()
        rc = self.lib.tvara_kv_append_tokens(self.h, seq, _ptr(k), _ptr(v), k.shape[0], 0, C.byref(applied))
        self.last_applied = applied.value
        self._check(rc)
        return applied.value

    def read(self, seq, layer, position, value=False):
        out = np.empty(self.kv_width, np.float32)
        self._check(self.lib.tvara_kv_read(self.h, seq, layer, position, int(value), _ptr(out)))
        return out

    def read_all(self, seq, layer, value=False):
        n = self.length(seq)
        out = np.empty(max(1, n * self.kv_width), np.float32)
        self._check(self.lib.tvara_kv_read_all(self.h, seq, layer, int(value), _ptr(out), out.size))
        return out[: n * self.kv_width]

    def drop(self, seq):
        self._check(self.lib.tvara_kv_drop(self.h, seq))

    def fork(self, seq):
        s = self.lib.tvara_kv_fork(self.h, seq)
        if not s:
            _capi.raise_last(self.lib)
        return s

    def truncate(self, seq, length):
        self._check(self.lib.tvara_kv_truncate(self.h, seq, length))

    def truncate_batch(self, seqs, lengths):
        """truncate(seqs[i], lengths[i]) for every i, in order, in one call;
        raises (after applying the prefix) at the first failure."""
        if not (isinstance(seqs, np.ndarray) and seqs.dtype == np.uint64 and seqs.flags.c_contiguous):
            seqs = np.ascontiguousarray(seqs, dtype=np.uint64)
        lengths = np.ascontiguousarray(lengths, dtype=np.uintp)
        if lengths.shape != seqs.shape:
            raise InvalidArgument("sequences and lengths differ in length")
        applied = C.c_size_t()
        rc = self.lib.tvara_kv_truncate_batch(self.h, C.cast(seqs.ctypes.data, _u64p),
                                              lengths.ctypes.data_as(C.POINTER(C.c_size_t)), seqs.size,
                                              C.byref(applied))
        self.last_applied = applied.value
        self._check(rc)
        return applied.value

    def audit(self, external=None):
        if external is None:
            self._check(self.lib.tvara_kv_audit(self.h, None, 0))
        else:
            ext = np.ascontiguousarray(external, dtype=np.uint64)
            self._check(self.lib.tvara_kv_audit(self.h, ext.ctypes.data_as(C.POINTER(C.c_size_t)), ext.size))

    def import_sequence(self, blocks, source_length, length):
        arr = (Handle * max(1, len(blocks)))(*[Handle(*b) for b in blocks])
        s = self.lib.tvara_kv_import_sequence(self.h, arr, len(blocks), source_length, length)
        if not s:
            _capi.raise_last(self.lib)
        return s

    def state(self):
        """Exact allocator and table state, in the oracle's format."""
        n = self.max_blocks
        refs = np.zeros(n, np.uint64)
        gens = np.zeros(n, np.uint64)
        free = np.zeros(n, np.uint64)
        count = C.c_size_t()
        self._check(
            self.lib.tvara_kv_pool_state(self.h, refs.ctypes.data_as(C.POINTER(C.c_size_t)),
                                         gens.ctypes.data_as(C.POINTER(C.c_uint64)),
                                         free.ctypes.data_as(C.POINTER(C.c_size_t)), C.byref(count))
        )
        tables = {s: self._sequence(s) for s in self.sequence_ids()}
        return {"refs": refs.tolist(), "generations": gens.tolist(), "free": free[: count.value].tolist(),
                "tables": tables}

    # ------------------------------------------------------------ attention
    def fused_paged_attention(self, q, seq, layer, heads, context, tail_key=None, tail_value=None, visible=None):
        from .attention import fused_paged_attention

        return fused_paged_attention(q, self, seq, layer, heads, context, tail_key, tail_value, visible)

    def fused_prompt_attention(self, queries, seq, layer, start, count, heads, context, precision="f32"):
        from .attention import fused_prompt_attention

        return fused_prompt_attention(queries, self, seq, layer, start, count, heads, context, precision)
