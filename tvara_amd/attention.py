"""Paged attention over a device ``PagedCache`` (libtvara_capi.so).

* ``fused_paged_attention`` -- attention.hpp:57-83, one query row;
* ``decode_batch`` -- the same for many sequences in one launch;
* ``fused_prompt_attention`` / ``prefill_batch`` -- attention.hpp:85-89, a
  causal chunk over cached positions, in f32 (reference semantics) or on bf16
  MFMA tiles;
* ``DecodePlan`` -- resident block tables for repeated device launches.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _capi
from ._capi import InvalidArgument

_fp = C.POINTER(C.c_float)
_sz = C.c_size_t
_NO_CAP = (1 << 64) - 1
_PRECISION = {"f32": _capi.ATTN_F32, "bf16": _capi.ATTN_BF16, "f32x3": _capi.ATTN_F32X3}


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return a.ctypes.data_as(_fp) if a is not None else None


def decode_batch(cache, q, seqs, layer, heads, context, tail_keys=None, tail_values=None, visible=None):
    """fused_paged_attention for every listed sequence: q [n, heads*head_dim]."""
    seqs = np.ascontiguousarray(seqs, dtype=np.uint64).reshape(-1)
    n = seqs.size
    hidden = heads * cache.head_dim
    q = _f32(q).reshape(n, hidden) if n else _f32(q)
    tk = _f32(tail_keys).reshape(n, cache.kv_width) if tail_keys is not None else None
    tv = _f32(tail_values).reshape(n, cache.kv_width) if tail_values is not None else None
    vis = None
    if visible is not None:
        vis = np.ascontiguousarray(np.broadcast_to(np.asarray(visible, dtype=np.uint64), (n,)))
    out = np.empty((max(n, 1), hidden), np.float32)
    rc = cache.lib.tvara_attn_decode(cache.h, seqs.ctypes.data_as(C.POINTER(C.c_uint64)), n, layer, heads, context,
                                     _ptr(q), _ptr(tk), _ptr(tv),
                                     vis.ctypes.data_as(C.POINTER(_sz)) if vis is not None else None, _ptr(out), 0)
    _capi.check(rc)
    return out[:n]


def fused_paged_attention(q, cache, sequence, layer, heads, context, tail_key=None, tail_value=None, visible=None):
    """fused_paged_attention (attention.hpp:57-83): one row of heads*head_dim."""
    tk = None if tail_key is None else _f32(tail_key).reshape(1, -1)
    tv = None if tail_value is None else _f32(tail_value).reshape(1, -1)
    vis = None if visible is None else [visible]
    return decode_batch(cache, _f32(q).reshape(1, -1), [sequence], layer, heads, context, tk, tv, vis)[0]


def prefill_batch(cache, queries, seqs, starts, counts, layer, heads, context, precision="f32"):
    """fused_prompt_attention for several sequences; queries packed by sequence."""
    seqs = np.ascontiguousarray(seqs, dtype=np.uint64).reshape(-1)
    starts = np.ascontiguousarray(starts, dtype=np.uint64).reshape(-1)
    counts = np.ascontiguousarray(counts, dtype=np.uint64).reshape(-1)
    if precision not in _PRECISION:
        raise InvalidArgument("unknown attention precision")
    hidden = heads * cache.head_dim
    rows = int(counts.sum())
    q = _f32(queries).reshape(rows, hidden)
    out = np.empty((max(rows, 1), hidden), np.float32)
    rc = cache.lib.tvara_attn_prefill(cache.h, seqs.ctypes.data_as(C.POINTER(C.c_uint64)), seqs.size, layer, heads,
                                      context, starts.ctypes.data_as(C.POINTER(_sz)),
                                      counts.ctypes.data_as(C.POINTER(_sz)), _ptr(q), _ptr(out),
                                      _PRECISION[precision], 0)
    _capi.check(rc)
    return out[:rows]


def fused_prompt_attention(queries, cache, sequence, layer, start, count, heads, context, precision="f32"):
    """fused_prompt_attention (attention.hpp:85-89): rows start .. start+count-1."""
    return prefill_batch(cache, queries, [sequence], [start], [count], layer, heads, context, precision).reshape(-1)


def prefill_batch_device(cache, q_ptr, out_ptr, seqs, starts, counts, layer, heads, context, precision="bf16"):
    """prefill_batch over device buffers (synchronous)."""
    seqs = np.ascontiguousarray(seqs, dtype=np.uint64).reshape(-1)
    starts = np.ascontiguousarray(starts, dtype=np.uint64).reshape(-1)
    counts = np.ascontiguousarray(counts, dtype=np.uint64).reshape(-1)
    rc = cache.lib.tvara_attn_prefill(cache.h, seqs.ctypes.data_as(C.POINTER(C.c_uint64)), seqs.size, layer, heads,
                                      context, starts.ctypes.data_as(C.POINTER(_sz)),
                                      counts.ctypes.data_as(C.POINTER(_sz)), C.cast(q_ptr, _fp),
                                      C.cast(out_ptr, _fp), _PRECISION[precision], 1)
    _capi.check(rc)


class DecodePlan:
    """Resident block tables for one batch of sequences (tvara_attn_plan_*)."""

    def __init__(self, cache, seqs, heads, context, visible=None, with_tail=False):
        self.cache = cache
        self.lib = cache.lib
        seqs = np.ascontiguousarray(seqs, dtype=np.uint64).reshape(-1)
        vis = None
        if visible is not None:
            vis = np.ascontiguousarray(np.broadcast_to(np.asarray(visible, dtype=np.uint64), seqs.shape))
        self.h = self.lib.tvara_attn_plan_create(cache.h, seqs.ctypes.data_as(C.POINTER(C.c_uint64)), seqs.size, heads,
                                                 context, vis.ctypes.data_as(C.POINTER(_sz)) if vis is not None else None,
                                                 int(with_tail))
        if not self.h:
            _capi.raise_last()
        split, items, kv = _sz(), _sz(), _sz()
        _capi.check(self.lib.tvara_attn_plan_info(self.h, C.byref(split), C.byref(items), C.byref(kv)))
        self.split_tokens, self.items, self.kv_bytes = split.value, items.value, kv.value

    def launch(self, layer, q_ptr, out_ptr, tail_k_ptr=None, tail_v_ptr=None, stream=None):
        """Asynchronous launch over device pointers (ints)."""
        _capi.check(self.lib.tvara_attn_plan_decode(self.h, layer, q_ptr, tail_k_ptr, tail_v_ptr, out_ptr, stream))

    def check(self):
        _capi.check(self.lib.tvara_attn_plan_check(self.h))

    def close(self):
        if getattr(self, "h", None):
            self.lib.tvara_attn_plan_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


class PrefillPlan:
    """Resident block tables for one chunked-prefill batch (tvara_prefill_plan_*):
    sequence i attends its rows starts[i] .. starts[i] + counts[i] - 1."""

    def __init__(self, cache, seqs, starts, counts, heads, context, precision="bf16"):
        self.cache = cache
        self.lib = cache.lib
        seqs = np.ascontiguousarray(seqs, dtype=np.uint64).reshape(-1)
        starts = np.ascontiguousarray(starts, dtype=np.uint64).reshape(-1)
        counts = np.ascontiguousarray(counts, dtype=np.uint64).reshape(-1)
        if not (seqs.size == starts.size == counts.size):
            raise ValueError("seqs, starts and counts differ in length")
        self.rows = int(counts.sum())
        self.h = self.lib.tvara_prefill_plan_create(cache.h, seqs.ctypes.data_as(C.POINTER(C.c_uint64)), seqs.size,
                                                    heads, context, starts.ctypes.data_as(C.POINTER(_sz)),
                                                    counts.ctypes.data_as(C.POINTER(_sz)), _PRECISION[precision])
        if not self.h:
            _capi.raise_last()

    def launch(self, layer, q_ptr, out_ptr, stream=None):
        """Asynchronous launch over device pointers (ints)."""
        _capi.check(self.lib.tvara_prefill_plan_launch(self.h, layer, q_ptr, out_ptr, stream))

    def check(self):
        _capi.check(self.lib.tvara_prefill_plan_check(self.h))

    def close(self):
        if getattr(self, "h", None):
            self.lib.tvara_prefill_plan_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


def profile_enable(on=True):
    _capi.check(_capi.lib().tvara_profile_enable(int(on)))


def profile_reset():
    _capi.check(_capi.lib().tvara_profile_reset())


def profile_read(kernel=None):
    ms, n = C.c_double(), _sz()
    _capi.check(_capi.lib().tvara_profile_read(kernel.encode() if kernel else None, C.byref(ms), C.byref(n)))
    return ms.value, n.value
