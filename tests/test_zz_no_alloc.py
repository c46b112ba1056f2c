"""tvara_attn_decode_noalloc, the decode entry point that allocates nothing,
against tvara_attn_decode on device buffers (device_ptrs = 1).  Both build
the same plan and run the same kernels, so the outputs must be bit-identical;
the first call is the full 64-sequence Llama-3.2-1B batch with tails, the
second a smaller batch (5 rows, no tails, a visible cap) that reuses the
scratch the first one left behind.  A batch whose plan exceeds the scratch is
refused before anything runs."""

import ctypes as C
import sys

import numpy as np
import pytest

from tvara_amd import _capi, attention, hip, synth, workloads

pytestmark = pytest.mark.gpu
_u64p = C.POINTER(C.c_uint64)
_szp = C.POINTER(C.c_size_t)
_fp = C.POINTER(C.c_float)


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def _decode(lib, fn, cache, seqs, heads, context, q, tk, tv, visible, out):
    seqs = np.ascontiguousarray(seqs, dtype=np.uint64)
    vis = None if visible is None else np.ascontiguousarray(visible, dtype=np.uint64)
    ptr = (lambda p: C.cast(p, _fp)) if fn == "tvara_attn_decode" else (lambda p: p)  # float* argtypes there
    args = [cache.h, seqs.ctypes.data_as(_u64p), seqs.size, 0, heads, context, ptr(q.ptr),
            ptr(tk.ptr) if tk is not None else None, ptr(tv.ptr) if tv is not None else None,
            vis.ctypes.data_as(_szp) if vis is not None else None, ptr(out.ptr)]
    if fn == "tvara_attn_decode":
        args.append(1)
    return getattr(lib, fn)(*args)


def _both(cache, seqs, heads, context, q, tk=None, tv=None, visible=None):
    lib = cache.lib
    n = len(seqs)
    dq = hip.DeviceArray.from_numpy(q)
    dtk = hip.DeviceArray.from_numpy(tk) if tk is not None else None
    dtv = hip.DeviceArray.from_numpy(tv) if tv is not None else None
    outs = []
    for fn in ("tvara_attn_decode", "tvara_attn_decode_noalloc"):
        out = hip.DeviceArray((n, q.shape[1]))
        out.zero()
        _capi.check(_decode(lib, fn, cache, seqs, heads, context, dq, dtk, dtv, visible, out))
        outs.append(out.numpy())
    return outs


def test_noalloc_matches_decode_twice(device):
    w = workloads.decode_c2()
    say("no-alloc decode", w.name)
    g = (w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks)
    cache = device.PagedCache(*g)
    seqs = workloads.fill_decode(cache, w)
    q = w.queries()
    kvw = w.kv_heads * w.head_dim
    tk = synth.normal(7, "tk", len(seqs) * kvw).reshape(len(seqs), kvw)
    tv = synth.normal(7, "tv", len(seqs) * kvw).reshape(len(seqs), kvw)
    ref, got = _both(cache, seqs, w.heads, w.context, q, tk, tv)
    assert np.isfinite(ref).all()
    assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))
    # second call, smaller: five rows, no tails, a visible cap on two of them
    small = [seqs[3], seqs[17], seqs[40], seqs[41], seqs[63]]
    lengths = [cache.length(s) for s in small]
    visible = [lengths[0], 100, lengths[2] // 2, lengths[3], 1]
    say("no-alloc decode, second call", lengths)
    ref2, got2 = _both(cache, small, w.heads, w.context, q[[3, 17, 40, 41, 63]], visible=visible)
    assert np.array_equal(ref2.view(np.uint32), got2.view(np.uint32))
    # and the host-pointer entry point agrees with both
    host = attention.decode_batch(cache, q[[3, 17, 40, 41, 63]], small, 0, w.heads, w.context, visible=visible)
    assert np.array_equal(host.view(np.uint32), got2.view(np.uint32))


def test_noalloc_rejects_batches_above_the_scratch(device):
    lib = _capi.lib()
    limit = lib.tvara_attn_decode_noalloc_limit()
    assert limit == 32 << 20
    cache = device.PagedCache(1, 1, 64, 16, 4)
    s = cache.create_sequence()
    cache.append_many(s, np.ones((16, 64)), np.ones((16, 64)))
    rows = limit // 256 + 1  # one work item of 256 bytes of block ids per row at least
    say("no-alloc limit", limit, "rows", rows)
    q = hip.DeviceArray((rows, 64))
    out = hip.DeviceArray((rows, 64))
    rc = _decode(lib, "tvara_attn_decode_noalloc", cache, [s] * rows, 1, 4096, q, None, None, None, out)
    assert rc == _capi.INVALID
    assert "no-allocation scratch" in _capi.last_error()


def _free_bytes():
    hip.synchronize()
    free, total = C.c_size_t(), C.c_size_t()
    hip.check(hip.runtime().hipMemGetInfo(C.byref(free), C.byref(total)))
    return free.value


def test_noalloc_leaves_device_memory_unchanged(device):
    """The device's free memory is the same before and after the no-allocation
    call on a fresh cache and batch, while tvara_attn_decode on the same batch
    then grows its plan buffers (the control: the probe sees an allocation of
    the batch's size)."""
    w = workloads.decode_c2()
    say("no-alloc free-memory probe", w.name)
    g = (w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks)
    cache = device.PagedCache(*g)
    seqs = workloads.fill_decode(cache, w)
    q = hip.DeviceArray.from_numpy(w.queries())
    out = hip.DeviceArray((len(seqs), w.heads * w.head_dim))
    lib = cache.lib
    before = _free_bytes()
    for _ in range(3):
        _capi.check(_decode(lib, "tvara_attn_decode_noalloc", cache, seqs, w.heads, w.context, q, None, None, None,
                            out))
    after = _free_bytes()
    assert after == before, (before, after)
    _capi.check(_decode(lib, "tvara_attn_decode", cache, seqs, w.heads, w.context, q, None, None, None, out))
    control = _free_bytes()
    say("free bytes: before", before, "after no-alloc", after, "after tvara_attn_decode", control)
    assert control < after, (after, control)
