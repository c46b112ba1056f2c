"""Paged decode attention on the GPU against the oracle (the reference's fused
paged attention restated in FP64).  Bar: |gpu - ref| <= 1e-4 * (1 + |ref|)
for f32 blocks (the tolerance form of tests/core/prefill_support.hpp:7-9)."""

import sys
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import refmath
from tvara_amd import attention, synth, workloads

pytestmark = pytest.mark.gpu
TOL = 1e-4


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def build_pair(device, oracle, w, fmt=None):
    g = (w.layers, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks)
    dev = device.PagedCache(*g, fmt=fmt if fmt is not None else device.F32)
    ref = oracle.Cache(*g)
    ds = workloads.fill_decode(dev, w)
    rs = workloads.fill_decode(ref, w)
    assert ds == rs
    return dev, ref, ds


def oracle_rows(ref, seqs, q, w, **kw):
    return np.stack([ref.fused_paged_attention(q[i], s, 0, w.heads, w.context, **kw) for i, s in enumerate(seqs)])


def test_c1_smollm2_shape(device, oracle):
    w = workloads.decode_c1()
    say("decode", w.name)
    dev, ref, seqs = build_pair(device, oracle, w)
    assert dev.state() == ref.state()  # the seeded placement reproduced exactly
    q = w.queries()
    got = attention.decode_batch(dev, q, seqs, 0, w.heads, w.context)
    want = oracle_rows(ref, seqs, q, w)
    assert refmath.close(got, want, TOL), refmath.max_rel(got, want)


def test_c2_llama32_batch(device, oracle):
    w = workloads.decode_c2()
    say("decode", w.name, "tokens", w.total_tokens)
    dev, ref, seqs = build_pair(device, oracle, w)
    q = w.queries()
    got = attention.decode_batch(dev, q, seqs, 0, w.heads, w.context)
    want = oracle_rows(ref, seqs, q, w)
    assert refmath.close(got, want, TOL), refmath.max_rel(got, want)
    # the same through a resident plan on device buffers, launched twice
    from tvara_amd import hip

    plan = attention.DecodePlan(dev, seqs, w.heads, w.context)
    dq = hip.DeviceArray.from_numpy(q)
    out = hip.DeviceArray(q.shape)
    for _ in range(2):
        out.zero()
        plan.launch(0, dq.ptr, out.ptr)
        plan.check()
        assert np.array_equal(out.numpy(), got)


def test_plan_on_a_non_blocking_stream(device, oracle):
    # The cache queues its appends, copies and zero-fills on its own stream
    # (the null stream here); a plan launched on a non-blocking stream is not
    # ordered against it by HIP.  The launch must still see every appended
    # row, and block writes queued after it (a truncate, then appends that
    # reuse the freed blocks) must not overtake its reads.
    from tvara_amd import hip

    heads, kv_heads, dim, tpb, n, length = 32, 8, 64, 16, 8, 3000
    g = (1, kv_heads, dim, tpb, n * (length // tpb + 1) + 8)
    dev, ref = device.PagedCache(*g), oracle.Cache(*g)
    w = kv_heads * dim
    seqs = []
    for i in range(n):
        k = synth.normal(40 + i, "k", length * w).reshape(length, w)
        v = synth.normal(40 + i, "v", length * w).reshape(length, w)
        sd, sr = dev.create_sequence(), ref.create_sequence()
        dev.append_many(sd, k, v)  # queued, not waited for
        ref.append_many(sr, k, v)
        seqs.append((sd, sr))
    q = synth.normal(49, "q", n * heads * dim).reshape(n, heads * dim)
    want = np.stack([ref.fused_paged_attention(q[i], sr, 0, heads, 8192) for i, (_, sr) in enumerate(seqs)])
    stream = hip.Stream(non_blocking=True)
    dq = hip.DeviceArray.from_numpy(q)
    for rnd in range(3):
        say("non-blocking stream round", rnd)
        plan = attention.DecodePlan(dev, [sd for sd, _ in seqs], heads, 8192)
        out = hip.DeviceArray(q.shape)
        plan.launch(0, dq.ptr, out.ptr, stream=stream.h)
        # block writes queued behind the launch on the cache's stream
        victim = dev.create_sequence()
        junk = np.full((length, w), np.nan, np.float32)
        dev.truncate(seqs[rnd][0], 0)
        dev.append_many(victim, junk, junk)
        plan.check()
        got = out.numpy()
        assert refmath.close(got, want, TOL), (rnd, refmath.max_rel(got, want))
        # restore the truncated sequence for the next round
        dev.drop(victim)
        k = synth.normal(40 + rnd, "k", length * w).reshape(length, w)
        v = synth.normal(40 + rnd, "v", length * w).reshape(length, w)
        dev.append_many(seqs[rnd][0], k, v)


def _single(device, oracle, heads, kv_heads, dim, tpb, length, seed, tail=False, visible=None, fmt=None,
            layers=1, layer=0):
    g = (layers, kv_heads, dim, tpb, length // tpb + 3)
    dev = device.PagedCache(*g, fmt=fmt if fmt is not None else device.F32)
    ref = oracle.Cache(*g)
    w = layers * kv_heads * dim
    k = synth.normal(seed, "k", length * w).reshape(length, w)
    v = synth.normal(seed, "v", length * w).reshape(length, w)
    if fmt == device.Q8_0:  # the oracle holds the dequantised values
        k = oracle.dequantize_q8_0(oracle.quantize_q8_0(k)).reshape(length, w)
        v = oracle.dequantize_q8_0(oracle.quantize_q8_0(v)).reshape(length, w)
    sd, sr = dev.create_sequence(), ref.create_sequence()
    dev.append_many(sd, k, v)
    ref.append_many(sr, k, v)
    q = synth.normal(seed, "q", heads * dim)
    kw = {}
    if tail:
        kw = {"tail_key": synth.normal(seed, "tk", kv_heads * dim), "tail_value": synth.normal(seed, "tv", kv_heads * dim)}
    if visible is not None:
        kw["visible"] = visible
    got = attention.fused_paged_attention(q, dev, sd, layer, heads, 1 << 20, **kw)
    want = ref.fused_paged_attention(q, sr, layer, heads, 1 << 20, **kw)
    return got, want


# groups above eight (16: Llama-3.1-405B's 128 / 8 heads) run as slices of at
# most eight heads, each a virtual KV head of the fast kernels; head_dims 80,
# 96 and 256 (Phi-2, Phi-3, Gemma) run it with up to four heads a slice
@pytest.mark.parametrize("dim,kv_heads,group", [(64, 8, 1), (64, 8, 2), (64, 3, 3), (64, 2, 4), (64, 4, 8), (64, 2, 7),
                                                (64, 3, 5), (128, 8, 4), (128, 2, 8), (128, 4, 5), (8, 1, 8), (32, 2, 2),
                                                (16, 4, 1), (64, 2, 16), (128, 2, 16), (64, 1, 12), (128, 1, 10),
                                                (64, 1, 32), (32, 2, 9), (256, 2, 2), (256, 1, 4), (256, 1, 3),
                                                (256, 2, 8), (96, 4, 1), (96, 2, 3), (96, 1, 8), (80, 4, 1),
                                                (80, 1, 4)])
@pytest.mark.parametrize("length", [1, 15, 16, 17, 100, 1031])
def test_shapes_and_gqa_ratios(device, oracle, dim, kv_heads, group, length):
    say("decode shape", dim, kv_heads, group, length)
    got, want = _single(device, oracle, kv_heads * group, kv_heads, dim, 16, length, seed=dim + length)
    assert refmath.close(got, want, TOL), refmath.max_rel(got, want)


# Q8_0 groups of 32 columns never straddle a head: head_dim is a multiple of 32
Q8_SHAPES = [(64, 8, 1), (64, 8, 2), (64, 3, 3), (64, 2, 4), (64, 4, 8), (64, 2, 6), (64, 2, 7), (128, 8, 4),
             (128, 2, 8), (128, 4, 5), (128, 2, 6), (128, 3, 7), (32, 2, 2), (32, 1, 8), (64, 2, 16), (128, 2, 16),
             (128, 1, 12), (256, 2, 2), (256, 1, 4), (256, 2, 8)]


@pytest.mark.parametrize("dim,kv_heads,group", Q8_SHAPES)
@pytest.mark.parametrize("length", [1, 17, 1031, 20000])
def test_q8_shapes(device, oracle, dim, kv_heads, group, length):
    # Q8_0 blocks against the oracle holding the dequantised values; the
    # 20,000-token row is cut into hundreds of splits (several merge passes)
    say("decode q8", dim, kv_heads, group, length)
    got, want = _single(device, oracle, kv_heads * group, kv_heads, dim, 16, length, seed=dim + length, tail=True,
                        fmt=device.Q8_0)
    assert refmath.close(got, want, TOL), refmath.max_rel(got, want)


def test_c5_q8_full_batch(device, oracle):
    # the whole 16 x 32,768-token Q8_0 batch in one launch; every row against
    # the oracle on the dequantised values, and against the original f32
    # values within the quantisation bar (2e-3)
    w = workloads.decode_c5()
    say("decode", w.name)
    dev = device.PagedCache(1, w.kv_heads, w.head_dim, 16, w.pool_blocks, fmt=device.Q8_0)
    seqs = workloads.fill_decode(dev, w)
    q = w.queries()
    got = attention.decode_batch(dev, q, seqs, 0, w.heads, w.context)

    def row(i):  # the oracle's calls release the GIL: rows run in threads
        k, v = w.keys(i), w.values(i)
        n = len(k)
        ref = oracle.Cache(1, w.kv_heads, w.head_dim, 16, n // 16 + 1)
        s = ref.create_sequence()
        ref.append_many(s, oracle.dequantize_q8_0(oracle.quantize_q8_0(k)).reshape(n, -1),
                        oracle.dequantize_q8_0(oracle.quantize_q8_0(v)).reshape(n, -1))
        want = ref.fused_paged_attention(q[i], s, 0, w.heads, w.context)
        del ref
        exact = oracle.Cache(1, w.kv_heads, w.head_dim, 16, n // 16 + 1)
        s = exact.create_sequence()
        exact.append_many(s, k, v)
        orig = exact.fused_paged_attention(q[i], s, 0, w.heads, w.context)
        return want, orig

    with ThreadPoolExecutor(max_workers=8) as pool:
        for i, (want, orig) in enumerate(pool.map(row, range(w.sequences))):
            assert refmath.close(got[i], want, TOL), (i, refmath.max_rel(got[i], want))
            assert refmath.close(got[i], orig, 2e-3), (i, refmath.max_rel(got[i], orig))
            say("row", i, "vs dequantised", refmath.max_rel(got[i], want), "vs f32", refmath.max_rel(got[i], orig))


@pytest.mark.parametrize("make", [workloads.decode_gqa16, lambda: workloads.decode_gqa16(q8=True),
                                  workloads.decode_gemma2, workloads.decode_phi3],
                         ids=["gqa16-f32", "gqa16-q8_0", "gemma2-d256", "phi3-d96"])
def test_wide_shapes_full_batch(device, oracle, make):
    # the 16 x 4,096-token batches of the shapes the fast kernels take by
    # slicing (Llama-3.1-405B's sixteen query heads per KV head) or by wider
    # token groups (head_dim 256 and 96): every row against the oracle (Q8_0:
    # on the dequantised values)
    w = make()
    say("decode", w.name)
    fmt = device.Q8_0 if w.q8 else device.F32
    dev = device.PagedCache(1, w.kv_heads, w.head_dim, 16, w.pool_blocks, fmt=fmt)
    seqs = workloads.fill_decode(dev, w)
    q = w.queries()
    got = attention.decode_batch(dev, q, seqs, 0, w.heads, w.context)

    def row(i):  # the oracle's calls release the GIL: rows run in threads
        k, v = w.keys(i), w.values(i)
        n = len(k)
        if w.q8:
            k = oracle.dequantize_q8_0(oracle.quantize_q8_0(k)).reshape(n, -1)
            v = oracle.dequantize_q8_0(oracle.quantize_q8_0(v)).reshape(n, -1)
        ref = oracle.Cache(1, w.kv_heads, w.head_dim, 16, n // 16 + 1)
        s = ref.create_sequence()
        ref.append_many(s, k, v)
        return ref.fused_paged_attention(q[i], s, 0, w.heads, w.context)

    with ThreadPoolExecutor(max_workers=8) as pool:
        for i, want in enumerate(pool.map(row, range(w.sequences))):
            assert refmath.close(got[i], want, TOL), (i, refmath.max_rel(got[i], want))


@pytest.mark.parametrize("tpb", [7, 5, 4, 32, 1])
def test_block_sizes(device, oracle, tpb):
    # block sizes that do not divide the length (prefill_t171.cpp, prefill_t180.cpp)
    for dim in (8, 64):
        got, want = _single(device, oracle, 4, 2, dim, tpb, 53, seed=tpb)
        assert refmath.close(got, want, TOL), refmath.max_rel(got, want)


@pytest.mark.parametrize("dim", [8, 64, 128])
def test_tail_and_visible(device, oracle, dim):
    for length, visible in [(0, None), (53, None), (53, 54), (53, 20), (300, 1), (300, 299)]:
        say("tail", dim, length, visible)
        got, want = _single(device, oracle, 8, 2, dim, 16, max(length, 0), seed=3, tail=True, visible=visible) \
            if length else (None, None)
        if length == 0:  # an empty cache with a tail attends to the tail alone
            g = (1, 2, dim, 16, 4)
            dev = device.PagedCache(*g)
            s = dev.create_sequence()
            tv = synth.normal(4, "tv", 2 * dim)
            out = attention.fused_paged_attention(synth.normal(4, "q", 8 * dim), dev, s, 0, 8, 64,
                                                  synth.normal(4, "tk", 2 * dim), tv)
            assert np.array_equal(out.reshape(8, dim), np.repeat(tv.reshape(2, dim), 4, axis=0))
            continue
        assert refmath.close(got, want, TOL), refmath.max_rel(got, want)


def test_layers(device, oracle):
    for layer in range(3):
        got, want = _single(device, oracle, 8, 4, 64, 16, 77, seed=layer, layers=3, layer=layer)
        assert refmath.close(got, want, TOL), refmath.max_rel(got, want)


def test_long_contexts(device, oracle):
    # fused vs reference through 8192 positions (prefill_t177.cpp)
    for length in (127, 1024, 4097, 8192):
        for dim in (16, 64):
            got, want = _single(device, oracle, 4, 2, dim, 16, length, seed=length)
            assert refmath.close(got, want, TOL), (length, dim, refmath.max_rel(got, want))


def test_nan_poisoned_unused_slots(device, oracle):
    # NaN in unused tail slots and junk in recycled blocks never leak (prefill_t174.cpp)
    for dim in (8, 64):
        for length in (1, 15, 16, 17, 31, 32, 33):
            g = (1, 2, dim, 16, 8)
            dev = device.PagedCache(*g)
            old = dev.create_sequence()
            junk = synth.signal(2 * dim, 100)
            dev.append_many(old, np.tile(junk, (48, 1)), np.tile(junk, (48, 1)))
            dev.drop(old)
            s = dev.create_sequence()
            k = synth.signal(length * 2 * dim).reshape(length, 2 * dim)
            v = synth.signal(length * 2 * dim, 2).reshape(length, 2 * dim)
            dev.append_many(s, k, v)
            h = dev.physical_block(s, length - 1)
            for slot in range(length % 16 or 16, 16):
                for kind in (0, 1):
                    dev.block_write(h, dev.kv_offset(0, kind, slot), np.full(2 * dim, np.nan, np.float32))
            q = synth.signal(4 * dim, 3)
            got = attention.fused_paged_attention(q, dev, s, 0, 4, 128)
            assert refmath.close(got, refmath.attention(q, k, v, 4, 2, dim), TOL)
            dev.audit()


def test_rejections(device):
    dev = device.PagedCache(1, 2, 64, 16, 8)
    s = dev.create_sequence()
    x = synth.normal(1, "x", 10 * 128).reshape(10, 128)
    dev.append_many(s, x, x)
    q = synth.normal(1, "q", 4 * 64)
    with pytest.raises(device.InvalidArgument):  # empty attention
        attention.fused_paged_attention(q, dev, s, 0, 4, 64, visible=0)
    with pytest.raises(device.InvalidArgument):  # length beyond context
        attention.fused_paged_attention(q, dev, s, 0, 4, 8)
    with pytest.raises(device.InvalidArgument):  # heads not a multiple of kv heads
        attention.fused_paged_attention(synth.normal(1, "q3", 3 * 64), dev, s, 0, 3, 64)
    with pytest.raises(device.InvalidArgument):  # bad layer
        attention.fused_paged_attention(q, dev, s, 1, 4, 64)
    with pytest.raises(device.InvalidArgument):  # unknown sequence
        attention.fused_paged_attention(q, dev, 99, 0, 4, 64)
    with pytest.raises(device.InvalidArgument):  # non-finite score (attention.hpp:11)
        attention.fused_paged_attention(np.full_like(q, np.inf), dev, s, 0, 4, 64)
    # the error flag is cleared: a valid call after it succeeds
    assert np.isfinite(attention.fused_paged_attention(q, dev, s, 0, 4, 64)).all()
    plan = attention.DecodePlan(dev, [s], 4, 64)
    dev.append(s, x[0], x[0])
    from tvara_amd import hip

    dq = hip.DeviceArray.from_numpy(q)
    with pytest.raises(device.InvalidArgument):  # the cache changed under the plan
        plan.launch(0, dq.ptr, dq.ptr)


def test_huge_scores_stay_finite(device, oracle):
    # scores near 1e4 (prefill_t170.cpp:4): the running maximum must move
    g = (1, 2, 64, 16, 8)
    dev, ref = device.PagedCache(*g), oracle.Cache(*g)
    sd, sr = dev.create_sequence(), ref.create_sequence()
    k = synth.normal(2, "k", 60 * 128).reshape(60, 128) * np.float32(300.0)
    v = synth.normal(2, "v", 60 * 128).reshape(60, 128)
    dev.append_many(sd, k, v)
    ref.append_many(sr, k, v)
    q = synth.normal(2, "q", 4 * 64)
    got = attention.fused_paged_attention(q, dev, sd, 0, 4, 64)
    want = ref.fused_paged_attention(q, sr, 0, 4, 64)
    assert np.isfinite(got).all() and refmath.close(got, want, TOL)


def _q8_sequence(device, oracle, kv_heads, dim, length, k, v, pool=8):
    """A Q8_0 cache holding one sequence of k/v (already dequantised Q8_0 values)."""
    dev = device.PagedCache(1, kv_heads, dim, 16, pool, fmt=device.Q8_0)
    s = dev.create_sequence()
    dev.append_many(s, k, v)
    return dev, s


def _q8_values(oracle, x):
    return oracle.dequantize_q8_0(oracle.quantize_q8_0(x)).reshape(x.shape)


@pytest.mark.parametrize("dim,group", [(64, 4), (128, 4), (128, 2), (128, 6), (128, 8)])
def test_q8_tail_and_visible(device, oracle, dim, group):
    for length, visible in [(53, None), (53, 54), (53, 20), (300, 1), (300, 299), (64, 33)]:
        say("q8 tail", dim, group, length, visible)
        got, want = _single(device, oracle, 2 * group, 2, dim, 16, length, seed=7, tail=True, visible=visible,
                            fmt=device.Q8_0)
        assert refmath.close(got, want, TOL), refmath.max_rel(got, want)
    # an empty Q8_0 cache with a tail attends to the (f32) tail alone
    dev = device.PagedCache(1, 2, dim, 16, 4, fmt=device.Q8_0)
    s = dev.create_sequence()
    tv = synth.normal(4, "tv", 2 * dim)
    out = attention.fused_paged_attention(synth.normal(4, "q", 2 * group * dim), dev, s, 0, 2 * group, 64,
                                          synth.normal(4, "tk", 2 * dim), tv)
    assert np.array_equal(out.reshape(2 * group, dim), np.repeat(tv.reshape(2, dim), group, axis=0))


def test_q8_zero_query_is_mean_of_values(device, oracle):
    # q = 0 gives every position the same score, so each query head returns the
    # mean of its KV head's values (tests/core/test_model.cpp:46-51)
    for dim, kv_heads, group, length in [(64, 2, 4, 77), (128, 8, 4, 300), (128, 4, 2, 33), (64, 3, 3, 16)]:
        say("q8 zero query", dim, kv_heads, group, length)
        w = kv_heads * dim
        k = _q8_values(oracle, synth.normal(11, "k", length * w).reshape(length, w))
        v = _q8_values(oracle, synth.normal(11, "v", length * w).reshape(length, w))
        dev, s = _q8_sequence(device, oracle, kv_heads, dim, length, k, v, pool=length // 16 + 2)
        heads = kv_heads * group
        got = attention.fused_paged_attention(np.zeros(heads * dim, np.float32), dev, s, 0, heads, 4096)
        want = np.repeat(v.astype(np.float64).reshape(length, kv_heads, dim).mean(axis=0), group, axis=0).reshape(-1)
        assert refmath.close(got, want, TOL), refmath.max_rel(got, want)


def test_q8_unused_slots_and_junk_never_leak(device, oracle):
    # Q8_0 form of prefill_t174.cpp: NaN group scales and junk int8 in the
    # unused slots of the last block, for the int8-MFMA score path (group <= 4)
    # and the vector path (group 8)
    nan_group = np.concatenate([np.frombuffer(np.float16(np.nan).tobytes(), np.uint8), np.full(32, 0x81, np.uint8)])
    for dim, kv_heads, group in [(64, 2, 4), (128, 2, 4), (128, 2, 3), (128, 1, 8)]:
        for length in (1, 15, 16, 17, 31, 32, 33, 47):
            say("q8 poison", dim, kv_heads, group, length)
            w = kv_heads * dim
            k = _q8_values(oracle, synth.signal(length * w).reshape(length, w))
            v = _q8_values(oracle, synth.signal(length * w, 2).reshape(length, w))
            dev, s = _q8_sequence(device, oracle, kv_heads, dim, length, k, v)
            h = dev.physical_block(s, length - 1)
            gpr = w // 32
            for slot in range(length % 16 or 16, 16):
                for kind in (0, 1):
                    dev.block_write(h, ((kind * 16 + slot) * gpr) * 34, np.tile(nan_group, gpr))
            heads = kv_heads * group
            q = synth.signal(heads * dim, 3)
            got = attention.fused_paged_attention(q, dev, s, 0, heads, 128)
            assert refmath.close(got, refmath.attention(q, k, v, heads, kv_heads, dim), TOL)
            dev.audit()


def test_q8_wide_ranges(device, oracle):
    # per-token magnitudes from 1e-4 to 1e1 (group scales from ~1e-6, fp16
    # subnormals, to ~0.3; scores up to ~1e2, so the running maximum moves),
    # queries with one large head and one near-zero head; against float64
    # attention on the dequantised values
    for dim, kv_heads, group in [(128, 2, 4), (64, 2, 4), (128, 4, 1)]:
        length = 200
        say("q8 ranges", dim, kv_heads, group)
        w = kv_heads * dim
        mag = np.float32(10.0) ** np.linspace(-4, 1, length, dtype=np.float32)[synth.permutation(5, "m", length)]
        k = _q8_values(oracle, synth.normal(5, "k", length * w).reshape(length, w) * mag[:, None])
        v = _q8_values(oracle, synth.normal(5, "v", length * w).reshape(length, w) * mag[:, None])
        dev, s = _q8_sequence(device, oracle, kv_heads, dim, length, k, v, pool=length // 16 + 2)
        heads = kv_heads * group
        q = synth.normal(5, "q", heads * dim).reshape(heads, dim)
        q[0] *= np.float32(4.0)
        q[-1] *= np.float32(1e-5)
        got = attention.fused_paged_attention(q.reshape(-1), dev, s, 0, heads, 4096)
        want = refmath.attention(q.reshape(-1), k, v, heads, kv_heads, dim)
        assert np.isfinite(got).all() and refmath.close(got, want, TOL), refmath.max_rel(got, want)


def test_prompt_chunk_f32(device, oracle):
    # fused_prompt_attention (prefill_t173.cpp): rows see their own prefix only
    g = (1, 1, 8, 7, 20)
    dev, ref = device.PagedCache(*g), oracle.Cache(*g)
    sd, sr = dev.create_sequence(), ref.create_sequence()
    k = synth.signal(39 * 8).reshape(39, 8)
    v = synth.signal(39 * 8, 2).reshape(39, 8)
    dev.append_many(sd, k, v)
    ref.append_many(sr, k, v)
    qs = synth.signal(13 * 32, 3)
    got = attention.fused_prompt_attention(qs, dev, sd, 0, 11, 13, 4, 128)
    want = ref.fused_prompt_attention(qs, sr, 0, 11, 13, 4, 128)
    assert refmath.close(got, want, TOL)
    h = dev.physical_block(sd, 38)
    dev.block_write(h, 0, np.full(dev.elements_per_block, 99999, np.float32))
    assert np.array_equal(attention.fused_prompt_attention(qs, dev, sd, 0, 11, 13, 4, 128), got)
    with pytest.raises(device.InvalidArgument):
        attention.fused_prompt_attention(qs, dev, sd, 0, 30, 13, 4, 128)


@pytest.mark.parametrize("split", [0, 1024], ids=["merge-launch", "merge-in-kernel"])
@pytest.mark.parametrize("fmt_name,dim,kv_heads,group", [("F32", 64, 8, 4), ("F32", 128, 4, 8), ("Q8_0", 128, 2, 8),
                                                         ("Q8_0", 128, 2, 5), ("F32", 64, 4, 8)])
def test_plan_back_to_back_launches(device, oracle, monkeypatch, fmt_name, dim, kv_heads, group, split):
    # rows of several splits: with the default split the launch fills the GPU
    # and merge_kernel combines them; 1,024-token splits give a launch of a few
    # dozen workgroups, where the last workgroup of each row merges (it counts
    # the row's finished splits and resets the count).  48 launches queued
    # without a wait, alternating two layers, all equal the first launch of
    # their layer byte for byte and match the oracle
    from tvara_amd import hip

    if split:
        monkeypatch.setenv("TVARA_SPLIT_TOKENS", str(split))

    fmt = getattr(device, fmt_name)
    heads, layers, tpb = kv_heads * group, 2, 16
    lengths = [97, 3000, 640, 1, 2049, 1500, 4096, 33, 800, 2500, 16, 1234]
    g = (layers, kv_heads, dim, tpb, sum((n + tpb - 1) // tpb for n in lengths) + 4)
    dev, ref = device.PagedCache(*g, fmt=fmt), oracle.Cache(*g)
    w = layers * kv_heads * dim
    seqs = []
    for i, n in enumerate(lengths):
        k = synth.normal(31, f"k{i}", n * w).reshape(n, w)
        v = synth.normal(31, f"v{i}", n * w).reshape(n, w)
        if fmt_name == "Q8_0":
            k = oracle.dequantize_q8_0(oracle.quantize_q8_0(k)).reshape(n, w)
            v = oracle.dequantize_q8_0(oracle.quantize_q8_0(v)).reshape(n, w)
        s, r = dev.create_sequence(), ref.create_sequence()
        dev.append_many(s, k, v)
        ref.append_many(r, k, v)
        assert s == r
        seqs.append(s)
    q = synth.normal(31, "q", len(lengths) * heads * dim).reshape(len(lengths), heads * dim)
    plan = attention.DecodePlan(dev, seqs, heads, 1 << 20)
    assert plan.items > len(lengths)  # some rows have several splits
    assert (plan.items < 64) == bool(split)
    say("back-to-back", fmt_name, dim, kv_heads, group, "split", plan.split_tokens, "items", plan.items)
    dq = hip.DeviceArray.from_numpy(q)
    outs = [hip.DeviceArray(q.shape) for _ in range(48)]
    for i, o in enumerate(outs):
        plan.launch(i % 2, dq.ptr, o.ptr)
    plan.check()
    got = [o.numpy() for o in outs]
    for i in range(2, len(got)):
        assert np.array_equal(got[i], got[i % 2]), i
    # Q8_0 blocks hold exactly the oracle's dequantised values, so both formats meet the f32 bar
    for layer in (0, 1):
        want = np.stack([ref.fused_paged_attention(q[i], s, layer, heads, 1 << 20) for i, s in enumerate(seqs)])
        assert refmath.close(got[layer], want, TOL), refmath.max_rel(got[layer], want)


@pytest.mark.parametrize("scale", ["fill", "small"], ids=["merge-launch", "merge-in-kernel"])
def test_ragged_rows_with_tail_only_rows(device, oracle, scale):
    # rows with no cached token (the tail is their only position), one-token
    # rows and rows ending on and off block edges, in a launch that fills the
    # GPU (merge_kernel combines the splits) and in a small one (the last
    # workgroup of each row merges them)
    if scale == "fill":
        lengths = [0, 1, 16, 17, 4096, 0, 300, 2047, 64, 65, 1000, 3001, 5, 0, 777, 2500] * 4
    else:
        lengths = [0, 1, 16, 17, 100, 0, 300, 47, 64, 65, 200, 31, 5, 0, 77, 250] * 3
    kv_heads, dim, group, tpb = 8, 64, 4, 16
    heads = kv_heads * group
    g = (1, kv_heads, dim, tpb, sum((n + tpb - 1) // tpb for n in lengths) + 4)
    dev, ref = device.PagedCache(*g), oracle.Cache(*g)
    w = kv_heads * dim
    seqs = []
    for i, n in enumerate(lengths):
        s, r = dev.create_sequence(), ref.create_sequence()
        if n:
            k = synth.normal(41, f"k{i}", n * w).reshape(n, w)
            v = synth.normal(41, f"v{i}", n * w).reshape(n, w)
            dev.append_many(s, k, v)
            ref.append_many(r, k, v)
        seqs.append(s)
    rows = len(lengths)
    q = synth.normal(41, "q", rows * heads * dim).reshape(rows, heads * dim)
    tk = synth.normal(41, "tk", rows * w).reshape(rows, w)
    tv = synth.normal(41, "tv", rows * w).reshape(rows, w)
    plan = attention.DecodePlan(dev, seqs, heads, 1 << 20, with_tail=True)
    assert (plan.items <= 128) == (scale == "small")
    say("ragged rows", scale, "rows", rows, "tokens", sum(lengths), "items", plan.items)
    got = attention.decode_batch(dev, q, seqs, 0, heads, 1 << 20, tail_keys=tk, tail_values=tv)
    want = np.stack([ref.fused_paged_attention(q[i], s, 0, heads, 1 << 20, tail_key=tk[i], tail_value=tv[i])
                     for i, s in enumerate(seqs)])
    assert refmath.close(got, want, TOL), refmath.max_rel(got, want)


@pytest.mark.parametrize("kv_heads,group", [(8, 4), (8, 1), (8, 2), (8, 3), (8, 8), (4, 4), (4, 8), (16, 2), (16, 4),
                                            (16, 7)])
def test_row_major_kernel(device, oracle, monkeypatch, kv_heads, group):
    # The row-major f32 kernel (head_dim 64; 4, 8 or 16 KV heads) takes launches
    # of more than 128 work items.  64-token splits over rows of every kind
    # (no cached token, one token, block edges, partial last blocks, long
    # rows) with each row's uncommitted token as its last position; three
    # launches in a row agree byte for byte and match the oracle.
    from tvara_amd import hip

    monkeypatch.setenv("TVARA_SPLIT_TOKENS", "64")
    dim, tpb = 64, 16
    heads = kv_heads * group
    rng = np.random.default_rng(61 + kv_heads * 10 + group)
    lengths = [0, 1, 15, 16, 17, 2047, 63, 64, 65, 100] + [int(x) for x in rng.integers(1, 1500, 14)]
    g = (2, kv_heads, dim, tpb, sum((n + tpb - 1) // tpb for n in lengths) + 4)
    dev, ref = device.PagedCache(*g), oracle.Cache(*g)
    w = 2 * kv_heads * dim
    seqs = []
    for i, n in enumerate(lengths):
        s, r = dev.create_sequence(), ref.create_sequence()
        if n:
            k = synth.normal(63, f"k{i}", n * w).reshape(n, w)
            v = synth.normal(63, f"v{i}", n * w).reshape(n, w)
            dev.append_many(s, k, v)
            ref.append_many(r, k, v)
        seqs.append(s)
    rows = len(lengths)
    q = synth.normal(63, "q", rows * heads * dim).reshape(rows, heads * dim)
    tk = synth.normal(63, "tk", rows * kv_heads * dim).reshape(rows, kv_heads * dim)
    tv = synth.normal(63, "tv", rows * kv_heads * dim).reshape(rows, kv_heads * dim)
    dq, dtk, dtv = (hip.DeviceArray.from_numpy(x) for x in (q, tk, tv))
    plan = attention.DecodePlan(dev, seqs, heads, 1 << 20, with_tail=True)
    assert plan.items > 128
    say("row-major", kv_heads, group, "items", plan.items)
    outs = [hip.DeviceArray(q.shape) for _ in range(3)]
    for o in outs:
        plan.launch(1, dq.ptr, o.ptr, dtk.ptr, dtv.ptr)
    plan.check()
    got = [o.numpy() for o in outs]
    for o in got[1:]:
        assert np.array_equal(o, got[0])
    want = np.stack([ref.fused_paged_attention(q[i], s, 1, heads, 1 << 20, tail_key=tk[i], tail_value=tv[i])
                     for i, s in enumerate(seqs)])
    assert refmath.close(got[0], want, TOL), refmath.max_rel(got[0], want)


@pytest.mark.parametrize("tpb", [32, 64, 256])
@pytest.mark.parametrize("dim,kv_heads,group", [(32, 2, 2), (32, 4, 8), (64, 8, 4), (64, 2, 7), (128, 4, 4),
                                                (128, 2, 8)])
def test_large_blocks_fast_kernels(device, oracle, tpb, dim, kv_heads, group):
    # f32 blocks of 32 to 256 tokens and head_dim 32 stream through the fast
    # kernels (splits start on a block); lengths ending inside and on a block,
    # with and without the uncommitted token, and a visible cap
    for length, kw in [(1, {}), (tpb - 1, {}), (tpb, {"tail": True}), (3 * tpb + 5, {}),
                       (2500, {"tail": True}), (2500, {"visible": 1300})]:
        got, want = _single(device, oracle, kv_heads * group, kv_heads, dim, tpb, length, seed=tpb + length, **kw)
        assert refmath.close(got, want, TOL), (length, kw, refmath.max_rel(got, want))


@pytest.mark.parametrize("tpb", [32, 64, 128, 1024])
def test_row_major_large_blocks(device, oracle, monkeypatch, tpb):
    # the row-major kernel over 32- to 1,024-token blocks: a 16-row tile is a
    # quarter or half of a block at 32 and 64; at 128 and 1,024 a 64-token
    # split covers part of one block, so a tile's block and its offset inside
    # it both come from the tile index
    from tvara_amd import hip

    monkeypatch.setenv("TVARA_SPLIT_TOKENS", "64")
    kv_heads, dim, group = 8, 64, 4
    heads = kv_heads * group
    # splits are whole blocks, so the larger blocks need more tokens to give
    # the row-major kernel its launch of more than 128 work items
    if tpb <= 64:
        lengths = [1, 31, 32, 33, 63, 64, 65, 200, 1000, 3000] * 3
    elif tpb == 128:
        lengths = [1, 31, 32, 33, 63, 64, 65, 200, 1000, 3000] * 4
    else:
        lengths = [1, tpb - 1, tpb, tpb + 1, 2 * tpb - 1, 2 * tpb, 2 * tpb + 1, 3000, 5000, 9000] * 5
    g = (1, kv_heads, dim, tpb, sum((n + tpb - 1) // tpb for n in lengths) + 4)
    dev, ref = device.PagedCache(*g), oracle.Cache(*g)
    w = kv_heads * dim
    seqs = []
    for i, n in enumerate(lengths):
        s, r = dev.create_sequence(), ref.create_sequence()
        k = synth.normal(71, f"k{i}", n * w).reshape(n, w)
        v = synth.normal(71, f"v{i}", n * w).reshape(n, w)
        dev.append_many(s, k, v)
        ref.append_many(r, k, v)
        seqs.append(s)
    q = synth.normal(71, "q", len(lengths) * heads * dim).reshape(len(lengths), heads * dim)
    plan = attention.DecodePlan(dev, seqs, heads, 1 << 20)
    assert plan.items > 128
    dq, out = hip.DeviceArray.from_numpy(q), hip.DeviceArray(q.shape)
    plan.launch(0, dq.ptr, out.ptr)
    plan.check()
    want = np.stack([ref.fused_paged_attention(q[i], s, 0, heads, 1 << 20) for i, s in enumerate(seqs)])
    got = out.numpy()
    assert refmath.close(got, want, TOL), refmath.max_rel(got, want)


def test_t176_shape(device, oracle):
    # tests/core/prefill_t176.cpp: 1,025 appends of one K/V row to a 2-KV-head,
    # head_dim 32 cache of 16-token blocks, one 4-head query (synth.signal is
    # the reference's signal(), tests/core/prefill_support.hpp:11-13)
    g = (1, 2, 32, 16, 128)
    dev, ref = device.PagedCache(*g), oracle.Cache(*g)
    k, v, q = synth.signal(64), synth.signal(64, 2), synth.signal(128, 3)
    sd, sr = dev.create_sequence(), ref.create_sequence()
    dev.append_many(sd, np.tile(k, (1025, 1)), np.tile(v, (1025, 1)))
    ref.append_many(sr, np.tile(k, (1025, 1)), np.tile(v, (1025, 1)))
    got = attention.fused_paged_attention(q, dev, sd, 0, 4, 2048)
    want = ref.fused_paged_attention(q, sr, 0, 4, 2048)
    # every key is the same row, so each head's output is that head's V row
    assert np.allclose(want.reshape(4, 32), np.repeat(v.reshape(2, 32), 2, axis=0), rtol=1e-6, atol=1e-6)
    assert refmath.close(got, want, TOL), refmath.max_rel(got, want)


@pytest.mark.parametrize("fmt_name,dim,kv_heads,group,split", [("F32", 64, 8, 4, 0), ("F32", 64, 4, 8, 0),
                                                               ("F32", 64, 16, 2, 0), ("F32", 128, 8, 4, 0),
                                                               ("F32", 64, 8, 4, 256), ("Q8_0", 128, 8, 4, 0),
                                                               ("Q8_0", 64, 2, 4, 0)])
def test_zero_query_counts_every_token(device, oracle, monkeypatch, fmt_name, dim, kv_heads, group, split):
    # q = 0: every score is 0 and every weight exp2(0) = 1, so with V of
    # integers (exact in f32 and in Q8_0 with one 127 per 32-column group) each
    # output row is the exact mean of the row's V rows and its tail row, through
    # any split and merge.  A dropped or repeated token moves the mean by at
    # least 1/(2n) of a unit, far above the 1e-6 bar -- the 1e-4 bar of the
    # N(0,1) tests can miss one token of 4,096.  Rows of the C2 length
    # distribution (launches that fill the GPU: the row-major, int8-MFMA and
    # head-major kernels with their split merges).
    if split:
        monkeypatch.setenv("TVARA_SPLIT_TOKENS", str(split))
    fmt = getattr(device, fmt_name)
    heads, tpb = kv_heads * group, 16
    lengths = [int(x) for x in synth.integers(2, "ctx", 64, 128, 4096)[:48]] + [1, 15, 16, 17]
    g = (1, kv_heads, dim, tpb, sum((n + tpb - 1) // tpb for n in lengths) + 4)
    dev = device.PagedCache(*g, fmt=fmt)
    w = kv_heads * dim
    rng = np.random.default_rng(91 + dim + kv_heads + group)
    seqs, vals = [], []
    for i, n in enumerate(lengths):
        v = rng.integers(-4, 5, size=(n, w)).astype(np.float32)
        v[:, ::32] = 127.0
        k = synth.normal(91, f"k{i}", n * w).reshape(n, w)
        s = dev.create_sequence()
        dev.append_many(s, k, v)
        seqs.append(s)
        vals.append(v)
    rows = len(lengths)
    tv = rng.integers(-4, 5, size=(rows, w)).astype(np.float32)
    tk = synth.normal(91, "tk", rows * w).reshape(rows, w)
    q = np.zeros((rows, heads * dim), np.float32)
    plan = attention.DecodePlan(dev, seqs, heads, 1 << 20, with_tail=True)
    say("zero query", fmt_name, dim, kv_heads, group, "items", plan.items, "split", plan.split_tokens)
    got = attention.decode_batch(dev, q, seqs, 0, heads, 1 << 20, tail_keys=tk, tail_values=tv)
    got = got.reshape(rows, heads, dim)
    for i, n in enumerate(lengths):
        want = (vals[i].astype(np.float64).sum(axis=0) + tv[i]) / (n + 1)
        want = want.reshape(kv_heads, dim)
        for h in range(heads):
            assert np.allclose(got[i, h], want[h // group], rtol=1e-6, atol=1e-6), (i, n, h)


@pytest.mark.parametrize("dim,kv_heads,group", [(64, 8, 4), (64, 3, 3), (128, 8, 4), (64, 2, 8), (128, 2, 3),
                                                (32, 4, 2), (64, 1, 16)])
def test_wave_split_chunks_count_every_token(device, oracle, dim, kv_heads, group):
    # Launches of at most 32 (row, KV head) pairs run wave splits: one
    # workgroup per pair when a row is short, else chunks of one memory round
    # trip a wave whose partials the merge kernel combines.  q = 0 and integer
    # V make every output the exact mean of the row's V rows and its tail, so
    # a token dropped or counted twice by a chunk boundary, an empty trailing
    # chunk (rows shorter than the longest) or the tail's early request shows
    # (the bar is 1e-6, a token moves the mean by at least 1/(2n)).
    heads, tpb = kv_heads * group, 16
    vkv = kv_heads * (2 if group > 8 else 1)  # groups above eight run as two slices
    for lengths in ([8192], [1], [40], [700], [2049, 31, 600, 8192, 1, 5000][:max(1, 32 // vkv)]):
        g = (1, kv_heads, dim, tpb, sum((n + tpb - 1) // tpb for n in lengths) + 4)
        dev = device.PagedCache(*g)
        w = kv_heads * dim
        rng = np.random.default_rng(7 * dim + kv_heads + group + len(lengths))
        seqs, vals = [], []
        for i, n in enumerate(lengths):
            v = rng.integers(-4, 5, size=(n, w)).astype(np.float32)
            s = dev.create_sequence()
            dev.append_many(s, synth.normal(17, f"k{i}", n * w).reshape(n, w), v)
            seqs.append(s)
            vals.append(v)
        rows = len(lengths)
        tv = rng.integers(-4, 5, size=(rows, w)).astype(np.float32)
        tk = synth.normal(17, "tk", rows * w).reshape(rows, w)
        plan = attention.DecodePlan(dev, seqs, heads, 1 << 20, with_tail=True)
        say("wave-split chunks", dim, kv_heads, group, lengths, "items", plan.items, "split", plan.split_tokens)
        if max(lengths) == 8192 and dim * group <= 512:
            assert plan.items > 8 * rows  # several chunks a row
        got = attention.decode_batch(dev, np.zeros((rows, heads * dim), np.float32), seqs, 0, heads, 1 << 20,
                                     tail_keys=tk, tail_values=tv).reshape(rows, heads, dim)
        for i, n in enumerate(lengths):
            want = ((vals[i].astype(np.float64).sum(axis=0) + tv[i]) / (n + 1)).reshape(kv_heads, dim)
            for h in range(heads):
                assert np.allclose(got[i, h], want[h // group], rtol=1e-6, atol=1e-6), (lengths, i, h)


@pytest.mark.parametrize("dim,kv_heads,group", [(64, 8, 4), (128, 8, 4), (64, 3, 3), (64, 2, 7)])
@pytest.mark.parametrize("length", [33, 700, 2048, 8192])
def test_wave_split_chunks_against_reference(device, oracle, dim, kv_heads, group, length):
    # one row (the single-sequence model step) with its tail, N(0,1) inputs,
    # through one or many chunks, against the oracle within the f32 bar
    say("wave-split row", dim, kv_heads, group, length)
    got, want = _single(device, oracle, kv_heads * group, kv_heads, dim, 16, length, seed=length + dim, tail=True)
    assert refmath.close(got, want, TOL), refmath.max_rel(got, want)
