"""Paged chunked-prefill attention on the GPU against the oracle's
fused_prompt_attention (attention.hpp:85-89, FP64).

f32 path: |gpu - ref| <= 1e-4 * (1 + |ref|).

f32x3 path (the MFMA tiles with every operand split as hi + lo and three
products, hi*hi + hi*lo + lo*hi): the score operands q*log2(e)/sqrt(d) and K
as fp16 parts (22 significant bits), V and the probabilities as bf16 parts
(16 bits), the dropped lo*lo term below 2^-16 of its product, so every
rounding term below shrinks by 2^7 or more against the bf16 path: the
short-row worst case becomes ~8e-2 / 128 ~ 6e-4 at |ref| ~ 5, within the f32
bar's 1e-4 * (1 + |ref|), and the long rows sit two orders below it.  The
f32 bar applies.

bf16 MFMA path.  q*log2(e)/sqrt(d), K, V and the probabilities P are rounded
to bf16 (unit roundoff u = 2^-9); products and sums are f32.  To first order
the output error of one row is
    sum_t w_t * (dv_t + v_t * dp_t + (v_t - o) * ds_t)
with |dv_t| <= u|v_t|, |dp_t| <= u, and a score error ds_t (natural-log units)
that is a sum of d independent rounding terms, so its standard deviation is
    sigma_s = u / sqrt(3) * sqrt(2 * sum_i (q_i k_i)^2) / sqrt(d)  ~ 2^-9 * 0.8
for N(0,1) inputs at d = 64.  The three terms are independent across keys:
  * a row with few visible keys keeps them whole: with |v| <= 5 (the largest of
    ~10^6 N(0,1) draws) and |v - o| <= 10, a 4-sigma score error gives
    10 * 4 * 1.6e-3 + 2 * 5 * u ~ 8e-2 in the worst element, and the batch RMS
    is ~ |v| * sigma_s ~ 2e-3;
  * a row of the chunked-prefill shape sees >= 2,049 keys; N(0,1) scores give
    n_eff = n / e >= 750 effective keys, so every term shrinks by
    1/sqrt(n_eff) < 0.04: the worst element stays below 1e-2 and the RMS below
    1e-3.
Bars: short rows  max |gpu - ref| <= 8e-2 * (1 + |ref|), RMS <= 2e-3;
      long rows   max |gpu - ref| <= 1e-2 * (1 + |ref|), RMS <= 1e-3.
"""

import sys

import numpy as np
import pytest

import refmath
from tvara_amd import attention, synth, workloads

pytestmark = pytest.mark.gpu
TOL_F32 = 1e-4
SHORT_ROWS = (8e-2, 2e-3)
LONG_ROWS = (1e-2, 1e-3)


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def bf16_ok(got, want, bars):
    d = np.asarray(got, np.float64) - np.asarray(want, np.float64)
    rms = float(np.sqrt(np.mean(d * d)))
    return refmath.close(got, want, bars[0]) and rms <= bars[1], (refmath.max_rel(got, want), rms)


def build(device, oracle, heads, kv_heads, dim, specs, seed, tpb=16, q8=False):
    """specs: (cached tokens, chunk start, chunk rows) per sequence.  q8: Q8_0
    blocks, with the oracle holding the dequantised values."""
    nb = sum((n + tpb - 1) // tpb for n, _, _ in specs) + 4
    dev = device.PagedCache(1, kv_heads, dim, tpb, nb, fmt=device.Q8_0 if q8 else device.F32)
    ref = oracle.Cache(1, kv_heads, dim, tpb, nb)
    w = kv_heads * dim
    ds, rs, qs = [], [], []
    for i, (n, start, rows) in enumerate(specs):
        k = synth.normal(seed, f"k{i}", n * w).reshape(n, w)
        v = synth.normal(seed, f"v{i}", n * w).reshape(n, w)
        if q8:
            k = oracle.dequantize_q8_0(oracle.quantize_q8_0(k)).reshape(n, w)
            v = oracle.dequantize_q8_0(oracle.quantize_q8_0(v)).reshape(n, w)
        sd, sr = dev.create_sequence(), ref.create_sequence()
        dev.append_many(sd, k, v)
        ref.append_many(sr, k, v)
        ds.append(sd)
        rs.append(sr)
        qs.append(synth.normal(seed, f"q{i}", rows * heads * dim).reshape(rows, heads * dim))
    return dev, ref, ds, rs, qs


@pytest.mark.parametrize("fmt", ["f32", "q8_0"])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("group", [1, 2, 3, 4, 5, 6, 7, 8, 10, 16])  # 10, 16: slices of 5 and 8 heads
def test_bf16_small_shapes(device, oracle, group, dim, fmt):
    heads, kv_heads = 2 * group, 2
    specs = [(137, 100, 37), (64, 0, 64), (20, 3, 17)]
    say("prefill bf16 group", group, "dim", dim, fmt)
    dev, ref, ds, rs, qs = build(device, oracle, heads, kv_heads, dim, specs, seed=group, q8=fmt == "q8_0")
    starts = [s for _, s, _ in specs]
    counts = [r for _, _, r in specs]
    got = attention.prefill_batch(dev, np.concatenate(qs), ds, starts, counts, 0, heads, 4096, precision="bf16")
    f32 = attention.prefill_batch(dev, np.concatenate(qs), ds, starts, counts, 0, heads, 4096, precision="f32")
    want = np.concatenate([ref.fused_prompt_attention(q, s, 0, st, c, heads, 4096).reshape(c, -1)
                           for q, s, st, c in zip(qs, rs, starts, counts)])
    assert refmath.close(f32, want, TOL_F32), refmath.max_rel(f32, want)
    ok, err = bf16_ok(got, want, SHORT_ROWS)
    assert ok, err


@pytest.mark.parametrize("fmt", ["f32", "q8_0"])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("tpb", [32, 64, 128, 1024])
def test_bf16_block_sizes(device, oracle, tpb, dim, fmt):
    """Blocks above 16 tokens: a 64-key tile lies inside one block (tpb >= 64)
    or spans several (32); at 128 and 1,024 a block holds several tiles, so a
    key's slot depends on the tile index as well as its row."""
    heads, kv_heads = 8, 2
    specs = [(1100, 900, 200), (300, 0, 300), (20, 3, 17)]
    say("prefill bf16 tpb", tpb, "dim", dim, fmt)
    dev, ref, ds, rs, qs = build(device, oracle, heads, kv_heads, dim, specs, seed=tpb + dim, tpb=tpb,
                                 q8=fmt == "q8_0")
    starts = [s for _, s, _ in specs]
    counts = [r for _, _, r in specs]
    got = attention.prefill_batch(dev, np.concatenate(qs), ds, starts, counts, 0, heads, 4096, precision="bf16")
    f32 = attention.prefill_batch(dev, np.concatenate(qs), ds, starts, counts, 0, heads, 4096, precision="f32")
    want = np.concatenate([ref.fused_prompt_attention(q, s, 0, st, c, heads, 4096).reshape(c, -1)
                           for q, s, st, c in zip(qs, rs, starts, counts)])
    assert refmath.close(f32, want, TOL_F32), refmath.max_rel(f32, want)
    ok, err = bf16_ok(got, want, SHORT_ROWS)
    assert ok, err


@pytest.mark.parametrize("fmt", ["f32", "q8_0"])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("group", [1, 2, 3, 4, 5, 6, 7, 8, 10, 16])
def test_f32x3_small_shapes(device, oracle, group, dim, fmt):
    # Q8_0 blocks: d * q dequantised when staged, against the oracle over the
    # dequantised values the blocks hold
    heads, kv_heads = 2 * group, 2
    specs = [(137, 100, 37), (64, 0, 64), (20, 3, 17), (1, 0, 1)]
    say("prefill f32x3 group", group, "dim", dim, fmt)
    dev, ref, ds, rs, qs = build(device, oracle, heads, kv_heads, dim, specs, seed=50 + group, q8=fmt == "q8_0")
    starts = [s for _, s, _ in specs]
    counts = [r for _, _, r in specs]
    got = attention.prefill_batch(dev, np.concatenate(qs), ds, starts, counts, 0, heads, 4096, precision="f32x3")
    want = np.concatenate([ref.fused_prompt_attention(q, s, 0, st, c, heads, 4096).reshape(c, -1)
                           for q, s, st, c in zip(qs, rs, starts, counts)])
    say("f32x3 max rel", refmath.max_rel(got, want))
    assert refmath.close(got, want, TOL_F32), refmath.max_rel(got, want)


@pytest.mark.parametrize("fmt", ["f32", "q8_0"])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("tpb", [32, 64, 128, 1024])
def test_f32x3_block_sizes(device, oracle, tpb, dim, fmt):
    heads, kv_heads = 8, 2
    specs = [(1100, 900, 200), (300, 0, 300), (20, 3, 17)]
    say("prefill f32x3 tpb", tpb, "dim", dim, fmt)
    dev, ref, ds, rs, qs = build(device, oracle, heads, kv_heads, dim, specs, seed=60 + tpb + dim, tpb=tpb,
                                 q8=fmt == "q8_0")
    starts = [s for _, s, _ in specs]
    counts = [r for _, _, r in specs]
    got = attention.prefill_batch(dev, np.concatenate(qs), ds, starts, counts, 0, heads, 4096, precision="f32x3")
    want = np.concatenate([ref.fused_prompt_attention(q, s, 0, st, c, heads, 4096).reshape(c, -1)
                           for q, s, st, c in zip(qs, rs, starts, counts)])
    assert refmath.close(got, want, TOL_F32), refmath.max_rel(got, want)


@pytest.mark.parametrize("dim", [64, 128])
def test_f32x3_sharp_scores(device, oracle, dim):
    # queries and keys of N(0, 36) put the scores' standard deviation near 36:
    # a score's error enters the softmax's exponent unscaled, so score
    # operands carried in two bf16 parts (16 bits) leave 4.1e-4 on these rows
    # at d=64 (a float64 simulation of the split products), over the f32 bar;
    # with fp16 parts (22 bits) the same simulation gives 1.1e-5
    heads, kv_heads = 8, 2
    w = kv_heads * dim
    specs = [(700, 500, 200), (130, 0, 130)]
    nb = sum((n + 15) // 16 for n, _, _ in specs) + 4
    dev = device.PagedCache(1, kv_heads, dim, 16, nb)
    ref = oracle.Cache(1, kv_heads, dim, 16, nb)
    ds, rs, qs = [], [], []
    for i, (n, _, rows) in enumerate(specs):
        k = (6.0 * synth.normal(90, f"k{i}", n * w)).astype(np.float32).reshape(n, w)
        v = synth.normal(90, f"v{i}", n * w).reshape(n, w)
        sd, sr = dev.create_sequence(), ref.create_sequence()
        dev.append_many(sd, k, v)
        ref.append_many(sr, k, v)
        ds.append(sd)
        rs.append(sr)
        qs.append((6.0 * synth.normal(90, f"q{i}", rows * heads * dim)).astype(np.float32).reshape(rows, -1))
    starts = [s for _, s, _ in specs]
    counts = [r for _, _, r in specs]
    say("prefill f32x3 sharp", dim)
    got = attention.prefill_batch(dev, np.concatenate(qs), ds, starts, counts, 0, heads, 4096, precision="f32x3")
    want = np.concatenate([ref.fused_prompt_attention(q, s, 0, st, c, heads, 4096).reshape(c, -1)
                           for q, s, st, c in zip(qs, rs, starts, counts)])
    say("f32x3 sharp max rel", refmath.max_rel(got, want))
    assert refmath.close(got, want, TOL_F32), refmath.max_rel(got, want)


def test_f32x3_refusals(device):
    # the three-product tiles take the bf16 tiles' shapes: head_dim 64 or 128
    # and power-of-two blocks of 16 to 1,024 tokens; the f32 rows take the rest
    for dim, tpb in [(32, 16), (64, 24)]:
        dev = device.PagedCache(1, 2, dim, tpb, 8, fmt=device.Q8_0)
        s = dev.create_sequence()
        x = synth.normal(1, "x", 20 * 2 * dim).reshape(20, -1)
        dev.append_many(s, x, x)
        q = synth.normal(1, "q", 4 * 4 * dim).reshape(4, -1)
        with pytest.raises(device.InvalidArgument):
            attention.prefill_batch(dev, q, [s], [10], [4], 0, 4, 64, precision="f32x3")
        assert np.isfinite(attention.prefill_batch(dev, q, [s], [10], [4], 0, 4, 64, precision="f32")).all()


def bf16_rne(x):
    """float32 -> the nearest bfloat16 (ties to even), as float32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("tpb", [16, 64])
@pytest.mark.parametrize("fmt", ["f32", "q8_0"])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("group", [1, 4, 8])
def test_bf16_against_bf16_operands(device, oracle, group, dim, fmt, tpb):
    """The MFMA path against the FP64 oracle run on the operands the kernel
    actually multiplies: K and V rounded to bf16 (Q8_0: d * q rounded), and
    the query bf16(q * log2(e)/sqrt(d)) carried back to natural units.  The
    scores then agree to f32 summation error, and what is left is the bf16
    rounding of the probabilities, p~ = p (1 + e), |e| <= u = 2^-9, which
    enters numerator and normaliser alike:
        |o~ - o| = |sum w e (v - o)| / (1 + sum w e) <= u (max|v| + |o|) / (1 - u).
    A dropped or duplicated key in a short row, a wrong scale or a stale
    running maximum breaks this bound by far."""
    heads, kv_heads = 2 * group, 2
    specs = [(137, 100, 37), (64, 0, 64), (20, 3, 17), (300, 250, 50)]
    say("prefill bf16 operands group", group, "dim", dim, fmt, "tpb", tpb)
    nb = sum((n + tpb - 1) // tpb for n, _, _ in specs) + 4
    q8 = fmt == "q8_0"
    dev = device.PagedCache(1, kv_heads, dim, tpb, nb, fmt=device.Q8_0 if q8 else device.F32)
    ref = oracle.Cache(1, kv_heads, dim, tpb, nb)
    w, seed = kv_heads * dim, 100 + group + dim + tpb
    qscale = np.float32(1.4426950408889634 / np.sqrt(float(dim)))
    ds, rs, qs, qo, vmax = [], [], [], [], 0.0
    for i, (n, start, rows) in enumerate(specs):
        k = synth.normal(seed, f"k{i}", n * w).reshape(n, w)
        v = synth.normal(seed, f"v{i}", n * w).reshape(n, w)
        kr, vr = k, v
        if q8:
            kr = oracle.dequantize_q8_0(oracle.quantize_q8_0(k)).reshape(n, w)
            vr = oracle.dequantize_q8_0(oracle.quantize_q8_0(v)).reshape(n, w)
        kr, vr = bf16_rne(kr), bf16_rne(vr)
        vmax = max(vmax, float(np.abs(vr).max()))
        sd, sr = dev.create_sequence(), ref.create_sequence()
        dev.append_many(sd, k, v)
        ref.append_many(sr, kr, vr)
        ds.append(sd)
        rs.append(sr)
        q = synth.normal(seed, f"q{i}", rows * heads * dim).reshape(rows, heads * dim)
        qs.append(q)
        qb = bf16_rne((q * qscale).astype(np.float32))
        qo.append((qb.astype(np.float64) * np.sqrt(float(dim)) / 1.4426950408889634).astype(np.float32))
    starts = [s for _, s, _ in specs]
    counts = [r for _, _, r in specs]
    got = attention.prefill_batch(dev, np.concatenate(qs), ds, starts, counts, 0, heads, 4096, precision="bf16")
    want = np.concatenate([ref.fused_prompt_attention(q, s, 0, st, c, heads, 4096).reshape(c, -1)
                           for q, s, st, c in zip(qo, rs, starts, counts)])
    u = 2.0 ** -9
    bound = u * (vmax + np.abs(want).astype(np.float64)) / (1 - u) + 1e-5
    err = np.abs(np.asarray(got, np.float64) - want)
    assert np.all(err <= bound), (float((err / bound).max()), float(err.max()))
    say("bf16 operands: worst error / bound", float((err / bound).max()), "max error", float(err.max()))


@pytest.mark.parametrize("make,fmt", [(workloads.prefill_c4, "f32"), (workloads.prefill_8b, "f32"),
                                      (workloads.prefill_c4, "q8_0")], ids=["d64", "d128", "d64-q8_0"])
def test_bf16_c4_shape(device, oracle, make, fmt):
    w = make()
    say("prefill", w.name, fmt)
    g = (1, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks())
    q8 = fmt == "q8_0"
    dev, ref = device.PagedCache(*g, fmt=device.Q8_0 if q8 else device.F32), oracle.Cache(*g)
    ds = workloads.fill_prefill(dev, w)
    q = np.concatenate([w.chunk_queries(i) for i in range(w.sequences)])
    got = attention.prefill_batch(dev, q, ds, [w.prefix] * w.sequences, [w.chunk] * w.sequences, 0, w.heads,
                                  w.context, precision="bf16").reshape(w.sequences, w.chunk, -1)
    f32 = attention.prefill_batch(dev, q, ds, [w.prefix] * w.sequences, [w.chunk] * w.sequences, 0, w.heads,
                                  w.context, precision="f32").reshape(w.sequences, w.chunk, -1)
    # every 37th row and the last, 24 seeded random rows per sequence, and a
    # seeded run of 256 consecutive rows (whole query tiles) in one sequence
    rng = np.random.default_rng(4242)
    run_seq, run_at = int(rng.integers(w.sequences)), int(rng.integers(w.chunk - 256 + 1))
    want, gsel, fsel = [], [], []
    for i in range(w.sequences):
        rows = sorted(set(range(0, w.chunk, 37)) | {w.chunk - 1} |
                      set(rng.choice(w.chunk, 24, replace=False).tolist()))
        s = ref.create_sequence()
        k, v = w.keys(i), w.values(i)
        if q8:  # the oracle holds the dequantised values the Q8_0 blocks store
            k = oracle.dequantize_q8_0(oracle.quantize_q8_0(k)).reshape(k.shape)
            v = oracle.dequantize_q8_0(oracle.quantize_q8_0(v)).reshape(v.shape)
        ref.append_many(s, k, v)
        qi = w.chunk_queries(i)
        for r in rows:
            want.append(ref.fused_prompt_attention(qi[r], s, 0, w.prefix + r, 1, w.heads, w.context))
            gsel.append(got[i, r])
            fsel.append(f32[i, r])
        if i == run_seq:
            run = ref.fused_prompt_attention(qi[run_at:run_at + 256], s, 0, w.prefix + run_at, 256, w.heads,
                                             w.context).reshape(256, -1)
            want.extend(run)
            gsel.extend(got[i, run_at:run_at + 256])
            fsel.extend(f32[i, run_at:run_at + 256])
        ref.drop(s)
    want = np.stack(want)
    assert refmath.close(np.stack(fsel), want, TOL_F32), refmath.max_rel(np.stack(fsel), want)
    ok, err = bf16_ok(np.stack(gsel), want, LONG_ROWS)
    assert ok, err
    say("c4 bf16 vs oracle (max rel, rms):", err)
    # over the whole batch the bf16 path tracks the f32 path
    ok, err = bf16_ok(got, f32, LONG_ROWS)
    assert ok, err
    say("c4 bf16 vs f32 path (max rel, rms):", err)


@pytest.mark.parametrize("make,fmt", [(workloads.prefill_c4, "f32"), (workloads.prefill_8b, "f32"),
                                      (workloads.prefill_c4, "q8_0")], ids=["d64", "d128", "d64-q8_0"])
def test_c4_every_row_against_reference(device, oracle, ref, make, fmt):
    # every one of the batch's 8 x 512 rows, on both paths, against the
    # reference's own fused_prompt_attention (attention.hpp:85-89, built from
    # its sources in oracle/_ref) run over the same K/V on the host's threads:
    # the f32 path within the f32 bar, the bf16 path within its derived bars
    import os

    w = make()
    say("prefill every row", w.name, fmt)
    g = (1, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks())
    q8 = fmt == "q8_0"
    dev = device.PagedCache(*g, fmt=device.Q8_0 if q8 else device.F32)
    ds = workloads.fill_prefill(dev, w)
    q = np.concatenate([w.chunk_queries(i) for i in range(w.sequences)])
    args = (ds, [w.prefix] * w.sequences, [w.chunk] * w.sequences, 0, w.heads, w.context)
    got = attention.prefill_batch(dev, q, *args, precision="bf16").reshape(w.sequences, w.chunk, -1)
    f32 = attention.prefill_batch(dev, q, *args, precision="f32").reshape(w.sequences, w.chunk, -1)
    x3 = attention.prefill_batch(dev, q, *args, precision="f32x3").reshape(f32.shape)
    threads = max(1, min(16, os.cpu_count() or 1))
    rc = ref.RefCache(*g)
    want = np.empty_like(f32)
    for i in range(w.sequences):
        k, v = w.keys(i), w.values(i)
        if q8:  # the reference holds the dequantised values the Q8_0 blocks store
            k = oracle.dequantize_q8_0(oracle.quantize_q8_0(k)).reshape(k.shape)
            v = oracle.dequantize_q8_0(oracle.quantize_q8_0(v)).reshape(v.shape)
        s = rc.create_sequence()
        rc.append_many(s, k, v)
        want[i] = rc.prompt_batch(w.chunk_queries(i), s, 0, w.prefix, w.chunk, w.heads, w.context, 16,
                                  threads).reshape(w.chunk, -1)
        rc.drop(s)
    assert refmath.close(f32, want, TOL_F32), refmath.max_rel(f32, want)
    ok, err = bf16_ok(got, want, LONG_ROWS)
    assert ok, err
    say("every row: f32 max rel", refmath.max_rel(f32, want), "bf16 (max rel, rms)", err)
    say("every row: f32x3 max rel", refmath.max_rel(x3, want))
    assert refmath.close(x3, want, TOL_F32), refmath.max_rel(x3, want)


@pytest.mark.parametrize("precision", ["bf16", "f32", "f32x3"])
def test_prefill_plan_matches_call(device, oracle, precision):
    # a resident plan launched on two layers gives the one-shot call's bytes,
    # and refuses to run once the cache has changed
    from tvara_amd import hip

    heads, kv_heads, dim = 8, 2, 64
    specs = [(137, 100, 37), (64, 0, 64), (20, 3, 17)]
    g = (2, kv_heads, dim, 16, 40)
    dev = device.PagedCache(*g)
    w = 2 * kv_heads * dim
    ds, qs = [], []
    for i, (n, _, rows) in enumerate(specs):
        s = dev.create_sequence()
        dev.append_many(s, synth.normal(9, f"k{i}", n * w).reshape(n, w), synth.normal(9, f"v{i}", n * w).reshape(n, w))
        ds.append(s)
        qs.append(synth.normal(9, f"q{i}", rows * heads * dim).reshape(rows, heads * dim))
    q = np.concatenate(qs)
    starts, counts = [st for _, st, _ in specs], [r for _, _, r in specs]
    plan = attention.PrefillPlan(dev, ds, starts, counts, heads, 4096, precision)
    dq, out = hip.DeviceArray.from_numpy(q), hip.DeviceArray(q.shape)
    for layer in (1, 0):
        want = attention.prefill_batch(dev, q, ds, starts, counts, layer, heads, 4096, precision=precision)
        out.zero()
        plan.launch(layer, dq.ptr, out.ptr)
        plan.check()
        assert np.array_equal(out.numpy(), want.reshape(q.shape))
    dev.append(ds[0], synth.normal(9, "x", w), synth.normal(9, "y", w))
    with pytest.raises(device.InvalidArgument):
        plan.launch(0, dq.ptr, out.ptr)


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("group", [1, 4])
def test_bf16_nan_poisoned_unused_slots(device, oracle, group, dim):
    # prefill_t174.cpp for the MFMA path: NaN in the unused slots of the last
    # block (past the cached length, inside the last 64-key tile) never reaches
    # a row; chunks that end at the cache end, 16-key boundaries and mid-block
    heads, kv_heads = 2 * group, 2
    w = kv_heads * dim
    for n, rows in [(137, 37), (33, 33), (80, 16), (1, 1)]:
        say("prefill bf16 poison", group, dim, n, rows)
        dev = device.PagedCache(1, kv_heads, dim, 16, n // 16 + 3)
        ref = oracle.Cache(1, kv_heads, dim, 16, n // 16 + 3)
        k = synth.normal(21, "k", n * w).reshape(n, w)
        v = synth.normal(21, "v", n * w).reshape(n, w)
        sd, sr = dev.create_sequence(), ref.create_sequence()
        dev.append_many(sd, k, v)
        ref.append_many(sr, k, v)
        h = dev.physical_block(sd, n - 1)
        for slot in range(n % 16 or 16, 16):
            for kind in (0, 1):
                dev.block_write(h, dev.kv_offset(0, kind, slot), np.full(w, np.nan, np.float32))
        q = synth.normal(21, "q", rows * heads * dim).reshape(rows, heads * dim)
        got = attention.prefill_batch(dev, q, [sd], [n - rows], [rows], 0, heads, 4096, precision="bf16")
        want = ref.fused_prompt_attention(q, sr, 0, n - rows, rows, heads, 4096).reshape(rows, -1)
        assert np.isfinite(got).all()
        ok, err = bf16_ok(got.reshape(rows, -1), want, SHORT_ROWS)
        assert ok, err


def test_bf16_rejections(device):
    dev = device.PagedCache(1, 2, 32, 16, 8)
    s = dev.create_sequence()
    x = synth.normal(1, "x", 20 * 64).reshape(20, 64)
    dev.append_many(s, x, x)
    q = synth.normal(1, "q", 4 * 4 * 32)
    with pytest.raises(device.InvalidArgument):  # bf16 tile kernels cover head_dim 64 and 128
        attention.prefill_batch(dev, q, [s], [10], [4], 0, 4, 64, precision="bf16")
    dev = device.PagedCache(1, 2, 64, 16, 8)
    s = dev.create_sequence()
    x = synth.normal(1, "x", 20 * 128).reshape(20, 128)
    dev.append_many(s, x, x)
    q = synth.normal(1, "q", 4 * 4 * 64).reshape(4, -1)
    q[1, 3] = np.inf
    with pytest.raises(device.InvalidArgument):  # non-finite input
        attention.prefill_batch(dev, q, [s], [10], [4], 0, 4, 64, precision="bf16")
    with pytest.raises(device.InvalidArgument):  # chunk past the cached tokens
        attention.prefill_batch(dev, q, [s], [18], [4], 0, 4, 64, precision="bf16")
    q[1, 3] = 0.0
    for tpb in (8, 24):  # bf16 tile kernels take power-of-two blocks of 16 to 1,024 tokens
        dev = device.PagedCache(1, 2, 64, tpb, 8)
        s = dev.create_sequence()
        dev.append_many(s, x, x)
        with pytest.raises(device.InvalidArgument):
            attention.prefill_batch(dev, q, [s], [10], [4], 0, 4, 64, precision="bf16")
        f32 = attention.prefill_batch(dev, q, [s], [10], [4], 0, 4, 64, precision="f32")
        assert np.all(np.isfinite(f32))


@pytest.mark.parametrize("dim", [64, 128])
def test_x3_range(device, dim):
    # f32x3 carries queries and keys as fp16 parts: a visible key beyond the
    # fp16 range (65,504), or a query beyond it once multiplied by
    # log2(e)/sqrt(head_dim) (1e6 at both widths), makes scores non-finite and
    # the launch fails as a non-finite input does; the f32 rows take the same
    # inputs
    heads, kv_heads = 4, 2
    w = kv_heads * dim
    x = synth.normal(2, "x", 20 * w).reshape(20, w)
    q = synth.normal(2, "q", 4 * heads * dim).reshape(4, -1)
    for where in ("key", "query"):
        dev = device.PagedCache(1, kv_heads, dim, 16, 8)
        s = dev.create_sequence()
        k, qq = x.copy(), q.copy()
        if where == "key":
            k[5, 7] = 7e4
        else:
            qq[2, dim + 3] = -1e6
        dev.append_many(s, k, x)
        say("prefill x3 range", dim, where)
        with pytest.raises(device.InvalidArgument):
            attention.prefill_batch(dev, qq, [s], [10], [4], 0, heads, 4096, precision="f32x3")
        f32 = attention.prefill_batch(dev, qq, [s], [10], [4], 0, heads, 4096, precision="f32")
        assert np.isfinite(f32).all()
        # within the range the launch goes through
        k[5, 7], qq[2, dim + 3] = 6e4, -6e4
        dev.block_write(dev.physical_block(s, 5), dev.kv_offset(0, 0, 5), k[5])
        got = attention.prefill_batch(dev, qq, [s], [10], [4], 0, heads, 4096, precision="f32x3")
        assert np.isfinite(got).all()


@pytest.mark.parametrize("precision", ["bf16", "f32", "f32x3"])
@pytest.mark.parametrize("dim", [64, 128])
def test_chunk_invariant_under_future_tokens(device, precision, dim):
    # prefill_t173.cpp:6: tokens appended after a chunk (here huge and NaN
    # values, in the chunk's last block and in new blocks) leave the chunk's
    # rows byte-identical
    heads, kv_heads, tpb = 8, 2, 16
    w = kv_heads * dim
    dev = device.PagedCache(1, kv_heads, dim, tpb, 24)
    s = dev.create_sequence()
    n, start, rows = 150, 110, 40
    dev.append_many(s, synth.normal(41, "k", n * w).reshape(n, w), synth.normal(41, "v", n * w).reshape(n, w))
    q = synth.normal(41, "q", rows * heads * dim).reshape(rows, heads * dim)
    before = attention.prefill_batch(dev, q, [s], [start], [rows], 0, heads, 4096, precision=precision)
    junk = np.full((60, w), 3e4, np.float32)
    junk[::3] = np.nan
    dev.append_many(s, junk, junk)
    after = attention.prefill_batch(dev, q, [s], [start], [rows], 0, heads, 4096, precision=precision)
    assert np.isfinite(before).all()
    assert np.array_equal(before, after)


@pytest.mark.parametrize("precision", ["bf16", "f32", "f32x3"])
@pytest.mark.parametrize("fmt", ["f32", "q8_0"])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("group", [1, 3, 4, 8, 12])
def test_zero_query_averages_every_visible_key(device, oracle, group, dim, fmt, precision):
    # With q = 0 every score is 0, every probability exp2(0) = 1 exactly, and
    # with V of integers (exact in bf16, Q8_0 and every f32 partial sum) each
    # output row is the exact mean of the V rows its causal mask admits.
    # A dropped or repeated key moves the mean by at least 1/(2n) of a unit,
    # far above the 1e-6 bar, so the mask boundary of every row, the chunk
    # tiling, the GQA row mapping and the paged block walk are checked exactly
    # (the bf16 bars above cannot see a single key among thousands).  The f32
    # path (decode kernels, split merges) is exact here too.
    heads, kv_heads = 2 * group, 2
    w = kv_heads * dim
    specs = [(1100, 1000, 100), (300, 0, 300), (77, 60, 17), (2100, 1600, 500)]
    nb = sum((n + 15) // 16 for n, _, _ in specs) + 4
    q8 = fmt == "q8_0"
    dev = device.PagedCache(1, kv_heads, dim, 16, nb, fmt=device.Q8_0 if q8 else device.F32)
    ref = oracle.Cache(1, kv_heads, dim, 16, nb)
    rng = np.random.default_rng(83 + group + dim)
    ds, rs, vals = [], [], []
    for i, (n, _, _) in enumerate(specs):
        k = synth.normal(83, f"k{i}", n * w).reshape(n, w)
        # integers (exact in bf16); one 127 per 32-column group makes the
        # Q8_0 scale exactly 1, so the blocks hold the same integers
        v = rng.integers(-4, 5, size=(n, w)).astype(np.float32)
        v[:, ::32] = 127.0
        if q8:
            k = oracle.dequantize_q8_0(oracle.quantize_q8_0(k)).reshape(n, w)
            assert np.array_equal(oracle.dequantize_q8_0(oracle.quantize_q8_0(v)).reshape(n, w), v)
        sd, sr = dev.create_sequence(), ref.create_sequence()
        dev.append_many(sd, k, v)
        ref.append_many(sr, k, v)
        ds.append(sd)
        rs.append(sr)
        vals.append(v)
    starts = [s for _, s, _ in specs]
    counts = [r for _, _, r in specs]
    rows = sum(counts)
    q = np.zeros((rows, heads * dim), np.float32)
    say("prefill zero query", group, dim, fmt, precision)
    got = attention.prefill_batch(dev, q, ds, starts, counts, 0, heads, 4096, precision=precision)
    got = got.reshape(rows, heads, dim)
    at = 0
    for i, (n, start, cnt) in enumerate(specs):
        csum = np.cumsum(vals[i].reshape(n, kv_heads, dim).astype(np.float64), axis=0)
        for r in range(cnt):
            want = csum[start + r] / (start + r + 1)  # keys 0 .. start + r
            for h in range(heads):
                assert np.allclose(got[at + r, h], want[h // group], rtol=1e-6, atol=1e-6), (i, r, h)
        at += cnt


def _every_kernel(monkeypatch, run):
    """run() under TVARA_PREFILL_PIPE = 0 (prefill_bf16_kernel) and 1 (the
    software-pipelined kernel)."""
    out = []
    for flag in ("0", "1"):
        monkeypatch.setenv("TVARA_PREFILL_PIPE", flag)
        out.append(run())
    monkeypatch.delenv("TVARA_PREFILL_PIPE")
    return out


def _same_bits(plain, *others):
    return all(np.array_equal(plain.view(np.uint32), o.view(np.uint32)) for o in others)


@pytest.mark.parametrize("make,fmt", [(workloads.prefill_c4, "f32"), (workloads.prefill_c4, "q8_0"),
                                      (workloads.prefill_8b, "f32")], ids=["d64", "d64-q8_0", "d128"])
def test_pipelined_kernel_matches_plain_kernel(device, monkeypatch, make, fmt):
    """The pipelined kernels perform the plain kernel's products, exponentials
    and rescales in the same order, so the whole chunked-prefill batch must
    agree bit for bit (the plain kernel is pinned to the oracle above)."""
    w = make()
    say("pipelined vs plain prefill", w.name, fmt)
    g = (1, w.kv_heads, w.head_dim, w.tokens_per_block, w.pool_blocks())
    dev = device.PagedCache(*g, fmt=device.Q8_0 if fmt == "q8_0" else device.F32)
    ds = workloads.fill_prefill(dev, w)
    q = np.concatenate([w.chunk_queries(i) for i in range(w.sequences)])
    plain, pipe = _every_kernel(monkeypatch, lambda: attention.prefill_batch(
        dev, q, ds, [w.prefix] * w.sequences, [w.chunk] * w.sequences, 0, w.heads, w.context, precision="bf16"))
    assert np.isfinite(plain).all()
    assert _same_bits(plain, pipe)


@pytest.mark.parametrize("tpb", [16, 32, 1024])
@pytest.mark.parametrize("group", [1, 3, 4, 8])
def test_pipelined_kernel_ragged_chunks(device, oracle, monkeypatch, group, tpb):
    """Ragged chunks (a row alone, chunks ending inside a tile, a chunk with no
    cached prefix, odd and even tile counts) through every kernel: equal bits,
    and the pipelined ones within the short-row bars of the oracle."""
    heads, kv_heads, dim = 2 * group, 2, 64
    specs = [(1, 0, 1), (65, 64, 1), (200, 137, 63), (129, 0, 129), (700, 300, 400)]
    say("pipelined prefill ragged, group", group, "tpb", tpb)
    dev, ref, ds, rs, qs = build(device, oracle, heads, kv_heads, dim, specs, seed=31 + group, tpb=tpb)
    starts = [s for _, s, _ in specs]
    counts = [r for _, _, r in specs]
    plain, pipe = _every_kernel(monkeypatch, lambda: attention.prefill_batch(
        dev, np.concatenate(qs), ds, starts, counts, 0, heads, 4096, precision="bf16"))
    assert _same_bits(plain, pipe)
    want = np.concatenate([ref.fused_prompt_attention(q, s, 0, st, c, heads, 4096).reshape(c, -1)
                           for q, s, st, c in zip(qs, rs, starts, counts)])
    ok, err = bf16_ok(pipe, want, SHORT_ROWS)
    assert ok, err
