// Paged decode attention for gfx950: fused_paged_attention
// (core/include/tvara/attention.hpp:57-83) over f32 or Q8_0 blocks.
//
// Work decomposition.  A row (one query vector with `heads` heads) walks its
// sequence's block table.  The host cuts each row's cached tokens into splits
// of `split_tokens`; one workgroup handles one split for a group of KV heads,
// one wave per KV head.  Within a wave, LPT lanes share one token (a "token
// group") and each lane owns E = head_dim / LPT consecutive-in-memory columns,
// so one dwordx4 per lane reads whole 64-128 byte row segments and the whole
// workgroup streams contiguous 2 KiB slot rows of a block.  The G query heads
// of a GQA group are evaluated on every K/V element loaded (the reference
// re-reads the rows once per query head, attention.hpp:72).
//
// Softmax.  Scores are in log2 units (q is pre-scaled by log2(e)/sqrt(d)).
// Each lane keeps the running maximum of its head slot; the accumulators are
// only rescaled when a score exceeds the running maximum by more than
// kThreshold, so exp2(s - m) stays below 2^kThreshold and the rescale runs a
// handful of times per split instead of once per tile.
//
// Splits are merged by log-sum-exp: in merge_kernel / merge_wave_kernel, or
// for launches of at most 128 workgroups in the last workgroup of each row
// (merge_row_splits).  A non-finite score sets *err, matching
// OnlineAttention::update's rejection (attention.hpp:11).
#include <algorithm>
#include <cstdlib>
#include <string>
#include <type_traits>

#include "common.hpp"
#include "q8.hpp"
#include "device_util.hpp"

namespace tvara_amd {
namespace {

constexpr float kThreshold = 8.0f;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// K/V rows (non-temporal loads measured no faster on MI355X)
__device__ __forceinline__ float4 stream_load(const float* p) { return *reinterpret_cast<const float4*>(p); }

// Transpose-reduce: lane c of every LPT-lane group returns the sum over the
// group of v[c].  Pairings use DPP (quad permutes, half-row mirror).
template <int LPT>
__device__ __forceinline__ float transpose_reduce(const float (&v)[LPT], int c);

template <>
__device__ __forceinline__ float transpose_reduce<4>(const float (&v)[4], int c) {
    const bool b2 = (c & 2) != 0, b1 = (c & 1) != 0;
    const float r0 = (b2 ? v[2] : v[0]) + dpp<0x4E>(b2 ? v[0] : v[2]);
    const float r1 = (b2 ? v[3] : v[1]) + dpp<0x4E>(b2 ? v[1] : v[3]);
    return (b1 ? r1 : r0) + dpp<0xB1>(b1 ? r0 : r1);
}

template <>
__device__ __forceinline__ float transpose_reduce<8>(const float (&v)[8], int c) {
    const bool b4 = (c & 4) != 0;
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = (b4 ? v[i + 4] : v[i]) + dpp<0x141>(b4 ? v[i] : v[i + 4]);
    return transpose_reduce<4>(r, c & 3);
}

// Sixteen-lane groups (a DPP row, head_dim 256): lane c pairs with 15 - c
// (row_mirror), which holds the other half of columns, then the eight-lane
// reduce finishes within each half-row.
template <>
__device__ __forceinline__ float transpose_reduce<16>(const float (&v)[16], int c) {
    const bool b8 = (c & 8) != 0;
    float r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (b8 ? v[i + 8] : v[i]) + dpp<0x140>(b8 ? v[i] : v[i + 8]);
    return transpose_reduce<8>(r, c & 7);
}

// value of lane (token group base + h)
template <int LPT>
__device__ __forceinline__ float group_bcast(float v, int h, int lane);

template <>
__device__ __forceinline__ float group_bcast<4>(float v, int h, int) {
    switch (h) {
        case 0: return dpp<0x00>(v);
        case 1: return dpp<0x55>(v);
        case 2: return dpp<0xAA>(v);
        default: return dpp<0xFF>(v);
    }
}

// Eight-lane groups: broadcast lane h%4 within every quad, then copy the
// quad that holds lane h onto the other quad of its group (row_shr:4 writes
// banks 1 and 3 from banks 0 and 2; row_shl:4 the reverse).
template <>
__device__ __forceinline__ float group_bcast<8>(float v, int h, int) {
    const int b = __builtin_bit_cast(int, group_bcast<4>(v, h & 3, 0));
    if (h < 4) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(b, b, 0x114, 0xF, 0xA, false));
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(b, b, 0x104, 0xF, 0x5, false));
}

// Sixteen-lane groups: row_newbcast broadcasts lane h of every row
template <>
__device__ __forceinline__ float group_bcast<16>(float v, int h, int) {
    switch (h) {
        case 0: return dpp<0x150>(v);
        case 1: return dpp<0x151>(v);
        case 2: return dpp<0x152>(v);
        case 3: return dpp<0x153>(v);
        case 4: return dpp<0x154>(v);
        case 5: return dpp<0x155>(v);
        case 6: return dpp<0x156>(v);
        default: return dpp<0x157>(v);
    }
}

__device__ __forceinline__ float wave_max_across(float v, int from) {
    for (int o = from; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ float wave_sum_across(float v, int from) {
    for (int o = from; o < 64; o <<= 1) v += __shfl_xor(v, o);
    return v;
}

struct RowState {
    float m = -INFINITY;  // running max of this lane's head slot (log2 units)
    float l = 0.f;        // partial normaliser of this lane's head slot
    bool bad = false;
};

// Online-softmax update for one tile: `s` is this lane's full score for head
// slot c (valid when `own`); rescales acc when the maximum moves by more than
// kThreshold; returns p = exp2(s - m).
template <int G, int LPT, int E>
__device__ __forceinline__ float softmax_step(float s, bool own, int lane, RowState& st, float (&acc)[G][E]) {
    s = own ? s : -INFINITY;
    st.bad |= own && !__builtin_isfinite(s);
    const bool need = own && (s > st.m + kThreshold);
    if (__any(need)) {
        const float mnew = fmaxf(st.m, wave_max_across(s, LPT));
        const float alpha = (mnew == -INFINITY) ? 1.f : fast_exp2(st.m - mnew);
        st.m = mnew;
        st.l *= alpha;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float ah = group_bcast<LPT>(alpha, h, lane);
#pragma unroll
            for (int e = 0; e < E; ++e) acc[h][e] *= ah;
        }
    }
    const float p = own ? fast_exp2(s - st.m) : 0.f;
    st.l += p;
    return p;
}

// sum over the token groups of a wave that share head slot / column lane c
template <int LPT>
__device__ __forceinline__ float token_group_sum(float v) {
    v += dpp<0x128>(v);                          // row_ror:8
    if constexpr (LPT == 4) v += dpp<0x124>(v);  // row_ror:4
    return cross_row_sum(v);
}

// Reduce the token groups of a wave and write the split's result: the
// normalised output when the row has one split, otherwise the partial
// (acc, m, l) that merge_kernel combines.  `col(c, e4)` is the head-local
// column of lane slot c's e4-th float4.
// With a.row_done set, the last workgroup of a row's splits merges them in
// the same launch.  Each workgroup stores its partials with agent-scope
// relaxed atomic stores, waits for them (vmcnt counts stores on gfx9), and
// counts its split with one agent-scope acquire-release fetch_add.  On gfx950
// the release half writes the XCD's L2 back before the add, so the partials
// reach memory shared by all eight XCDs; the acquire half invalidates the
// finishing workgroup's L2 before it reads every partial with agent-scope
// loads.  The merge combines the splits in split order (the result does not
// depend on which workgroup finished last) and resets the counter for the
// next launch.  The L2 write-backs serialise across workgroups, so the
// launcher enables this only for launches of at most
// kInKernelMergeMaxWorkgroups workgroups, where it saves the second launch;
// larger launches take merge_kernel.
// Launches that share a plan must not overlap.
template <int D, int G>
__device__ __forceinline__ void merge_row_splits(const DecodeArgs& a, int lane, int kh, int first, int row,
                                                 int nsplit) {
    constexpr int U = 8;  // splits requested together
    const size_t head0 = static_cast<size_t>(kh) * G;
    float* out = a.out + (static_cast<size_t>(row) * a.heads + head0) * D;
    auto ld = [](const float* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    for (int o4 = lane; o4 < G * D / 4; o4 += 64) {
        const int h = (4 * o4) / D;
        float M = -INFINITY, L = 0.f;
        float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int s0 = 0; s0 < nsplit; s0 += U) {
            float m[U], l[U];
            float4 x[U];
#pragma unroll
            for (int k = 0; k < U; ++k) {
                const size_t it = static_cast<size_t>(first + min(s0 + k, nsplit - 1));
                const float* ml = a.part_ml + (it * a.heads + head0 + h) * 2;
                const float* pa = a.part_acc + (it * a.heads + head0) * D + 4 * o4;
                m[k] = ld(ml);
                l[k] = ld(ml + 1);
                x[k] = make_float4(ld(pa), ld(pa + 1), ld(pa + 2), ld(pa + 3));
            }
            float mc = M;
#pragma unroll
            for (int k = 0; k < U; ++k)
                if (s0 + k < nsplit) mc = fmaxf(mc, m[k]);
            const float sc = M == -INFINITY ? 0.f : fast_exp2(M - mc);
            L *= sc;
            sum.x *= sc;
            sum.y *= sc;
            sum.z *= sc;
            sum.w *= sc;
#pragma unroll
            for (int k = 0; k < U; ++k) {
                const float w = s0 + k < nsplit ? fast_exp2(m[k] - mc) : 0.f;
                L = fmaf(w, l[k], L);
                sum.x = fmaf(w, x[k].x, sum.x);
                sum.y = fmaf(w, x[k].y, sum.y);
                sum.z = fmaf(w, x[k].z, sum.z);
                sum.w = fmaf(w, x[k].w, sum.w);
            }
            M = mc;
        }
        const float inv = 1.f / L;
        *reinterpret_cast<float4*>(out + 4 * o4) = make_float4(sum.x * inv, sum.y * inv, sum.z * inv, sum.w * inv);
    }
}

template <int D, int G, int LPT, int E, bool kWS = false, class Col>
__device__ __forceinline__ void finish_split(const DecodeArgs& a, float (&acc)[G][E], RowState& st, int lane, int wave,
                                             int nwaves, int kh, int item, int first, int row, int nsplit, Col col) {
    extern __shared__ float lds[];
    const int c = lane & (LPT - 1);
    st.l = wave_sum_across(st.l, LPT);
    // token groups sharing a 16-lane row are summed with DPP row rotates, so
    // only the four row sums go through LDS
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < E; ++e) {
            float v = acc[h][e];
            if constexpr (LPT < 16) v += dpp<0x128>(v);  // row_ror:8
            if constexpr (LPT == 4) v += dpp<0x124>(v);  // row_ror:4
            acc[h][e] = v;
        }
    float* red = lds + static_cast<size_t>(wave) * 4 * G * D;
    float* ml = lds + static_cast<size_t>(nwaves) * 4 * G * D + wave * 2 * G;
    if ((lane & 15) < LPT) {
        const int row = lane >> 4;
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int e4 = 0; e4 < E / 4; ++e4)
                *reinterpret_cast<float4*>(red + (row * G + h) * D + col(c, e4)) =
                    make_float4(acc[h][4 * e4], acc[h][4 * e4 + 1], acc[h][4 * e4 + 2], acc[h][4 * e4 + 3]);
    }
    if (lane < G) {
        ml[c] = st.m;
        ml[G + c] = st.l;
    }
    __syncthreads();
    if constexpr (kWS) {
        // the waves hold consecutive splits of one (row, KV head): combine
        // their partials by log-sum-exp in split order, in LDS
        const float* ml0 = lds + static_cast<size_t>(nwaves) * 4 * G * D;
        float* outw = a.out + (static_cast<size_t>(row) * a.heads + static_cast<size_t>(kh) * G) * D;
        for (int o = static_cast<int>(threadIdx.x); o < G * D; o += static_cast<int>(blockDim.x)) {
            const int h = o / D;
            float M = -INFINITY;
            for (int w = 0; w < nwaves; ++w) M = fmaxf(M, ml0[w * 2 * G + h]);
            float L = 0.f, sum = 0.f;
            for (int w = 0; w < nwaves; ++w) {
                const float mw = ml0[w * 2 * G + h];
                const float wt = mw == -INFINITY ? 0.f : fast_exp2(mw - M);
                const float* r = lds + static_cast<size_t>(w) * 4 * G * D + o;
                L = fmaf(wt, ml0[w * 2 * G + G + h], L);
                sum = fmaf(wt, r[0] + r[G * D] + r[2 * G * D] + r[3 * G * D], sum);
            }
            if (a.ws_chunks > 1) {
                // the chunk's partial, [chunk][heads] (chunk = row * chunks +
                // c = blockIdx.x), for merge_wave_kernel or, with row_done
                // set, the row's last chunk in this launch (agent-scope
                // stores, as below)
                const size_t at = static_cast<size_t>(blockIdx.x) * a.heads + static_cast<size_t>(kh) * G + h;
                float* pa = a.part_acc + at * D + (o - h * D);
                if (a.row_done)
                    __hip_atomic_store(pa, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else
                    *pa = sum;
                if (o == h * D) {
                    if (a.row_done) {
                        __hip_atomic_store(a.part_ml + 2 * at, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        __hip_atomic_store(a.part_ml + 2 * at + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    } else {
                        a.part_ml[2 * at] = M;
                        a.part_ml[2 * at + 1] = L;
                    }
                }
            } else {
                outw[o] = sum / L;
            }
        }
        if (__any(st.bad) && lane == 0) *a.err = 1;
        if (a.ws_chunks > 1 && a.row_done) {
            // the (row, KV head)'s last chunk merges them all, in chunk order,
            // as the split merge below does
            __shared__ int last_chunk;
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __syncthreads();
            if (threadIdx.x == 0) {
                int* done = a.row_done + static_cast<size_t>(row) * a.lay.kv_heads + kh;
                const int prev = __hip_atomic_fetch_add(done, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
                last_chunk = prev == a.ws_chunks - 1;
                if (last_chunk) __hip_atomic_store(done, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();
            if (last_chunk && wave == 0) merge_row_splits<D, G>(a, lane, kh, row * a.ws_chunks, row, a.ws_chunks);
        }
        return;
    }
    const size_t head0 = static_cast<size_t>(kh) * G;
    float* out = a.out + (static_cast<size_t>(row) * a.heads + head0) * D;
    for (int o4 = lane; o4 < G * D / 4; o4 += 64) {
        float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float4 x = *reinterpret_cast<const float4*>(red + t * G * D + 4 * o4);
            sum.x += x.x;
            sum.y += x.y;
            sum.z += x.z;
            sum.w += x.w;
        }
        if (nsplit == 1) {
            const float l = ml[G + (4 * o4) / D];
            *reinterpret_cast<float4*>(out + 4 * o4) = make_float4(sum.x / l, sum.y / l, sum.z / l, sum.w / l);
        } else if (a.row_done) {
            float* p = a.part_acc + (static_cast<size_t>(item) * a.heads + head0) * D + 4 * o4;
            __hip_atomic_store(p, sum.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p + 1, sum.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p + 2, sum.z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p + 3, sum.w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            *reinterpret_cast<float4*>(a.part_acc + (static_cast<size_t>(item) * a.heads + head0) * D + 4 * o4) = sum;
        }
    }
    if (nsplit > 1 && lane < G) {
        float* o = a.part_ml + (static_cast<size_t>(item) * a.heads + head0 + lane) * 2;
        __hip_atomic_store(o, ml[lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(o + 1, ml[G + lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (__any(st.bad) && lane == 0) *a.err = 1;
    if (nsplit > 1 && a.row_done) {
        __shared__ int last;
        // every wave waits for its own partial stores (gfx9's vmcnt counts
        // stores) before the barrier; the signal fences keep the compiler
        // from moving a store past the wait
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __syncthreads();
        if (threadIdx.x == 0) {
            int* done = a.row_done + static_cast<size_t>(row) * (a.lay.kv_heads / nwaves) + kh / nwaves;
            // release publishes this workgroup's partials at device scope;
            // acquire orders the last arriver's reads of the others'
            const int prev = __hip_atomic_fetch_add(done, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            last = prev == nsplit - 1;
            if (last) __hip_atomic_store(done, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (last) merge_row_splits<D, G>(a, lane, kh, first, row, nsplit);
    }
}

// ------------------------------------------------------------- f32 blocks

// Above four query heads per KV head a workgroup has at most two waves and
// the query and accumulator registers alone (2 * G * D / LPT per lane) fill
// 256 VGPRs: the 128-thread bound lets the compiler keep the rest in AGPRs
// (one wave per SIMD) instead of scratch (Llama-3-70B shape, d=128: 120
// against 469 us; Q8_0 73 against 510 us).
//
// kWS (wave splits): a workgroup takes one (row, KV head) and its waves take
// the row's consecutive splits (the plan gives every row as many splits as
// the workgroup has waves), merged in LDS: no second launch and no global
// round trip, for launches too small to fill the GPU.
template <int D, int G, int LPT, int NB, bool kWS>
__global__ __launch_bounds__(G > 4 && !kWS ? 128 : 512) void decode_f32_kernel(
    const DecodeArgs a, const std::conditional_t<kWS, WsItems, WorkOrder> order) {
    constexpr int E = D / LPT, NV = E / 4, TT = 64 / LPT;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int groups = kWS ? 1 : a.lay.kv_heads / nwaves;
    // the launch order (a kernel argument, so no dependent load) maps this
    // workgroup to its work item
    const int slot = static_cast<int>(blockIdx.x) / groups;
    // wave splits: blockIdx.x is the (row, chunk), blockIdx.y the KV head
    int item;
    if constexpr (kWS)
        item = static_cast<int>(blockIdx.x) * nwaves + wave;
    else
        item = order.n ? static_cast<int>(order.item[slot]) : slot;
    const int kh = kWS ? static_cast<int>(blockIdx.y) : (static_cast<int>(blockIdx.x) % groups) * nwaves + wave;
    // the item's descriptor and block ids: from the kernel arguments (wave
    // splits of few items, at fixed strides so that no argument read comes
    // first), else in two independent loads
    bool inl = false;
    if constexpr (kWS) inl = order.n != 0;
    int4 it;  // row, first token, end token, tail | splits << 1
    int bids = 0;
    if constexpr (kWS) {
        if (inl) {
            const int at = static_cast<int>(blockIdx.x) * kWsInlineWaves + __builtin_amdgcn_readfirstlane(wave);
            it = order.item[at];
            bids = order.ids[at * kWsInlinePer + (lane & (kWsInlinePer - 1))];
        }
    }
    if (!inl) {
        it = a.work[item];
        bids = a.work_blocks[static_cast<size_t>(item) * kMaxSplitBlocks + lane];
    }
    const int nsplit = it.w >> 1;
    const bool tail = (it.w & 1) != 0;
    const int t0 = it.y, t1 = it.z;
    const int c = lane & (LPT - 1), tg = lane / LPT;
    const int kvw = a.lay.kv_width;

    float q[G][E];
    {
        const float* qr = a.q + (static_cast<size_t>(it.x) * a.heads + static_cast<size_t>(kh) * G) * D + 4 * c;
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int m = 0; m < NV; ++m) {
                // scaled in the score, not here: a use of q before the first
                // tile would make the prologue wait for every tile load
                const float4 x = *reinterpret_cast<const float4*>(qr + h * D + 4 * LPT * m);
                q[h][4 * m] = x.x;
                q[h][4 * m + 1] = x.y;
                q[h][4 * m + 2] = x.z;
                q[h][4 * m + 3] = x.w;
            }
    }
    // wave splits: the row's uncommitted K/V (attention.hpp:80) is requested
    // with the query, not after the last tile, so it costs no round trip of
    // its own
    const bool tok = tail && tg == 0;
    float4 tka[kWS ? NV : 1], tva[kWS ? NV : 1];
    if constexpr (kWS) {
        const size_t toff = static_cast<size_t>(it.x) * kvw + static_cast<size_t>(kh / a.kv_share) * D + 4 * c;
#pragma unroll
        for (int m = 0; m < NV; ++m) {
            tka[m] = tok ? *reinterpret_cast<const float4*>(a.tail_k + toff + 4 * LPT * m) : make_float4(0.f, 0.f, 0.f, 0.f);
            tva[m] = tok ? *reinterpret_cast<const float4*>(a.tail_v + toff + 4 * LPT * m) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    float acc[G][E];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[h][e] = 0.f;
    RowState st;

    const float* pool = reinterpret_cast<const float*>(a.pool);
    const size_t bstride = a.lay.stride / sizeof(float);
    // bids holds the split's block ids, one per lane (a split spans at most 64
    // blocks); a tile's id is read from the owning lane, so the loop issues no
    // table loads

    // blocks of tpb = 2^tsh tokens (16 to 1,024); a split starts on a block
    const int tpb = a.lay.tpb, tsh = __builtin_ctz(static_cast<unsigned>(tpb));
    const int kvh = kh / a.kv_share;  // the KV head whose K/V this (virtual) head reads
    const size_t koff = static_cast<size_t>(a.layer) * 2 * tpb * kvw + static_cast<size_t>(kvh) * D + 4 * c;
    const size_t voff = koff + static_cast<size_t>(tpb) * kvw;

    auto load = [&](int tb, float4 (&kk)[NV], float4 (&vv)[NV], bool ok) {
        const int bid = __builtin_amdgcn_readlane(bids, (tb - t0) >> tsh);
        const float* base =
            pool + static_cast<size_t>(bid) * bstride + static_cast<size_t>((tb & (tpb - 1)) + tg) * kvw;
#pragma unroll
        for (int m = 0; m < NV; ++m) {
            kk[m] = ok ? stream_load(base + koff + 4 * LPT * m) : make_float4(0.f, 0.f, 0.f, 0.f);
            vv[m] = ok ? stream_load(base + voff + 4 * LPT * m) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto process = [&](const float4 (&kk)[NV], const float4 (&vv)[NV], bool ok) {
        float part[LPT];
#pragma unroll
        for (int h = 0; h < LPT; ++h) part[h] = 0.f;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float s = 0.f;
#pragma unroll
            for (int m = 0; m < NV; ++m) {
                s = fmaf(q[h][4 * m], kk[m].x, s);
                s = fmaf(q[h][4 * m + 1], kk[m].y, s);
                s = fmaf(q[h][4 * m + 2], kk[m].z, s);
                s = fmaf(q[h][4 * m + 3], kk[m].w, s);
            }
            part[h] = s;
        }
        const float s = transpose_reduce<LPT>(part, c) * a.qscale;
        const float p = softmax_step<G, LPT, E>(s, ok && c < G, lane, st, acc);
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float ph = group_bcast<LPT>(p, h, lane);
#pragma unroll
            for (int m = 0; m < NV; ++m) {
                acc[h][4 * m] = fmaf(ph, vv[m].x, acc[h][4 * m]);
                acc[h][4 * m + 1] = fmaf(ph, vv[m].y, acc[h][4 * m + 1]);
                acc[h][4 * m + 2] = fmaf(ph, vv[m].z, acc[h][4 * m + 2]);
                acc[h][4 * m + 3] = fmaf(ph, vv[m].w, acc[h][4 * m + 3]);
            }
        }
    };

    // Full tiles stream with NB in flight (tile i+NB is requested as soon as
    // tile i is consumed) and unmasked loads; a partial last tile is masked.
    // The prefetches are unconditional: past the last full tile they re-read
    // it and the result is masked out.  (A conditional prefetch leaves a phi
    // at the join whose register copies wait for the load just issued.)
    const int nfull = max(t1 - t0, 0) / TT;
    if (nfull > 0) {
        const int last = nfull - 1;
        float4 kbuf[NB][NV], vbuf[NB][NV];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            load(t0 + min(j, last) * TT, kbuf[j], vbuf[j], true);
            asm volatile("" ::: "memory");  // issue order = use order
        }
        for (int i = 0; i < nfull; i += NB) {
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                process(kbuf[j], vbuf[j], i + j < nfull);
                load(t0 + min(i + j + NB, last) * TT, kbuf[j], vbuf[j], true);
                // keep the prefetch here: without this the compiler sinks it
                // past the next tile's wait and only one tile is in flight
                asm volatile("" ::: "memory");
            }
        }
    }
    float4 ka[NV], va[NV];
    if (t0 + nfull * TT < t1) {
        const bool ok = t0 + nfull * TT + tg < t1;
        load(t0 + nfull * TT, ka, va, ok);
        process(ka, va, ok);
    }
    if (tail) {  // the current token's uncommitted K/V is the last position (attention.hpp:80)
        if constexpr (kWS) {
            process(tka, tva, tok);
        } else {
            const bool ok = tg == 0;
            const float* tk = a.tail_k + static_cast<size_t>(it.x) * kvw + static_cast<size_t>(kvh) * D + 4 * c;
            const float* tv = a.tail_v + static_cast<size_t>(it.x) * kvw + static_cast<size_t>(kvh) * D + 4 * c;
#pragma unroll
            for (int m = 0; m < NV; ++m) {
                ka[m] = ok ? *reinterpret_cast<const float4*>(tk + 4 * LPT * m) : make_float4(0.f, 0.f, 0.f, 0.f);
                va[m] = ok ? *reinterpret_cast<const float4*>(tv + 4 * LPT * m) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
            process(ka, va, ok);
        }
    }
    finish_split<D, G, LPT, E, kWS>(a, acc, st, lane, wave, nwaves, kh, item, item - t0 / a.split_tokens, it.x,
                                    nsplit, [](int cc, int e4) { return 4 * cc + 4 * LPT * e4; });
}

// ------------------------------------- f32 blocks, row-major waves (head_dim 64)
//
// A workgroup of eight waves takes one work item for all of its KV heads
// (kv_heads = 4P, P = 1, 2 or 4) and reads each 16-token block in steps of
// 8 KiB of consecutive slot rows: load m of wave w covers floats
// [(8m + w) * 256, +256) of the block's K (and V) section, i.e. slot row
// m*R + w/P (R = 8/P rows a step, M = 2P loads per block and section) and
// the half-, quarter- or whole row of KV heads hb..hb+3, hb = 4 (w % P).
// Every workgroup-wide load is then one contiguous 8 KiB run (a 64 KiB block
// in eight K and eight V loads), which HBM serves at 6.3 TB/s where the
// head-major layout of decode_f32_kernel (16 strided 64-byte pieces a load)
// gets 5.9 TB/s (MI355X, the C2 block placement, loads without arithmetic).
//
// Lane l of a wave owns columns 4(l%16)..+3 of KV head hb + l/16 in every row
// it reads, so a DPP row (16 lanes) is one KV head.  A wave's R-way token
// phase w/P sees every R-th token of the item; the phases' softmax states
// are merged in LDS at the end of the item (log-sum-exp), by the phase-0
// waves, which write the output row or the split's partial.
//
// Scores: the lane's partial dots for (row, query head) pairs are
// transpose-reduced over the 16 lanes of the DPP row (row_mirror,
// row_half_mirror, quad permutes), so after four levels each lane holds the
// full score of one pair (VP = 16 pairs at a time; fewer pairs leave copies on
// neighbouring lanes).  Online softmax in log2 units with the lazy rescale of
// decode_f32_kernel; probabilities go back to the row with row_newbcast.

// DPP row_ror:d (0 < d < 16)
template <int D_>
__device__ __forceinline__ float row_ror(float v) {
    return dpp<0x120 + D_>(v);
}

// lane L of each DPP row receives lane L0 of that row
template <int L0>
__device__ __forceinline__ float row_bcast(float v) {
    return dpp<0x150 + L0>(v);
}

// lane L of each DPP row receives lane (j << SH) & 15 of that row (j folds to
// a constant once the caller's loops are unrolled)
template <int SH>
__device__ __forceinline__ float row_bcast_dyn(float v, int j) {
    switch ((j << SH) & 15) {
        case 0: return row_bcast<0>(v);
        case 1: return row_bcast<1>(v);
        case 2: return row_bcast<2>(v);
        case 3: return row_bcast<3>(v);
        case 4: return row_bcast<4>(v);
        case 5: return row_bcast<5>(v);
        case 6: return row_bcast<6>(v);
        case 7: return row_bcast<7>(v);
        case 8: return row_bcast<8>(v);
        case 9: return row_bcast<9>(v);
        case 10: return row_bcast<10>(v);
        case 11: return row_bcast<11>(v);
        case 12: return row_bcast<12>(v);
        case 13: return row_bcast<13>(v);
        case 14: return row_bcast<14>(v);
        default: return row_bcast<15>(v);
    }
}

// Pairing of the lanes of a DPP row that differ in lane bit BIT: row_mirror
// (bit 3), row_half_mirror (bit 2), quad permutes (bits 1 and 0).  Partners
// agree on every higher bit, so they hold the same values at each level.
template <int BIT>
constexpr int row_pair_ctrl() {
    return BIT == 8 ? 0x140 : BIT == 4 ? 0x141 : BIT == 2 ? 0x4E : 0xB1;
}

template <int N, int BIT>
__device__ __forceinline__ void row_sum_level(float (&a)[16], int i) {
    constexpr int C = row_pair_ctrl<BIT>();
    if constexpr (N > 1) {
        // keep this lane's half of the values, plus the partner's copy of it
        const bool up = (i & BIT) != 0;
#pragma unroll
        for (int j = 0; j < N / 2; ++j) a[j] = (up ? a[j + N / 2] : a[j]) + dpp<C>(up ? a[j] : a[j + N / 2]);
    } else {
        a[0] += dpp<C>(a[0]);
    }
    if constexpr (BIT > 1) row_sum_level<(N > 1 ? N / 2 : 1), BIT / 2>(a, i);
}

// Sum over the 16 lanes of a DPP row of N = 2^k values per lane (N <= 16):
// lane i of the row returns the sum of value i >> (4 - k).
template <int N>
__device__ __forceinline__ float row_transpose_sum(const float (&v)[N], int i) {
    float a[16];
#pragma unroll
    for (int j = 0; j < N; ++j) a[j] = v[j];
    row_sum_level<N, 8>(a, i);
    return a[0];
}

constexpr int pad_heads(int g) { return g == 1 ? 1 : g == 2 ? 2 : g <= 4 ? 4 : 8; }
constexpr int ilog2(int n) { return n <= 1 ? 0 : 1 + ilog2(n / 2); }

// LDS floats of a row-major decode workgroup: the partial accumulators and
// (max, normaliser) pairs of the token phases 1 .. R-1
__host__ __device__ constexpr size_t rows_lds_floats(int G, int P) {
    return static_cast<size_t>(8 / P - 1) * P * 4 * G * (64 + 2);
}

template <int G, int P, int NB>
__global__ __launch_bounds__(512) void decode_rows_kernel(const DecodeArgs a, const WorkOrder order) {
    constexpr int D = 64, R = 8 / P, M = 2 * P;
    constexpr int GP = pad_heads(G), LGP = ilog2(GP);
    constexpr int MC = M * GP <= 16 ? M : 16 / GP;  // block rows scored together
    constexpr int VP = MC * GP, SH = 4 - ilog2(VP);
    static_assert(M % MC == 0 && VP <= 16, "row-major decode: shape");
    extern __shared__ float lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = lane & 15, kvrow = lane >> 4, c0 = 4 * i;
    const int ph = wave / P, wp = wave % P, hb = wp * 4, kh = hb + kvrow;
    // the value this lane holds after a transpose-sum: (row mq of the chunk,
    // query head gq); `prim` marks the first of its copies
    const int jq = i >> SH, gq = jq % GP, mq = jq / GP;
    const bool prim = (i & ((1 << SH) - 1)) == 0;

    const int slot = static_cast<int>(blockIdx.x);
    const int item = order.n ? static_cast<int>(order.item[slot]) : slot;
    const int4 it = a.work[item];  // row, first token, end token, tail | splits << 1
    const int bids = a.work_blocks[static_cast<size_t>(item) * kMaxSplitBlocks + lane];
    const int nsplit = it.w >> 1;
    const bool tail = (it.w & 1) != 0;
    const int n = max(it.z - it.y, 0), nfull = n / 16;
    const int kvw = a.lay.kv_width;

    float q[G][4];
    {
        const float* qr = a.q + (static_cast<size_t>(it.x) * a.heads + static_cast<size_t>(kh) * G) * D + c0;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            // scaled in the score, not here (see decode_f32_kernel)
            const float4 x = *reinterpret_cast<const float4*>(qr + g * D);
            q[g][0] = x.x;
            q[g][1] = x.y;
            q[g][2] = x.z;
            q[g][3] = x.w;
        }
    }
    float acc[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[g][c] = 0.f;
    float ms = -INFINITY, ls = 0.f;  // this lane's query head gq (on prim lanes)
    bool bad = false;

    const float* pool = reinterpret_cast<const float*>(a.pool);
    const size_t bstride = a.lay.stride / sizeof(float);
    // blocks of tpb = 16 * 2^bsh tokens; the kernel's tiles are 16 rows
    const int tpb = a.lay.tpb, bsh = __builtin_ctz(static_cast<unsigned>(tpb)) - 4;
    const size_t kbase = static_cast<size_t>(a.layer) * 2 * tpb * kvw + static_cast<size_t>(ph) * kvw + hb * D + 4 * lane;
    const size_t vsec = static_cast<size_t>(tpb) * kvw, rstep = static_cast<size_t>(R) * kvw;

    // rows m*R + ph of a full block (unconditional loads: a select on a load
    // makes the compiler wait for it where the loop carries the registers)
    auto load = [&](const float* base, float4 (&kk)[M], float4 (&vv)[M]) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            kk[m] = stream_load(base + m * rstep);
            vv[m] = stream_load(base + vsec + m * rstep);
        }
    };
    // the same rows of a partial block: rows at or past `valid` read as zero
    auto load_part = [&](const float* base, float4 (&kk)[M], float4 (&vv)[M], int valid) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const bool ok = m * R + ph < valid;
            kk[m] = ok ? stream_load(base + m * rstep) : make_float4(0.f, 0.f, 0.f, 0.f);
            vv[m] = ok ? stream_load(base + vsec + m * rstep) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    // tile b: rows 16 (b mod 2^bsh) .. of the split's block b >> bsh
    auto block_base = [&](int b) __attribute__((always_inline)) {
        return pool + static_cast<size_t>(__builtin_amdgcn_readlane(bids, b >> bsh)) * bstride +
               static_cast<size_t>((b & ((1 << bsh) - 1)) * 16) * kvw + kbase;
    };
    auto process = [&](const float4 (&kk)[M], const float4 (&vv)[M], int valid) __attribute__((always_inline)) {
#pragma unroll
        for (int ch = 0; ch < M / MC; ++ch) {
            float part[VP];
#pragma unroll
            for (int mm = 0; mm < MC; ++mm)
#pragma unroll
                for (int g = 0; g < GP; ++g) {
                    float d = 0.f;
                    if (g < G) {
                        const float4 k = kk[ch * MC + mm];
                        d = fmaf(q[g][0], k.x, d);
                        d = fmaf(q[g][1], k.y, d);
                        d = fmaf(q[g][2], k.z, d);
                        d = fmaf(q[g][3], k.w, d);
                    }
                    part[mm * GP + g] = d;
                }
            float sc = row_transpose_sum<VP>(part, i) * a.qscale;
            const bool own = prim && gq < G && (ch * MC + mq) * R + ph < valid;
            sc = own ? sc : -INFINITY;
            bad |= own && !__builtin_isfinite(sc);
            if (__any(own && sc > ms + kThreshold)) {
                float mx = sc;
#pragma unroll
                for (int d = 1 << (SH + LGP); d < 16; d <<= 1) {
                    if (d == 1) mx = fmaxf(mx, row_ror<1>(mx));
                    if (d == 2) mx = fmaxf(mx, row_ror<2>(mx));
                    if (d == 4) mx = fmaxf(mx, row_ror<4>(mx));
                    if (d == 8) mx = fmaxf(mx, row_ror<8>(mx));
                }
                const float mnew = fmaxf(ms, mx);
                const float alpha = mnew == -INFINITY ? 1.f : fast_exp2(ms - mnew);
                ms = mnew;
                ls *= alpha;
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float ag = row_bcast_dyn<SH>(alpha, g);
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[g][c] *= ag;
                }
            }
            const float p = own ? fast_exp2(sc - ms) : 0.f;
            ls += p;
#pragma unroll
            for (int mm = 0; mm < MC; ++mm) {
                const float4 v = vv[ch * MC + mm];
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float pg = row_bcast_dyn<SH>(p, mm * GP + g);
                    acc[g][0] = fmaf(pg, v.x, acc[g][0]);
                    acc[g][1] = fmaf(pg, v.y, acc[g][1]);
                    acc[g][2] = fmaf(pg, v.z, acc[g][2]);
                    acc[g][3] = fmaf(pg, v.w, acc[g][3]);
                }
            }
        }
    };

    // full blocks, NB in flight; unconditional prefetches (past the last
    // full block they re-read it and the result is masked out), as in
    // decode_f32_kernel
    if (nfull > 0) {
        const int last = nfull - 1;
        float4 kb[NB][M], vb[NB][M];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            load(block_base(min(j, last)), kb[j], vb[j]);
            asm volatile("" ::: "memory");  // issue order = use order
        }
        for (int b = 0; b < nfull; b += NB) {
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                process(kb[j], vb[j], b + j < nfull ? 16 : 0);
                load(block_base(min(b + j + NB, last)), kb[j], vb[j]);
                asm volatile("" ::: "memory");  // keep the prefetch here
            }
        }
    }
    float4 ka[M], va[M];
    if (n > nfull * 16) {  // the partial last block: unused slots are never read
        load_part(block_base(nfull), ka, va, n - nfull * 16);
        process(ka, va, n - nfull * 16);
    }
    if (tail) {  // the row's uncommitted K/V is its last position (attention.hpp:80), row 0 of phase 0
        const size_t toff = static_cast<size_t>(it.x) * kvw + hb * D + 4 * lane;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const bool ok = m == 0 && ph == 0;
            ka[m] = ok ? *reinterpret_cast<const float4*>(a.tail_k + toff) : make_float4(0.f, 0.f, 0.f, 0.f);
            va[m] = ok ? *reinterpret_cast<const float4*>(a.tail_v + toff) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        process(ka, va, 1);
    }

    // the phases' states: normalisers summed over this row's token lanes,
    // phases 1 .. R-1 into LDS, combined by phase 0
    float lt = ls;
#pragma unroll
    for (int d = 1 << (SH + LGP); d < 16; d <<= 1) {
        if (d == 1) lt += row_ror<1>(lt);
        if (d == 2) lt += row_ror<2>(lt);
        if (d == 4) lt += row_ror<4>(lt);
        if (d == 8) lt += row_ror<8>(lt);
    }
    float* accs = lds;
    float* mls = lds + static_cast<size_t>(R - 1) * P * 4 * G * 64;
    if (ph > 0) {
        const int pw = ((ph - 1) * P + wp) * 4 + kvrow;
#pragma unroll
        for (int g = 0; g < G; ++g)
            *reinterpret_cast<float4*>(accs + (static_cast<size_t>(pw) * G + g) * 64 + c0) =
                make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
        if (prim && mq == 0 && gq < G) {
            mls[(pw * G + gq) * 2] = ms;
            mls[(pw * G + gq) * 2 + 1] = lt;
        }
    }
    __syncthreads();
    if (ph == 0) {
        const size_t head0 = static_cast<size_t>(kh) * G;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float m0 = row_bcast_dyn<SH>(ms, g), l0 = row_bcast_dyn<SH>(lt, g);
            float mx = m0;
#pragma unroll
            for (int r = 1; r < R; ++r) mx = fmaxf(mx, mls[((((r - 1) * P + wp) * 4 + kvrow) * G + g) * 2]);
            const float w0 = m0 == -INFINITY ? 0.f : fast_exp2(m0 - mx);
            float l = w0 * l0;
            float4 o = make_float4(w0 * acc[g][0], w0 * acc[g][1], w0 * acc[g][2], w0 * acc[g][3]);
#pragma unroll
            for (int r = 1; r < R; ++r) {
                const int pw = ((r - 1) * P + wp) * 4 + kvrow;
                const float mr = mls[(pw * G + g) * 2];
                const float wr = mr == -INFINITY ? 0.f : fast_exp2(mr - mx);
                l = fmaf(wr, mls[(pw * G + g) * 2 + 1], l);
                const float4 x = *reinterpret_cast<const float4*>(accs + (static_cast<size_t>(pw) * G + g) * 64 + c0);
                o.x = fmaf(wr, x.x, o.x);
                o.y = fmaf(wr, x.y, o.y);
                o.z = fmaf(wr, x.z, o.z);
                o.w = fmaf(wr, x.w, o.w);
            }
            if (nsplit == 1) {
                float* out = a.out + (static_cast<size_t>(it.x) * a.heads + head0 + g) * D + c0;
                *reinterpret_cast<float4*>(out) = make_float4(o.x / l, o.y / l, o.z / l, o.w / l);
            } else {
                *reinterpret_cast<float4*>(a.part_acc + (static_cast<size_t>(item) * a.heads + head0 + g) * D + c0) = o;
                if (i == 0) {
                    float* pm = a.part_ml + (static_cast<size_t>(item) * a.heads + head0 + g) * 2;
                    pm[0] = mx;
                    pm[1] = l;
                }
            }
        }
    }
    if (__any(bad) && lane == 0) *a.err = 1;
}

// ------------------------------------------------------------- Q8_0 blocks

__device__ __forceinline__ void unpack_i8(uint4 w, float (&f)[16]) {
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[4 * j] = sbyte_to_float<0>(words[j]);
        f[4 * j + 1] = sbyte_to_float<1>(words[j]);
        f[4 * j + 2] = sbyte_to_float<2>(words[j]);
        f[4 * j + 3] = sbyte_to_float<3>(words[j]);
    }
}

// Each lane owns 16 consecutive columns (one dwordx4 of int8) = half a Q8_0
// group, so a token's row of head_dim columns is LPT = head_dim/16 lanes.
template <int D, int G>  // launch bounds: as decode_f32_kernel
__global__ __launch_bounds__(G > 4 ? 128 : 512) void decode_q8_kernel(const DecodeArgs a) {
    constexpr int LPT = D / 16, TT = 64 / LPT, E = 16;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int groups = a.lay.kv_heads / nwaves;
    const int item = static_cast<int>(blockIdx.x) / groups;
    const int kh = (static_cast<int>(blockIdx.x) % groups) * nwaves + wave;
    // the item's descriptor and block ids come in two independent loads
    const int4 it = a.work[item];  // row, first token, end token, tail | splits << 1
    const int bids = a.work_blocks[static_cast<size_t>(item) * kMaxSplitBlocks + lane];
    const int nsplit = it.w >> 1;
    const bool tail = (it.w & 1) != 0;
    const int t0 = it.y, t1 = it.z;
    const int c = lane & (LPT - 1), tg = lane / LPT;
    const int kvw = a.lay.kv_width;

    float q[G][E];
    {
        const float* qr = a.q + (static_cast<size_t>(it.x) * a.heads + static_cast<size_t>(kh) * G) * D + 16 * c;
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const float4 x = *reinterpret_cast<const float4*>(qr + h * D + 4 * m);
                q[h][4 * m] = x.x * a.qscale;
                q[h][4 * m + 1] = x.y * a.qscale;
                q[h][4 * m + 2] = x.z * a.qscale;
                q[h][4 * m + 3] = x.w * a.qscale;
            }
    }
    float acc[G][E];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[h][e] = 0.f;
    RowState st;

    // bids holds the split's block ids, one per lane (a split spans at most 64
    // blocks); a tile's id is read from the owning lane, so the loop issues no
    // table loads

    const size_t sec = a.lay.section;
    const int kvh = kh / a.kv_share;  // the KV head whose K/V this (virtual) head reads
    const size_t qcol = static_cast<size_t>(kvh) * D + 16 * c;  // column in the f32 tail row
    // this head's run of the section: int8 [16][D], then fp16 scales [16][D/32]
    const size_t qoff = static_cast<size_t>(kvh) * a.lay.head_bytes + 16 * c;
    const size_t soff = static_cast<size_t>(kvh) * a.lay.head_bytes + 16 * D + (16 * c / 32) * 2;
    const size_t ksec = static_cast<size_t>(a.layer) * 2 * sec, vsec = ksec + sec;

    struct Tile {
        uint4 kq, vq;
        uint16_t ks, vs;
        bool ok;
    };
    auto load = [&](int tb, Tile& x, bool ok) {
        x.ok = ok;
        const int bid = __builtin_amdgcn_readlane(bids, (tb - t0) >> 4);
        const int slot = (tb & 15) + tg;
        const char* base = a.pool + static_cast<size_t>(bid) * a.lay.stride;
        if (ok) {
            x.kq = *reinterpret_cast<const uint4*>(base + ksec + qoff + static_cast<size_t>(slot) * D);
            x.vq = *reinterpret_cast<const uint4*>(base + vsec + qoff + static_cast<size_t>(slot) * D);
            x.ks = *reinterpret_cast<const uint16_t*>(base + ksec + soff + static_cast<size_t>(slot) * (D / 16));
            x.vs = *reinterpret_cast<const uint16_t*>(base + vsec + soff + static_cast<size_t>(slot) * (D / 16));
        } else {
            x.kq = x.vq = make_uint4(0, 0, 0, 0);
            x.ks = x.vs = 0;
        }
    };
    auto process_f = [&](const float (&kf)[16], float ks, const float (&vf)[16], float vs, bool ok) {
        float part[LPT];
#pragma unroll
        for (int h = 0; h < LPT; ++h) part[h] = 0.f;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) s = fmaf(q[h][e], kf[e], s);
            part[h] = s * ks;
        }
        const float s = transpose_reduce<LPT>(part, c);
        const float p = softmax_step<G, LPT, E>(s, ok && c < G, lane, st, acc);
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float w = group_bcast<LPT>(p, h, lane) * vs;
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[h][e] = fmaf(w, vf[e], acc[h][e]);
        }
    };
    auto process = [&](const Tile& x) {
        float kf[16], vf[16];
        unpack_i8(x.kq, kf);
        unpack_i8(x.vq, vf);
        process_f(kf, half_bits_to_float(x.ks), vf, half_bits_to_float(x.vs), x.ok);
    };

    // Two tiles in flight.  The prefetches are unconditional (past the last
    // full tile they re-read it and the result is masked out): a conditional
    // load lets the compiler pull the byte unpacking up to the load, which then
    // has to wait for the data at once.
    const int nfull = max(t1 - t0, 0) / TT;
    const int last = max(nfull - 1, 0);
    Tile ta, tb2;
    if (nfull > 0) {
        load(t0, ta, true);
        asm volatile("" ::: "memory");  // issue order = use order
        load(t0 + min(1, last) * TT, tb2, true);
        asm volatile("" ::: "memory");
    }
    for (int i = 0; i < nfull; i += 2) {
        process(ta);
        load(t0 + min(i + 2, last) * TT, ta, true);
        asm volatile("" ::: "memory");  // keep the prefetch ahead of the next tile's wait
        tb2.ok = i + 1 < nfull;
        process(tb2);
        load(t0 + min(i + 3, last) * TT, tb2, true);
        asm volatile("" ::: "memory");
    }
    if (t0 + nfull * TT < t1) {
        load(t0 + nfull * TT, ta, t0 + nfull * TT + tg < t1);
        process(ta);
    }
    if (tail) {  // the uncommitted token arrives as f32
        const bool ok = tg == 0;
        const float* tk = a.tail_k + static_cast<size_t>(it.x) * kvw + qcol;
        const float* tv = a.tail_v + static_cast<size_t>(it.x) * kvw + qcol;
        float kf[16], vf[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            kf[e] = ok ? tk[e] : 0.f;
            vf[e] = ok ? tv[e] : 0.f;
        }
        process_f(kf, 1.f, vf, 1.f, ok);
    }
    finish_split<D, G, LPT, E>(a, acc, st, lane, wave, nwaves, kh, item, item - t0 / a.split_tokens, it.x, nsplit,
                               [](int cc, int e4) { return 16 * cc + 4 * e4; });
}

// ------------------------------------------- Q8_0 blocks, scores on int8 MFMA
//
// The score side runs on the int8 matrix cores.  v_mfma_i32_16x16x32_i8
// multiplies a 16 x 32 int8 A by a 32 x 16 int8 B into exact int32 sums; lane
// l supplies row (A) or column (B) l%16 at k-slots 8(l/16)..+7 and receives
// rows 4(l/16)..+3 of column l%16.  One Q8_0 group (32 columns) is one k
// range, so each group's sums can take that group's scale d[t][g].
//   B: the raw int8 K bytes of 16 tokens (column = token).  A wave loads its
//      head's K run contiguously (16 bytes per lane) and restages it in LDS,
//      because the operand layout puts consecutive lanes on different tokens.
//   A: the query, split exactly into four base-128 int8 pieces,
//      x = q * 127 / max|q| = a0 + a1/128 + a2/128^2 + a3/128^3 (|a0| <= 127,
//      |aj| <= 64, remainder below 2^-22 of max|q|), one row per
//      (head h, piece j) = 4h + j.
// Lane (u, t) then holds the four pieces of head u for token t; the score is
// qscale * max|q_u|/127 * sum_g d[t][g] * sum_j 128^-j C_g[j], one score per
// lane (16 tokens x 4 heads per MFMA group).
//
// The value side stays on the vector ALUs in f32, as decode_q8_kernel: a
// 16-bit operand cannot carry p * d for every fp16 group scale d.  The
// weights w[t][g][h] = p[t][h] * dV[t][g] go from the score layout to the
// value layout (lane = token group x 16 columns) through LDS.  Against
// decode_q8_kernel this removes the K conversions and the G x head_dim f32
// products per token, about half of the vector instructions.

__device__ __forceinline__ float readlane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// max / sum over the 16 lanes of a DPP row (every lane receives the result)
__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dpp<0xB1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp<0x4E>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp<0x124>(v));  // row_ror:4
    return fmaxf(v, dpp<0x128>(v));  // row_ror:8
}

__device__ __forceinline__ float row_sum16(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x124>(v);
    return v + dpp<0x128>(v);
}

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// LDS bytes per wave: the K rows of a 32-token tile ([32][D + 16] int8) and
// the weights w[32 tokens][groups][4 heads]
template <int D>
constexpr size_t q8_mma_wave_lds() {
    return 32 * (D + 16) + 32 * (D / 32) * 4 * sizeof(float);
}

template <int D, int G>
__global__ __launch_bounds__(512) void decode_q8_mma_kernel(const DecodeArgs a) {
    constexpr int NG = D / 32;                      // Q8_0 groups per head row
    constexpr int LPT = D / 16, TT = 64 / LPT, E = 16;
    constexpr int VP = 32 / TT;                     // value passes per 32-token tile
    constexpr int KP = D / 64;                      // 16-byte K chunks per lane and block
    constexpr int KRS = D + 16;                     // LDS row of one token's K (padded against bank conflicts)
    static_assert(G >= 1 && G <= 4, "four query heads per KV head at most");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    // a wave takes G query heads of one KV head (q8_mma_heads): the group's
    // heads come in group / G slices over as many waves
    const int halves = a.group / G;
    const int groups = a.lay.kv_heads * halves / nwaves;
    const int item = static_cast<int>(blockIdx.x) / groups;
    const int slot = (static_cast<int>(blockIdx.x) % groups) * nwaves + wave;
    const int kh = slot / halves;
    const size_t qh0 = static_cast<size_t>(kh) * a.group + static_cast<size_t>(slot % halves) * G;  // first query head
    // the item's descriptor and block ids come in two independent loads
    const int4 it = a.work[item];  // row, first token, end token, tail | splits << 1
    const int bids = a.work_blocks[static_cast<size_t>(item) * kMaxSplitBlocks + lane];
    const int nsplit = it.w >> 1;
    const bool tail = (it.w & 1) != 0;
    const int t0 = it.y, t1 = it.z;
    const int n = max(t1 - t0, 0);
    const int kvw = a.lay.kv_width;
    const int u = lane >> 4, t16 = lane & 15;         // score layout: head u, token t16
    const int c = lane & (LPT - 1), tg = lane / LPT;  // value layout: token group, 16 columns

    extern __shared__ float lds[];
    char* kl = reinterpret_cast<char*>(lds) + static_cast<size_t>(wave) * q8_mma_wave_lds<D>();  // [32][D + 16] int8
    float* wl = reinterpret_cast<float*>(kl + 32 * KRS);  // [32 tokens][NG][4 heads]

    // query pieces: lane (u, r) holds piece r%4 of head r/4 at columns 32g + 8u .. +7
    long qa[NG];
    float wsc;  // qscale * max|q| / 127 of head u
    {
        const int hq = t16 >> 2, jp = t16 & 3;
        const bool hv = hq < G;
        const float* qr = a.q + (static_cast<size_t>(it.x) * a.heads + qh0 + (hv ? hq : 0)) * D;
        float qv[NG][8];
        float mx = 0.f;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const float4 x0 = hv ? *reinterpret_cast<const float4*>(qr + 32 * g + 8 * u) : make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 x1 = hv ? *reinterpret_cast<const float4*>(qr + 32 * g + 8 * u + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
            qv[g][0] = x0.x; qv[g][1] = x0.y; qv[g][2] = x0.z; qv[g][3] = x0.w;
            qv[g][4] = x1.x; qv[g][5] = x1.y; qv[g][6] = x1.z; qv[g][7] = x1.w;
#pragma unroll
            for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(qv[g][e]));
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float inv = mx > 0.f ? 127.f / mx : 0.f;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            uint32_t w[2] = {0u, 0u};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = qv[g][e] * inv;
                const float a0 = __builtin_rintf(x);
                float r = (x - a0) * 128.f;  // exact: |x - a0| <= 1/2, power-of-two scaling
                const float a1 = __builtin_rintf(r);
                r = (r - a1) * 128.f;
                const float a2 = __builtin_rintf(r);
                r = (r - a2) * 128.f;
                const float a3 = __builtin_rintf(r);
                const float pc = jp == 0 ? a0 : (jp == 1 ? a1 : (jp == 2 ? a2 : a3));
                w[e >> 2] |= (static_cast<uint32_t>(static_cast<int>(pc)) & 0xffu) << (8 * (e & 3));
            }
            qa[g] = static_cast<long>((static_cast<uint64_t>(w[1]) << 32) | w[0]);
        }
        // the max of head h sits in every lane whose row is 4h + j: take lane 4h
        const float m0 = readlane_f(mx, 0), m1 = readlane_f(mx, 4), m2 = readlane_f(mx, 8), m3 = readlane_f(mx, 12);
        const float mh = u == 0 ? m0 : (u == 1 ? m1 : (u == 2 ? m2 : m3));
        wsc = a.qscale * (mh / 127.f);
    }

    float acc[G][E];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[h][e] = 0.f;
    float mv = -INFINITY, lv = 0.f;  // head u's running max (row-uniform); this lane's share of the normaliser
    bool bad = false;

    const int nblk = (n + 15) >> 4;
    const size_t sec = a.lay.section;
    // this head's run of a section: int8 [16][D] then fp16 scales [16][NG]
    const int kvh = kh / a.kv_share;  // the KV head whose K/V this (virtual) head reads
    const size_t ksec = static_cast<size_t>(a.layer) * 2 * sec + static_cast<size_t>(kvh) * a.lay.head_bytes;
    const size_t vsec = ksec + sec;
    const size_t kcol = static_cast<size_t>(kvh) * D;  // column of the f32 tail row

    // Loads are contiguous: lane i takes bytes 16i (+1024m) of a head's int8
    // plane, and the 16 tokens' scales are one 16 * NG * 2 byte run.
    struct Tile {
        u32x4_t kq[2][KP];   // K int8 of each half, natural order (staged in LDS for the MFMA operand)
        uint2 ks[2], vs[2];  // the NG group scales of token t16 (K and V)
        uint4 vq[VP];        // value layout: token k * TT + tg, columns 16c .. +15
    };
    auto block_base = [&](int i, int b) {
        const int bid = __builtin_amdgcn_readlane(bids, min(2 * i + b, nblk - 1));
        return a.pool + static_cast<size_t>(bid) * a.lay.stride;
    };
    auto load = [&](Tile& x, int i) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const char* kb = block_base(i, b) + ksec;
            const char* vb = kb + sec;
#pragma unroll
            for (int m = 0; m < KP; ++m) x.kq[b][m] = *reinterpret_cast<const u32x4_t*>(kb + 1024 * m + 16 * lane);
            const size_t so = 16 * D + static_cast<size_t>(t16) * NG * 2;
            if constexpr (NG >= 4) {
                x.ks[b] = *reinterpret_cast<const uint2*>(kb + so);
                x.vs[b] = *reinterpret_cast<const uint2*>(vb + so);
            } else {
                x.ks[b] = make_uint2(*reinterpret_cast<const uint32_t*>(kb + so), 0u);
                x.vs[b] = make_uint2(*reinterpret_cast<const uint32_t*>(vb + so), 0u);
            }
        }
#pragma unroll
        for (int k = 0; k < VP; ++k) {
            const int b = (k * TT) >> 4;
            x.vq[k] = *reinterpret_cast<const uint4*>(block_base(i, b) + vsec + static_cast<size_t>((k * TT) & 15) * D +
                                                      16 * lane);
        }
    };
    auto scale_of = [](uint2 s, int g) {
        const uint32_t w = g < 2 ? s.x : s.y;
        return half_bits_to_float(static_cast<uint16_t>((g & 1) ? (w >> 16) : (w & 0xffffu)));
    };
    // online-softmax step for one row-uniform tile maximum tm of head u
    auto rescale = [&](float tm) {
        if (__any(tm > mv + kThreshold)) {
            const float mnew = fmaxf(mv, tm);
            const float alpha = (mnew == -INFINITY) ? 1.f : fast_exp2(mv - mnew);
            mv = mnew;
            lv *= alpha;
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float ah = readlane_f(alpha, 16 * h);
#pragma unroll
                for (int e = 0; e < E; ++e) acc[h][e] *= ah;
            }
        }
    };
    auto process = [&](const Tile& x, int i) {
        // K rows of both halves into LDS; lane (u, t) then reads its 8-byte k-slots of token t
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int m = 0; m < KP; ++m) {
                const int byte = 1024 * m + 16 * lane;
                *reinterpret_cast<u32x4_t*>(kl + (16 * b + byte / D) * KRS + byte % D) = x.kq[b][m];
            }
        float s[2];
        bool ok[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            float sc = 0.f;
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                const uint2 kv = *reinterpret_cast<const uint2*>(kl + (16 * b + t16) * KRS + 32 * g + 8 * u);
                i32x4_t r = {0, 0, 0, 0};
                r = __builtin_amdgcn_mfma_i32_16x16x32_i8(qa[g], __builtin_bit_cast(long, kv), r, 0, 0, 0);
                const float xg = fmaf(static_cast<float>(r[3]), 0x1p-21f,
                                      fmaf(static_cast<float>(r[2]), 0x1p-14f,
                                           fmaf(static_cast<float>(r[1]), 0x1p-7f, static_cast<float>(r[0]))));
                sc = fmaf(scale_of(x.ks[b], g), xg, sc);
            }
            sc *= wsc;
            ok[b] = (32 * i + 16 * b + t16 < n) && u < G;
            bad |= ok[b] && !__builtin_isfinite(sc);
            s[b] = ok[b] ? sc : -INFINITY;
        }
        rescale(row_max16(fmaxf(s[0], s[1])));
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const float p = ok[b] ? fast_exp2(s[b] - mv) : 0.f;
            lv += p;
#pragma unroll
            for (int g = 0; g < NG; ++g)
                wl[((16 * b + t16) * NG + g) * 4 + u] = ok[b] ? p * scale_of(x.vs[b], g) : 0.f;
        }
#pragma unroll
        for (int k = 0; k < VP; ++k) {
            const float4 w4 = *reinterpret_cast<const float4*>(wl + ((k * TT + tg) * NG + (c >> 1)) * 4);
            const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
            float vf[16];
            unpack_i8(x.vq[k], vf);
#pragma unroll
            for (int h = 0; h < G; ++h)
#pragma unroll
                for (int e = 0; e < E; ++e) acc[h][e] = fmaf(wv[h], vf[e], acc[h][e]);
        }
    };

    // Two tiles of 32 tokens (two blocks) in flight; prefetches past the last
    // tile re-read it, and a tile past the end is fully masked.
    const int ntiles = (n + 31) >> 5;
    if (ntiles > 0) {
        const int last = ntiles - 1;
        Tile ta, tb;
        load(ta, 0);
        asm volatile("" ::: "memory");
        load(tb, min(1, last));
        asm volatile("" ::: "memory");
        for (int i = 0; i < ntiles; i += 2) {
            process(ta, i);
            load(ta, min(i + 2, last));
            asm volatile("" ::: "memory");
            process(tb, i + 1);
            load(tb, min(i + 3, last));
            asm volatile("" ::: "memory");
        }
    }
    if (tail) {  // the uncommitted token arrives as f32 and is the last position (attention.hpp:80)
        constexpr int CPL = D / 16;
        float part = 0.f;
        if (u < G) {
            const float* qh = a.q + (static_cast<size_t>(it.x) * a.heads + qh0 + u) * D + t16 * CPL;
            const float* tk = a.tail_k + static_cast<size_t>(it.x) * kvw + kcol + t16 * CPL;
#pragma unroll
            for (int e = 0; e < CPL; ++e) part = fmaf(qh[e], tk[e], part);
        }
        float st = row_sum16(part) * a.qscale;
        const bool okt = u < G;
        bad |= okt && !__builtin_isfinite(st);
        st = okt ? st : -INFINITY;
        rescale(st);
        const float p = okt ? fast_exp2(st - mv) : 0.f;
        lv += t16 == 0 ? p : 0.f;
        float ph[G];
#pragma unroll
        for (int h = 0; h < G; ++h) ph[h] = readlane_f(p, 16 * h);
        if (tg == 0) {
            const float* tv = a.tail_v + static_cast<size_t>(it.x) * kvw + kcol + 16 * c;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float v = tv[e];
#pragma unroll
                for (int h = 0; h < G; ++h) acc[h][e] = fmaf(ph[h], v, acc[h][e]);
            }
        }
    }
    // Sum the token groups in registers (DPP within a 16-lane row, permlane
    // swaps across the four rows): lane c < LPT then holds columns 16c .. 16c+15 of
    // every head, so the split needs neither LDS nor a workgroup barrier.
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < E; ++e) {
            acc[h][e] = token_group_sum<LPT>(acc[h][e]);
        }
    const float lsum = row_sum16(lv);
    float mh[G], lh[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        mh[h] = readlane_f(mv, 16 * h);
        lh[h] = readlane_f(lsum, 16 * h);
    }
    const size_t head0 = qh0;
    if (lane < LPT) {
        float* dst = nsplit == 1 ? a.out + (static_cast<size_t>(it.x) * a.heads + head0) * D
                                 : a.part_acc + (static_cast<size_t>(item) * a.heads + head0) * D;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float sc = nsplit == 1 ? 1.f / lh[h] : 1.f;
#pragma unroll
            for (int e4 = 0; e4 < E / 4; ++e4)
                *reinterpret_cast<float4*>(dst + h * D + 16 * c + 4 * e4) =
                    make_float4(acc[h][4 * e4] * sc, acc[h][4 * e4 + 1] * sc, acc[h][4 * e4 + 2] * sc,
                                acc[h][4 * e4 + 3] * sc);
        }
    }
    if (nsplit > 1 && lane < G) {
        float m = mh[0], l = lh[0];
#pragma unroll
        for (int h = 1; h < G; ++h) {
            m = lane == h ? mh[h] : m;
            l = lane == h ? lh[h] : l;
        }
        float* o = a.part_ml + (static_cast<size_t>(item) * a.heads + head0 + lane) * 2;
        o[0] = m;
        o[1] = l;
    }
    if (__any(bad) && lane == 0) *a.err = 1;
}

// --------------------------------------------------- any shape (one wave per head)

__device__ __forceinline__ float element(const DecodeArgs& a, int block, int kind, int slot, int column) {
    const char* base = a.pool + static_cast<size_t>(block) * a.lay.stride;
    const int kvw = a.lay.kv_width;
    if (a.lay.format == kF32)
        return reinterpret_cast<const float*>(base)[(static_cast<size_t>(a.layer * 2 + kind) * a.lay.tpb + slot) * kvw +
                                                    column];
    const char* sec = base + static_cast<size_t>(a.layer * 2 + kind) * a.lay.section;
    const int8_t qv = reinterpret_cast<const int8_t*>(sec)[q8_byte_offset(a.lay, slot, column)];
    const uint16_t d = *reinterpret_cast<const uint16_t*>(sec + q8_scale_offset(a.lay, slot, column / 32));
    return half_bits_to_float(d) * static_cast<float>(qv);
}

constexpr int kGenericMaxDim = 512;

__global__ __launch_bounds__(64) void decode_generic_kernel(const DecodeArgs a) {
    __shared__ float qs[kGenericMaxDim];
    const int lane = threadIdx.x;
    const int h = blockIdx.y, kh = h / (a.group * a.kv_share);  // the KV head (group: a slice when kv_share > 1)
    const int D = a.lay.head_dim, kvw = a.lay.kv_width, tpb = a.lay.tpb;
    const int2 it = a.items[blockIdx.x];
    const int4 en = a.entries[it.x];
    const int nsplit = en.z >> 1;
    const bool tail = (en.z & 1) && it.y == nsplit - 1;
    const int t0 = it.y * a.split_tokens;
    const int t1 = min(t0 + a.split_tokens, en.y);
    const int ntok = max(t1 - t0, 0) + (tail ? 1 : 0);
    const int32_t* tab = a.tables + en.x;
    const float* qr = a.q + (static_cast<size_t>(it.x) * a.heads + h) * D;
    for (int d = lane; d < D; d += 64) qs[d] = qr[d] * a.qscale;
    __syncthreads();
    const float* tk = tail ? a.tail_k + static_cast<size_t>(it.x) * kvw + static_cast<size_t>(kh) * D : nullptr;
    const float* tv = tail ? a.tail_v + static_cast<size_t>(it.x) * kvw + static_cast<size_t>(kh) * D : nullptr;
    float m = -INFINITY, l = 0.f, acc[kGenericMaxDim / 64];
    for (int i = 0; i < kGenericMaxDim / 64; ++i) acc[i] = 0.f;
    bool bad = false;
    for (int base = 0; base < ntok; base += 64) {
        const int j = base + lane;
        const bool ok = j < ntok;
        float s = -INFINITY;
        if (ok) {
            s = 0.f;
            const int p = t0 + j;
            if (p < t1) {
                const int bid = tab[p / tpb], slot = p % tpb;
                for (int d = 0; d < D; ++d) s = fmaf(qs[d], element(a, bid, 0, slot, kh * D + d), s);
            } else {
                for (int d = 0; d < D; ++d) s = fmaf(qs[d], tk[d], s);
            }
            bad |= !__builtin_isfinite(s);
        }
        float mx = s;
        for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const float mnew = fmaxf(m, mx);
        const float alpha = (mnew == -INFINITY) ? 1.f : exp2f(m - mnew);
        const float pj = ok ? exp2f(s - mnew) : 0.f;
        float ps = pj;
        for (int o = 32; o >= 1; o >>= 1) ps += __shfl_xor(ps, o);
        l = l * alpha + ps;
        m = mnew;
        for (int i = 0; i < kGenericMaxDim / 64; ++i) acc[i] *= alpha;
        const int count = min(64, ntok - base);
        for (int jj = 0; jj < count; ++jj) {
            const float w = __shfl(pj, jj);
            const int p = t0 + base + jj;
            if (p < t1) {
                const int bid = tab[p / tpb], slot = p % tpb;
                for (int i = 0; i * 64 + lane < D; ++i)
                    acc[i] = fmaf(w, element(a, bid, 1, slot, kh * D + i * 64 + lane), acc[i]);
            } else {
                for (int i = 0; i * 64 + lane < D; ++i) acc[i] = fmaf(w, tv[i * 64 + lane], acc[i]);
            }
        }
    }
    if (nsplit == 1) {
        float* o = a.out + (static_cast<size_t>(it.x) * a.heads + h) * D;
        for (int i = 0; i * 64 + lane < D; ++i) o[i * 64 + lane] = acc[i] / l;
    } else {
        float* o = a.part_acc + (static_cast<size_t>(blockIdx.x) * a.heads + h) * D;
        for (int i = 0; i * 64 + lane < D; ++i) o[i * 64 + lane] = acc[i];
        if (lane == 0) {
            a.part_ml[(static_cast<size_t>(blockIdx.x) * a.heads + h) * 2] = m;
            a.part_ml[(static_cast<size_t>(blockIdx.x) * a.heads + h) * 2 + 1] = l;
        }
    }
    if (__any(bad) && lane == 0) *a.err = 1;
}

// ---------------------------------------------------------- split merge

// Log-sum-exp merge of a row's split partials, one 256-lane workgroup per
// (row, head).  The partial row of a split is cut into `nu` units of V floats;
// lane (r, u) takes unit u (and u + 64, ... when nu > 64) of splits r, r + R,
// ... where R = 256 / min(64, nu), U splits at a time with every load issued
// before the first is used, so a row of up to R * U splits costs one memory
// round trip.  Each lane keeps an online maximum over its splits; the R lanes
// of a unit are combined through LDS.
template <int V, int UPL, int U, bool kInline>
__global__ __launch_bounds__(256) void merge_kernel(const DecodeArgs a, const RowSplits rs) {
    using T = typename std::conditional<V == 4, float4, float>::type;
    __shared__ float sm[256], sl[256];
    __shared__ T sa[256][UPL];
    const int row = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int2 en = kInline ? rs.r[row] : make_int2(a.entries[row].w, a.entries[row].z >> 1);  // first item, splits
    const int nsplit = en.y;
    if (nsplit <= 1) return;
    const int D = a.lay.head_dim, nu = D / V;
    const int lpr = min(64, nu), R = 256 / lpr;
    const int u0 = lane % lpr, r = lane / lpr;
    const size_t step = static_cast<size_t>(a.heads);
    const float* ml = a.part_ml + (static_cast<size_t>(en.x) * step + h) * 2;
    const float* pa = a.part_acc + (static_cast<size_t>(en.x) * step + h) * D;

    auto zero = [] {
        if constexpr (V == 4) return make_float4(0.f, 0.f, 0.f, 0.f);
        else return 0.f;
    };
    auto axpy = [](float w, const T& x, T& y) {
        if constexpr (V == 4) {
            y.x = fmaf(w, x.x, y.x);
            y.y = fmaf(w, x.y, y.y);
            y.z = fmaf(w, x.z, y.z);
            y.w = fmaf(w, x.w, y.w);
        } else {
            y = fmaf(w, x, y);
        }
    };
    float M = -INFINITY, L = 0.f;
    T acc[UPL];
#pragma unroll
    for (int j = 0; j < UPL; ++j) acc[j] = zero();
    for (int s0 = 0; s0 < nsplit; s0 += R * U) {
        float m[U], l[U];
        T x[U][UPL];
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int sp = s0 + k * R + r;
            const bool ok = r < R && sp < nsplit;
            m[k] = ok ? ml[sp * step * 2] : -INFINITY;
            l[k] = ok ? ml[sp * step * 2 + 1] : 0.f;
#pragma unroll
            for (int j = 0; j < UPL; ++j) {
                const int u = u0 + 64 * j;
                x[k][j] = ok && u < nu ? *reinterpret_cast<const T*>(pa + sp * step * D + u * V) : zero();
            }
        }
        float mc = M;
#pragma unroll
        for (int k = 0; k < U; ++k) mc = fmaxf(mc, m[k]);
        if (mc != -INFINITY) {  // this lane holds a split
            const float sc = fast_exp2(M - mc);  // 0 while M is still -inf
            L *= sc;
#pragma unroll
            for (int j = 0; j < UPL; ++j) {
                T z = zero();
                axpy(sc, acc[j], z);
                acc[j] = z;
            }
#pragma unroll
            for (int k = 0; k < U; ++k) {
                const float w = fast_exp2(m[k] - mc);  // 0 for an empty slot
                L = fmaf(w, l[k], L);
#pragma unroll
                for (int j = 0; j < UPL; ++j) axpy(w, x[k][j], acc[j]);
            }
            M = mc;
        }
    }
    sm[lane] = M;
    sl[lane] = L;
#pragma unroll
    for (int j = 0; j < UPL; ++j) sa[lane][j] = acc[j];
    __syncthreads();
    if (r != 0) return;
    float Mt = M;
    for (int rr = 1; rr < R; ++rr) Mt = fmaxf(Mt, sm[rr * lpr + u0]);
    float Lt = 0.f;
    T at[UPL];
#pragma unroll
    for (int j = 0; j < UPL; ++j) at[j] = zero();
    for (int rr = 0; rr < R; ++rr) {
        const int src = rr * lpr + u0;
        const float w = sm[src] == -INFINITY ? 0.f : fast_exp2(sm[src] - Mt);
        Lt = fmaf(w, sl[src], Lt);
#pragma unroll
        for (int j = 0; j < UPL; ++j) axpy(w, sa[src][j], at[j]);
    }
    const float inv = 1.f / Lt;
    float* o = a.out + (static_cast<size_t>(row) * a.heads + h) * D;
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
        const int u = u0 + 64 * j;
        if (u >= nu) break;
        T y = zero();
        axpy(inv, at[j], y);
        *reinterpret_cast<T*>(o + u * V) = y;
    }
}

// The same merge with one wave per (row, head) and four heads per
// workgroup, for head_dim = 4 * LPR with LPR a power of two up to 64: lane
// (r, u) holds float4 u of splits r, r + R, ... (R = 64 / LPR), U of them
// per memory round trip, and the R slots combine by shuffles.
template <int LPR, int U, bool kInline>
__global__ __launch_bounds__(256) void merge_wave_kernel(const DecodeArgs a, const RowSplits rs) {
    constexpr int R = 64 / LPR, D = 4 * LPR;
    const int lane = threadIdx.x & 63, h = blockIdx.y * 4 + (threadIdx.x >> 6);
    const int row = blockIdx.x;
    if (h >= a.heads) return;
    // (first item, splits) of the row: from the kernel arguments when the
    // plan has few rows (no dependent load before the partials), else from HBM
    const int2 en = kInline ? rs.r[row] : make_int2(a.entries[row].w, a.entries[row].z >> 1);
    const int nsplit = en.y;
    if (nsplit <= 1) return;
    const int u = lane % LPR, r = lane / LPR;
    const size_t step = static_cast<size_t>(a.heads);
    const float* ml = a.part_ml + (static_cast<size_t>(en.x) * step + h) * 2;
    const float* pa = a.part_acc + (static_cast<size_t>(en.x) * step + h) * D;
    float M = -INFINITY, L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < nsplit; s0 += R * U) {
        float m[U], l[U];
        float4 x[U];
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int sp = s0 + k * R + r;
            const bool ok = sp < nsplit;
            m[k] = ok ? ml[sp * step * 2] : -INFINITY;
            l[k] = ok ? ml[sp * step * 2 + 1] : 0.f;
            x[k] = ok ? *reinterpret_cast<const float4*>(pa + sp * step * D + 4 * u) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        float mc = M;
#pragma unroll
        for (int k = 0; k < U; ++k) mc = fmaxf(mc, m[k]);
        if (mc != -INFINITY) {
            const float sc = fast_exp2(M - mc);  // 0 while M is still -inf
            L *= sc;
            acc.x *= sc;
            acc.y *= sc;
            acc.z *= sc;
            acc.w *= sc;
#pragma unroll
            for (int k = 0; k < U; ++k) {
                const float w = fast_exp2(m[k] - mc);  // 0 for an empty slot
                L = fmaf(w, l[k], L);
                acc.x = fmaf(w, x[k].x, acc.x);
                acc.y = fmaf(w, x[k].y, acc.y);
                acc.z = fmaf(w, x[k].z, acc.z);
                acc.w = fmaf(w, x[k].w, acc.w);
            }
            M = mc;
        }
    }
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) {
        const float Mo = __shfl_xor(M, off), Lo = __shfl_xor(L, off);
        const float4 ao = make_float4(__shfl_xor(acc.x, off), __shfl_xor(acc.y, off), __shfl_xor(acc.z, off),
                                      __shfl_xor(acc.w, off));
        const float Mt = fmaxf(M, Mo);
        const float w1 = M == -INFINITY ? 0.f : fast_exp2(M - Mt);
        const float w2 = Mo == -INFINITY ? 0.f : fast_exp2(Mo - Mt);
        L = fmaf(w1, L, w2 * Lo);
        acc.x = fmaf(w1, acc.x, w2 * ao.x);
        acc.y = fmaf(w1, acc.y, w2 * ao.y);
        acc.z = fmaf(w1, acc.z, w2 * ao.z);
        acc.w = fmaf(w1, acc.w, w2 * ao.w);
        M = Mt;
    }
    if (r) return;
    const float inv = 1.f / L;
    *reinterpret_cast<float4*>(a.out + (static_cast<size_t>(row) * a.heads + h) * D + 4 * u) =
        make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
}

template <bool kInline>
void launch_merge_t(const DecodeArgs& a, const RowSplits& rs, int nrows, hipStream_t s) {
    const int D = a.lay.head_dim;
    const dim3 grid(nrows, a.heads), block(256);
    // one wave per (row, head), four heads per workgroup (sixteen measured
    // no faster on the Llama-3.2-1B batch and slower on the Llama-3-8B one);
    // a wave requests 16 splits at d=64 and 32 at d=128 before using any, so
    // rows of up to that many splits cost one memory round trip (Llama-3-8B
    // batch, 32 splits a row: 4.5 against 4.8-4.9 us with 16 at d=128)
    const dim3 wgrid(nrows, (a.heads + 3) / 4), wblock(256);
    if (D == 64)
        launch("paged_decode_merge", merge_wave_kernel<16, 4, kInline>, wgrid, wblock, 0, s, a, rs);
    else if (D == 128)
        launch("paged_decode_merge", merge_wave_kernel<32, 16, kInline>, wgrid, wblock, 0, s, a, rs);
    else if (D == 256)
        launch("paged_decode_merge", merge_wave_kernel<64, 8, kInline>, wgrid, wblock, 0, s, a, rs);
    else if (D == 32)
        launch("paged_decode_merge", merge_wave_kernel<8, 4, kInline>, wgrid, wblock, 0, s, a, rs);
    else if (D % 4 == 0 && D <= 256)
        launch("paged_decode_merge", merge_kernel<4, 1, 8, kInline>, grid, block, 0, s, a, rs);
    else if (D % 4 == 0)
        launch("paged_decode_merge", merge_kernel<4, 2, 8, kInline>, grid, block, 0, s, a, rs);
    else
        launch("paged_decode_merge", merge_kernel<1, 8, 4, kInline>, grid, block, 0, s, a, rs);
}

void launch_merge(const DecodeArgs& a, const RowSplits* inline_rows, int nrows, hipStream_t s) {
    if (inline_rows && nrows <= kInlineRows)
        launch_merge_t<true>(a, *inline_rows, nrows, s);
    else
        launch_merge_t<false>(a, RowSplits{}, nrows, s);
}

template <int D, int G, int LPT>
void launch_f32(const DecodeArgs& a, int nitems, int waves, const WorkOrder& order, hipStream_t s) {
    const size_t lds = (static_cast<size_t>(waves) * 4 * G * D + waves * 2 * G) * sizeof(float);
    const dim3 grid(nitems * (a.lay.kv_heads / waves)), block(64 * waves);
    // two tiles in flight: a third needs more than the 256 VGPRs that keep two
    // waves per SIMD, and measured slower
    WorkOrder o;
    o.n = a.lay.kv_heads == waves && order.n == nitems ? order.n : 0;
    if (o.n) std::copy(order.item, order.item + o.n, o.item);
    launch("paged_decode", decode_f32_kernel<D, G, LPT, 2, false>, grid, block, lds, s, a, o);
}

template <int G, int P>
void launch_rows(const DecodeArgs& a, int nitems, const WorkOrder& order, hipStream_t s) {
    WorkOrder o;
    o.n = order.n == nitems ? order.n : 0;
    if (o.n) std::copy(order.item, order.item + o.n, o.item);
    launch("paged_decode", decode_rows_kernel<G, P, 2>, dim3(nitems), dim3(512), rows_lds_floats(G, P) * sizeof(float),
           s, a, o);
}

template <int P>
bool dispatch_rows_p(const DecodeArgs& a, int nitems, const WorkOrder& order, hipStream_t s) {
    switch (a.group) {
        case 1: launch_rows<1, P>(a, nitems, order, s); return true;
        case 2: launch_rows<2, P>(a, nitems, order, s); return true;
        case 3: launch_rows<3, P>(a, nitems, order, s); return true;
        case 4: launch_rows<4, P>(a, nitems, order, s); return true;
        case 5: launch_rows<5, P>(a, nitems, order, s); return true;
        case 6: launch_rows<6, P>(a, nitems, order, s); return true;
        case 7: launch_rows<7, P>(a, nitems, order, s); return true;
        case 8: launch_rows<8, P>(a, nitems, order, s); return true;
        default: return false;
    }
}

bool dispatch_rows(const DecodeArgs& a, int nitems, const WorkOrder& order, hipStream_t s) {
    switch (a.lay.kv_heads) {
        case 4: return dispatch_rows_p<1>(a, nitems, order, s);
        case 8: return dispatch_rows_p<2>(a, nitems, order, s);
        case 16: return dispatch_rows_p<4>(a, nitems, order, s);
        default: return false;
    }
}

template <int D, int G, int LPT>
void launch_f32_ws(const DecodeArgs& a, int nrows, const WsItems& items, hipStream_t s) {
    const int waves = a.wave_splits;
    const size_t lds = (static_cast<size_t>(waves) * 4 * G * D + waves * 2 * G) * sizeof(float);
    launch("paged_decode", decode_f32_kernel<D, G, LPT, 2, true>, dim3(nrows * a.ws_chunks, a.lay.kv_heads),
           dim3(64 * waves), lds, s, a, items);
}

template <int D>
void dispatch_ws(const DecodeArgs& a, int nrows, const WsItems& it, hipStream_t s) {
    constexpr int LPT = D == 128 ? 8 : 4;
    switch (a.group) {
        case 1: launch_f32_ws<D, 1, LPT>(a, nrows, it, s); return;
        case 2: launch_f32_ws<D, 2, LPT>(a, nrows, it, s); return;
        case 3: launch_f32_ws<D, 3, LPT>(a, nrows, it, s); return;
        case 4: launch_f32_ws<D, 4, LPT>(a, nrows, it, s); return;
        default: break;
    }
    if constexpr (D != 128) {
        switch (a.group) {
            case 5: launch_f32_ws<D, 5, 8>(a, nrows, it, s); return;
            case 6: launch_f32_ws<D, 6, 8>(a, nrows, it, s); return;
            case 7: launch_f32_ws<D, 7, 8>(a, nrows, it, s); return;
            case 8: launch_f32_ws<D, 8, 8>(a, nrows, it, s); return;
            default: break;
        }
    }
    throw std::logic_error("wave-split decode: unsupported shape");
}

template <int D, int G>
void launch_q8(const DecodeArgs& a, int nitems, int waves, hipStream_t s) {
    const size_t lds = (static_cast<size_t>(waves) * 4 * G * D + waves * 2 * G) * sizeof(float);
    launch("paged_decode", decode_q8_kernel<D, G>, dim3(nitems * (a.lay.kv_heads / waves)), dim3(64 * waves), lds, s,
           a);
}

template <int D, int G>
void launch_q8_mma(const DecodeArgs& a, int nitems, int waves, hipStream_t s) {
    const size_t lds = static_cast<size_t>(waves) * q8_mma_wave_lds<D>();
    const int slots = a.lay.kv_heads * (a.group / G);
    launch("paged_decode", decode_q8_mma_kernel<D, G>, dim3(nitems * (slots / waves)), dim3(64 * waves), lds, s, a);
}

// Q8_0 scores on the int8 matrix cores: a wave takes up to four query heads
// of a KV head, the group's heads in one slice or, for six and eight, two of
// three and four; five and seven run one head a wave at head_dim 64 (the
// vector kernel gives a token D/16 lanes, one head slot each, so four at 64)
// and stay on the vector kernel at 128.  Returns the heads per wave, 0 for
// the vector kernel.  TVARA_Q8_DECODE=valu selects the vector kernel where it
// applies.
int q8_mma_heads(int group, int head_dim) {
    static const bool valu = [] {
        const char* env = std::getenv("TVARA_Q8_DECODE");
        return env && std::string(env) == "valu";
    }();
    if (head_dim != 64 && head_dim != 128) return 0;
    if (group == 6 || group == 8) return valu ? 0 : group / 2;
    if (group == 5 || group == 7) return head_dim == 64 ? 1 : 0;
    return group <= 4 && !valu ? group : 0;
}

bool q8_mma_shape(int group, int format, int head_dim) {
    return format != kF32 && q8_mma_heads(group, head_dim) > 0;
}

// Up to four query heads per KV head the f32 kernel gives a token D/16 lanes
// (four at head_dim 64); five to eight take eight lanes a token at either
// head_dim, so the queries and accumulators of a lane stay at 2 * G * D / 8.
template <int D>
bool dispatch_fast(const DecodeArgs& a, int nitems, int waves, const WorkOrder& order, hipStream_t s) {
    // head_dims 80, 96 and 256 (Phi-2, Phi-3, Gemma): f32 blocks (and Q8_0 at
    // 256) and up to four query heads per KV head (three at 80), a token on
    // 4, 8 or 16 lanes
    constexpr bool kF32Only = D == 80 || D == 96 || D == 256;
    constexpr int LPT = D == 256 ? 16 : (D == 128 || D == 96 ? 8 : 4);
    const int G = a.group;
    if (G > 8) return false;
    if constexpr (kF32Only) {
        if (a.lay.format != kF32) {
            // Q8_0 (head_dim a multiple of 32): the vector kernel, a token on
            // D/16 = 16 lanes at 256
            if constexpr (D == 256) {
                switch (G) {
                    case 1: launch_q8<D, 1>(a, nitems, waves, s); return true;
                    case 2: launch_q8<D, 2>(a, nitems, waves, s); return true;
                    case 3: launch_q8<D, 3>(a, nitems, waves, s); return true;
                    case 4: launch_q8<D, 4>(a, nitems, waves, s); return true;
                    default: break;
                }
            }
            return false;
        }
        switch (G) {
            case 1: launch_f32<D, 1, LPT>(a, nitems, waves, order, s); return true;
            case 2: launch_f32<D, 2, LPT>(a, nitems, waves, order, s); return true;
            case 3: launch_f32<D, 3, LPT>(a, nitems, waves, order, s); return true;
            case 4:  // at head_dim 80 four heads' registers (four lanes a token) would spill
                if constexpr (D != 80) {
                    launch_f32<D, 4, LPT>(a, nitems, waves, order, s);
                    return true;
                }
                return false;
            default: return false;
        }
    } else {
        if constexpr (D != 32) {
            if (a.lay.format != kF32) {
                switch (q8_mma_heads(G, D)) {
                case 1: launch_q8_mma<D, 1>(a, nitems, waves, s); return true;
                case 2: launch_q8_mma<D, 2>(a, nitems, waves, s); return true;
                case 3: launch_q8_mma<D, 3>(a, nitems, waves, s); return true;
                case 4: launch_q8_mma<D, 4>(a, nitems, waves, s); return true;
                default: break;
                }
            }
        }
        if (a.lay.format == kF32) {
            switch (G) {
                case 1: launch_f32<D, 1, LPT>(a, nitems, waves, order, s); return true;
                case 2: launch_f32<D, 2, LPT>(a, nitems, waves, order, s); return true;
                case 3: launch_f32<D, 3, LPT>(a, nitems, waves, order, s); return true;
                case 4: launch_f32<D, 4, LPT>(a, nitems, waves, order, s); return true;
                default: break;
            }
            switch (G) {
                case 5: launch_f32<D, 5, 8>(a, nitems, waves, order, s); return true;
                case 6: launch_f32<D, 6, 8>(a, nitems, waves, order, s); return true;
                case 7: launch_f32<D, 7, 8>(a, nitems, waves, order, s); return true;
                case 8: launch_f32<D, 8, 8>(a, nitems, waves, order, s); return true;
                default: break;
            }
            return false;
        }
        if constexpr (D != 32) {
            switch (G) {
                case 1: launch_q8<D, 1>(a, nitems, waves, s); return true;
                case 2: launch_q8<D, 2>(a, nitems, waves, s); return true;
                case 3: launch_q8<D, 3>(a, nitems, waves, s); return true;
                case 4: launch_q8<D, 4>(a, nitems, waves, s); return true;
                default: break;
            }
        }
        if constexpr (LPT == 8) {  // the vector kernel's head slots: D/16 lanes a token
            switch (G) {
                case 5: launch_q8<D, 5>(a, nitems, waves, s); return true;
                case 6: launch_q8<D, 6>(a, nitems, waves, s); return true;
                case 7: launch_q8<D, 7>(a, nitems, waves, s); return true;
                case 8: launch_q8<D, 8>(a, nitems, waves, s); return true;
                default: break;
            }
        }
        return false;
    }
}

}  // namespace

// Waves per workgroup (one per KV head), measured on MI355X: eight for f32
// blocks (a workgroup streams whole 2 KiB slot rows; about one workgroup per
// CU is best), four for Q8_0 (the int8-MFMA kernel: 207 us against 210 us
// with eight on the Llama-3-8B batch; the vector kernel: more, shorter
// workgroups hide its longer per-tile arithmetic), at most two for groups
// above four query heads; a divisor of kv_heads whose LDS fits 64 KiB.
// TVARA_DECODE_WAVES overrides it for tuning.
int decode_slots(int kv_heads, int group, int format, int head_dim) {
    return kv_heads * (q8_mma_shape(group, format, head_dim) ? group / q8_mma_heads(group, head_dim) : 1);
}

int decode_waves(int kv_heads, int group, int format, int head_dim) {
    const bool mma = q8_mma_shape(group, format, head_dim);
    const int slots = decode_slots(kv_heads, group, format, head_dim);
    int w = format == kF32 ? 8 : 4;
    if (const char* env = std::getenv("TVARA_DECODE_WAVES")) w = std::atoi(env);
    if (group > 4 && !mma) w = std::min(w, 2);
    w = std::max(1, std::min(w, 8));
    auto lds = [&](int n) {
        return mma ? static_cast<size_t>(n) * (32 * (head_dim + 16) + 32 * (head_dim / 32) * 4 * sizeof(float))
                   : static_cast<size_t>(n) * (4 * group * head_dim + 2 * group) * sizeof(float);
    };
    while (w > 1 && (slots % w || lds(w) > 65536)) --w;
    return w;
}

// Workgroups per CU a decode launch is sized for (the split length is the
// shortest whose launch fits CUs x this): one for f32 blocks, two for the
// int8-MFMA Q8_0 kernel (two 8-wave workgroups' worth of registers per CU),
// four for the vector Q8_0 kernel; above four query heads per KV head two
// (head_dim 128) or four (64).
// TVARA_DECODE_BUDGET overrides it.
int decode_budget_per_cu(int group, int format, int head_dim) {
    if (const char* env = std::getenv("TVARA_DECODE_BUDGET")) return std::max(1, std::atoi(env));
    // above four query heads per KV head the vector kernels run two-wave
    // workgroups: at head_dim 128 one wave per SIMD, two workgroups per CU
    // (the Llama-3-70B shape: f32 94 against 120 us with one); at 64 (eight
    // lanes a token, two or three waves per SIMD) four (TinyLlama's shape,
    // 64 x 2,048 tokens: 42.8 against 45.6 us with two)
    if (group > 4 && !q8_mma_shape(group, format, head_dim)) return head_dim == 64 ? 4 : 2;
    if (format == kF32) return 1;
    return q8_mma_shape(group, format, head_dim) ? 2 : 4;
}

static int waves_for(const DecodeArgs& a) {
    return decode_waves(a.lay.kv_heads, a.group, a.lay.format, a.lay.head_dim);
}

// Wave splits, for launches of at most 32 (row, KV head) pairs on f32 blocks
// and the fast shapes that fit 512-thread workgroups: a workgroup per (row,
// KV head, chunk) whose waves take consecutive splits of the chunk, merged
// in LDS; with more than one chunk a row's chunks leave partials that
// merge_wave_kernel combines.  Such launches are latency-bound: the usual
// decomposition puts a (row, KV head) pair's waves on one CU, and a wave
// that holds more tokens than it has in flight (two tiles) pays a memory
// round trip per two tiles.  So a row of up to two round trips a wave over
// eight waves stays one workgroup; a longer one is cut into chunks of one
// round trip a wave (eight waves), as many as fill the CUs once, beyond
// which the splits grow (MI355X, one Llama-3.2-1B row, 32/8 heads: 2,048
// tokens 25.1 against about 6 us, 8,192 tokens 70.2 against about 9 us).
WaveSplitShape wave_split_shape(int rows, int kv_heads, int group, int format, int head_dim, int tpb,
                                size_t max_tokens, int cus) {
    WaveSplitShape none{};
    if (const char* env = std::getenv("TVARA_WAVE_SPLITS"); env && std::atoi(env) == 0) return none;
    if (format != kF32 || !decode_f32_blocks(tpb) || (head_dim != 32 && head_dim != 64 && head_dim != 128)) return none;
    if (group > 8 || (head_dim == 128 && group > 4)) return none;
    const size_t pairs = static_cast<size_t>(rows) * kv_heads;
    if (pairs > 32 || max_tokens == 0) return none;
    // tokens a wave has in flight (two tiles of 64 / LPT tokens, LPT as
    // dispatch_ws); at most eight waves, their partials in 64 KiB of LDS
    const int lpt = head_dim == 128 || group > 4 ? 8 : 4;
    const size_t flight = 2 * (64 / lpt);
    const size_t per_wave = (4 * static_cast<size_t>(group) * head_dim + 2 * group) * sizeof(float);
    const size_t wmax = std::min<size_t>(8, 65536 / per_wave);
    if (wmax < 1) return none;
    auto blocks_of = [&](size_t t) {
        const size_t b = static_cast<size_t>(tpb);
        return (std::max<size_t>(t, 16) + b - 1) / b * b;
    };
    WaveSplitShape w{};
    // (one workgroup of two round trips a wave measured as fast as two
    // chunks of one, 7.4 against 7.5 us plus the merge for the SmolLM2-135M
    // row, and faster than them from 384 tokens up to 512)
    if (max_tokens <= 2 * wmax * flight) {
        w.waves = static_cast<int>(std::min(wmax, (max_tokens + flight - 1) / flight));
        w.chunks = 1;
        w.tokens = blocks_of((max_tokens + w.waves - 1) / w.waves);
    } else {
        size_t t = blocks_of(flight);
        if (const char* env = std::getenv("TVARA_WS_TOKENS")) t = blocks_of(std::strtoull(env, nullptr, 10));
        auto chunks = [&](size_t sp) { return (max_tokens + wmax * sp - 1) / (wmax * sp); };
        while (pairs * chunks(t) > static_cast<size_t>(cus) && t < kMaxSplitTokens) t = blocks_of(2 * t);
        w.waves = static_cast<int>(wmax);
        w.chunks = static_cast<int>(chunks(t));
        w.tokens = t;
    }
    // the kernels keep a split's block ids in one register per lane
    if (w.tokens > kMaxSplitTokens || w.tokens / tpb > static_cast<size_t>(kMaxSplitBlocks)) return none;
    // every chunk of a row's waves must cover the row
    if (static_cast<size_t>(w.waves) * w.chunks * w.tokens < max_tokens) return none;
    return w;
}

// the largest decode launch whose splits are merged in the kernel
// (TVARA_INKERNEL_MERGE_MAX overrides it for tuning)
constexpr int kInKernelMergeMaxWorkgroups = 128;

static int in_kernel_merge_max() {
    static const int max_wgs = [] {
        const char* env = std::getenv("TVARA_INKERNEL_MERGE_MAX");
        return env ? std::atoi(env) : kInKernelMergeMaxWorkgroups;
    }();
    return max_wgs;
}

bool decode_f32_blocks(int tpb) { return tpb >= 16 && tpb <= 1024 && (tpb & (tpb - 1)) == 0; }

bool decode_rows_shape(int kv_heads, int group, int format, int head_dim, int tpb) {
    if (const char* env = std::getenv("TVARA_ROW_MAJOR"); env && std::atoi(env) == 0) return false;
    return format == kF32 && head_dim == 64 && decode_f32_blocks(tpb) && (kv_heads == 4 || kv_heads == 8 || kv_heads == 16) &&
           group >= 1 && group <= 8;
}

// f32 blocks: head_dim 32, 64 or 128, any power-of-two block of 16 to 1,024
// tokens; Q8_0 blocks: head_dim 64 or 128, 16-token blocks
bool decode_fast_path(const DecodeArgs& a) {
    if (a.group > 8) return false;
    if (a.lay.format == kF32)
        return decode_f32_blocks(a.lay.tpb) &&
               (a.lay.head_dim == 32 || a.lay.head_dim == 64 || a.lay.head_dim == 128 ||
                ((a.lay.head_dim == 96 || a.lay.head_dim == 256) && a.group <= 4) ||
                (a.lay.head_dim == 80 && a.group <= 3));
    return a.lay.tpb == 16 && (a.lay.head_dim == 64 || a.lay.head_dim == 128 || (a.lay.head_dim == 256 && a.group <= 4));
}

void launch_decode(const DecodeArgs& a, int nitems, int nrows, bool need_merge, const RowSplits* inline_rows,
                   const WorkOrder* order, hipStream_t s, const WsItems* ws_items) {
    static const WorkOrder identity = [] {
        WorkOrder o;
        o.n = 0;
        return o;
    }();
    const WorkOrder& ord = order ? *order : identity;
    if (nitems <= 0) return;
    if (a.wave_splits) {  // the plan chose wave splits (wave_split_shape): merged in LDS
        static const WsItems none = [] {
            WsItems w{};
            w.n = 0;
            return w;
        }();
        const WsItems& it = ws_items ? *ws_items : none;
        // chunk partials: merged by the (row, KV head)'s last chunk in
        // launches of at most 64 workgroups, else by the merge kernel
        // (MI355X, one Llama-3.2-1B row: 1,024 tokens 10.4 -> 9.5 us and
        // 2,048 tokens 10.4 -> 9.8 us in 64 workgroups; 4,096 tokens 10.7
        // against 11.1 us in 128)
        DecodeArgs b = a;
        const bool in_kernel = a.ws_chunks > 1 && a.row_done &&
                               nrows * a.ws_chunks * a.lay.kv_heads <= std::min(64, in_kernel_merge_max());
        if (!in_kernel) b.row_done = nullptr;
        b.lay.head_dim == 64    ? dispatch_ws<64>(b, nrows, it, s)
        : b.lay.head_dim == 128 ? dispatch_ws<128>(b, nrows, it, s)
                                : dispatch_ws<32>(b, nrows, it, s);
        TVARA_HIP(hipGetLastError());
        if (a.ws_chunks > 1 && !in_kernel) {  // (first chunk, chunks) per row
            if (!inline_rows || nrows > kInlineRows) throw std::logic_error("wave-split decode: rows not inline");
            launch_merge(b, inline_rows, nrows, s);
            TVARA_HIP(hipGetLastError());
        }
        return;
    }
    if (a.row_major) {  // the plan chose the row-major kernel: merge_kernel merges
        DecodeArgs b = a;
        b.row_done = nullptr;
        if (!dispatch_rows(b, nitems, ord, s)) throw std::logic_error("row-major decode: unsupported shape");
        TVARA_HIP(hipGetLastError());
        if (need_merge) {
            launch_merge(b, inline_rows, nrows, s);
            TVARA_HIP(hipGetLastError());
        }
        return;
    }
    // Small launches of the f32 and vector Q8_0 kernels merge a row's splits
    // in its last workgroup: there the second launch is pure latency (the
    // SmolLM2-135M row: 7.7 against 8.3 us per step).  A launch that fills
    // the GPU keeps merge_kernel: every workgroup waiting for its partials to
    // reach the point of coherence and for its count costs more than the
    // launch (the Llama-3.2-1B batch of 253 workgroups: 105.5 against 102.8 us).
    // The int8-MFMA Q8_0 and generic kernels always leave it to merge_kernel.
    const bool fast = decode_fast_path(a);
    const int wgs = fast ? nitems * (decode_slots(a.lay.kv_heads, a.group, a.lay.format, a.lay.head_dim) / waves_for(a))
                         : nitems * a.heads;
    const bool in_kernel = fast && a.row_done && !q8_mma_shape(a.group, a.lay.format, a.lay.head_dim) &&
                           wgs <= in_kernel_merge_max();
    DecodeArgs b = a;
    if (!in_kernel) b.row_done = nullptr;
    bool merged = false;
    {
        bool done = false;
        if (fast) {
            const int waves = waves_for(b);
            done = b.lay.head_dim == 64    ? dispatch_fast<64>(b, nitems, waves, ord, s)
                   : b.lay.head_dim == 128 ? dispatch_fast<128>(b, nitems, waves, ord, s)
                   : b.lay.head_dim == 256 ? dispatch_fast<256>(b, nitems, waves, ord, s)
                   : b.lay.head_dim == 96  ? dispatch_fast<96>(b, nitems, waves, ord, s)
                   : b.lay.head_dim == 80  ? dispatch_fast<80>(b, nitems, waves, ord, s)
                                           : dispatch_fast<32>(b, nitems, waves, ord, s);
        }
        if (!done) {
            if (b.lay.head_dim > kGenericMaxDim) throw std::invalid_argument("head_dim above 512 is not supported");
            b.row_done = nullptr;
            launch("paged_decode", decode_generic_kernel, dim3(nitems, b.heads), dim3(64), 0, s, b);
        }
        TVARA_HIP(hipGetLastError());
        merged = done && in_kernel;
    }
    if (need_merge && !merged) {
        launch_merge(b, inline_rows, nrows, s);
        TVARA_HIP(hipGetLastError());
    }
}

}  // namespace tvara_amd
