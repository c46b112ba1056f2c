// Paged chunked-prefill attention on CDNA4 MFMA: the causal chunk of
// fused_prompt_attention (core/include/tvara/attention.hpp:85-89), with bf16
// operands and f32 accumulation.
//
// A workgroup takes 8 waves x 32 query rows of one (sequence, KV head); a row
// is one (chunk position, query head of the GQA group), so the G heads that
// share a KV head share every K/V tile.  Key tiles of 64 positions (four
// blocks of 16 tokens, two of 32, or part of one larger block) are read from
// the pool (f32 or Q8_0) by all the waves, rounded to bf16 and staged in
// double-buffered LDS: K as [key][d], V transposed as [d][key].
//
// Each wave computes S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (A = K from
// LDS, B = Q^T held in registers), so the score of row r and key k sits in the
// lane that owns row r: lane l holds rows 16*nt + l%16 and keys
// 16*mt + 4*(l/16) + i.  Those registers are exactly the B operand of
// O^T = V^T P^T when the 32-key K dimension of the second product is ordered
// {4g..4g+3, 16+4g..16+4g+3} for lane group g, so P never leaves registers;
// the A operand (V^T) is read from LDS in the same key order.  Online softmax
// runs in log2 units with the lazy rescale of the decode kernels; the S^T
// accumulators start at -m (the row's running maximum), so the MFMA returns
// score - m ready for exp2, and the normaliser is one more MFMA tile whose A
// operand is a row of ones.  The causal mask is applied on tiles that reach
// past a row's own position.
#include <cstdlib>

#include "common.hpp"
#include "device_util.hpp"
#include "q8.hpp"

namespace tvara_amd {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kThreshold = 8.0f;
constexpr int kRows = 32, kKeys = 64;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef short i16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 on an LDS address
__device__ __forceinline__ bf16x4 tr16_read(const __bf16* p) {
    typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
    return __builtin_bit_cast(bf16x4, v);
}

__device__ __forceinline__ bf16x4 to_bf16(float4 v) {
    const f32x4 f = {v.x, v.y, v.z, v.w};
    return __builtin_convertvector(f, bf16x4);
}

__device__ __forceinline__ bf16x4 to_bf16(f32x4 v) { return __builtin_convertvector(v, bf16x4); }

// word 3 of a raw buffer descriptor (32-bit data format, no swizzle)
constexpr int kBufferWord3 = 0x00020000;

// kQ8: Q8_0 blocks (the head's int8 plane and fp16 group scales), dequantised
// to bf16 when staged; otherwise f32 blocks.
// TPB: 16 for blocks of 16 tokens (block arithmetic folded at compile time),
// 0 for any power of two from 16 to 1,024 read from the layout
template <int D, int G, int kWaves, bool kQ8, int TPB>
__global__ __launch_bounds__(64 * kWaves) void prefill_bf16_kernel(const PrefillArgs a) {
    constexpr int PW = kRows / G;        // chunk positions per wave; rows PW*G .. 31 are padding (G = 3, 5, 6, 7)
    constexpr int QT = kWaves * PW;      // chunk positions per workgroup
    constexpr int KC = D / 32;           // K-dimension chunks of S^T
    constexpr int DT = D / 16;           // output column tiles
    constexpr int KSTR = D + 8;          // LDS row pitch of K (bf16): 144 B, conflict-free b128 operand reads
    constexpr int VSTR = D + 16;         // LDS row pitch of V (bf16): 160 B, conflict-free transposing reads
    static_assert(D == 64 || D == 128, "head_dim 64 or 128");
    constexpr int LPR = D / 4;                // staging lanes per key row (4 columns each)
    constexpr int KPP = 64 * kWaves / LPR;    // keys per staging pass
    constexpr int SP = kKeys / KPP;           // staging passes per tile
    static_assert(SP >= 1 && SP * KPP == kKeys, "the staging map covers whole key rows");
    __shared__ __attribute__((aligned(16))) __bf16 klds[2][kKeys * KSTR];
    __shared__ __attribute__((aligned(16))) __bf16 vlds[2][kKeys * VSTR];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r16 = lane & 15;
    // XCD-aware order: workgroups are dispatched to the 8 XCDs round-robin by
    // id, so the chunk tiles of one (sequence, KV head) pair get ids of one
    // residue mod 8 and share that XCD's L2 for their common K/V tiles.
    const int id = static_cast<int>(blockIdx.x), xcd = id & 7, k = id >> 3;
    const int pair = (k / a.chunk_tiles) * 8 + xcd, ct = k % a.chunk_tiles;
    if (pair >= a.pairs) return;
    const int kh = pair % a.lay.kv_heads;
    const int4 sd = a.seqs[pair / a.lay.kv_heads];  // table offset, start, rows, first query row
    const int start = sd.y, nrows = sd.z;
    const int q0 = ct * QT;
    if (q0 >= nrows) return;  // the whole workgroup: chunk_tiles covers the longest chunk
    const int kmax = start + min(q0 + QT, nrows);  // keys this workgroup reads: [0, kmax)
    const int ntiles = (kmax + kKeys - 1) / kKeys;
    const int pw0 = q0 + wave * PW;
    const int wave_kmax = pw0 < nrows ? start + min(pw0 + PW, nrows) : 0;
    const int kvw = a.lay.kv_width;
    const int32_t* tab = a.tables + sd.x;

    // Q^T as the B operand: row n = 16*nt + r16, columns 32*kc + 8*g .. +7
    bf16x8 qop[2][KC];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int r = 16 * nt + r16, pos = pw0 + r / G, head = kh * G + r % G;
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
            float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
            if (pos < nrows && r < PW * G) {
                const float* qp = a.q + (static_cast<size_t>(sd.w + pos) * a.heads + head) * D + 32 * kc + 8 * g;
                x0 = *reinterpret_cast<const float4*>(qp);
                x1 = *reinterpret_cast<const float4*>(qp + 4);
            }
            const float s = a.qscale;
            const bf16x4 lo = to_bf16(make_float4(x0.x * s, x0.y * s, x0.z * s, x0.w * s));
            const bf16x4 hi = to_bf16(make_float4(x1.x * s, x1.y * s, x1.z * s, x1.w * s));
            qop[nt][kc] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
    }

    // staging map: D/4 lanes per key row (4 columns each), KPP keys per pass,
    // SP passes per 64-key tile.  A wave's rows in a pass are 64/LPR aligned
    // consecutive keys, so they lie in one paged block: the block id and base
    // address are wave-uniform (scalar registers) and a lane's offset within
    // the block depends only on its row and the pass.  The block ids are loaded
    // two tiles ahead of the K/V rows, so no wave waits on a table lookup
    // before issuing its loads.
    const int skey = tid / LPR, col = 4 * (tid % LPR);
    const int wkey = __builtin_amdgcn_readfirstlane(skey);  // the wave's first row in a pass
    // Blocks hold tpb = 2^tsh tokens (16 to 1,024).  The pass start
    // kt * 64 + KPP * p is a multiple of KPP (a power of two) and skey < KPP,
    // so key kt * 64 + KPP * p + skey sits in slot
    // ((kt * 64 + KPP * p) & (tpb - 1)) + (skey & (tpb - 1)) of its block: the
    // first term is wave-uniform and goes into the loads' scalar offsets, the
    // second gives the loop-invariant lane offsets roff (the lane's four
    // columns within the block's K or V run of this head: f32, or Q8_0 int8)
    // and soff (Q8_0: their group's scale).
    const int tpb = TPB ? TPB : a.lay.tpb, tsh = __builtin_ctz(static_cast<unsigned>(tpb));
    const int lslot = skey & (tpb - 1);
    const unsigned roff =
        static_cast<unsigned>(kQ8 ? lslot * D + col : (lslot * kvw + col) * static_cast<int>(sizeof(float)));
    const unsigned soff = static_cast<unsigned>(tpb * D + (lslot * (D / 32) + col / 32) * 2);
    // K/V rows are read through a buffer descriptor per block (base = the
    // block's K run of this layer and head, V one section further, 32-bit lane
    // offsets, reads bounded by the block's end)
    const int kvh = kh / a.kv_share;  // the KV head whose K/V this (virtual) head reads
    const size_t kbytes = kQ8 ? static_cast<size_t>(a.layer) * 2 * a.lay.section + static_cast<size_t>(kvh) * a.lay.head_bytes
                              : (static_cast<size_t>(a.layer) * 2 * tpb * kvw + static_cast<size_t>(kvh) * D) * sizeof(float);
    const int vsec = static_cast<int>(kQ8 ? a.lay.section : static_cast<size_t>(tpb) * kvw * sizeof(float));
    const int brange = static_cast<int>(a.lay.stride - kbytes);
    // register stages of K/V rows in flight: two (even / odd tiles) at head_dim
    // 64, one at 128, where two would not fit beside the accumulators
    constexpr int kStages = D == 64 ? 2 : 1;
    f32x4 kA[SP], vA[SP], kB[kStages == 2 ? SP : 1], vB[kStages == 2 ? SP : 1];
    int bA[SP], bB[kStages == 2 ? SP : 1];
    // Every load is unconditional: rows of a pass past the chunk's reach read
    // the last reachable block (any slot of it: in bounds, possibly stale or
    // never written).  A load under a branch makes the compiler wait for all
    // outstanding loads where the branches join.  Such keys lie past every
    // row's causal limit, so their scores are masked; their V rows are zeroed
    // when staged, so a non-finite value there cannot reach a row as 0 * NaN.
    auto tabload = [&](int kt, int (&b)[SP]) {
#pragma unroll
        for (int p = 0; p < SP; ++p) b[p] = tab[min(kt * kKeys + KPP * p + wkey, kmax - 1) >> tsh];
    };
    // tile kt's rows, from the block ids tabload put in b
    auto gload = [&](int kt, const int (&b)[SP], f32x4 (&kreg)[SP], f32x4 (&vreg)[SP]) {
#pragma unroll
        for (int p = 0; p < SP; ++p) {
            const int base = (kt * kKeys + KPP * p) & (tpb - 1);  // the pass's first slot in its block
            const int rso = base * (kQ8 ? D : kvw * static_cast<int>(sizeof(float))), sso = base * (D / 32) * 2;
            const char* blk =
                a.pool + static_cast<size_t>(__builtin_amdgcn_readfirstlane(b[p])) * a.lay.stride + kbytes;
            const __amdgpu_buffer_rsrc_t r =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(blk), 0, brange, kBufferWord3);
            if constexpr (kQ8) {  // four int8 and their scale's bits, dequantised when staged
                const unsigned kq = __builtin_amdgcn_raw_buffer_load_b32(r, roff, rso, 0);
                const unsigned ks = __builtin_amdgcn_raw_buffer_load_b16(r, soff, sso, 0);
                const unsigned vq = __builtin_amdgcn_raw_buffer_load_b32(r, roff, vsec + rso, 0);
                const unsigned vs = __builtin_amdgcn_raw_buffer_load_b16(r, soff, vsec + sso, 0);
                kreg[p] = f32x4{__builtin_bit_cast(float, kq), __builtin_bit_cast(float, ks), 0.f, 0.f};
                vreg[p] = f32x4{__builtin_bit_cast(float, vq), __builtin_bit_cast(float, vs), 0.f, 0.f};
            } else {
                kreg[p] = __builtin_amdgcn_raw_buffer_load_b128(r, roff, rso, 0);
                vreg[p] = __builtin_amdgcn_raw_buffer_load_b128(r, roff, vsec + rso, 0);
            }
        }
    };
    auto values = [](f32x4 x) {  // the staged f32 values (Q8_0: d * q, as dequantize_q8_0)
        if constexpr (kQ8) {
            // elements copied to scalars first: a bit cast of a vector element
            // directly reads element 0 under this compiler
            const float x0 = x[0], x1 = x[1];
            const uint32_t q = __builtin_bit_cast(uint32_t, x0);
            const float d = half_bits_to_float(static_cast<uint16_t>(__builtin_bit_cast(uint32_t, x1)));
            return f32x4{sbyte_to_float<0>(q) * d, sbyte_to_float<1>(q) * d, sbyte_to_float<2>(q) * d,
                         sbyte_to_float<3>(q) * d};
        } else {
            return x;
        }
    };
    auto lstore = [&](int kt, int buf, const f32x4 (&kreg)[SP], f32x4 (&vreg)[SP]) {
        if (kt * kKeys + kKeys > kmax) {  // the chunk's last tile: zero V past its reach
#pragma unroll
            for (int p = 0; p < SP; ++p)
                if (kt * kKeys + KPP * p + skey >= kmax) vreg[p] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int p = 0; p < SP; ++p) {
            *reinterpret_cast<bf16x4*>(&klds[buf][(KPP * p + skey) * KSTR + col]) = to_bf16(values(kreg[p]));
            *reinterpret_cast<bf16x4*>(&vlds[buf][(KPP * p + skey) * VSTR + col]) = to_bf16(values(vreg[p]));
        }
    };

    // acc[DT] is the normaliser: A = a row of ones (A row l%16 comes from lane
    // l, so lanes 0, 16, 32, 48 hold row 0) times P^T sums the bf16
    // probabilities the output tiles use
    f32x4 acc[DT + 1][2];
#pragma unroll
    for (int dt = 0; dt <= DT; ++dt) acc[dt][0] = acc[dt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    const __bf16 one = r16 == 0 ? static_cast<__bf16>(1.f) : static_cast<__bf16>(0.f);
    const bf16x8 ones = bf16x8{one, one, one, one, one, one, one, one};
    float m[2] = {-INFINITY, -INFINITY};
    int lim[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) lim[nt] = start + pw0 + (16 * nt + r16) / G;  // last visible key of the row

    // Tile t's K/V rows are requested two iterations before they are written
    // to LDS (register stages A for even tiles, B for odd), its block ids four
    // iterations before; every load is unconditional (past the last tile they
    // re-read it), so no branch makes the compiler wait for them early.
    auto compute = [&](int kt, int buf) {
        const int kbase = kt * kKeys;
        if (kbase < wave_kmax) {
            // scores arrive as score - m: the accumulators start at -m (the
            // running maximum), 0 on a wave's first tile when m is still -inf
            const bool first = m[0] == -INFINITY;
            f32x4 s[4][2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const float c0 = first ? 0.f : -m[nt];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) s[mt][nt] = f32x4{c0, c0, c0, c0};
            }
            // every K operand of the tile is read before the first product, so
            // the reads' latency is paid once
            bf16x8 kop[KC][4];
#pragma unroll
            for (int kc = 0; kc < KC; ++kc)
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
                    kop[kc][mt] = *reinterpret_cast<const bf16x8*>(&klds[buf][(16 * mt + r16) * KSTR + 32 * kc + 8 * g]);
#pragma unroll
            for (int kc = 0; kc < KC; ++kc)
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) {
                    s[mt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[kc][mt], qop[0][kc], s[mt][0], 0, 0, 0);
                    s[mt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[kc][mt], qop[1][kc], s[mt][1], 0, 0, 0);
                }
            // the causal mask only on tiles that reach past a row's own position
            if (kbase + kKeys - 1 > start + pw0) {
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (kbase + 16 * mt + 4 * g + i > lim[nt]) s[mt][nt][i] = -INFINITY;
            }
            float rmax[2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                float mx = -INFINITY;
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[mt][nt][i]);
                rmax[nt] = cross_row_max(mx);
            }
            if (first) {
                // every row sees key 0 here, so its maximum is finite
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    m[nt] = rmax[nt];
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) s[mt][nt] -= rmax[nt];
                }
            } else if (__any(rmax[0] > kThreshold || rmax[1] > kThreshold)) {
                // rmax is relative to m: raise m where the tile exceeds it
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    const float up = fmaxf(rmax[nt], 0.f);
                    const float alpha = fast_exp2(-up);
                    m[nt] += up;
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) s[mt][nt] -= up;
#pragma unroll
                    for (int dt = 0; dt <= DT; ++dt) acc[dt][nt] *= alpha;
                }
            }
            // P^T as the B operand of O^T = V^T P^T: keys {4g+i, 16+4g+i} of each
            // 32-key half kc (s already holds score - m; a masked score gives
            // exp2(-inf) = 0).  Row half 1's probabilities for a key half are
            // computed between the two halves' products, so the vector ALU
            // works while the matrix core runs half 0's MFMAs.
            auto probs = [&](int nt, int kc) {
                float p[2][4];
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int i = 0; i < 4; ++i) p[h][i] = fast_exp2(s[2 * kc + h][nt][i]);
                const bf16x4 lo = to_bf16(make_float4(p[0][0], p[0][1], p[0][2], p[0][3]));
                const bf16x4 hi = to_bf16(make_float4(p[1][0], p[1][1], p[1][2], p[1][3]));
                return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            };
            bf16x8 pop0[2];
            pop0[0] = probs(0, 0);
            pop0[1] = probs(0, 1);
            // V^T operand by transposing LDS reads (ds_read_b64_tr_b16): within
            // each 16-lane group, lane i receives element i%4 of the chunk that
            // lane 4j + i/4 addresses, as its element j; lane 16g + 4j + q
            // addresses key row 4g + j (+16 for the second half), columns
            // 16dt + 4q, so lane (g, i) gets column 16dt + i of keys 4g + j
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) {
                bf16x8 vop[DT];
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    const __bf16* vrow = &vlds[buf][(32 * kc + 4 * g + (r16 >> 2)) * VSTR + 16 * dt + 4 * (r16 & 3)];
                    const bf16x4 lo = tr16_read(vrow);
                    const bf16x4 hi = tr16_read(vrow + 16 * VSTR);
                    vop[dt] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
                    acc[dt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop[dt], pop0[kc], acc[dt][0], 0, 0, 0);
                acc[DT][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pop0[kc], acc[DT][0], 0, 0, 0);
                const bf16x8 pop1 = probs(1, kc);
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
                    acc[dt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop[dt], pop1, acc[dt][1], 0, 0, 0);
                acc[DT][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pop1, acc[DT][1], 0, 0, 0);
            }
        }
    };
    auto tile = [&](int t) { return min(t, ntiles - 1); };
    if constexpr (kStages == 2) {
        tabload(0, bA);
        gload(0, bA, kA, vA);
        tabload(tile(1), bB);
        gload(tile(1), bB, kB, vB);
        tabload(tile(2), bA);
        tabload(tile(3), bB);
        lstore(0, 0, kA, vA);
        __syncthreads();
        for (int kt = 0; kt < ntiles; kt += 2) {
            gload(tile(kt + 2), bA, kA, vA);
            tabload(tile(kt + 4), bA);
            compute(kt, 0);
            lstore(tile(kt + 1), 1, kB, vB);
            __syncthreads();
            if (kt + 1 >= ntiles) break;
            gload(tile(kt + 3), bB, kB, vB);
            tabload(tile(kt + 5), bB);
            compute(kt + 1, 1);
            lstore(tile(kt + 2), 0, kA, vA);
            __syncthreads();
        }
    } else {
        // one register stage: tile t + 1 is requested before tile t's products
        tabload(0, bA);
        gload(0, bA, kA, vA);
        tabload(tile(1), bA);
        lstore(0, 0, kA, vA);
        __syncthreads();
        for (int kt = 0; kt < ntiles; ++kt) {
            gload(tile(kt + 1), bA, kA, vA);
            tabload(tile(kt + 2), bA);
            compute(kt, kt & 1);
            lstore(tile(kt + 1), (kt + 1) & 1, kA, vA);
            __syncthreads();
        }
    }

    bool bad = false;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        // row 0 of the normaliser tile: lane r16 (group 0), element 0
        const float l = __shfl(acc[DT][nt][0], r16);
        const int r = 16 * nt + r16, pos = pw0 + r / G, head = kh * G + r % G;
        if (pos >= nrows || r >= PW * G) continue;
        float* o = a.out + (static_cast<size_t>(sd.w + pos) * a.heads + head) * D + 4 * g;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const f32x4 v = acc[dt][nt] / l;
            bad |= !__builtin_isfinite(v[0]) || !__builtin_isfinite(v[1]) || !__builtin_isfinite(v[2]) ||
                   !__builtin_isfinite(v[3]);
            *reinterpret_cast<float4*>(o + 16 * dt) = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
    if (__any(bad) && lane == 0) *a.err = 1;
}

// eight waves per workgroup (measured on MI355X against four: 158 against 225
// us on the 8 x (2,048 + 512) chunk; K/V tiles are re-read by half as many
// workgroups) and 64-key tiles (128-key tiles measured 177 us)
template <int D, int G, int W, int TPB>
void launch_gw(const PrefillArgs& a, int nseqs, int max_rows, hipStream_t s) {
    const bool q8 = a.lay.format == kQ8;
    constexpr int QT = W * (kRows / G);
    PrefillArgs b = a;
    b.chunk_tiles = (max_rows + QT - 1) / QT;
    b.pairs = nseqs * a.lay.kv_heads;
    const int groups8 = (b.pairs + 7) / 8;  // ids = 8 XCDs x pair groups x chunk tiles
    const dim3 grid(8 * groups8 * b.chunk_tiles), block(64 * W);
    if (q8)
        launch("paged_prefill_bf16", prefill_bf16_kernel<D, G, W, true, TPB>, grid, block, 0, s, b);
    else
        launch("paged_prefill_bf16", prefill_bf16_kernel<D, G, W, false, TPB>, grid, block, 0, s, b);
}

// waves per workgroup (TVARA_PREFILL_WAVES: 4 or 8, for blocks of 16 tokens;
// other block sizes take 8)
template <int G>
void launch_g(const PrefillArgs& a, int nseqs, int max_rows, hipStream_t s) {
    static const int waves = [] {
        const char* env = std::getenv("TVARA_PREFILL_WAVES");
        return env && std::atoi(env) == 4 ? 4 : 8;
    }();
    if (a.lay.tpb != 16) {
        if (a.lay.head_dim == 128)
            launch_gw<128, G, 8, 0>(a, nseqs, max_rows, s);
        else
            launch_gw<64, G, 8, 0>(a, nseqs, max_rows, s);
    } else if (a.lay.head_dim == 128) {
        waves == 4 ? launch_gw<128, G, 4, 16>(a, nseqs, max_rows, s) : launch_gw<128, G, 8, 16>(a, nseqs, max_rows, s);
    } else {
        waves == 4 ? launch_gw<64, G, 4, 16>(a, nseqs, max_rows, s) : launch_gw<64, G, 8, 16>(a, nseqs, max_rows, s);
    }
}

}  // namespace

bool prefill_bf16_supported(const BlockLayout& lay, int group) {
    // the staging reads take 32-bit offsets within a block
    return (lay.format == kF32 || lay.format == kQ8) && decode_f32_blocks(lay.tpb) &&
           (lay.head_dim == 64 || lay.head_dim == 128) &&
           lay.stride < (size_t(1) << 31) && group >= 1 && group <= 8;
}

void launch_prefill_bf16(const PrefillArgs& a, int nseqs, int max_rows, hipStream_t s) {
    if (!prefill_bf16_supported(a.lay, a.group))
        throw std::invalid_argument(
            "bf16 prefill needs f32 or Q8_0 blocks of 16 to 1,024 tokens (a power of two, under 2 GiB), "
            "head_dim 64 or 128, and a GQA slice of 1-8 heads");
    if (nseqs <= 0 || max_rows <= 0) return;
    switch (a.group) {
        case 1: launch_g<1>(a, nseqs, max_rows, s); break;
        case 2: launch_g<2>(a, nseqs, max_rows, s); break;
        case 3: launch_g<3>(a, nseqs, max_rows, s); break;
        case 4: launch_g<4>(a, nseqs, max_rows, s); break;
        case 5: launch_g<5>(a, nseqs, max_rows, s); break;
        case 6: launch_g<6>(a, nseqs, max_rows, s); break;
        case 7: launch_g<7>(a, nseqs, max_rows, s); break;
        default: launch_g<8>(a, nseqs, max_rows, s); break;
    }
    TVARA_HIP(hipGetLastError());
}

}  // namespace tvara_amd
