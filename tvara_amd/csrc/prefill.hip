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
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

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
// kX3: f32 inputs carried as three products of split operands.  The score
// operands Q and K are split into fp16 parts, x = hi + lo (hi = fp16(x),
// lo = fp16(x - hi): 22 significant bits, lo subnormal for small x, which the
// MFMA keeps), V and the probabilities into bf16 parts (16 bits, the range of
// f32), and every product takes hi*hi + hi*lo + lo*hi in f32.  A score then
// carries about 2^-22 relative error per term (bf16 parts gave 2^-15, which
// exceeded the 1e-4 bar on rows whose scores spread over tens of units) and
// the output about 2^-16 per term.  Keys, and queries once scaled by
// log2(e)/sqrt(D), must lie within the fp16 range (65,504): beyond it a score
// is not finite and the launch fails as a non-finite input does.  LDS holds the lo planes of K and V beside the hi
// ones.
template <int D, int G, int kWaves, bool kQ8, int TPB, bool kX3 = false>
__global__ __launch_bounds__(64 * kWaves) void prefill_bf16_kernel(const PrefillArgs a) {
    constexpr int PW = kRows / G;        // chunk positions per wave; rows PW*G .. 31 are padding (G = 3, 5, 6, 7)
    constexpr int QT = kWaves * PW;      // chunk positions per workgroup
    constexpr int KC = D / 32;           // K-dimension chunks of S^T
    constexpr int DT = D / 16;           // output column tiles
    // LDS row pitches of K and V (bf16): 160 B at d=64, 288 B at d=128.  With
    // these SQ_LDS_BANK_CONFLICT reads zero on the C4 batch; a K pitch of
    // D + 8 put 28% of the LDS-active cycles in bank conflicts, D + 24 44%
    // (the kernel time moved by under 2%: the LDS reads are latency-, not
    // conflict-bound)
    constexpr int KSTR = D + 16;
    constexpr int VSTR = D + 16;
    static_assert(D == 64 || D == 128, "head_dim 64 or 128");
    constexpr int LPR = D / 4;                // staging lanes per key row (4 columns each)
    constexpr int KPP = 64 * kWaves / LPR;    // keys per staging pass
    constexpr int SP = kKeys / KPP;           // staging passes per tile
    static_assert(SP >= 1 && SP * KPP == kKeys, "the staging map covers whole key rows");
    __shared__ __attribute__((aligned(16))) __bf16 klds[2][kKeys * KSTR];
    __shared__ __attribute__((aligned(16))) __bf16 vlds[2][kKeys * VSTR];
    __shared__ __attribute__((aligned(16))) __bf16 klo[kX3 ? 2 : 1][kX3 ? kKeys * KSTR : 8];
    __shared__ __attribute__((aligned(16))) __bf16 vlo[kX3 ? 2 : 1][kX3 ? kKeys * VSTR : 8];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r16 = lane & 15;
    // XCD-aware order: workgroups are dispatched to the 8 XCDs round-robin by
    // id, so the chunk tiles of one (sequence, KV head) pair get ids of one
    // residue mod 8 and share that XCD's L2 for their common K/V tiles.
    // Within an XCD the ids run from the last chunk tile to the first (the
    // most keys to the fewest), pairs fastest: the dispatcher hands the next
    // id to the first CU that frees up, so the heaviest tiles start first and
    // the lightest fill in behind them (measured: 111.6 against 114.5 us on
    // the 8 x (2,048 + 512) chunk).
    const int id = static_cast<int>(blockIdx.x), xcd = id & 7, k = id >> 3;
    const int groups8 = (a.pairs + 7) >> 3;
    const int pair = (k % groups8) * 8 + xcd, ct = a.chunk_tiles - 1 - k / groups8;
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
    // (kX3: qop and qlo the fp16 parts)
    bf16x8 qop[2][KC];
    bf16x8 qlo[kX3 ? 2 : 1][kX3 ? KC : 1];
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
            const f32x4 y0 = {x0.x * s, x0.y * s, x0.z * s, x0.w * s}, y1 = {x1.x * s, x1.y * s, x1.z * s, x1.w * s};
            if constexpr (kX3) {
                // fp16 parts (11 + 11 significant bits; the MFMA keeps fp16
                // subnormals), kept in the bf16x8 registers as bits
                const f16x4 h0 = __builtin_convertvector(y0, f16x4), h1 = __builtin_convertvector(y1, f16x4);
                const f16x4 l0 = __builtin_convertvector(y0 - __builtin_convertvector(h0, f32x4), f16x4);
                const f16x4 l1 = __builtin_convertvector(y1 - __builtin_convertvector(h1, f32x4), f16x4);
                qop[nt][kc] = __builtin_bit_cast(bf16x8, f16x8{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]});
                qlo[nt][kc] = __builtin_bit_cast(bf16x8, f16x8{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]});
            } else {
                const bf16x4 lo = to_bf16(y0);
                const bf16x4 hi = to_bf16(y1);
                qop[nt][kc] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
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
            const f32x4 kv = values(kreg[p]), vv = values(vreg[p]);
            const bf16x4 vb = to_bf16(vv);
            *reinterpret_cast<bf16x4*>(&vlds[buf][(KPP * p + skey) * VSTR + col]) = vb;
            if constexpr (kX3) {
                // K as fp16 parts (the score operands), V as bf16 parts
                const f16x4 kh = __builtin_convertvector(kv, f16x4);
                *reinterpret_cast<f16x4*>(&klds[buf][(KPP * p + skey) * KSTR + col]) = kh;
                *reinterpret_cast<f16x4*>(&klo[buf][(KPP * p + skey) * KSTR + col]) =
                    __builtin_convertvector(kv - __builtin_convertvector(kh, f32x4), f16x4);
                *reinterpret_cast<bf16x4*>(&vlo[buf][(KPP * p + skey) * VSTR + col]) =
                    to_bf16(vv - __builtin_convertvector(vb, f32x4));
            } else {
                *reinterpret_cast<bf16x4*>(&klds[buf][(KPP * p + skey) * KSTR + col]) = to_bf16(kv);
            }
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
            if constexpr (kX3) {
                // per 32-column step: the hi and lo K operands, then hi*hi,
                // hi*lo and lo*hi into each score tile
#pragma unroll
                for (int kc = 0; kc < KC; ++kc) {
                    f16x8 khi[4], klw[4];
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) {
                        khi[mt] = *reinterpret_cast<const f16x8*>(&klds[buf][(16 * mt + r16) * KSTR + 32 * kc + 8 * g]);
                        klw[mt] = *reinterpret_cast<const f16x8*>(&klo[buf][(16 * mt + r16) * KSTR + 32 * kc + 8 * g]);
                    }
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                        for (int nt = 0; nt < 2; ++nt) {
                            const f16x8 qh = __builtin_bit_cast(f16x8, qop[nt][kc]);
                            const f16x8 ql = __builtin_bit_cast(f16x8, qlo[nt][kc]);
                            s[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(khi[mt], qh, s[mt][nt], 0, 0, 0);
                            s[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(khi[mt], ql, s[mt][nt], 0, 0, 0);
                            s[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(klw[mt], qh, s[mt][nt], 0, 0, 0);
                        }
                }
            } else {
                // every K operand of the tile is read before the first product, so
                // the reads' latency is paid once
                bf16x8 kop[KC][4];
#pragma unroll
                for (int kc = 0; kc < KC; ++kc)
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt)
                        kop[kc][mt] =
                            *reinterpret_cast<const bf16x8*>(&klds[buf][(16 * mt + r16) * KSTR + 32 * kc + 8 * g]);
#pragma unroll
                for (int kc = 0; kc < KC; ++kc)
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) {
                        s[mt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[kc][mt], qop[0][kc], s[mt][0], 0, 0, 0);
                        s[mt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[kc][mt], qop[1][kc], s[mt][1], 0, 0, 0);
                    }
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
            // each lane's own maximum decides the rescale (some lane's exceeds
            // the threshold exactly when some row's does); the cross-lane row
            // maximum is taken only on the first tile and the rare tile that
            // raises m, as the pipelined kernel does
            float lmax[2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                float mx = -INFINITY;
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[mt][nt][i]);
                lmax[nt] = mx;
            }
            if (first) {
                // every row sees key 0 here, so its maximum is finite
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    const float rmax = cross_row_max(lmax[nt]);
                    m[nt] = rmax;
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) s[mt][nt] -= rmax;
                }
            } else if (__any(lmax[0] > kThreshold || lmax[1] > kThreshold)) {
                // the row maximum is relative to m: raise m where the tile exceeds it
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    const float up = fmaxf(cross_row_max(lmax[nt]), 0.f);
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
            // V^T operand by transposing LDS reads (ds_read_b64_tr_b16): within
            // each 16-lane group, lane i receives element i%4 of the chunk that
            // lane 4j + i/4 addresses, as its element j; lane 16g + 4j + q
            // addresses key row 4g + j (+16 for the second half), columns
            // 16dt + 4q, so lane (g, i) gets column 16dt + i of keys 4g + j
            auto vread = [&](const __bf16* plane, int kc, int dt) {
                const __bf16* vrow = plane + (32 * kc + 4 * g + (r16 >> 2)) * VSTR + 16 * dt + 4 * (r16 & 3);
                const bf16x4 lo = tr16_read(vrow);
                const bf16x4 hi = tr16_read(vrow + 16 * VSTR);
                return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            };
            if constexpr (kX3) {
                // probabilities as hi + lo; O += Vh Ph + Vh Pl + Vl Ph and the
                // normaliser sums Ph + Pl
#pragma unroll
                for (int kc = 0; kc < 2; ++kc) {
                    bf16x8 ph[2], pl[2];
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) {
                        f32x4 p0, p1;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            p0[i] = fast_exp2(s[2 * kc][nt][i]);
                            p1[i] = fast_exp2(s[2 * kc + 1][nt][i]);
                        }
                        const bf16x4 h0 = to_bf16(p0), h1 = to_bf16(p1);
                        const bf16x4 l0 = to_bf16(p0 - __builtin_convertvector(h0, f32x4));
                        const bf16x4 l1 = to_bf16(p1 - __builtin_convertvector(h1, f32x4));
                        ph[nt] = bf16x8{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
                        pl[nt] = bf16x8{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
                    }
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) {
                        const bf16x8 vh = vread(vlds[buf], kc, dt), vl = vread(vlo[buf], kc, dt);
#pragma unroll
                        for (int nt = 0; nt < 2; ++nt) {
                            acc[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, ph[nt], acc[dt][nt], 0, 0, 0);
                            acc[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, pl[nt], acc[dt][nt], 0, 0, 0);
                            acc[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl, ph[nt], acc[dt][nt], 0, 0, 0);
                        }
                    }
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) {
                        acc[DT][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, ph[nt], acc[DT][nt], 0, 0, 0);
                        acc[DT][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pl[nt], acc[DT][nt], 0, 0, 0);
                    }
                }
                return;
            }
            bf16x8 pop0[2];
            pop0[0] = probs(0, 0);
            pop0[1] = probs(0, 1);
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) {
                bf16x8 vop[DT];
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) vop[dt] = vread(vlds[buf], kc, dt);
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

// The same tiles and arithmetic, software-pipelined within each wave.
// Iteration kt issues tile kt+1's S^T MFMAs beside the exponentials of tile
// kt, then tile kt's PV MFMAs beside the scan of tile kt+1's scores.  The
// rescale test takes each lane's own maximum: some lane's maximum exceeds the
// threshold exactly when some row's does, so the cross-lane reduction runs
// only on the rare tile that raises a running maximum.  Every product,
// exponential and rescale is the one prefill_bf16_kernel performs, in the
// same order, so the two kernels give the same bits.
//
// On MI355X this gains about 3% on the 8 x (2,048 + 512) chunk: a SIMD's
// MFMA and vector work add up rather than overlap (16 MFMAs and 32
// exponentials of one wave take 443 cycles against 264 and 275 apart, 405 of
// 240 and 255 with two waves per SIMD), so the order within a wave matters
// little.  What sets the time is the sum per 64-key tile and wave: 36 MFMAs
// (576 cycles), 24 LDS operand reads, 32 exponentials and the staging.
//
// LDS keeps K one tile ahead of V: iteration kt reads K of tile kt+1 (buffer
// (kt+1)&1) and V of tile kt (buffer kt&1), and writes K of tile kt+2 and V
// of tile kt+1 into the other two, so one barrier per tile suffices.  The
// rows written in iteration kt were requested from HBM one iteration before.
template <int D, int G, int kWaves, int NT, bool kQ8, int TPB>
__global__ __launch_bounds__(64 * kWaves) void prefill_pipe_kernel(const PrefillArgs a) {
    constexpr int WR = 16 * NT;  // rows per wave: NT tiles of 16
    constexpr int PW = WR / G;
    constexpr int QT = kWaves * PW;
    constexpr int KC = D / 32;
    constexpr int DT = D / 16;
    constexpr int KSTR = D + 16;  // as prefill_bf16_kernel
    constexpr int VSTR = D + 16;
    static_assert(D == 64 || D == 128, "head_dim 64 or 128");
    constexpr int LPR = D / 4;
    constexpr int KPP = 64 * kWaves / LPR;
    constexpr int SP = kKeys / KPP;
    static_assert(SP >= 1 && SP * KPP == kKeys, "the staging map covers whole key rows");
    __shared__ __attribute__((aligned(16))) __bf16 klds[2][kKeys * KSTR];
    __shared__ __attribute__((aligned(16))) __bf16 vlds[2][kKeys * VSTR];

    // the wave index is uniform: in a scalar register, every branch on a
    // wave's rows and every block-table lookup is scalar
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    // workgroup order as in prefill_bf16_kernel
    const int id = static_cast<int>(blockIdx.x), xcd = id & 7, k = id >> 3;
    const int groups8 = (a.pairs + 7) >> 3;
    const int pair = (k % groups8) * 8 + xcd, ct = a.chunk_tiles - 1 - k / groups8;
    if (pair >= a.pairs) return;
    const int kh = pair % a.lay.kv_heads;
    const int4 sd = a.seqs[pair / a.lay.kv_heads];
    const int start = sd.y, nrows = sd.z;
    const int q0 = ct * QT;
    if (q0 >= nrows) return;
    const int kmax = start + min(q0 + QT, nrows);
    const int ntiles = (kmax + kKeys - 1) / kKeys;
    const int pw0 = q0 + wave * PW;
    const int wave_kmax = pw0 < nrows ? start + min(pw0 + PW, nrows) : 0;
    const int wtiles = (wave_kmax + kKeys - 1) / kKeys;  // tiles this wave's rows see (0: no rows)
    const int kvw = a.lay.kv_width;
    const int32_t* tab = a.tables + sd.x;

    bf16x8 qop[NT][KC];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
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

    // staging map and block addressing as in prefill_bf16_kernel
    const int skey = tid / LPR, col = 4 * (tid % LPR);
    const int wkey = __builtin_amdgcn_readfirstlane(skey);
    const int tpb = TPB ? TPB : a.lay.tpb, tsh = __builtin_ctz(static_cast<unsigned>(tpb));
    const int lslot = skey & (tpb - 1);
    const unsigned roff =
        static_cast<unsigned>(kQ8 ? lslot * D + col : (lslot * kvw + col) * static_cast<int>(sizeof(float)));
    const unsigned soff = static_cast<unsigned>(tpb * D + (lslot * (D / 32) + col / 32) * 2);
    const int kvh = kh / a.kv_share;
    const size_t kbytes = kQ8 ? static_cast<size_t>(a.layer) * 2 * a.lay.section + static_cast<size_t>(kvh) * a.lay.head_bytes
                              : (static_cast<size_t>(a.layer) * 2 * tpb * kvw + static_cast<size_t>(kvh) * D) * sizeof(float);
    const int vsec = static_cast<int>(kQ8 ? a.lay.section : static_cast<size_t>(tpb) * kvw * sizeof(float));
    const int brange = static_cast<int>(a.lay.stride - kbytes);
    // Loads are unconditional: rows past the chunk's reach read the last
    // reachable block (see prefill_bf16_kernel); tiles past the last re-read it.
    auto tile = [&](int t) { return min(t, ntiles - 1); };
    auto blocks = [&](int kt, int (&b)[SP]) {
#pragma unroll
        for (int p = 0; p < SP; ++p) b[p] = tab[min(kt * kKeys + KPP * p + wkey, kmax - 1) >> tsh];
    };
    // one half (K: sec 0, V: sec vsec) of tile kt's rows
    auto load = [&](int kt, const int (&b)[SP], int sec, f32x4 (&reg)[SP]) {
#pragma unroll
        for (int p = 0; p < SP; ++p) {
            const int base = (kt * kKeys + KPP * p) & (tpb - 1);
            const int rso = base * (kQ8 ? D : kvw * static_cast<int>(sizeof(float))), sso = base * (D / 32) * 2;
            const char* blk =
                a.pool + static_cast<size_t>(__builtin_amdgcn_readfirstlane(b[p])) * a.lay.stride + kbytes;
            const __amdgpu_buffer_rsrc_t r =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(blk), 0, brange, kBufferWord3);
            if constexpr (kQ8) {
                const unsigned q = __builtin_amdgcn_raw_buffer_load_b32(r, roff, sec + rso, 0);
                const unsigned sc = __builtin_amdgcn_raw_buffer_load_b16(r, soff, sec + sso, 0);
                reg[p] = f32x4{__builtin_bit_cast(float, q), __builtin_bit_cast(float, sc), 0.f, 0.f};
            } else {
                reg[p] = __builtin_amdgcn_raw_buffer_load_b128(r, roff, sec + rso, 0);
            }
        }
    };
    auto values = [](f32x4 x) {
        if constexpr (kQ8) {
            const float x0 = x[0], x1 = x[1];
            const uint32_t q = __builtin_bit_cast(uint32_t, x0);
            const float d = half_bits_to_float(static_cast<uint16_t>(__builtin_bit_cast(uint32_t, x1)));
            return f32x4{sbyte_to_float<0>(q) * d, sbyte_to_float<1>(q) * d, sbyte_to_float<2>(q) * d,
                         sbyte_to_float<3>(q) * d};
        } else {
            return x;
        }
    };
    auto kstore = [&](int buf, const f32x4 (&reg)[SP]) {
#pragma unroll
        for (int p = 0; p < SP; ++p)
            *reinterpret_cast<bf16x4*>(&klds[buf][(KPP * p + skey) * KSTR + col]) = to_bf16(values(reg[p]));
    };
    auto vstore = [&](int kt, int buf, f32x4 (&reg)[SP]) {
        if (kt * kKeys + kKeys > kmax) {  // the chunk's last tile: zero V past its reach
#pragma unroll
            for (int p = 0; p < SP; ++p)
                if (kt * kKeys + KPP * p + skey >= kmax) reg[p] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int p = 0; p < SP; ++p)
            *reinterpret_cast<bf16x4*>(&vlds[buf][(KPP * p + skey) * VSTR + col]) = to_bf16(values(reg[p]));
    };

    f32x4 acc[DT + 1][NT];
#pragma unroll
    for (int dt = 0; dt <= DT; ++dt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const __bf16 one = r16 == 0 ? static_cast<__bf16>(1.f) : static_cast<__bf16>(0.f);
    const bf16x8 ones = bf16x8{one, one, one, one, one, one, one, one};
    float m[NT];
    int lim[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        m[nt] = -INFINITY;
        lim[nt] = start + pw0 + (16 * nt + r16) / G;
    }

    typedef f32x4 Scores[4][NT];
    typedef bf16x8 KOps[KC][4];
    typedef bf16x8 VOps[2][DT];
    // every K operand of the tile in K buffer kb, and every V operand (V^T by
    // transposing reads, in the probabilities' key order: lane (g, i) gets
    // column 16dt + i of keys 4g + j and 16 + 4g + j of key half kc) of the
    // tile in V buffer vb
    auto kops = [&](int kb, KOps& k) {
#pragma unroll
        for (int kc = 0; kc < KC; ++kc)
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
                k[kc][mt] = *reinterpret_cast<const bf16x8*>(&klds[kb][(16 * mt + r16) * KSTR + 32 * kc + 8 * g]);
    };
    auto vops = [&](int vb, VOps& v) {
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const __bf16* vrow = &vlds[vb][(32 * kc + 4 * g + (r16 >> 2)) * VSTR + 16 * dt + 4 * (r16 & 3)];
                const bf16x4 lo = tr16_read(vrow);
                const bf16x4 hi = tr16_read(vrow + 16 * VSTR);
                v[kc][dt] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
    };
    // S^T of row tile nt: accumulators starting at -m (0 before the first tile)
    auto scores = [&](const KOps& k, Scores& s, int nt, bool first) {
        const float c = first ? 0.f : -m[nt];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) s[mt][nt] = f32x4{c, c, c, c};
#pragma unroll
        for (int kc = 0; kc < KC; ++kc)
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
                s[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k[kc][mt], qop[nt][kc], s[mt][nt], 0, 0, 0);
    };
    // the causal mask, for tiles that reach past a row's own position
    auto mask = [&](int kbase, Scores& s) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (kbase + 16 * mt + 4 * g + i > lim[nt]) s[mt][nt][i] = -INFINITY;
    };
    auto lane_max = [](const Scores& s, int nt) {
        float mx = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[mt][nt][i]);
        return mx;
    };
    // raise each row's running maximum to the tile's (the tile's scores are
    // relative to the old one) and rescale what was accumulated
    auto rescale = [&](Scores& s) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const float up = fmaxf(cross_row_max(lane_max(s, nt)), 0.f);
            const float alpha = fast_exp2(-up);
            m[nt] += up;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) s[mt][nt] -= up;
#pragma unroll
            for (int dt = 0; dt <= DT; ++dt) acc[dt][nt] *= alpha;
        }
    };
    // P^T (B operand of O^T = V^T P^T) for key half kc and row tile nt
    auto probs = [](const Scores& s, int nt, int kc) {
        float p[2][4];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) p[h][i] = fast_exp2(s[2 * kc + h][nt][i]);
        const bf16x4 lo = to_bf16(make_float4(p[0][0], p[0][1], p[0][2], p[0][3]));
        const bf16x4 hi = to_bf16(make_float4(p[1][0], p[1][1], p[1][2], p[1][3]));
        return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    // Prologue: K and V of tile 0 and K of tile 1 in LDS, tile 0's scores in
    // registers.  Staging then runs K one tile ahead of V: iteration kt
    // writes K of tile kt+2 and V of tile kt+1, whose rows were requested
    // from HBM one iteration earlier (requesting them two iterations earlier,
    // in alternating register sets, measured no faster).
    f32x4 kreg[SP], vreg[SP];
    int bK[SP], bV[SP];  // block ids of the next loads (K of tile kt+3, V of tile kt+2)
    Scores s;            // the current tile's scores, score - m, updated in place
    {
        f32x4 k0[SP], v0[SP], k1[SP];
        int b0[SP], b1[SP], b2[SP];
        blocks(0, b0);
        blocks(tile(1), b1);
        blocks(tile(2), b2);
        load(0, b0, 0, k0);
        load(0, b0, vsec, v0);
        load(tile(1), b1, 0, k1);
        load(tile(2), b2, 0, kreg);
        load(tile(1), b1, vsec, vreg);
        blocks(tile(3), bK);
        blocks(tile(2), bV);
        kstore(0, k0);
        vstore(0, 0, v0);
        kstore(1, k1);
    }
    __syncthreads();
    if (wtiles > 0) {
        KOps k;
        kops(0, k);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) scores(k, s, nt, true);
        if (kKeys - 1 > start + pw0) mask(0, s);
        // every row sees key 0 in tile 0, so its maximum is finite
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            m[nt] = cross_row_max(lane_max(s, nt));
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) s[mt][nt] -= m[nt];
        }
    }
    __syncthreads();  // tile 0's K is read before iteration 0 overwrites it

    // Iteration kt (cb = kt & 1: reads K of tile kt+1 from buffer nb, V of
    // tile kt from buffer cb; writes K of tile kt+2 to cb and V of tile kt+1
    // to nb).  The row tiles go in two halves: half h's probabilities of tile
    // kt leave s as bf16, then tile kt+1's scores for those rows are computed
    // into the same registers while the other half is exponentiated.  Tile
    // kt+1's scores are computed even past the wave's last tile (from
    // whatever K buffer nb then holds, never used), so that every product and
    // exponential of the iteration shares one basic block and one schedule.
    constexpr int H = NT / 2;
    auto step = [&](int kt, const int cb) {
        const int nb = cb ^ 1;
        if (kt < wtiles) {
            KOps k;
            VOps v;
            kops(nb, k);
            vops(cb, v);
            bf16x8 pop[2][NT];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int nt = h * H; nt < h * H + H; ++nt) {
                    pop[0][nt] = probs(s, nt, 0);
                    pop[1][nt] = probs(s, nt, 1);
                }
#pragma unroll
                for (int nt = h * H; nt < h * H + H; ++nt) scores(k, s, nt, false);
            }
#pragma unroll
            for (int kc = 0; kc < 2; ++kc)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt)
                        acc[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v[kc][dt], pop[kc][nt], acc[dt][nt], 0, 0, 0);
                    acc[DT][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pop[kc][nt], acc[DT][nt], 0, 0, 0);
                }
            const int kn = (kt + 1) * kKeys;
            if (kn + kKeys - 1 > start + pw0) mask(kn, s);  // a tile reaching past a row's own position
            bool up = false;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) up |= lane_max(s, nt) > kThreshold;
            if (kt + 1 < wtiles && __any(up)) rescale(s);
        }
        kstore(cb, kreg);
        vstore(tile(kt + 1), nb, vreg);
        load(tile(kt + 3), bK, 0, kreg);
        load(tile(kt + 2), bV, vsec, vreg);
        blocks(tile(kt + 4), bK);
        blocks(tile(kt + 3), bV);
        __syncthreads();
    };
    // Both halves always run (the second's products are skipped past the
    // last tile by kt < wtiles; its staging then re-reads the last tile):
    // a break between them would give the loop a path on which the first
    // half's loads are still in flight at the top, and the compiler would
    // wait for them there.
    for (int kt = 0; kt < ntiles; kt += 2) {
        step(kt, 0);
        step(kt + 1, 1);
    }

    bool bad = false;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
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

// Kernel choice, TVARA_PREFILL_PIPE (read on every launch, so one process
// can compare them; results are bit-identical): 0 prefill_bf16_kernel, 1
// prefill_pipe_kernel; unset, the pipelined kernel at head_dim 64 and the
// plain one at 128, where the pipelined kernel's operand sets do not fit in
// registers beside its accumulators.  Both run eight waves of 32 rows, 256
// rows per workgroup, over 64-key tiles (eight waves of the plain kernel
// measured 158 against 225 us for four on the 8 x (2,048 + 512) chunk;
// 128-key tiles 177 us).
//
// x3 (three products per product) always takes the plain kernel, over f32
// or Q8_0 blocks (d * q dequantised when staged, then split).
template <int D, int G, int TPB>
void launch_gt(const PrefillArgs& a, int nseqs, int max_rows, bool x3, hipStream_t s) {
    const char* env = std::getenv("TVARA_PREFILL_PIPE");
    const bool pipe = env ? std::atoi(env) != 0 : D == 64;
    const bool q8 = a.lay.format == kQ8;
    constexpr int W = 8, QT = W * (kRows / G);  // chunk positions per workgroup
    PrefillArgs b = a;
    b.chunk_tiles = (max_rows + QT - 1) / QT;
    b.pairs = nseqs * a.lay.kv_heads;
    const int groups8 = (b.pairs + 7) / 8;  // ids = 8 XCDs x chunk tiles x pair groups
    const dim3 grid(8 * groups8 * b.chunk_tiles), block(64 * W);
    if (x3) {
        if (q8)
            launch("paged_prefill_x3", prefill_bf16_kernel<D, G, W, true, TPB, true>, grid, block, 0, s, b);
        else
            launch("paged_prefill_x3", prefill_bf16_kernel<D, G, W, false, TPB, true>, grid, block, 0, s, b);
    } else if (pipe) {
        if (q8)
            launch("paged_prefill_bf16", prefill_pipe_kernel<D, G, W, 2, true, TPB>, grid, block, 0, s, b);
        else
            launch("paged_prefill_bf16", prefill_pipe_kernel<D, G, W, 2, false, TPB>, grid, block, 0, s, b);
    } else if (q8) {
        launch("paged_prefill_bf16", prefill_bf16_kernel<D, G, W, true, TPB>, grid, block, 0, s, b);
    } else {
        launch("paged_prefill_bf16", prefill_bf16_kernel<D, G, W, false, TPB>, grid, block, 0, s, b);
    }
}

// blocks of 16 tokens fold the block arithmetic at compile time; other
// powers of two read it from the layout
template <int G>
void launch_g(const PrefillArgs& a, int nseqs, int max_rows, bool x3, hipStream_t s) {
    if (a.lay.head_dim == 128)
        a.lay.tpb == 16 ? launch_gt<128, G, 16>(a, nseqs, max_rows, x3, s)
                        : launch_gt<128, G, 0>(a, nseqs, max_rows, x3, s);
    else
        a.lay.tpb == 16 ? launch_gt<64, G, 16>(a, nseqs, max_rows, x3, s)
                        : launch_gt<64, G, 0>(a, nseqs, max_rows, x3, s);
}

}  // namespace

bool prefill_bf16_supported(const BlockLayout& lay, int group) {
    // the staging reads take 32-bit offsets within a block
    return (lay.format == kF32 || lay.format == kQ8) && decode_f32_blocks(lay.tpb) &&
           (lay.head_dim == 64 || lay.head_dim == 128) &&
           lay.stride < (size_t(1) << 31) && group >= 1 && group <= 8;
}

bool prefill_x3_supported(const BlockLayout& lay, int group) { return prefill_bf16_supported(lay, group); }

void launch_prefill_bf16(const PrefillArgs& a, int nseqs, int max_rows, hipStream_t s, bool x3) {
    if (!prefill_bf16_supported(a.lay, a.group))
        throw std::invalid_argument(
            "bf16 prefill needs f32 or Q8_0 blocks of 16 to 1,024 tokens (a power of two, under 2 GiB), "
            "head_dim 64 or 128, and a GQA slice of 1-8 heads");
    if (nseqs <= 0 || max_rows <= 0) return;
    switch (a.group) {
        case 1: launch_g<1>(a, nseqs, max_rows, x3, s); break;
        case 2: launch_g<2>(a, nseqs, max_rows, x3, s); break;
        case 3: launch_g<3>(a, nseqs, max_rows, x3, s); break;
        case 4: launch_g<4>(a, nseqs, max_rows, x3, s); break;
        case 5: launch_g<5>(a, nseqs, max_rows, x3, s); break;
        case 6: launch_g<6>(a, nseqs, max_rows, x3, s); break;
        case 7: launch_g<7>(a, nseqs, max_rows, x3, s); break;
        default: launch_g<8>(a, nseqs, max_rows, x3, s); break;
    }
    TVARA_HIP(hipGetLastError());
}

}  // namespace tvara_amd
