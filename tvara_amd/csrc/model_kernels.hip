// Device kernels of the Llama decode executor around the paged attention
// path: weight dequantisation at load, RMSNorm, matrix-vector products,
// rotary embedding and the SwiGLU gate (core/include/tvara/model.hpp:47-126,
// core/include/tvara/quant.hpp:14-71,178-184).
//
// Rounding follows the reference's: products and sums the reference rounds to
// float one at a time are written with __fmul_rn / __fsub_rn / __fadd_rn so
// the compiler does not contract them into FMAs; dot products and the RMS sum
// accumulate in double and round once, as quant::dot_f32 and rms_norm do.
#include <algorithm>

#include "model.hpp"
#include "q8.hpp"
#include "device_util.hpp"

namespace tvara_amd {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ void flag_bad(int* bad, float v) {
    if (!__builtin_isfinite(v)) atomicOr(bad, 1);
}

// ------------------------------------------------------------ dequantisation

__global__ void check_f32_kernel(const float* w, size_t n, int* bad) {
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        flag_bad(bad, w[i]);
}

__global__ void f16_kernel(const uint8_t* raw, size_t n, float* out, int* bad) {
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const uint16_t h = static_cast<uint16_t>(raw[2 * i] | (raw[2 * i + 1] << 8));
        const float v = half_bits_to_float(h);
        out[i] = v;
        flag_bad(bad, v);
    }
}

// Q8_0: 34-byte groups, x = d * q (quant.hpp:39-49)
__global__ void q8_0_kernel(const uint8_t* raw, size_t n, float* out, int* bad) {
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const uint8_t* g = raw + (i / 32) * 34;
        const float d = half_bits_to_float(static_cast<uint16_t>(g[0] | (g[1] << 8)));
        const float v = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(g[2 + i % 32])));
        out[i] = v;
        flag_bad(bad, v);
    }
}

// Q4_0: 18-byte groups; byte j holds elements j (low nibble) and j+16 (high),
// x = d * (q - 8) (quant.hpp:50-60)
__global__ void q4_0_kernel(const uint8_t* raw, size_t n, float* out, int* bad) {
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const uint8_t* g = raw + (i / 32) * 18;
        const int e = static_cast<int>(i % 32);
        const float d = half_bits_to_float(static_cast<uint16_t>(g[0] | (g[1] << 8)));
        const unsigned q = e < 16 ? (g[2 + e] & 15u) : (g[2 + e - 16] >> 4);
        const float v = __fmul_rn(d, static_cast<float>(static_cast<int>(q) - 8));
        out[i] = v;
        flag_bad(bad, v);
    }
}

// Q4_K: 144-byte super-blocks of 256: fp16 d, fp16 dmin, 12 bytes of 6-bit
// (scale, min) pairs for eight groups of 32, then 128 bytes of nibbles
// (group g reads byte 16 + (g/2)*32 + i, high nibble for odd g);
// x = d*scale*q - dmin*min (quant.hpp:62-85)
__global__ void q4_k_kernel(const uint8_t* raw, size_t n, float* out, int* bad) {
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const uint8_t* b = raw + (i / 256) * 144;
        const int e = static_cast<int>(i % 256), g = e / 32, k = e % 32;
        const float d = half_bits_to_float(static_cast<uint16_t>(b[0] | (b[1] << 8)));
        const float dmin = half_bits_to_float(static_cast<uint16_t>(b[2] | (b[3] << 8)));
        const uint8_t* s = b + 4;
        unsigned sc, mn;
        if (g < 4) {
            sc = s[g] & 63u;
            mn = s[g + 4] & 63u;
        } else {
            sc = (s[g + 4] & 15u) | ((s[g - 4] >> 6) << 4);
            mn = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
        }
        const unsigned packed = b[16 + (g / 2) * 32 + k];
        const unsigned q = (g & 1) ? (packed >> 4) : (packed & 15u);
        const float v = __fsub_rn(__fmul_rn(__fmul_rn(d, static_cast<float>(sc)), static_cast<float>(q)),
                                  __fmul_rn(dmin, static_cast<float>(mn)));
        out[i] = v;
        flag_bad(bad, v);
    }
}

// ------------------------------------------------------------------- RMSNorm

// out = x * float(1/sqrt(sum(x^2)/n + eps)) * w, the sum in double
// (model.hpp:54-61); one workgroup
__global__ __launch_bounds__(1024) void rmsnorm_kernel(const float* x, const float* w, float* out, int n, float eps) {
    __shared__ double part[1024 / 64];
    __shared__ float inv;
    x += static_cast<size_t>(blockIdx.x) * n;  // one workgroup per row of a batch
    out += static_cast<size_t>(blockIdx.x) * n;
    double sum = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) sum += static_cast<double>(x[i]) * x[i];
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0;
        for (int k = 0; k < static_cast<int>(blockDim.x >> 6); ++k) t += part[k];
        inv = static_cast<float>(1.0 / sqrt(t / static_cast<double>(n) + static_cast<double>(eps)));
    }
    __syncthreads();
    const float iv = inv;
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = __fmul_rn(__fmul_rn(x[i], iv), w[i]);
}

// ------------------------------------------------------------- matvec

// y = W v for row-major W [rows][cols]: one wave per row, double accumulation
// rounded once (quant::dot_f32); output rows are cut into up to three
// segments, each written to its own buffer, optionally as residual + y (the
// reference's x[j] += residual[j]).
struct MatvecArgs {
    const float* w;
    const float* v;
    int rows, cols;
    MatvecSegment seg[3];
    int nseg;
};

template <bool VEC>
__global__ __launch_bounds__(kThreads) void matvec_kernel(const MatvecArgs a) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const float* wr = a.w + static_cast<size_t>(row) * a.cols;
    double acc = 0;
    if constexpr (VEC) {
        const int c4 = a.cols / 4;
        for (int k = lane; k < c4; k += 64) {
            const float4 w4 = reinterpret_cast<const float4*>(wr)[k];
            const float4 v4 = reinterpret_cast<const float4*>(a.v)[k];
            acc = fma(static_cast<double>(w4.x), static_cast<double>(v4.x), acc);
            acc = fma(static_cast<double>(w4.y), static_cast<double>(v4.y), acc);
            acc = fma(static_cast<double>(w4.z), static_cast<double>(v4.z), acc);
            acc = fma(static_cast<double>(w4.w), static_cast<double>(v4.w), acc);
        }
    } else {
        for (int k = lane; k < a.cols; k += 64) acc = fma(static_cast<double>(wr[k]), static_cast<double>(a.v[k]), acc);
    }
    for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
    if (lane) return;
    int r = row, s = 0;
    while (s + 1 < a.nseg && r >= a.seg[s].rows) r -= a.seg[s++].rows;
    const float y = static_cast<float>(acc);
    float* out = a.seg[s].out;
    out[r] = a.seg[s].residual ? __fadd_rn(a.seg[s].residual[r], y) : y;
}

// Y[j] = W X[j] for a batch of vectors (one per sequence), as a skinny GEMM:
// a workgroup owns 64 rows of W and up to 64 vectors; K advances in chunks
// of 32 columns staged in LDS (W tile [64][32], X tile [64][32], double
// buffered), and each thread accumulates a 4-row x 4-vector micro-tile in
// f32.  Every weight is read from HBM once per launch; the X tile comes from
// L2.
constexpr int kTileRows = 64, kTileVecs = 64, kTileK = 32;

struct BatchMatvecArgs {
    const float* w;
    const float* x;  // [n][cols]
    int rows, cols, n;
    MatvecSegment seg[3];  // output j of segment s: seg.out[j * seg.rows + r]
    int nseg;
    int chunks_per_split;  // K chunks of kTileK per blockIdx.y
    float* partial;        // split-K: [gridDim.y][n_total][rows] partial sums, else null
    int n_total, j0;       // partial layout: vector stride and this launch's first vector
};

__global__ __launch_bounds__(256) void batch_matvec_kernel(const BatchMatvecArgs a) {
    __shared__ float ws[2][kTileRows][kTileK + 4];
    __shared__ float xs[2][kTileVecs][kTileK + 4];
    const int t = threadIdx.x;
    const int row0 = blockIdx.x * kTileRows;
    // staging map: thread t copies float4 (t % 8) of rows t/8 and t/8 + 32
    const int sc = (t % 8) * 4, sr = t / 8;
    // micro-tile: rows 4*(t%16) .. +3, vectors 4*(t/16) .. +3
    const int mr = (t % 16) * 4, mv = (t / 16) * 4;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
    auto stage = [&](int buf, int k0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int r = sr + 32 * h;
            float4 w = make_float4(0.f, 0.f, 0.f, 0.f), x = w;
            if (row0 + r < a.rows) w = *reinterpret_cast<const float4*>(a.w + static_cast<size_t>(row0 + r) * a.cols + k0 + sc);
            if (r < a.n) x = *reinterpret_cast<const float4*>(a.x + static_cast<size_t>(r) * a.cols + k0 + sc);
            *reinterpret_cast<float4*>(&ws[buf][r][sc]) = w;
            *reinterpret_cast<float4*>(&xs[buf][r][sc]) = x;
        }
    };
    const int kbeg = blockIdx.y * a.chunks_per_split;
    const int nk = min(a.cols / kTileK - kbeg, a.chunks_per_split);
    stage(0, kbeg * kTileK);
    __syncthreads();
    for (int kc = 0; kc < nk; ++kc) {
        const int buf = kc & 1;
        if (kc + 1 < nk) stage(buf ^ 1, (kbeg + kc + 1) * kTileK);
#pragma unroll
        for (int k = 0; k < kTileK; k += 4) {
            float4 w4[4], x4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) w4[i] = *reinterpret_cast<const float4*>(&ws[buf][mr + i][k]);
#pragma unroll
            for (int j = 0; j < 4; ++j) x4[j] = *reinterpret_cast<const float4*>(&xs[buf][mv + j][k]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j] = fmaf(w4[i].x, x4[j].x, acc[i][j]);
                    acc[i][j] = fmaf(w4[i].y, x4[j].y, acc[i][j]);
                    acc[i][j] = fmaf(w4[i].z, x4[j].z, acc[i][j]);
                    acc[i][j] = fmaf(w4[i].w, x4[j].w, acc[i][j]);
                }
        }
        __syncthreads();
    }
    if (a.partial) {  // split-K: the fixed-order sum happens afterwards
        float* p = a.partial + static_cast<size_t>(blockIdx.y) * a.n_total * a.rows;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (row0 + mr + i < a.rows && mv + j < a.n)
                    p[static_cast<size_t>(a.j0 + mv + j) * a.rows + row0 + mr + i] = acc[i][j];
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = row0 + mr + i;
        if (row >= a.rows) break;
        int rr = row, sg = 0;
        while (sg + 1 < a.nseg && rr >= a.seg[sg].rows) rr -= a.seg[sg++].rows;
        const MatvecSegment& S = a.seg[sg];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (mv + j >= a.n) break;
            const size_t at = static_cast<size_t>(mv + j) * S.rows + rr;
            S.out[at] = S.residual ? __fadd_rn(S.residual[at], acc[i][j]) : acc[i][j];
        }
    }
}

// y[j][r] = sum over splits s (in order) of partial[s][j][r], to the segments
__global__ void split_sum_kernel(const BatchMatvecArgs a, int splits) {
    const size_t total = static_cast<size_t>(a.n) * a.rows;
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        float sum = 0.f;
        for (int sp = 0; sp < splits; ++sp) sum += a.partial[static_cast<size_t>(sp) * total + i];
        const int j = static_cast<int>(i / a.rows);
        int rr = static_cast<int>(i % a.rows), sg = 0;
        while (sg + 1 < a.nseg && rr >= a.seg[sg].rows) rr -= a.seg[sg++].rows;
        const MatvecSegment& S = a.seg[sg];
        const size_t at = static_cast<size_t>(j) * S.rows + rr;
        S.out[at] = S.residual ? __fadd_rn(S.residual[at], sum) : sum;
    }
}

// out[j] = table[idx[j]] (embedding rows of a batch)
__global__ void gather_embedding_kernel(const float* table, const uint32_t* idx, int n, int h, float* out) {
    const size_t total = static_cast<size_t>(n) * h;
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        out[i] = table[static_cast<size_t>(idx[i / h]) * h + i % h];
}

// [layers][n][kv] -> [n][layers][kv] (one token row per sequence for the append)
__global__ void interleave_layers_kernel(const float* src, float* dst, int layers, int n, int kv) {
    const size_t total = static_cast<size_t>(layers) * n * kv;
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const size_t e = i % kv, j = (i / kv) % n, l = i / (static_cast<size_t>(kv) * n);
        dst[(j * layers + l) * kv + e] = src[i];
    }
}

// ------------------------------------------------------------- RoPE

// rotate pair i of every head of q and k by the (cos, sin) of this position
// (model.hpp:63-72): interleaved pairs (2i, 2i+1) or split (i, i+dim/2)
__global__ void rope_kernel(float* q, int qheads, float* k, int kheads, int dim, const float* cs, int interleaved) {
    const int half = dim / 2;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (qheads + kheads) * half) return;
    // row blockIdx.y of a batch: its own position's (cos, sin)
    q += static_cast<size_t>(blockIdx.y) * qheads * dim;
    k += static_cast<size_t>(blockIdx.y) * kheads * dim;
    cs += static_cast<size_t>(blockIdx.y) * dim;
    const int h = t / half, i = t % half;
    float* x = h < qheads ? q + static_cast<size_t>(h) * dim : k + static_cast<size_t>(h - qheads) * dim;
    const int ia = interleaved ? 2 * i : i, ib = interleaved ? 2 * i + 1 : i + half;
    const float c = cs[2 * i], s = cs[2 * i + 1];
    const float left = x[ia], right = x[ib];
    x[ia] = __fsub_rn(__fmul_rn(left, c), __fmul_rn(right, s));
    x[ib] = __fadd_rn(__fmul_rn(right, c), __fmul_rn(left, s));
}

// ------------------------------------------------------------- SwiGLU

// gate = gate * (sigmoid(gate) * up), the sigmoid in the overflow-free form
// of model.hpp:111-116
__global__ void swiglu_kernel(float* gate, const float* up, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float g = gate[i];
    const float small = expf(-fabsf(g));
    const float one = __fadd_rn(1.f, small);
    const float sig = g >= 0 ? __fdiv_rn(1.f, one) : __fdiv_rn(small, one);
    gate[i] = __fmul_rn(g, __fmul_rn(sig, up[i]));
}

// ------------------------------------------------------------- Q8_0 weights

// one thread per (row, group): the 34-byte GGUF group to its tile slots
__global__ void q8_repack_kernel(const uint8_t* raw, int rows, int groups, int row0, int stride, uint8_t* q,
                                 uint16_t* d, int* bad) {
    const int pairs = (groups + 1) / 2;
    const size_t total = static_cast<size_t>(rows) * groups;
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const int r = static_cast<int>(i / groups), g = static_cast<int>(i % groups);
        const uint8_t* src = raw + i * 34;
        const int row = row0 + r * stride, rr = row % 16;
        const size_t block = static_cast<size_t>(row / 16) * pairs + g / 2;
        const uint16_t h = static_cast<uint16_t>(src[0] | (src[1] << 8));
        d[(block * 16 + rr) * 2 + g % 2] = h;
        if (!__builtin_isfinite(half_bits_to_float(h))) atomicOr(bad, 1);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint8_t* dst = q + (block * 64 + rr + 16 * j) * 16 + (g % 2) * 8;
#pragma unroll
            for (int b = 0; b < 8; ++b) dst[b] = src[2 + 8 * j + b];
        }
    }
}

struct Q8MatvecArgs {
    const uint4* q;
    const uint32_t* d;  // the two groups' fp16 scales of a row, per (tile, pair)
    const float* v;     // the input, or x when norm_w is set
    const float* norm_w;  // RMSNorm weight: the input is rms_norm(x) * norm_w
    float eps;
    int rows, tiles, groups, pairs, cols;
    MatvecSegment seg[3];
    int nseg;
    // epilogue on adjacent row pairs (2i, 2i+1): rotate the first rope_rows
    // rows by rope_cs (interleaved RoPE over rope_dim-wide heads), or, with
    // swiglu, write gate * (sigmoid(gate) * up) of rows (gate i, up i) to
    // seg[0].out[i]
    const float* rope_cs;
    int rope_dim, rope_rows;
    int swiglu;
};

// sum of 8 int8 (two dwords) times 8 floats, in f32
__device__ __forceinline__ float dot8(uint32_t lo, uint32_t hi, float4 a, float4 b) {
    float s = sbyte_to_float<0>(lo) * a.x;
    s = fmaf(sbyte_to_float<1>(lo), a.y, s);
    s = fmaf(sbyte_to_float<2>(lo), a.z, s);
    s = fmaf(sbyte_to_float<3>(lo), a.w, s);
    s = fmaf(sbyte_to_float<0>(hi), b.x, s);
    s = fmaf(sbyte_to_float<1>(hi), b.y, s);
    s = fmaf(sbyte_to_float<2>(hi), b.z, s);
    return fmaf(sbyte_to_float<3>(hi), b.w, s);
}

__device__ __forceinline__ void write_segment(const MatvecSegment* seg, int nseg, int row, size_t col_offset_rows,
                                              float y) {
    int r = row, s = 0;
    while (s + 1 < nseg && r >= seg[s].rows) r -= seg[s++].rows;
    const size_t at = col_offset_rows * seg[s].rows + r;
    seg[s].out[at] = seg[s].residual ? __fadd_rn(seg[s].residual[at], y) : y;
}

// y = W v over Q8_0 tiles: a workgroup per RT 16-row tiles, its W waves
// taking contiguous shares of the group pairs, U pairs a step with every
// load issued first (16 bytes of weights per lane per tile and pair).  The
// input vector is staged in LDS first -- normalised there when the product
// follows an RMSNorm (model.hpp:54-61: sum of squares in double, the scale
// rounded to float, (x * s) * w), which each workgroup computes for itself.
// Lane l accumulates row l%16 of each tile over its eight columns of each
// group: the eight products in f32, times the group's d, added in double;
// lanes and waves are then summed in double and each row rounds to float
// once.  Pairs past the share, and the zero group that completes an odd
// count, are selected away rather than multiplied (their loads stay in
// bounds).
template <int W, int RT>
__global__ __launch_bounds__(W * 64) void matvec_q8_kernel(const Q8MatvecArgs a) {
    constexpr int U = 2;
    extern __shared__ float vs[];  // cols floats
    __shared__ double red[W][RT][16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int P = a.pairs, G = a.groups, C = a.cols;
    const int per = (P + W - 1) / W;
    const int p0 = min(P, wave * per), p1 = min(P, p0 + per);
    int tl[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) tl[r] = min(static_cast<int>(blockIdx.x) * RT + r, a.tiles - 1);
    // U pairs of every tile from pair p on, clamped to the wave's last pair
    // (a wave without pairs reads pair P - 1 and adds nothing)
    auto load = [&](int p, uint4 (&qq)[RT][U], uint32_t (&dd)[RT][U]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int pc = min(p + u, p1 - 1);
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const size_t blk = static_cast<size_t>(tl[r]) * P + pc;
                qq[r][u] = a.q[blk * 64 + lane];
                dd[r][u] = a.d[blk * 16 + (lane & 15)];
            }
        }
    };
    // the first step's weights are requested before the input is staged
    uint4 qq[RT][U];
    uint32_t dd[RT][U];
    load(p0, qq, dd);
    if (a.norm_w) {
        // one pass over the input and the norm weights, both staged in LDS as
        // float4s (two per thread a step, all four loads requested first);
        // each thread then rescales the elements it staged
        float* ws = vs + C;
        constexpr int S = 4 * W * 64;
        double sq = 0;
        for (int k0 = 4 * static_cast<int>(threadIdx.x); k0 < C; k0 += 2 * S) {
            const int k1 = min(k0 + S, C - 4);
            const float4 x0 = *reinterpret_cast<const float4*>(a.v + k0);
            const float4 w0 = *reinterpret_cast<const float4*>(a.norm_w + k0);
            const float4 x1 = *reinterpret_cast<const float4*>(a.v + k1);
            const float4 w1 = *reinterpret_cast<const float4*>(a.norm_w + k1);
            sq += static_cast<double>(x0.x) * x0.x + static_cast<double>(x0.y) * x0.y +
                  static_cast<double>(x0.z) * x0.z + static_cast<double>(x0.w) * x0.w;
            *reinterpret_cast<float4*>(vs + k0) = x0;
            *reinterpret_cast<float4*>(ws + k0) = w0;
            if (k0 + S < C) {
                sq += static_cast<double>(x1.x) * x1.x + static_cast<double>(x1.y) * x1.y +
                      static_cast<double>(x1.z) * x1.z + static_cast<double>(x1.w) * x1.w;
                *reinterpret_cast<float4*>(vs + k1) = x1;
                *reinterpret_cast<float4*>(ws + k1) = w1;
            }
        }
        for (int o = 32; o >= 1; o >>= 1) sq += __shfl_xor(sq, o);
        if (lane == 0) red[wave][0][0] = sq;
        __syncthreads();
        double t = 0;
        for (int w = 0; w < W; ++w) t += red[w][0][0];
        const float inv = static_cast<float>(1.0 / sqrt(t / static_cast<double>(C) + static_cast<double>(a.eps)));
        for (int k = 4 * static_cast<int>(threadIdx.x); k < C; k += S) {
            float4 x = *reinterpret_cast<const float4*>(vs + k);
            const float4 w = *reinterpret_cast<const float4*>(ws + k);
            x.x = __fmul_rn(__fmul_rn(x.x, inv), w.x);
            x.y = __fmul_rn(__fmul_rn(x.y, inv), w.y);
            x.z = __fmul_rn(__fmul_rn(x.z, inv), w.z);
            x.w = __fmul_rn(__fmul_rn(x.w, inv), w.w);
            *reinterpret_cast<float4*>(vs + k) = x;
        }
        __syncthreads();  // red is reused below
    } else {
        for (int k = 4 * threadIdx.x; k < C; k += 4 * W * 64)
            *reinterpret_cast<float4*>(vs + k) = *reinterpret_cast<const float4*>(a.v + k);
    }
    __syncthreads();
    const float* vp = vs + 8 * (lane >> 4);
    double acc[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[r] = 0;
    for (int p = p0; p < p1; p += U) {
        // the next step's weights are in flight while this step is summed
        // (unconditional, clamped: the last step re-reads its own pairs)
        uint4 nq[RT][U];
        uint32_t nd[RT][U];
        load(min(p + U, p1 - 1), nq, nd);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int pc = min(p + u, p1 - 1);
            const bool live = p + u < p1, second = 2 * pc + 1 < G;
            const int c0 = 64 * pc, c1 = second ? c0 + 32 : c0;
            const float4 v0 = *reinterpret_cast<const float4*>(vp + c0);
            const float4 v1 = *reinterpret_cast<const float4*>(vp + c0 + 4);
            const float4 v2 = *reinterpret_cast<const float4*>(vp + c1);
            const float4 v3 = *reinterpret_cast<const float4*>(vp + c1 + 4);
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const double s0 = static_cast<double>(half_bits_to_float(static_cast<uint16_t>(dd[r][u] & 0xffff))) *
                                  dot8(qq[r][u].x, qq[r][u].y, v0, v1);
                const double s1 = static_cast<double>(half_bits_to_float(static_cast<uint16_t>(dd[r][u] >> 16))) *
                                  dot8(qq[r][u].z, qq[r][u].w, v2, v3);
                const double t = second ? s0 + s1 : s0;
                acc[r] += live ? t : 0.0;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                qq[r][u] = nq[r][u];
                dd[r][u] = nd[r][u];
            }
    }
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        acc[r] += __shfl_xor(acc[r], 16);
        acc[r] += __shfl_xor(acc[r], 32);
        if (lane < 16) red[wave][r][lane] = acc[r];
    }
    __syncthreads();
    if (wave || lane >= 16) return;
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        double t = red[0][r][lane];
#pragma unroll
        for (int w = 1; w < W; ++w) t += red[w][r][lane];
        const int tile = static_cast<int>(blockIdx.x) * RT + r, row = tile * 16 + lane;
        float y = static_cast<float>(t);
        const float other = __shfl_xor(y, 1);  // the row-pair partner (lanes 0..15 all take part)
        if (a.swiglu) {
            // model.hpp:111-116, with the overflow-free sigmoid
            if (!(lane & 1) && tile < a.tiles && row + 1 < a.rows) {
                const float small = expf(-fabsf(y));
                const float one = __fadd_rn(1.f, small);
                const float sig = y >= 0 ? __fdiv_rn(1.f, one) : __fdiv_rn(small, one);
                a.seg[0].out[row / 2] = __fmul_rn(y, __fmul_rn(sig, other));
            }
            continue;
        }
        if (a.rope_cs && row < a.rope_rows) {  // model.hpp:63-72
            const int i = (row % a.rope_dim) / 2;
            const float c = a.rope_cs[2 * i], sn = a.rope_cs[2 * i + 1];
            y = lane & 1 ? __fadd_rn(__fmul_rn(y, c), __fmul_rn(other, sn))
                         : __fsub_rn(__fmul_rn(y, c), __fmul_rn(other, sn));
        }
        if (tile < a.tiles && row < a.rows) write_segment(a.seg, a.nseg, row, 0, y);
    }
}

// The batched product runs on fp16 MFMAs.  int8 weights are exact in fp16;
// each activation vector is scaled by a power of two (max |x| into
// [2^13, 2^14), exact) and split as x = hi + lo with hi = fp16(x) and
// lo = fp16(x - hi), which keeps 22 of its 24 bits.  One 16x16x32 MFMA then
// covers exactly one Q8_0 group: C = A*Bhi + A*Blo in f32, and the
// accumulator takes d * C.  Element k of vector j sits where lane
// (j%16) + 16((k%32)/8) of vector tile j/16 reads it as a B operand:
// halves[((vt*groups + k/32)*2 + part)*64 + lane][k%8], part 0 = hi, 1 = lo.
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Elements k0 .. k0 + 7 of vector j (k0 % 8 == 0, already scaled): one
// 16-byte store each for the hi and the lo halves
__device__ __forceinline__ void put_halves8(_Float16* halves, int groups, int j, int k0, const float (&v)[8]) {
    half8 hi, lo;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        hi[i] = static_cast<_Float16>(v[i]);
        lo[i] = static_cast<_Float16>(v[i] - static_cast<float>(hi[i]));
    }
    const int lane = (j % 16) + 16 * ((k0 % 32) / 8);
    const size_t at = ((static_cast<size_t>(j / 16) * groups + k0 / 32) * 2 * 64 + lane) * 8;
    *reinterpret_cast<half8*>(halves + at) = hi;
    *reinterpret_cast<half8*>(halves + at + 64 * 8) = lo;
}

__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}

__device__ __forceinline__ void store8(float* p, const float (&v)[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// the power of two that brings max |x| into [2^13, 2^14) (1 for 0 or a
// non-finite maximum, which then propagates)
__device__ __forceinline__ int halves_shift(float m) {
    int e = 0;
    if (m > 0.f && __builtin_isfinite(m)) {
        frexpf(m, &e);
        return 14 - e;
    }
    return 0;
}

// max over the workgroup (every thread gets it); scratch holds a float per wave
__device__ __forceinline__ float block_max(float m, float* scratch) {
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = m;
    __syncthreads();
    float r = scratch[0];
    for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) r = fmaxf(r, scratch[w]);
    return r;
}

// The per-vector epilogues run a workgroup per vector; a thread takes
// eight consecutive elements a chunk (float4 loads, 16-byte halves stores),
// at most kEpiChunks chunks: rows of up to 16,384 at 1,024 threads.
constexpr int kEpiChunks = 2;

// threads for a row of h elements: one chunk each up to 1,024 threads
inline int epi_threads(int h) { return std::min(1024, std::max(64, ((h / 8 + 63) / 64) * 64)); }

// halves of vector j = blockIdx.x (a row of cols floats)
__global__ __launch_bounds__(1024) void split_halves_kernel(const float* x, int cols, int groups, _Float16* halves,
                                                             float* unscale) {
    __shared__ float part[16];
    const int j = blockIdx.x, T = blockDim.x;
    const float* xr = x + static_cast<size_t>(j) * cols;
    float v[kEpiChunks][8];
    float m = 0.f;
#pragma unroll
    for (int c = 0; c < kEpiChunks; ++c) {
        const int e0 = 8 * (static_cast<int>(threadIdx.x) + T * c);
        if (e0 < cols) {
            load8(xr + e0, v[c]);
#pragma unroll
            for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[c][i]));
        }
    }
    const int shift = halves_shift(block_max(m, part));
    const float up = ldexpf(1.f, shift);
    if (threadIdx.x == 0) unscale[j] = ldexpf(1.f, -shift);
#pragma unroll
    for (int c = 0; c < kEpiChunks; ++c) {
        const int e0 = 8 * (static_cast<int>(threadIdx.x) + T * c);
        if (e0 < cols) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[c][i] *= up;
            put_halves8(halves, groups, j, e0, v[c]);
        }
    }
}

// eight int8 (two dwords) to eight fp16: each byte b, offset by 128, becomes
// the fp16 1024 + (b ^ 0x80) (0x64 above the byte), from which 1152 is
// subtracted exactly
__device__ __forceinline__ half8 i8x8_to_half8(uint2 q) {
    const uint32_t x = q.x ^ 0x80808080u, y = q.y ^ 0x80808080u;
    const uint32_t w[4] = {__builtin_amdgcn_perm(0x64646464u, x, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u),
                           __builtin_amdgcn_perm(0x64646464u, y, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, y, 0x04030402u)};
    const half2v bias = {static_cast<_Float16>(1152.f), static_cast<_Float16>(1152.f)};
    half8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2v h = __builtin_bit_cast(half2v, w[i]) - bias;
        r[2 * i] = h[0];
        r[2 * i + 1] = h[1];
    }
    return r;
}

struct Q8BatchArgs {
    const uint4* q;
    const uint16_t* d;
    const uint4* halves;  // 8 fp16 per lane, see put_halves8
    const float* unscale;
    int rows, tiles, groups, pairs;  // tiles: one past the last row tile of this launch
    int tile0;                       // its first row tile (blockIdx.x counts from it)
    int n, vt0;                      // vectors in this launch, first vector tile
    int n_total;
    int n_total_tiles;  // vector tiles the halves hold
    int groups_per_split;
    float* out;  // [gridDim.y][n_total][rows]
};

// A workgroup of NT waves covers RT row tiles (RT x 16 rows) over a share of
// the groups; wave w owns vector tile w (16 vectors).  The operands are taken as
// C^T = X W^T: A = the wave's fp16 activation halves (registers, straight
// from global memory), B = the row tiles' int8 weights, converted to fp16 once
// per workgroup and shared through LDS, so lane l accumulates weight row l%16
// of each tile for vectors 4(l/16) + i and needs one scale per tile and
// group.  K advances in chunks of two group pairs: the int8 tiles and scales
// of chunk c + 2 are requested while chunk c is multiplied (two register
// sets), staged into the other LDS buffer after it (one barrier per chunk);
// the activations of chunk c + 1 are requested after chunk c's barrier.
// Prefetches are unconditional (clamped to the last chunk) so that the
// compiler keeps them ahead of the arithmetic.
//
// Every operand is read through a buffer descriptor: a thread keeps a fixed
// byte offset per load slot and a chunk adds one scalar offset, so the loads
// cost no vector address arithmetic.  The weight and scale views cover this
// workgroup's row tiles only and the activation view this wave's vector
// tile; reads past a view return zero.  The groups past the split's end (a
// last chunk of fewer than four) read their activations past the view, so
// they multiply zeros and add exactly nothing.
constexpr int kBufferWord3 = 0x00020000;  // gfx9 buffer descriptor, dword 3

__device__ __forceinline__ __amdgpu_buffer_rsrc_t view(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufferWord3);
}

template <int NT, int RT>
__global__ __launch_bounds__(256) void batch_q8_kernel(const Q8BatchArgs a) {
    constexpr int P = 2, CG = 2 * P;                 // pairs and groups per chunk
    constexpr int NTH = 64 * NT;
    constexpr int RAW = RT * P * 64;                 // uint4 of int8 per chunk
    constexpr int WPT = (RAW + NTH - 1) / NTH;       // per thread
    constexpr int DW = RT * P * 16;                  // scale dwords per chunk (16 rows x 2 groups each)
    constexpr int DPT = (DW + NTH - 1) / NTH;        // per thread
    __shared__ half8 ws[2][CG][RT][64];
    __shared__ uint32_t wd[2][RT][P][16];
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gbeg = static_cast<int>(blockIdx.y) * a.groups_per_split;
    const int gend = min(a.groups, gbeg + a.groups_per_split);
    const int pbeg = gbeg / 2;
    const int nchunks = (gend - gbeg + CG - 1) / CG;
    const int t0 = a.tile0 + static_cast<int>(blockIdx.x) * RT;
    const int tiles_here = min(RT, a.tiles - t0);
    const __amdgpu_buffer_rsrc_t qv =
        view(a.q + static_cast<size_t>(t0) * a.pairs * 64, static_cast<uint32_t>(tiles_here * a.pairs) * 1024u);
    const __amdgpu_buffer_rsrc_t dv = view(reinterpret_cast<const uint32_t*>(a.d) + static_cast<size_t>(t0) * a.pairs * 16,
                                           static_cast<uint32_t>(tiles_here * a.pairs) * 64u);
    const uint32_t xbytes = static_cast<uint32_t>(a.groups) * 2048u;
    const __amdgpu_buffer_rsrc_t xv = view(a.halves + static_cast<size_t>(a.vt0 + wave) * a.groups * 2 * 64, xbytes);
    // byte offsets of this thread's load slots within a chunk
    uint32_t qoff[WPT], doff[DPT];
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
        const int e = min(tid + NTH * i, RAW - 1);
        const int r = (e >> 6) / P, p = (e >> 6) % P;
        qoff[i] = static_cast<uint32_t>(((r * a.pairs + p) * 64 + (e & 63)) * 16);
    }
#pragma unroll
    for (int i = 0; i < DPT; ++i) {
        const int e = min(tid + NTH * i, DW - 1);
        const int r = e / (P * 16), p = (e / 16) % P;
        doff[i] = static_cast<uint32_t>(((r * a.pairs + p) * 16 + (e & 15)) * 4);
    }
    const uint32_t xoff = static_cast<uint32_t>(lane) * 16u;

    auto load_raw = [&](int chunk, uint4 (&raw)[WPT], uint32_t (&dr)[DPT]) {
        const int pc = pbeg + chunk * P;
#pragma unroll
        for (int i = 0; i < WPT; ++i)
            raw[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(qv, qoff[i], pc * 1024, 0));
#pragma unroll
        for (int i = 0; i < DPT; ++i) dr[i] = __builtin_amdgcn_raw_buffer_load_b32(dv, doff[i], pc * 64, 0);
    };
    auto stage = [&](int buf, const uint4 (&raw)[WPT], const uint32_t (&dr)[DPT]) {
#pragma unroll
        for (int i = 0; i < WPT; ++i) {
            const int e = tid + NTH * i;
            if (RAW % NTH && e >= RAW) break;
            const int r = (e >> 6) / P, p = (e >> 6) % P, l = e & 63;
            ws[buf][2 * p][r][l] = i8x8_to_half8(make_uint2(raw[i].x, raw[i].y));
            ws[buf][2 * p + 1][r][l] = i8x8_to_half8(make_uint2(raw[i].z, raw[i].w));
        }
#pragma unroll
        for (int i = 0; i < DPT; ++i) {
            const int e = tid + NTH * i;
            if (e < DW) wd[buf][e / (P * 16)][(e / 16) % P][e & 15] = dr[i];
        }
    };
    auto load_x = [&](int chunk, u32x4 (&x)[CG][2]) {
#pragma unroll
        for (int c = 0; c < CG; ++c) {
            const int g = gbeg + chunk * CG + c;
            const int so = g < gend ? g * 2048 : static_cast<int>(xbytes);  // past the split: zeros
            x[c][0] = __builtin_amdgcn_raw_buffer_load_b128(xv, xoff, so, 0);
            x[c][1] = __builtin_amdgcn_raw_buffer_load_b128(xv, xoff + 1024u, so, 0);
        }
    };
    float4v acc[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[r] = float4v{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int buf, const u32x4 (&x)[CG][2]) {
        uint32_t dd[RT][P];
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int p = 0; p < P; ++p) dd[r][p] = wd[buf][r][p][lane & 15];
#pragma unroll
        for (int c = 0; c < CG; ++c) {
            const half8 xh = __builtin_bit_cast(half8, x[c][0]), xl = __builtin_bit_cast(half8, x[c][1]);
            half8 w[RT];
#pragma unroll
            for (int r = 0; r < RT; ++r) w[r] = ws[buf][c][r][lane];
            float4v cc[RT];
#pragma unroll
            for (int r = 0; r < RT; ++r)
                cc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, w[r], float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < RT; ++r) cc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, w[r], cc[r], 0, 0, 0);
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const float d = half_bits_to_float(static_cast<uint16_t>(dd[r][c / 2] >> (c % 2 ? 16 : 0)));
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[r][i] = fmaf(d, cc[r][i], acc[r][i]);
            }
        }
    };

    uint4 rA[WPT], rB[WPT];
    uint32_t dA[DPT], dB[DPT];
    u32x4 xA[CG][2], xB[CG][2];
    const int c1 = min(1, nchunks - 1);
    load_raw(0, rA, dA);
    load_x(0, xA);
    load_raw(c1, rB, dB);
    stage(0, rA, dA);
    load_x(c1, xB);
    __syncthreads();
    for (int k = 0;; k += 2) {
        load_raw(min(k + 2, nchunks - 1), rA, dA);
        compute(0, xA);
        stage(1, rB, dB);
        __syncthreads();
        if (k + 1 >= nchunks) break;
        load_x(min(k + 2, nchunks - 1), xA);
        load_raw(min(k + 3, nchunks - 1), rB, dB);
        compute(1, xB);
        stage(0, rA, dA);
        __syncthreads();
        if (k + 2 >= nchunks) break;
        load_x(min(k + 3, nchunks - 1), xB);
    }
    // lane l holds row l%16 of each tile for vectors 4(l/16) + i of its tile
    float* out = a.out + static_cast<size_t>(blockIdx.y) * a.n_total * a.rows;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int jl = wave * 16 + 4 * (lane >> 4) + i;
        if (jl >= a.n) continue;
        const int j = a.vt0 * 16 + jl;
        const float us = a.unscale[j];
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const int row = (t0 + r) * 16 + (lane & 15);
            if (t0 + r < a.tiles && row < a.rows) out[static_cast<size_t>(j) * a.rows + row] = acc[r][i] * us;
        }
    }
}

// Weight-stationary form of the same product, for any number of vectors in
// one launch.  A workgroup of four waves owns RT row tiles over one K split
// of a.groups_per_split groups (a multiple of four): it first converts the
// split's int8 weights and scales into LDS, eight loads a thread requested
// before the first conversion, and then each wave multiplies them against
// its vector tiles in turn (tiles w, w + 4, ...), UG groups a step, the
// activation halves of the next step (the next tile's first, at a tile's
// end) in flight while a step is summed.  No barrier follows the staging.
// The arithmetic per group is the chunked kernel's, so the sums are the
// same.  LDS: groups_per_split * RT KiB of fp16 weights, then the scales.
template <int RT, int UG>
__global__ __launch_bounds__(256) void batch_q8_ws_kernel(const Q8BatchArgs a) {
    extern __shared__ half8 wsh[];  // [groups_per_split][RT][64], then scales [RT][pairs][16] dwords
    const int gps = a.groups_per_split, pps = gps / 2;
    uint32_t* wsd = reinterpret_cast<uint32_t*>(wsh + static_cast<size_t>(gps) * RT * 64);
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gbeg = static_cast<int>(blockIdx.y) * gps;
    const int gend = min(a.groups, gbeg + gps);
    const int pbeg = gbeg / 2;
    // every slot of the split's share is staged, the pairs past its end too
    // (the next split's bytes, or zeros past the view): each weight and
    // scale a dead group meets is finite, so its zero activations add zero
    const int np = pps;
    const int t0 = a.tile0 + static_cast<int>(blockIdx.x) * RT;
    const int tiles_here = min(RT, a.tiles - t0);
    const __amdgpu_buffer_rsrc_t qv =
        view(a.q + static_cast<size_t>(t0) * a.pairs * 64, static_cast<uint32_t>(tiles_here * a.pairs) * 1024u);
    const __amdgpu_buffer_rsrc_t dv = view(reinterpret_cast<const uint32_t*>(a.d) + static_cast<size_t>(t0) * a.pairs * 16,
                                           static_cast<uint32_t>(tiles_here * a.pairs) * 64u);
    // ---- staging: RT x np pairs x 64 lanes of int8, eight loads a thread a round
    {
        constexpr int B = 8;
        const int units = RT * np * 64;
        for (int e0 = tid; e0 < units; e0 += 256 * B) {
            uint4 raw[B];
#pragma unroll
            for (int i = 0; i < B; ++i) {
                const int e = e0 + 256 * i;  // past `units`: a read past the view (zeros), not stored
                const int l = e & 63, rp = e >> 6, r = rp / np, p = rp - r * np;
                raw[i] = __builtin_bit_cast(
                    uint4, __builtin_amdgcn_raw_buffer_load_b128(
                               qv, static_cast<uint32_t>(((r * a.pairs + p) * 64 + l) * 16), pbeg * 1024, 0));
            }
#pragma unroll
            for (int i = 0; i < B; ++i) {
                const int e = e0 + 256 * i;
                if (e >= units) break;
                const int l = e & 63, rp = e >> 6, r = rp / np, p = rp - r * np;
                wsh[((2 * p) * RT + r) * 64 + l] = i8x8_to_half8(make_uint2(raw[i].x, raw[i].y));
                wsh[((2 * p + 1) * RT + r) * 64 + l] = i8x8_to_half8(make_uint2(raw[i].z, raw[i].w));
            }
        }
        const int dunits = RT * np * 16;
        for (int e = tid; e < dunits; e += 256) {
            const int row = e & 15, rp = e >> 4, r = rp / np, p = rp - r * np;
            wsd[(r * pps + p) * 16 + row] = __builtin_amdgcn_raw_buffer_load_b32(
                dv, static_cast<uint32_t>(((r * a.pairs + p) * 16 + row) * 4), pbeg * 64, 0);
        }
    }
    __syncthreads();

    // ---- products: this wave's vector tiles (w, w + 4, ...), UG groups a
    // unit, one stream of (tile, unit) steps double-buffered across tiles
    const int ntv = (a.n + 15) / 16;
    const uint32_t xbytes = static_cast<uint32_t>(a.n_total_tiles) * static_cast<uint32_t>(a.groups) * 2048u;
    const __amdgpu_buffer_rsrc_t xv = view(a.halves, xbytes);
    const uint32_t xoff = static_cast<uint32_t>(lane) * 16u;
    const int nunits = (gend - gbeg + UG - 1) / UG;
    const int mytiles = wave < ntv ? (ntv - 1 - wave) / 4 + 1 : 0;
    const int steps = mytiles * nunits;
    auto load_x = [&](int jt, int u, u32x4 (&x)[UG][2]) {
        const int vt = wave + 4 * jt;
#pragma unroll
        for (int c = 0; c < UG; ++c) {
            const int g = gbeg + UG * u + c;
            const int so = g < gend ? ((a.vt0 + vt) * a.groups + g) * 2048 : static_cast<int>(xbytes);
            x[c][0] = __builtin_amdgcn_raw_buffer_load_b128(xv, xoff, so, 0);
            x[c][1] = __builtin_amdgcn_raw_buffer_load_b128(xv, xoff + 1024u, so, 0);
        }
    };
    float4v acc[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[r] = float4v{0.f, 0.f, 0.f, 0.f};
    float* out = a.out + static_cast<size_t>(blockIdx.y) * a.n_total * a.rows;
    auto step = [&](int jt, int u, const u32x4 (&x)[UG][2]) {
        uint32_t dd[RT][UG / 2];
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int p = 0; p < UG / 2; ++p)
                dd[r][p] = wsd[(r * pps + min((UG / 2) * u + p, pps - 1)) * 16 + (lane & 15)];
#pragma unroll
        for (int c = 0; c < UG; ++c) {
            const int gl = min(UG * u + c, gps - 1);  // a group past the split reads a staged one: its x is zero
            const half8 xh = __builtin_bit_cast(half8, x[c][0]), xl = __builtin_bit_cast(half8, x[c][1]);
            half8 w[RT];
#pragma unroll
            for (int r = 0; r < RT; ++r) w[r] = wsh[(gl * RT + r) * 64 + lane];
            float4v cc[RT];
#pragma unroll
            for (int r = 0; r < RT; ++r)
                cc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, w[r], float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < RT; ++r) cc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, w[r], cc[r], 0, 0, 0);
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const float d = half_bits_to_float(static_cast<uint16_t>(dd[r][c / 2] >> (c % 2 ? 16 : 0)));
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[r][i] = fmaf(d, cc[r][i], acc[r][i]);
            }
        }
        if (u + 1 < nunits) return;
        // the tile's last unit: lane l holds row l%16 of each row tile for
        // vectors 4(l/16) + i of vector tile vt
        const int vt = wave + 4 * jt;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int jl = vt * 16 + 4 * (lane >> 4) + i;
            if (jl >= a.n) continue;
            const int j = a.vt0 * 16 + jl;
            const float us = a.unscale[j];
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const int row = (t0 + r) * 16 + (lane & 15);
                if (t0 + r < a.tiles && row < a.rows) out[static_cast<size_t>(j) * a.rows + row] = acc[r][i] * us;
            }
        }
#pragma unroll
        for (int r = 0; r < RT; ++r) acc[r] = float4v{0.f, 0.f, 0.f, 0.f};
    };
    if (steps == 0) return;
    // the (tile, unit) of the next step to load and of the step to compute,
    // counted up rather than divided out of a flat index (8% of the
    // product's time at 256-512 vectors went to the divisions)
    u32x4 xa[UG][2], xb[UG][2];
    int jn = 0, un = 0, jc = 0, uc = 0;
    auto next_load = [&](u32x4 (&x)[UG][2]) {
        const bool past = jn >= mytiles;
        load_x(past ? mytiles - 1 : jn, past ? nunits - 1 : un, x);
        if (++un == nunits) {
            un = 0;
            ++jn;
        }
    };
    auto next_step = [&](const u32x4 (&x)[UG][2]) {
        step(jc, uc, x);
        if (++uc == nunits) {
            uc = 0;
            ++jc;
        }
    };
    next_load(xa);
    for (int k = 0;; k += 2) {
        next_load(xb);
        next_step(xa);
        if (k + 1 >= steps) break;
        next_load(xa);
        next_step(xb);
        if (k + 2 >= steps) break;
    }
}

// ---------------------------------------------------------- batch epilogues
//
// The batched products write f32 sums per K split, [splits][n][rows]; these
// kernels add the splits in order (from 0.f, as one split's value is itself)
// and apply what follows the product in the layer.

// The sum runs in split order.  The partials are read N at a time (N = 1, 2
// or 4 when that covers every split, else 8), all N requested before the
// first add; clamped indices keep the loads unconditional, and a select (not
// an add of 0.f) skips the surplus ones.
template <int N>
__device__ __forceinline__ float split_sum(const float* p, int splits, size_t stride, size_t at) {
    float s = 0.f;
    for (int k0 = 0; k0 < splits; k0 += N) {
        float v[N];
#pragma unroll
        for (int k = 0; k < N; ++k) v[k] = p[static_cast<size_t>(min(k0 + k, splits - 1)) * stride + at];
#pragma unroll
        for (int k = 0; k < N; ++k) s = k0 + k < splits ? s + v[k] : s;
    }
    return s;
}

__device__ __forceinline__ float split_total(const float* p, int splits, size_t stride, size_t at) {
    if (splits == 1) return split_sum<1>(p, splits, stride, at);
    if (splits == 2) return split_sum<2>(p, splits, stride, at);
    if (splits <= 4) return split_sum<4>(p, splits, stride, at);
    return split_sum<8>(p, splits, stride, at);
}

// the split sums of eight consecutive elements at p + at (16-byte aligned),
// in split order from 0.f, four splits' loads requested at a time
__device__ __forceinline__ void split_total8(const float* p, int splits, size_t stride, size_t at, float (&s)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) s[i] = 0.f;
    for (int k0 = 0; k0 < splits; k0 += 4) {
        float v[4][8];
#pragma unroll
        for (int k = 0; k < 4; ++k) load8(p + static_cast<size_t>(min(k0 + k, splits - 1)) * stride + at, v[k]);
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int i = 0; i < 8; ++i) s[i] = k0 + k < splits ? s[i] + v[k][i] : s[i];
    }
}

// Q|K|V rows of vector j: q and k rotated by row j's (cos, sin)
// (model.hpp:63-72), v copied; one thread per rotation pair or v element
__global__ void qkv_epilogue_kernel(const float* p, int splits, int n, int qheads, int kheads, int dim, int interleaved,
                                    const float* cs, float* q, float* k, float* v) {
    const int half = dim / 2, rows = (qheads + 2 * kheads) * dim, kw = kheads * dim;
    const int pairs = (qheads + kheads) * half, per = pairs + kw;
    const size_t stride = static_cast<size_t>(n) * rows;
    const size_t total = static_cast<size_t>(n) * per;
    for (size_t t = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; t < total;
         t += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const int j = static_cast<int>(t / per), e = static_cast<int>(t % per);
        const size_t base = static_cast<size_t>(j) * rows;
        if (e >= pairs) {
            const int c = e - pairs;
            v[static_cast<size_t>(j) * kw + c] = split_total(p, splits, stride, base + qheads * dim + kw + c);
            continue;
        }
        const int h = e / half, i = e % half;
        const int ia = interleaved ? 2 * i : i, ib = interleaved ? 2 * i + 1 : i + half;
        const float left = split_total(p, splits, stride, base + h * dim + ia);
        const float right = split_total(p, splits, stride, base + h * dim + ib);
        const float c = cs[static_cast<size_t>(j) * dim + 2 * i], s = cs[static_cast<size_t>(j) * dim + 2 * i + 1];
        float* x = h < qheads ? q + (static_cast<size_t>(j) * qheads + h) * dim
                              : k + (static_cast<size_t>(j) * kheads + (h - qheads)) * dim;
        x[ia] = __fsub_rn(__fmul_rn(left, c), __fmul_rn(right, s));
        x[ib] = __fadd_rn(__fmul_rn(right, c), __fmul_rn(left, s));
    }
}

// Vector j = blockIdx.x: x += the product's sum (the residual add, when p is
// given), then RMSNorm with w (model.hpp:54-61: sum of squares in double,
// scale rounded to float, (x * s) * w) into `norm` (when given) and, when
// `halves` is given, into the next product's fp16 halves.  A thread keeps
// its chunks in registers between the passes.
__global__ __launch_bounds__(1024) void resid_norm_kernel(const float* p, int splits, float* x, const float* w, int n,
                                                          int h, float eps, float* norm, _Float16* halves, int groups,
                                                          float* unscale) {
    __shared__ double part[16];
    __shared__ float mpart[16];
    const int j = blockIdx.x, T = blockDim.x;
    float* xr = x + static_cast<size_t>(j) * h;
    const size_t stride = static_cast<size_t>(n) * h;
    float y[kEpiChunks][8], wv[kEpiChunks][8];
    double sq = 0;
#pragma unroll
    for (int c = 0; c < kEpiChunks; ++c) {
        const int e0 = 8 * (static_cast<int>(threadIdx.x) + T * c);
        if (e0 < h) {
            load8(xr + e0, y[c]);
            load8(w + e0, wv[c]);
            if (p) {
                float t[8];
                split_total8(p, splits, stride, static_cast<size_t>(j) * h + e0, t);
#pragma unroll
                for (int i = 0; i < 8; ++i) y[c][i] = __fadd_rn(y[c][i], t[i]);
                store8(xr + e0, y[c]);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) sq += static_cast<double>(y[c][i]) * y[c][i];
        }
    }
    for (int o = 32; o >= 1; o >>= 1) sq += __shfl_xor(sq, o);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = sq;
    __syncthreads();
    double t = 0;
    for (int wave = 0; wave < T / 64; ++wave) t += part[wave];
    const float inv = static_cast<float>(1.0 / sqrt(t / static_cast<double>(h) + static_cast<double>(eps)));
    float mx = 0.f;
#pragma unroll
    for (int c = 0; c < kEpiChunks; ++c) {
        const int e0 = 8 * (static_cast<int>(threadIdx.x) + T * c);
        if (e0 < h) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                y[c][i] = __fmul_rn(__fmul_rn(y[c][i], inv), wv[c][i]);
                mx = fmaxf(mx, fabsf(y[c][i]));
            }
            if (norm) store8(norm + static_cast<size_t>(j) * h + e0, y[c]);
        }
    }
    if (!halves) return;
    const int shift = halves_shift(block_max(mx, mpart));
    const float up = ldexpf(1.f, shift);
    if (threadIdx.x == 0) unscale[j] = ldexpf(1.f, -shift);
#pragma unroll
    for (int c = 0; c < kEpiChunks; ++c) {
        const int e0 = 8 * (static_cast<int>(threadIdx.x) + T * c);
        if (e0 < h) {
#pragma unroll
            for (int i = 0; i < 8; ++i) y[c][i] *= up;
            put_halves8(halves, groups, j, e0, y[c]);
        }
    }
}

// Vector j = blockIdx.x of the fused gate|up product: gate * (sigmoid(gate)
// * up) (model.hpp:111-116) into `out` (when given) and, when given, the next
// product's halves
__global__ __launch_bounds__(1024) void swiglu_epilogue_kernel(const float* p, int splits, int n, int inter, float* out,
                                                               _Float16* halves, int groups, float* unscale,
                                                               int interleaved) {
    __shared__ float mpart[16];
    const int j = blockIdx.x, T = blockDim.x;
    const size_t stride = static_cast<size_t>(n) * 2 * inter, base = static_cast<size_t>(j) * 2 * inter;
    float val[kEpiChunks][8];
    float mx = 0.f;
#pragma unroll
    for (int c = 0; c < kEpiChunks; ++c) {
        const int e0 = 8 * (static_cast<int>(threadIdx.x) + T * c);
        if (e0 < inter) {
            float g[8], u[8];
            if (interleaved) {  // rows 2e (gate), 2e + 1 (up)
                float a[8], b[8];
                split_total8(p, splits, stride, base + 2 * static_cast<size_t>(e0), a);
                split_total8(p, splits, stride, base + 2 * static_cast<size_t>(e0) + 8, b);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    g[i] = a[2 * i], u[i] = a[2 * i + 1];
                    g[4 + i] = b[2 * i], u[4 + i] = b[2 * i + 1];
                }
            } else {
                split_total8(p, splits, stride, base + e0, g);
                split_total8(p, splits, stride, base + inter + e0, u);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float small = expf(-fabsf(g[i]));
                const float one = __fadd_rn(1.f, small);
                const float sig = g[i] >= 0 ? __fdiv_rn(1.f, one) : __fdiv_rn(small, one);
                val[c][i] = __fmul_rn(g[i], __fmul_rn(sig, u[i]));
                mx = fmaxf(mx, fabsf(val[c][i]));
            }
            if (out) store8(out + static_cast<size_t>(j) * inter + e0, val[c]);
        }
    }
    if (!halves) return;
    const int shift = halves_shift(block_max(mx, mpart));
    const float up = ldexpf(1.f, shift);
    if (threadIdx.x == 0) unscale[j] = ldexpf(1.f, -shift);
#pragma unroll
    for (int c = 0; c < kEpiChunks; ++c) {
        const int e0 = 8 * (static_cast<int>(threadIdx.x) + T * c);
        if (e0 < inter) {
#pragma unroll
            for (int i = 0; i < 8; ++i) val[c][i] *= up;
            put_halves8(halves, groups, j, e0, val[c]);
        }
    }
}

// element (j, c) of row idx[j] (or `row`) of a Q8_0 table
__global__ void gather_embedding_q8_kernel(const uint8_t* q, const uint16_t* d, int pairs, const uint32_t* idx,
                                           uint32_t row, int n, int h, float* out) {
    const size_t total = static_cast<size_t>(n) * h;
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const int j = static_cast<int>(i / h), c = static_cast<int>(i % h);
        const uint32_t r = idx ? idx[j] : row;
        const int g = c / 32;
        const size_t blk = static_cast<size_t>(r / 16) * pairs + g / 2;
        const int lane = static_cast<int>(r % 16) + 16 * ((c % 32) / 8);
        const float dv = half_bits_to_float(d[(blk * 16 + r % 16) * 2 + g % 2]);
        out[i] = __fmul_rn(dv, static_cast<float>(static_cast<int8_t>(q[(blk * 64 + lane) * 16 + (g % 2) * 8 + c % 8])));
    }
}

unsigned grid_for(size_t n) {
    return static_cast<unsigned>(std::min<size_t>((n + kThreads - 1) / kThreads, 8192));
}

}  // namespace

void launch_dequant(uint32_t type, const uint8_t* raw, size_t n, float* out, int* bad, hipStream_t s) {
    if (!n) return;
    switch (type) {
        case 0:  // f32 payloads are copied in place; only checked here
            launch("model_dequant", check_f32_kernel, dim3(grid_for(n)), dim3(kThreads), 0, s,
                   static_cast<const float*>(out), n, bad);
            break;
        case 1: launch("model_dequant", f16_kernel, dim3(grid_for(n)), dim3(kThreads), 0, s, raw, n, out, bad); break;
        case 2: launch("model_dequant", q4_0_kernel, dim3(grid_for(n)), dim3(kThreads), 0, s, raw, n, out, bad); break;
        case 8: launch("model_dequant", q8_0_kernel, dim3(grid_for(n)), dim3(kThreads), 0, s, raw, n, out, bad); break;
        case 12: launch("model_dequant", q4_k_kernel, dim3(grid_for(n)), dim3(kThreads), 0, s, raw, n, out, bad); break;
        default: throw std::invalid_argument("unsupported native weight type");
    }
    TVARA_HIP(hipGetLastError());
}

void launch_rmsnorm(const float* x, const float* w, float* out, int n, float eps, hipStream_t s, int rows) {
    launch("model_rmsnorm", rmsnorm_kernel, dim3(rows), dim3(1024), 0, s, x, w, out, n, eps);
    TVARA_HIP(hipGetLastError());
}

void launch_split_sum(const float* p, int splits, int n, int rows, float* out, hipStream_t s) {
    BatchMatvecArgs b{};
    b.rows = rows;
    b.n = n;
    b.nseg = 1;
    b.seg[0] = MatvecSegment{out, rows, nullptr};
    b.partial = const_cast<float*>(p);
    launch("model_matvec_sum", split_sum_kernel, dim3(grid_for(static_cast<size_t>(n) * rows)), dim3(kThreads), 0, s, b,
           splits);
    TVARA_HIP(hipGetLastError());
}

void launch_gather_embedding(const float* table, const uint32_t* idx, int n, int h, float* out, hipStream_t s) {
    launch("model_embedding", gather_embedding_kernel, dim3(grid_for(static_cast<size_t>(n) * h)), dim3(kThreads), 0, s,
           table, idx, n, h, out);
    TVARA_HIP(hipGetLastError());
}

void launch_interleave_layers(const float* src, float* dst, int layers, int n, int kv, hipStream_t s) {
    const size_t total = static_cast<size_t>(layers) * n * kv;
    launch("model_interleave", interleave_layers_kernel, dim3(grid_for(total)), dim3(kThreads), 0, s, src, dst, layers,
           n, kv);
    TVARA_HIP(hipGetLastError());
}

void launch_matvec(const float* w, int rows, int cols, const float* v, const MatvecSegment* seg, int nseg,
                   hipStream_t s) {
    MatvecArgs a{};
    a.w = w;
    a.v = v;
    a.rows = rows;
    a.cols = cols;
    a.nseg = nseg;
    for (int i = 0; i < nseg; ++i) a.seg[i] = seg[i];
    const dim3 grid((rows + kThreads / 64 - 1) / (kThreads / 64));
    if (cols % 4 == 0)
        launch("model_matvec", matvec_kernel<true>, grid, dim3(kThreads), 0, s, a);
    else
        launch("model_matvec", matvec_kernel<false>, grid, dim3(kThreads), 0, s, a);
    TVARA_HIP(hipGetLastError());
}

void launch_rope(float* q, int qheads, float* k, int kheads, int dim, const float* cs, bool interleaved,
                 hipStream_t s, int rows) {
    const int n = (qheads + kheads) * (dim / 2);
    launch("model_rope", rope_kernel, dim3((n + kThreads - 1) / kThreads, rows), dim3(kThreads), 0, s, q, qheads, k,
           kheads, dim, cs, interleaved ? 1 : 0);
    TVARA_HIP(hipGetLastError());
}

void launch_swiglu(float* gate, const float* up, int n, hipStream_t s) {
    launch("model_swiglu", swiglu_kernel, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, s, gate, up, n);
    TVARA_HIP(hipGetLastError());
}

void launch_q8_repack(const uint8_t* raw, int rows, int cols, int row0, int stride, Weight& w, int* bad,
                      hipStream_t s) {
    const size_t total = static_cast<size_t>(rows) * (cols / 32);
    if (!total) return;
    launch("model_q8_repack", q8_repack_kernel, dim3(grid_for(total)), dim3(kThreads), 0, s, raw, rows, cols / 32, row0,
           stride, static_cast<uint8_t*>(w.q.ptr), static_cast<uint16_t*>(w.d.ptr), bad);
    TVARA_HIP(hipGetLastError());
}

void launch_matvec_q8(const Weight& w, const float* v, const MatvecSegment* seg, int nseg, hipStream_t s,
                      const float* norm_w, float eps, const float* rope_cs, int rope_dim, int rope_rows) {
    if (w.cols > 15360) throw std::invalid_argument("Q8_0 matrix wider than 15,360 columns");
    Q8MatvecArgs a{};
    a.q = static_cast<const uint4*>(w.q.ptr);
    a.d = static_cast<const uint32_t*>(w.d.ptr);
    a.v = v;
    a.norm_w = norm_w;
    a.eps = eps;
    a.rows = w.rows;
    a.tiles = w.tiles();
    a.groups = w.groups();
    a.pairs = w.pairs();
    a.cols = w.cols;
    a.nseg = nseg;
    for (int i = 0; i < nseg; ++i) a.seg[i] = seg[i];
    a.rope_cs = rope_cs;
    a.rope_dim = rope_dim;
    a.rope_rows = rope_rows;
    a.swiglu = w.interleaved ? 1 : 0;
    // two tiles per workgroup (sharing the staged input) for the largest
    // matrices.  Waves per workgroup: up to about sixteen waves per CU over
    // the launch (4,096), at most sixteen, at least two when there is work
    // for two, and at least two group pairs a wave (MI355X, Llama-3.2-1B shapes, two pairs a step:
    // 16,384 x 2,048 gate|up in 11.2 us at one tile and four waves against
    // 12.3 at two tiles and eight; 2,048 x 8,192 down 8.6 us at sixteen;
    // 3,072 x 2,048 QKV 6.1-6.2 us at eight or sixteen; the 128,256-row
    // logits in 58 us at two waves against 65 at one)
    const int rt = a.tiles >= 4096 ? 2 : 1;
    const int wgs = (a.tiles + rt - 1) / rt;
    int want = 1;
    while (want < 16 && 2 * want * 2 <= a.pairs && (want < 2 || wgs * want * 2 <= 4096)) want *= 2;
    const dim3 grid(wgs);
    // the input, and the norm weights beside it when the product normalises
    const size_t lds = static_cast<size_t>(w.cols) * sizeof(float) * (norm_w ? 2 : 1);
    auto go = [&](auto kernel, int waves) { launch("model_matvec_q8", kernel, grid, dim3(64 * waves), lds, s, a); };
    if (rt == 2) {
        if (want >= 8) go(matvec_q8_kernel<8, 2>, 8);
        else if (want >= 4) go(matvec_q8_kernel<4, 2>, 4);
        else if (want >= 2) go(matvec_q8_kernel<2, 2>, 2);
        else go(matvec_q8_kernel<1, 2>, 1);
    } else {
        if (want >= 16) go(matvec_q8_kernel<16, 1>, 16);
        else if (want >= 8) go(matvec_q8_kernel<8, 1>, 8);
        else if (want >= 4) go(matvec_q8_kernel<4, 1>, 4);
        else if (want >= 2) go(matvec_q8_kernel<2, 1>, 2);
        else go(matvec_q8_kernel<1, 1>, 1);
    }
    TVARA_HIP(hipGetLastError());
}

namespace {
// one wave per vector tile
template <int RT>
void launch_batch_q8(int nt, dim3 grid, hipStream_t s, const Q8BatchArgs& a) {
    switch (nt) {
        case 1: launch("model_matvec_q8", batch_q8_kernel<1, RT>, grid, dim3(64), 0, s, a); break;
        case 2: launch("model_matvec_q8", batch_q8_kernel<2, RT>, grid, dim3(128), 0, s, a); break;
        case 3: launch("model_matvec_q8", batch_q8_kernel<3, RT>, grid, dim3(192), 0, s, a); break;
        default: launch("model_matvec_q8", batch_q8_kernel<4, RT>, grid, dim3(256), 0, s, a); break;
    }
}

// row tiles per workgroup and groups per K split of the batched Q8_0
// product: four row tiles from 1,024 tiles up, else two (more workgroups for
// the smaller matrices); the groups are split while the launch has fewer than
// 512 workgroups (two per CU), in whole chunks of four groups, never below
// eight groups and into at most eight splits (the epilogues read every split)
struct Q8Plan {
    int rt, gx, per, splits;
};
Q8Plan q8_plan(const Weight& w) {
    Q8Plan p{};
    const int tiles = w.tiles(), groups = w.groups();
    p.rt = tiles >= 1024 ? 4 : 2;
    p.gx = (tiles + p.rt - 1) / p.rt;
    const int want = p.gx >= 512 ? 1 : std::min({(512 + p.gx - 1) / p.gx, std::max(1, groups / 8), 8});
    p.per = (groups + want - 1) / want;
    p.per = (p.per + 3) / 4 * 4;  // whole chunks, so splits start on a group pair
    p.splits = (groups + p.per - 1) / p.per;
    return p;
}

struct F32Plan {
    int tiles, per, splits;
};
F32Plan f32_plan(int rows, int cols) {
    F32Plan p{};
    p.tiles = (rows + kTileRows - 1) / kTileRows;
    const int chunks = cols / kTileK;
    const int want = std::max(1, std::min(chunks, (512 + p.tiles - 1) / p.tiles));
    p.per = (chunks + want - 1) / want;
    p.splits = (chunks + p.per - 1) / p.per;
    return p;
}

// Weight-stationary plan: RT row tiles per workgroup (four from 1,024 row
// tiles up, else two) and the K split that keeps a workgroup's fp16 weights
// within 64 KiB of LDS, split further (in steps of four groups, never below
// eight) while the launch has fewer than 512 workgroups.
struct WsPlan {
    int rt, gps, gx, splits;
    size_t lds;
};
WsPlan ws_plan(const Weight& w) {
    WsPlan p{};
    const int tiles = w.tiles(), groups = w.groups();
    p.rt = tiles >= 1024 ? 4 : 2;
    p.gx = (tiles + p.rt - 1) / p.rt;
    const int cap = 64 / p.rt;  // groups of fp16 weights in 64 KiB
    int splits = (groups + cap - 1) / cap;
    while (p.gx * splits < 512 && (groups + splits) / (splits + 1) >= 8) ++splits;
    p.gps = (groups + splits - 1) / splits;
    p.gps = (p.gps + 3) / 4 * 4;
    if (p.gps > cap) p.gps = cap / 4 * 4;
    p.splits = (groups + p.gps - 1) / p.gps;
    p.lds = static_cast<size_t>(p.gps) * p.rt * 1024 + static_cast<size_t>(p.rt) * (p.gps / 2) * 64;
    return p;
}

// The weight-stationary kernel from 128 vectors (matrices under 1,024 row
// tiles) or 256 (under 4,096); the chunked kernel otherwise.  MI355X,
// Llama-3.2-1B shapes, weights from HBM: QKV / output / gate|up / down at 512
// vectors 35.6 / 28.8 / 117 / 70.8 us against 59.9 / 51.0 / 138.5 / 100.6;
// at 128 vectors 13.5 / 11.0 / 48.3 / 23.9 against 16.2 / 13.4 / 37.6 /
// 26.8; at 64 vectors, and for the 8,016-tile logits at every size, the
// chunked kernel is faster (gate|up 18.9 against 32.2 us at 64; logits 841
// against 862-891 us at 512).
bool ws_for(const Weight& w, int n) {
    const int t = w.tiles();
    return w.q8 && t < 4096 && (n >= 256 || (n >= 128 && t < 1024));
}

void launch_ws(const Weight& w, const WsPlan& p, int tile0, int tile1, const _Float16* halves, const float* unscale,
               int n, float* out, hipStream_t s) {
    Q8BatchArgs a{};
    a.q = static_cast<const uint4*>(w.q.ptr);
    a.d = static_cast<const uint16_t*>(w.d.ptr);
    a.halves = reinterpret_cast<const uint4*>(halves);
    a.unscale = unscale;
    a.rows = w.rows;
    a.tiles = tile1;
    a.tile0 = tile0;
    a.groups = w.groups();
    a.pairs = w.pairs();
    a.n = n;
    a.vt0 = 0;
    a.n_total = n;
    a.n_total_tiles = (n + 15) / 16;
    a.groups_per_split = p.gps;
    a.out = out;
    if (static_cast<double>(a.n_total_tiles) * a.groups * 2048 >= 2147483648.0)
        throw std::invalid_argument("batched product input above 2 GiB");
    const dim3 grid((tile1 - tile0 + p.rt - 1) / p.rt, p.splits);
    if (p.rt == 4)
        launch("model_matvec_q8", batch_q8_ws_kernel<4, 4>, grid, dim3(256), p.lds, s, a);
    else
        launch("model_matvec_q8", batch_q8_ws_kernel<2, 4>, grid, dim3(256), p.lds, s, a);
}
}  // namespace

int batch_splits(const Weight& w, int n) {
    if (!w.q8) return f32_plan(w.rows, w.cols).splits;
    return ws_for(w, n) ? ws_plan(w).splits : q8_plan(w).splits;
}

int batch_splits_max(const Weight& w) {
    if (!w.q8) return f32_plan(w.rows, w.cols).splits;
    return std::max(ws_plan(w).splits, q8_plan(w).splits);
}

void launch_batch_product(const Weight& w, const float* x, const _Float16* halves, const float* unscale, int n,
                          float* out, hipStream_t s) {
    if (ws_for(w, n)) {
        launch_ws(w, ws_plan(w), 0, w.tiles(), halves, unscale, n, out, s);
    } else if (w.q8) {
        const Q8Plan p = q8_plan(w);
        for (int j0 = 0; j0 < n; j0 += 64) {
            const int nj = std::min(64, n - j0);
            Q8BatchArgs a{};
            a.q = static_cast<const uint4*>(w.q.ptr);
            a.d = static_cast<const uint16_t*>(w.d.ptr);
            a.halves = reinterpret_cast<const uint4*>(halves);
            a.unscale = unscale;
            a.rows = w.rows;
            a.tiles = w.tiles();
            a.groups = w.groups();
            a.pairs = w.pairs();
            a.n = nj;
            a.vt0 = j0 / 16;
            a.n_total = n;
            a.groups_per_split = p.per;
            a.out = out;
            const dim3 grid(p.gx, p.splits);
            if (p.rt == 4)
                launch_batch_q8<4>((nj + 15) / 16, grid, s, a);
            else
                launch_batch_q8<2>((nj + 15) / 16, grid, s, a);
        }
    } else {
        if (w.cols % kTileK) throw std::invalid_argument("batched matvec needs a row width divisible by 32");
        const F32Plan p = f32_plan(w.rows, w.cols);
        for (int j0 = 0; j0 < n; j0 += kTileVecs) {
            BatchMatvecArgs a{};
            a.w = static_cast<const float*>(w.f32.ptr);
            a.x = x + static_cast<size_t>(j0) * w.cols;
            a.rows = w.rows;
            a.cols = w.cols;
            a.n = std::min(kTileVecs, n - j0);
            a.chunks_per_split = p.per;
            a.partial = out;
            a.n_total = n;
            a.j0 = j0;
            launch("model_matvec", batch_matvec_kernel, dim3(p.tiles, p.splits), dim3(256), 0, s, a);
        }
    }
    TVARA_HIP(hipGetLastError());
}

void launch_batch_product_tiles(const Weight& w, int tile0, int tile1, const _Float16* halves, const float* unscale,
                                int n, float* out, hipStream_t s) {
    if (!w.q8 || batch_splits(w, n) != 1 || tile0 < 0 || tile0 >= tile1 || tile1 > w.tiles())
        throw std::invalid_argument("row-tile range of a batched product needs an unsplit Q8_0 matrix");
    if (ws_for(w, n)) {
        launch_ws(w, ws_plan(w), tile0, tile1, halves, unscale, n, out, s);
        TVARA_HIP(hipGetLastError());
        return;
    }
    const Q8Plan p = q8_plan(w);
    for (int j0 = 0; j0 < n; j0 += 64) {
        const int nj = std::min(64, n - j0);
        Q8BatchArgs a{};
        a.q = static_cast<const uint4*>(w.q.ptr);
        a.d = static_cast<const uint16_t*>(w.d.ptr);
        a.halves = reinterpret_cast<const uint4*>(halves);
        a.unscale = unscale;
        a.rows = w.rows;
        a.tiles = tile1;
        a.tile0 = tile0;
        a.groups = w.groups();
        a.pairs = w.pairs();
        a.n = nj;
        a.vt0 = j0 / 16;
        a.n_total = n;
        a.groups_per_split = p.per;
        a.out = out;
        const dim3 grid((tile1 - tile0 + p.rt - 1) / p.rt, 1);
        if (p.rt == 4)
            launch_batch_q8<4>((nj + 15) / 16, grid, s, a);
        else
            launch_batch_q8<2>((nj + 15) / 16, grid, s, a);
    }
    TVARA_HIP(hipGetLastError());
}

void launch_split_halves(const float* x, int n, int cols, _Float16* halves, float* unscale, hipStream_t s) {
    if (cols % 32 || cols > 1024 * 8 * kEpiChunks) throw std::invalid_argument("batched decode width above 16384");
    launch("model_split_halves", split_halves_kernel, dim3(n), dim3(epi_threads(cols)), 0, s, x, cols, cols / 32, halves,
           unscale);
    TVARA_HIP(hipGetLastError());
}

void launch_qkv_epilogue(const float* p, int splits, int n, int qheads, int kheads, int dim, bool interleaved,
                         const float* cs, float* q, float* k, float* v, hipStream_t s) {
    const size_t total = static_cast<size_t>(n) * ((qheads + kheads) * (dim / 2) + kheads * dim);
    launch("model_qkv_epilogue", qkv_epilogue_kernel, dim3(grid_for(total)), dim3(kThreads), 0, s, p, splits, n, qheads,
           kheads, dim, interleaved ? 1 : 0, cs, q, k, v);
    TVARA_HIP(hipGetLastError());
}

void launch_resid_norm(const float* p, int splits, float* x, const float* w, int n, int h, float eps, float* norm,
                       _Float16* halves, float* unscale, hipStream_t s) {
    if (h % 32 || h > 1024 * 8 * kEpiChunks) throw std::invalid_argument("batched decode width above 16384");
    launch("model_resid_norm", resid_norm_kernel, dim3(n), dim3(epi_threads(h)), 0, s, p, splits, x, w, n, h, eps, norm,
           halves, h / 32, unscale);
    TVARA_HIP(hipGetLastError());
}

void launch_swiglu_epilogue(const float* p, int splits, int n, int inter, float* out, _Float16* halves,
                            float* unscale, hipStream_t s, bool interleaved) {
    if (inter % 32 || inter > 1024 * 8 * kEpiChunks) throw std::invalid_argument("batched decode width above 16384");
    launch("model_swiglu_epilogue", swiglu_epilogue_kernel, dim3(n), dim3(epi_threads(inter)), 0, s, p, splits, n, inter,
           out, halves, inter / 32, unscale, interleaved ? 1 : 0);
    TVARA_HIP(hipGetLastError());
}

void launch_gather_embedding_q8(const Weight& w, const uint32_t* idx, uint32_t row, int n, float* out,
                                hipStream_t s) {
    const size_t total = static_cast<size_t>(n) * w.cols;
    launch("model_embedding", gather_embedding_q8_kernel, dim3(grid_for(total)), dim3(kThreads), 0, s,
           static_cast<const uint8_t*>(w.q.ptr), static_cast<const uint16_t*>(w.d.ptr), w.pairs(), idx, row, n,
           w.cols, out);
    TVARA_HIP(hipGetLastError());
}

}  // namespace tvara_amd
