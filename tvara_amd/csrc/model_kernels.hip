// Device kernels of the Llama decode executor around the paged attention
// path: weight dequantisation at load, RMSNorm, matrix-vector products,
// rotary embedding and the SwiGLU gate (core/include/tvara/model.hpp:47-126,
// core/include/tvara/quant.hpp:14-71,178-184).
//
// Rounding follows the reference's: products and sums the reference rounds to
// float one at a time are written with __fmul_rn / __fsub_rn / __fadd_rn so
// the compiler does not contract them into FMAs; dot products and the RMS sum
// accumulate in double and round once, as quant::dot_f32 and rms_norm do.
#include "model.hpp"
#include "q8.hpp"

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

// ------------------------------------------------------------- RoPE

// rotate pair i of every head of q and k by the (cos, sin) of this position
// (model.hpp:63-72): interleaved pairs (2i, 2i+1) or split (i, i+dim/2)
__global__ void rope_kernel(float* q, int qheads, float* k, int kheads, int dim, const float* cs, int interleaved) {
    const int half = dim / 2;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (qheads + kheads) * half) return;
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

void launch_rmsnorm(const float* x, const float* w, float* out, int n, float eps, hipStream_t s) {
    launch("model_rmsnorm", rmsnorm_kernel, dim3(1), dim3(1024), 0, s, x, w, out, n, eps);
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
                 hipStream_t s) {
    const int n = (qheads + kheads) * (dim / 2);
    launch("model_rope", rope_kernel, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, s, q, qheads, k, kheads,
           dim, cs, interleaved ? 1 : 0);
    TVARA_HIP(hipGetLastError());
}

void launch_swiglu(float* gate, const float* up, int n, hipStream_t s) {
    launch("model_swiglu", swiglu_kernel, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, s, gate, up, n);
    TVARA_HIP(hipGetLastError());
}

}  // namespace tvara_amd
