// KV block management kernels for gfx950: block zero-fill / copy-on-write copy,
// token append (f32 rows, or quantise-on-append to Q8_0), row gather,
// canonical Q8_0 conversion and block checksums.
//
// Every kernel is a plain streaming copy or transform: bound by HBM, no MFMA.
// Threads walk 16-byte units (one dwordx4 per lane) so a wave moves 1 KiB per
// instruction.
#include "common.hpp"
#include "q8.hpp"

namespace tvara_amd {
namespace {

constexpr int kThreads = 256;

// Non-temporal 16-byte stores for block bytes: nothing in the same launch
// reads them back, so they skip allocation in the caches (a later decode or
// copy reads them from HBM).
__device__ inline void store_stream(uint4* p, const uint4 v) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<u32x4*>(p));
}

__device__ inline void store_stream(float4* p, const float4 v) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<f32x4*>(p));
}

// BlockPool::allocate zero-fill (kv.hpp:48) and PagedCache::append's
// whole-block copy (kv.hpp:99); grid.y = op, grid.x strides the block.
__global__ __launch_bounds__(kThreads) void block_init_kernel(char* pool, size_t stride,
                                                              const BlockInitOp* __restrict__ ops) {
    const BlockInitOp op = ops[blockIdx.y];
    uint4* dst = reinterpret_cast<uint4*>(pool + static_cast<size_t>(op.dst) * stride);
    const size_t units = stride / 16;
    const size_t step = static_cast<size_t>(gridDim.x) * blockDim.x;
    if (op.src >= 0) {
        const uint4* src = reinterpret_cast<const uint4*>(pool + static_cast<size_t>(op.src) * stride);
        for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < units; i += step)
            store_stream(dst + i, src[i]);
    } else {
        const uint4 zero = make_uint4(0, 0, 0, 0);
        for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < units; i += step)
            store_stream(dst + i, zero);
    }
}

// The same zero-fill / copy with the ops in the kernel arguments.
__global__ __launch_bounds__(kThreads) void block_init_inline_kernel(char* pool, size_t stride, const InlineInitOps ops) {
    const int2 op = ops.op[blockIdx.y];
    uint4* dst = reinterpret_cast<uint4*>(pool + static_cast<size_t>(op.x) * stride);
    const size_t units = stride / 16;
    const size_t step = static_cast<size_t>(gridDim.x) * blockDim.x;
    if (op.y >= 0) {
        const uint4* src = reinterpret_cast<const uint4*>(pool + static_cast<size_t>(op.y) * stride);
        for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < units; i += step)
            store_stream(dst + i, src[i]);
    } else {
        const uint4 zero = make_uint4(0, 0, 0, 0);
        for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < units; i += step)
            store_stream(dst + i, zero);
    }
}

// PagedCache::append row copies (kv.hpp:103-106) for f32 blocks with the ops
// in the kernel arguments.  grid.x = op, grid.y = chunk of kAppendUnroll *
// kThreads 16-byte units of the token's rows over every (layer, kind); each
// thread requests all its units before storing the first.  Requires
// kv_width % 4 == 0.
constexpr int kAppendUnroll = 4;

__global__ __launch_bounds__(kThreads) void append_rows_f32_inline_kernel(char* pool, BlockLayout lay,
                                                                          const InlineRowOps ops,
                                                                          const float* __restrict__ keys,
                                                                          const float* __restrict__ values) {
    const int2 op = ops.op[blockIdx.x];
    const int slot = op.y >> 16, src_row = op.y & 0xffff;
    const int row4 = lay.kv_width / 4;  // 16-byte units per (layer, kind) row
    const int units = lay.layers * 2 * row4;
    const float4* krow = reinterpret_cast<const float4*>(keys + static_cast<size_t>(src_row) * lay.layers * lay.kv_width);
    const float4* vrow = reinterpret_cast<const float4*>(values + static_cast<size_t>(src_row) * lay.layers * lay.kv_width);
    float4* block = reinterpret_cast<float4*>(pool + static_cast<size_t>(op.x) * lay.stride);
    const int u0 = blockIdx.y * (kAppendUnroll * kThreads) + threadIdx.x;
    float4 x[kAppendUnroll];
    int dst[kAppendUnroll];
#pragma unroll
    for (int j = 0; j < kAppendUnroll; ++j) {
        const int u = min(u0 + j * kThreads, units - 1);  // clamped: every load is issued
        const int r = u / row4, c4 = u - r * row4;        // r = layer * 2 + kind
        const int src = (r >> 1) * row4 + c4;
        x[j] = (r & 1) ? vrow[src] : krow[src];
        dst[j] = (r * lay.tpb + slot) * row4 + c4;
    }
#pragma unroll
    for (int j = 0; j < kAppendUnroll; ++j)
        if (u0 + j * kThreads < units) store_stream(block + dst[j], x[j]);
}

// PagedCache::append row copies (kv.hpp:103-106): grid.x = layer*2+kind,
// grid.y = op.  Source rows are [src_row][layers][kv_width].
__global__ __launch_bounds__(kThreads) void append_rows_f32_kernel(char* pool, BlockLayout lay,
                                                                   const RowOp* __restrict__ ops,
                                                                   const float* __restrict__ keys,
                                                                   const float* __restrict__ values) {
    const RowOp op = ops[blockIdx.y];
    const int layer = blockIdx.x >> 1, kind = blockIdx.x & 1;
    const float* src = (kind ? values : keys) + (static_cast<size_t>(op.src_row) * lay.layers + layer) * lay.kv_width;
    float* dst = reinterpret_cast<float*>(pool + static_cast<size_t>(op.block) * lay.stride) +
                 (static_cast<size_t>(layer * 2 + kind) * lay.tpb + op.slot) * lay.kv_width;
    if ((lay.kv_width & 3) == 0) {
        const float4* s4 = reinterpret_cast<const float4*>(src);
        float4* d4 = reinterpret_cast<float4*>(dst);
        for (int i = threadIdx.x; i < lay.kv_width / 4; i += blockDim.x) d4[i] = s4[i];
    } else {
        for (int i = threadIdx.x; i < lay.kv_width; i += blockDim.x) dst[i] = src[i];
    }
}

// One layer's rows of reserved tokens (DeviceCache::reserve_tokens): grid.x =
// op, grid.y = kind; source rows are [src_row][kv_width].  Plain stores: the
// attention of the same layer reads them next.
__global__ __launch_bounds__(kThreads) void write_layer_rows_kernel(char* pool, BlockLayout lay,
                                                                    const RowOp* __restrict__ ops, int layer,
                                                                    const float* __restrict__ keys,
                                                                    const float* __restrict__ values) {
    const RowOp op = ops[blockIdx.x];
    const int kind = blockIdx.y;
    const float* src = (kind ? values : keys) + static_cast<size_t>(op.src_row) * lay.kv_width;
    float* dst = reinterpret_cast<float*>(pool + static_cast<size_t>(op.block) * lay.stride) +
                 (static_cast<size_t>(layer * 2 + kind) * lay.tpb + op.slot) * lay.kv_width;
    if ((lay.kv_width & 3) == 0) {
        const float4* s4 = reinterpret_cast<const float4*>(src);
        float4* d4 = reinterpret_cast<float4*>(dst);
        for (int i = threadIdx.x; i < lay.kv_width / 4; i += blockDim.x) d4[i] = s4[i];
    } else {
        for (int i = threadIdx.x; i < lay.kv_width; i += blockDim.x) dst[i] = src[i];
    }
}

// Quantise-on-append into Q8_0 with the encoder of tools/make_api_fixture.py:131-137:
// one 32-lane half-wave per group; scale = max|x|/127 in f64, q = clip(rint(x/f32(scale)),
// -127, 127) with an IEEE f32 division, d = f16(scale) rounded to nearest even.
__global__ __launch_bounds__(kThreads) void append_rows_q8_kernel(char* pool, BlockLayout lay,
                                                                  const RowOp* __restrict__ ops,
                                                                  const float* __restrict__ keys,
                                                                  const float* __restrict__ values) {
    const RowOp op = ops[blockIdx.y];
    const int layer = blockIdx.x >> 1, kind = blockIdx.x & 1;
    const float* src = (kind ? values : keys) + (static_cast<size_t>(op.src_row) * lay.layers + layer) * lay.kv_width;
    char* sec = pool + static_cast<size_t>(op.block) * lay.stride + static_cast<size_t>(layer * 2 + kind) * lay.section;
    const int groups = lay.kv_width / 32;
    const int l32 = threadIdx.x & 31;
    for (int g = threadIdx.x >> 5; g < groups; g += blockDim.x >> 5) {
        const float x = src[g * 32 + l32];
        float amax = fabsf(x);
        for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
        uint16_t d;
        int8_t qv;
        q8_encode_element(x, amax, &d, &qv);
        reinterpret_cast<int8_t*>(sec)[q8_byte_offset(lay, op.slot, g * 32 + l32)] = qv;
        if (l32 == 0) *reinterpret_cast<uint16_t*>(sec + q8_scale_offset(lay, op.slot, g)) = d;
    }
}

__device__ __forceinline__ float load_element(const char* pool, const BlockLayout& lay, int block, int layer,
                                              int kind, int slot, int column) {
    const char* base = pool + static_cast<size_t>(block) * lay.stride;
    if (lay.format == kF32)
        return reinterpret_cast<const float*>(base)[(static_cast<size_t>(layer * 2 + kind) * lay.tpb + slot) *
                                                        lay.kv_width +
                                                    column];
    const char* sec = base + static_cast<size_t>(layer * 2 + kind) * lay.section;
    const int8_t q = reinterpret_cast<const int8_t*>(sec)[q8_byte_offset(lay, slot, column)];
    const uint16_t d = *reinterpret_cast<const uint16_t*>(sec + q8_scale_offset(lay, slot, column / 32));
    return half_bits_to_float(d) * static_cast<float>(q);  // dequantize_q8_0 (quant.hpp:43-47)
}

// PagedCache::read / read_all gather (kv.hpp:110-119): one workgroup per row
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(const char* pool, BlockLayout lay,
                                                               const int2* __restrict__ rows, int layer, int kind,
                                                               float* __restrict__ out) {
    const int2 r = rows[blockIdx.x];
    float* o = out + static_cast<size_t>(blockIdx.x) * lay.kv_width;
    for (int i = threadIdx.x; i < lay.kv_width; i += blockDim.x)
        o[i] = load_element(pool, lay, r.x, layer, kind, r.y, i);
}

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z ^= z >> 30;
    z *= 0xBF58476D1CE4E5B9ull;
    z ^= z >> 27;
    z *= 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// byte `j` of the canonical image of a Q8_0 block
__device__ __forceinline__ uint32_t canonical_q8_byte(const char* base, const BlockLayout& lay, size_t j) {
    const size_t group = j / 34, off = j % 34;
    const int gpr = lay.kv_width / 32;  // groups per slot row
    const size_t row = group / gpr;     // (layer*2+kind)*tpb + slot
    const int gcol = static_cast<int>(group % gpr);
    const int sec = static_cast<int>(row / lay.tpb), slot = static_cast<int>(row % lay.tpb);
    const unsigned char* s = reinterpret_cast<const unsigned char*>(base + static_cast<size_t>(sec) * lay.section);
    if (off < 2) return s[q8_scale_offset(lay, slot, gcol) + off];
    return s[q8_byte_offset(lay, slot, gcol * 32) + (off - 2)];
}

__device__ __forceinline__ size_t canonical_words(const BlockLayout& lay) {
    const size_t elements = static_cast<size_t>(lay.layers) * 2 * lay.tpb * lay.kv_width;
    return lay.format == kF32 ? elements : elements / 32 * 34 / 4;
}

// checksum of each listed block's canonical image; one workgroup per block
__global__ __launch_bounds__(kThreads) void checksum_kernel(const char* pool, BlockLayout lay,
                                                            const int64_t* __restrict__ ids,
                                                            uint64_t* __restrict__ out) {
    __shared__ uint64_t partial[kThreads / 64];
    const char* base = pool + static_cast<size_t>(ids[blockIdx.x]) * lay.stride;
    const size_t words = canonical_words(lay);
    uint64_t h = 0;
    for (size_t i = threadIdx.x; i < words; i += blockDim.x) {
        uint32_t w;
        if (lay.format == kF32) {
            w = reinterpret_cast<const uint32_t*>(base)[i];
        } else {
            w = canonical_q8_byte(base, lay, 4 * i) | (canonical_q8_byte(base, lay, 4 * i + 1) << 8) |
                (canonical_q8_byte(base, lay, 4 * i + 2) << 16) | (canonical_q8_byte(base, lay, 4 * i + 3) << 24);
        }
        h += mix64((static_cast<uint64_t>(i) << 32) | w);
    }
    for (int m = 32; m >= 1; m >>= 1) {
        const uint32_t lo = __shfl_xor(static_cast<uint32_t>(h), m), hi = __shfl_xor(static_cast<uint32_t>(h >> 32), m);
        h += (static_cast<uint64_t>(hi) << 32) | lo;
    }
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = h;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t total = 0;
        for (int w = 0; w < kThreads / 64; ++w) total += partial[w];
        out[blockIdx.x] = total;
    }
}

// one Q8_0 block to / from its canonical image (34-byte groups); one thread per group
__global__ __launch_bounds__(kThreads) void q8_to_canonical_kernel(const char* pool, BlockLayout lay, int64_t id,
                                                                   uint8_t* __restrict__ out) {
    const int gpr = lay.kv_width / 32;
    const size_t groups = static_cast<size_t>(lay.layers) * 2 * lay.tpb * gpr;
    const char* base = pool + static_cast<size_t>(id) * lay.stride;
    for (size_t g = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; g < groups;
         g += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const size_t row = g / gpr;
        const int gcol = static_cast<int>(g % gpr);
        const int sec = static_cast<int>(row / lay.tpb), slot = static_cast<int>(row % lay.tpb);
        const unsigned char* s = reinterpret_cast<const unsigned char*>(base + static_cast<size_t>(sec) * lay.section);
        const unsigned char* d = s + q8_scale_offset(lay, slot, gcol);
        const unsigned char* q = s + q8_byte_offset(lay, slot, gcol * 32);
        uint8_t* o = out + g * 34;
        o[0] = d[0];
        o[1] = d[1];
        for (int i = 0; i < 32; ++i) o[2 + i] = q[i];
    }
}

__global__ __launch_bounds__(kThreads) void canonical_to_q8_kernel(char* pool, BlockLayout lay, int64_t id,
                                                                   const uint8_t* __restrict__ in) {
    const int gpr = lay.kv_width / 32;
    const size_t groups = static_cast<size_t>(lay.layers) * 2 * lay.tpb * gpr;
    char* base = pool + static_cast<size_t>(id) * lay.stride;
    for (size_t g = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; g < groups;
         g += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const size_t row = g / gpr;
        const int gcol = static_cast<int>(g % gpr);
        const int sec = static_cast<int>(row / lay.tpb), slot = static_cast<int>(row % lay.tpb);
        unsigned char* s = reinterpret_cast<unsigned char*>(base + static_cast<size_t>(sec) * lay.section);
        unsigned char* d = s + q8_scale_offset(lay, slot, gcol);
        unsigned char* q = s + q8_byte_offset(lay, slot, gcol * 32);
        const uint8_t* i8 = in + g * 34;
        d[0] = i8[0];
        d[1] = i8[1];
        for (int i = 0; i < 32; ++i) q[i] = i8[2 + i];
    }
}

constexpr int kMaxGridY = 65535;

}  // namespace

void launch_block_init(char* pool, size_t stride, const BlockInitOp* ops, int n, hipStream_t s) {
    if (n <= 0) return;
    const size_t units = stride / 16;
    const unsigned gx = static_cast<unsigned>(std::min<size_t>((units + kThreads - 1) / kThreads, 512));
    for (int base = 0; base < n; base += kMaxGridY) {
        const int count = std::min(kMaxGridY, n - base);
        launch("kv_block_init", block_init_kernel, dim3(gx, count), dim3(kThreads), 0, s, pool, stride, ops + base);
    }
    TVARA_HIP(hipGetLastError());
}

void launch_block_init_inline(char* pool, size_t stride, const InlineInitOps& ops, int n, hipStream_t s) {
    if (n <= 0) return;
    const size_t units = stride / 16;
    const unsigned gx = static_cast<unsigned>(std::min<size_t>((units + kThreads - 1) / kThreads, 512));
    launch("kv_block_init", block_init_inline_kernel, dim3(gx, n), dim3(kThreads), 0, s, pool, stride, ops);
    TVARA_HIP(hipGetLastError());
}

void launch_append_rows_inline(char* pool, const BlockLayout& lay, const InlineRowOps& ops, int n, const float* keys,
                               const float* values, hipStream_t s) {
    if (n <= 0) return;
    const int units = lay.layers * 2 * (lay.kv_width / 4);
    const int chunks = (units + kAppendUnroll * kThreads - 1) / (kAppendUnroll * kThreads);
    launch("kv_append_rows", append_rows_f32_inline_kernel, dim3(n, chunks), dim3(kThreads), 0, s, pool, lay, ops,
           keys, values);
    TVARA_HIP(hipGetLastError());
}

void launch_append_rows(char* pool, const BlockLayout& lay, const RowOp* ops, int n, const float* keys,
                        const float* values, hipStream_t s) {
    if (n <= 0) return;
    const int threads = lay.format == kF32 ? (lay.kv_width >= 1024 ? 256 : 128) : 256;
    for (int base = 0; base < n; base += kMaxGridY) {
        const int count = std::min(kMaxGridY, n - base);
        if (lay.format == kF32)
            launch("kv_append_rows", append_rows_f32_kernel, dim3(lay.layers * 2, count), dim3(threads), 0, s, pool,
                   lay, ops + base, keys, values);
        else
            launch("kv_append_rows", append_rows_q8_kernel, dim3(lay.layers * 2, count), dim3(threads), 0, s, pool,
                   lay, ops + base, keys, values);
    }
    TVARA_HIP(hipGetLastError());
}

void launch_write_layer_rows(char* pool, const BlockLayout& lay, const RowOp* ops, int n, int layer,
                             const float* keys, const float* values, hipStream_t s) {
    if (n <= 0) return;
    const int threads = lay.kv_width >= 1024 ? 256 : (lay.kv_width >= 256 ? 128 : 64);
    launch("kv_append_rows", write_layer_rows_kernel, dim3(n, 2), dim3(threads), 0, s, pool, lay, ops, layer, keys,
           values);
    TVARA_HIP(hipGetLastError());
}

void launch_gather_rows(const char* pool, const BlockLayout& lay, const int2* rows, int n, int layer, int kind,
                        float* out, hipStream_t s) {
    if (n <= 0) return;
    launch("kv_gather_rows", gather_rows_kernel, dim3(n), dim3(128), 0, s, pool, lay, rows, layer, kind, out);
    TVARA_HIP(hipGetLastError());
}

void launch_checksums(const char* pool, const BlockLayout& lay, const int64_t* ids, int n, uint64_t* out,
                      hipStream_t s) {
    if (n <= 0) return;
    launch("kv_checksum", checksum_kernel, dim3(n), dim3(kThreads), 0, s, pool, lay, ids, out);
    TVARA_HIP(hipGetLastError());
}

void launch_q8_to_canonical(const char* pool, const BlockLayout& lay, int64_t id, uint8_t* out, hipStream_t s) {
    launch("kv_q8_to_canonical", q8_to_canonical_kernel, dim3(64), dim3(kThreads), 0, s, pool, lay, id, out);
    TVARA_HIP(hipGetLastError());
}

void launch_canonical_to_q8(char* pool, const BlockLayout& lay, int64_t id, const uint8_t* in, hipStream_t s) {
    launch("kv_canonical_to_q8", canonical_to_q8_kernel, dim3(64), dim3(kThreads), 0, s, pool, lay, id, in);
    TVARA_HIP(hipGetLastError());
}

}  // namespace tvara_amd
