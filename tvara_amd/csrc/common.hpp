// Internal declarations shared by the host allocator, the C ABI and the
// gfx950 kernels of libtvara_capi.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "kv_ledger.hpp"

namespace tvara_amd {

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
#define TVARA_HIP(x) ::tvara_amd::hip_check((x), #x)

enum Format : int { kF32 = 0, kQ8 = 1 };

// Where a (layer, kind, slot, column) element of a block lives in HBM.
//  f32: the reference layout, ((layer*2+kind)*tpb+slot)*kv_width+column floats
//       (kv.hpp:30-33), so block bytes are the reference's bytes.
//  Q8_0: one section per (layer, kind) of `section` bytes holding each KV head
//       in turn: the head's int8 plane [tpb][head_dim] followed by its fp16
//       scale plane [tpb][head_dim/32], `head_bytes` per head (16-byte
//       aligned).  A head's tokens in a block are then one contiguous run
//       (2,176 B for 16 tokens at head_dim 128), which is what one decode wave
//       reads.  The canonical image is the reference element order cut into
//       34-byte groups (little-endian fp16 d, then 32 int8).
struct BlockLayout {
    int format;
    int layers, kv_heads, head_dim, tpb, kv_width;
    size_t stride;      // bytes between consecutive blocks in the pool (256-aligned)
    size_t section;     // Q8_0: bytes per (layer, kind) section
    size_t head_bytes;  // Q8_0: bytes per KV head within a section
};

// Q8_0: offset within a section of the int8 of (slot, column) and of the
// fp16 scale of (slot, group of 32 columns), columns and groups counted
// across the whole kv_width row
__host__ __device__ inline size_t q8_byte_offset(const BlockLayout& lay, int slot, int column) {
    const int h = column / lay.head_dim;
    return static_cast<size_t>(h) * lay.head_bytes + static_cast<size_t>(slot) * lay.head_dim + (column - h * lay.head_dim);
}

__host__ __device__ inline size_t q8_scale_offset(const BlockLayout& lay, int slot, int group) {
    const int ng = lay.head_dim / 32, h = group / ng;
    return static_cast<size_t>(h) * lay.head_bytes + static_cast<size_t>(lay.tpb) * lay.head_dim +
           (static_cast<size_t>(slot) * ng + (group - h * ng)) * 2;
}

// Block work passed in the kernel arguments (no upload) when a call has at
// most kInlineOps of it: init ops as (dst, src or -1) int32 pairs, row ops as
// (block, slot << 16 | input row) with slot and row below 65,536.
constexpr int kInlineOps = 400;
struct InlineInitOps {
    int2 op[kInlineOps];
};
struct InlineRowOps {
    int2 op[kInlineOps];
};

// Decode work: one entry per attention row (a sequence for decode, a
// (sequence, position) pair for the f32 prompt path); work items split rows
// into chunks of `split_tokens` cached tokens.
// longest split a decode work item covers: 64 blocks of 16 tokens (the
// kernels hold a split's block ids one per lane of a wave)
constexpr size_t kMaxSplitTokens = 1024;
constexpr int kMaxSplitBlocks = 64;  // block ids per work item (16-token blocks)

// Per attention row: (first work item, number of splits), passed in the
// merge kernel's arguments when a plan has at most kInlineRows rows.
constexpr int kInlineRows = 128;
struct RowSplits {
    int2 r[kInlineRows];
};

// Launch order of a decode launch's work items when the plan has at most
// kOrderedItems of them and one workgroup per item: workgroup s runs item
// item[s] (n == 0: workgroup s runs item s).  Workgroups go to the XCDs
// round-robin by id, so the order sets how many tokens each XCD streams.
constexpr int kOrderedItems = 512;
struct WorkOrder {
    int n;
    uint16_t item[kOrderedItems];
};

// A wave-split launch of few work items passes every item's descriptor and
// block ids in its kernel arguments, so no dependent load precedes its K/V
// reads (n == 0: the kernel reads them from the plan in HBM).  Slot
// chunk * kWsInlineWaves + wave holds an item, kWsInlinePer ids a slot: a
// launch of up to eight (row, chunk) workgroups whose splits span at most
// four blocks.
constexpr int kWsInlineWaves = 8, kWsInlinePer = 4;
constexpr int kWsInlineItems = 64, kWsInlineIds = kWsInlineItems * kWsInlinePer;
struct WsItems {
    int n;  // items
    int4 item[kWsInlineItems];
    int32_t ids[kWsInlineIds];
};

struct DecodeArgs {
    const char* pool;
    BlockLayout lay;
    int layer;
    int heads, group;  // query heads, heads per kv head
    const int32_t* tables;
    const int4* entries;  // x: table offset, y: cached tokens, z: tail | nsplit<<1, w: first item
    const int2* items;    // x: row, y: split index
    int split_tokens;
    // 16-token blocks: per work item x: row, y: first token, z: end token,
    // w: tail (the row's uncommitted token is this item's last) | the row's splits << 1;
    // and the item's block ids, kMaxSplitBlocks per item
    const int4* work;
    const int32_t* work_blocks;
    // per (row, KV-head group of a workgroup): splits finished in this launch,
    // for kernels that merge a row's splits in its last workgroup (zero between
    // launches; null: merge_kernel merges)
    int* row_done;
    int wave_splits;  // > 0: each row's splits are the waves of ws_chunks workgroups per (row, KV head)
    int ws_chunks;    // wave splits: workgroups per (row, KV head); above 1 they leave partials per chunk
    int row_major;    // 1: decode_rows_kernel (one eight-wave workgroup per work item)
    // Query groups above eight run as slices: lay.kv_heads and group describe
    // kv_share virtual KV heads per KV head, and virtual head v reads the K/V
    // of head v / kv_share (1: no slicing)
    int kv_share;
    const float* q;
    const float* tail_k;  // [rows][kv_width] or null
    const float* tail_v;
    float* out;
    float* part_acc;  // [items][heads][head_dim]
    float* part_ml;   // [items][heads][2]: running max (log2 units), normaliser
    float qscale;     // log2(e)/sqrt(head_dim)
    int* err;
};

struct PrefillArgs {
    const char* pool;
    BlockLayout lay;
    int layer;
    int heads, group;
    const int32_t* tables;
    const int4* seqs;  // x: table offset, y: start, z: rows, w: first query row
    const float* q;    // [sum rows][heads][head_dim]
    float* out;
    float qscale;
    int* err;
    int chunk_tiles;  // query tiles per (sequence, KV head) pair (set by the launcher)
    int pairs;        // sequences x KV heads
    // as DecodeArgs::kv_share: lay.kv_heads and group describe kv_share
    // virtual KV heads per KV head (GQA groups above eight)
    int kv_share;
};

// launchers (kernels.hip)
void launch_block_init(char* pool, size_t stride, const BlockInitOp* ops, int n, hipStream_t s);
void launch_block_init_inline(char* pool, size_t stride, const InlineInitOps& ops, int n, hipStream_t s);
void launch_append_rows_inline(char* pool, const BlockLayout& lay, const InlineRowOps& ops, int n, const float* keys,
                               const float* values, hipStream_t s);
void launch_append_rows(char* pool, const BlockLayout& lay, const RowOp* ops, int n, const float* keys,
                        const float* values, hipStream_t s);
// one layer's K and V rows ([n][kv_width] floats) into the f32 slots of ops
void launch_write_layer_rows(char* pool, const BlockLayout& lay, const RowOp* ops, int n, int layer,
                             const float* keys, const float* values, hipStream_t s);
void launch_gather_rows(const char* pool, const BlockLayout& lay, const int2* rows, int n, int layer, int kind,
                        float* out, hipStream_t s);
void launch_checksums(const char* pool, const BlockLayout& lay, const int64_t* ids, int n, uint64_t* out,
                      hipStream_t s);
void launch_q8_to_canonical(const char* pool, const BlockLayout& lay, int64_t id, uint8_t* out, hipStream_t s);
void launch_canonical_to_q8(char* pool, const BlockLayout& lay, int64_t id, const uint8_t* in, hipStream_t s);
// decode.hip
void launch_decode(const DecodeArgs& a, int nitems, int nrows, bool need_merge, const RowSplits* inline_rows,
                   const WorkOrder* order, hipStream_t s, const WsItems* ws_items = nullptr);
int decode_waves(int kv_heads, int group, int format, int head_dim);
int decode_slots(int kv_heads, int group, int format, int head_dim);  // waves' worth of work per work item
// waves == 0: the usual decomposition
struct WaveSplitShape {
    int waves = 0;    // splits per chunk, the waves of its workgroup
    int chunks = 0;   // workgroups per (row, KV head)
    size_t tokens = 0;  // tokens per split (a whole number of blocks)
};
WaveSplitShape wave_split_shape(int rows, int kv_heads, int group, int format, int head_dim, int tpb,
                                size_t max_tokens, int cus);
int decode_budget_per_cu(int group, int format, int head_dim);
// Shapes the row-major f32 kernel takes (head_dim 64, 16-token blocks, 4, 8
// or 16 KV heads, up to eight query heads each); plans of such a shape whose
// launch has more than kRowMajorMinWorkgroups workgroups use it.
bool decode_rows_shape(int kv_heads, int group, int format, int head_dim, int tpb);
// block sizes the f32 decode kernels stream directly (powers of two from 16
// to 1,024 tokens); their splits start on a block
bool decode_f32_blocks(int tpb);
constexpr size_t kRowMajorMinWorkgroups = 128;
// prefill.hip
bool prefill_bf16_supported(const BlockLayout& lay, int group);
// x3: the f32-accurate variant (three products per product of split
// operands), on the blocks the bf16 tiles take
bool prefill_x3_supported(const BlockLayout& lay, int group);
void launch_prefill_bf16(const PrefillArgs& a, int nseqs, int max_rows, hipStream_t s, bool x3 = false);

// kernel timing (profile.cpp)
// Per-kernel timing for tvara_profile_*: while enabled, every launch made
// through launch() carries a start/stop event pair that the runtime stamps
// with the kernel's own start and end.
bool profile_events(hipEvent_t* start, hipEvent_t* stop);
void profile_record(const char* name, hipEvent_t start, hipEvent_t stop);

template <class Kernel, class... Args>
void launch(const char* name, Kernel kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, Args... args) {
    hipEvent_t start = nullptr, stop = nullptr;
    const bool timed = profile_events(&start, &stop);
    hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), s, start, stop, 0, args...);
    if (timed) profile_record(name, start, stop);
}

}  // namespace tvara_amd
