// Device paged KV cache: the reference's PagedCache/BlockPool rules
// (core/include/tvara/kv.hpp) kept on the host, block storage in one HBM
// allocation, and every byte movement done by gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <map>
#include <vector>

#include "common.hpp"

namespace tvara_amd {

// Grow-only device buffer.
struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    void* ensure(size_t n);
    ~DeviceBuffer();
};

// Grow-only pinned host buffer whose reuse waits for the last copy out of it.
struct PinnedBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    hipEvent_t done = nullptr;
    void* acquire(size_t n);
    void release(hipStream_t s);
    ~PinnedBuffer();
};

class DeviceCache {
public:
    DeviceCache(const Geometry& g, int format);
    ~DeviceCache();
    DeviceCache(const DeviceCache&) = delete;
    DeviceCache& operator=(const DeviceCache&) = delete;

    const Geometry& geometry() const { return meta_.geometry(); }
    int format() const { return format_; }
    const BlockLayout& layout() const { return lay_; }
    size_t canonical_block_bytes() const;
    char* pool() const { return pool_; }
    hipStream_t stream() const { return stream_; }
    void set_stream(hipStream_t s) { stream_ = s; }
    uint64_t epoch() const { return meta_.epoch(); }
    int compute_units() const { return cus_; }
    int xcds() const { return xcds_; }  // XCDs (L2 domains) the workgroups are dealt over
    void synchronize();

    // the host bookkeeping (pool and tables); prefix trees work on it directly
    KvLedger& ledger() { return meta_; }
    const KvLedger& ledger() const { return meta_; }

    // BlockPool (kv.hpp:36-75)
    Handle allocate() { return meta_.allocate(); }
    void retain(Handle h) { meta_.retain(h); }
    void release(Handle h) { meta_.release(h); }
    size_t references(Handle h) const { return meta_.references(h); }
    size_t references_by_id(size_t id) const { return meta_.references_by_id(id); }
    size_t available() const { return meta_.available(); }
    void pool_audit() const { meta_.pool_audit(); }
    void pool_state(size_t* refs, uint64_t* generations, size_t* free_pop_order, size_t* free_count) const {
        meta_.pool_state(refs, generations, free_pop_order, free_count);
    }
    void block_read(Handle h, void* out, size_t bytes);
    void block_write(Handle h, size_t offset, const void* data, size_t bytes);
    void checksums(const Handle* handles, size_t n, uint64_t* out);

    // PagedCache (kv.hpp:78-165)
    uint64_t create_sequence() { return meta_.create_sequence(); }
    const Table& sequence(uint64_t id) const { return meta_.sequence(id); }
    std::vector<uint64_t> sequence_ids() const { return meta_.sequence_ids(); }
    Handle physical_block(uint64_t id, size_t position) const { return meta_.physical_block(id, position); }
    // appends one token to each listed sequence in order; *applied receives the
    // number applied before the failure of the first one that could not be,
    // which is rethrown
    size_t append_batch(const uint64_t* seqs, size_t n, const float* keys, const float* values, bool device,
                        size_t* applied = nullptr);
    size_t append_tokens(uint64_t seq, const float* keys, const float* values, size_t count, bool device);
    // Layer-wise appends (f32 blocks): appends `count` tokens to `seq` in the
    // ledger and runs their block work (zero-fills, copy-on-write copies) but
    // writes no rows; the returned device list gives each token's (block,
    // slot), in order, for write_layer_rows().  The tokens hold stale bytes
    // until every layer's rows are written, so the caller writes them before
    // anything reads them, or truncates.  On failure the block work of the
    // appends that took effect still runs, then the error is rethrown and the
    // caller truncates.
    const RowOp* reserve_tokens(uint64_t seq, size_t count);
    // layer `layer`'s K and V rows ([n][kv_width] floats, row i for the
    // token of ops[i]) into their slots
    void write_layer_rows(const RowOp* ops, size_t n, int layer, const float* keys, const float* values);
    void read(uint64_t id, size_t layer, size_t position, bool value, float* out);
    void read_all(uint64_t id, size_t layer, bool value, float* out, size_t capacity);
    void drop(uint64_t id) { meta_.drop(id); }
    uint64_t fork(uint64_t id) { return meta_.fork(id); }
    void truncate(uint64_t id, size_t length) { meta_.truncate(id, length); }
    void audit(const size_t* external, size_t count) const { meta_.audit(external, count); }
    uint64_t import_sequence(const Handle* blocks, size_t count, size_t source_length, size_t length) {
        return meta_.import_sequence(blocks, count, source_length, length);
    }

    // zero-fill blocks handed out by allocate() that are still live (kernel
    // launches with their ops in the arguments: no upload, no allocation)
    void flush();
    // Work on another stream `s` that reads the pool: enter() makes `s` wait
    // for everything queued on the cache's stream (appends, copies,
    // zero-fills); leave() makes the cache's stream wait for what `s` has
    // queued, so a later write to a block cannot overtake a read of it.
    void enter(hipStream_t s);
    void leave(hipStream_t s);
    // device scratch owned by the cache
    DeviceBuffer& scratch(int i) { return scratch_[i]; }
    PinnedBuffer& pinned(int i) { return pinned_[i]; }
    int* error_flag() const { return err_; }

private:
    // zero-fills and copy-on-write copies of planned appends, on the stream
    void run_block_init(const std::vector<BlockInitOp>& init);

    KvLedger meta_;
    int format_;
    BlockLayout lay_{};
    char* pool_ = nullptr;
    hipStream_t stream_ = nullptr;
    int cus_ = 256, xcds_ = 1;
    hipEvent_t ordered_[2] = {nullptr, nullptr};
    DeviceBuffer scratch_[6];
    PinnedBuffer pinned_[6];
    int* err_ = nullptr;
};

// A batch of attention rows with resident block tables.  compute() builds the
// host image of the plan (block ids, per-row entries, work items); place()
// uploads it into buffers the plan owns, place_in() into one packed region of
// caller-provided device memory (no allocation).
struct AttnPlan {
    DeviceCache* cache = nullptr;
    uint64_t epoch = 0;
    int rows = 0, heads = 0, group = 0, items = 0, split_tokens = 0;
    // query groups above eight (f32 blocks: four at head_dims 96 and 256,
    // three at 80) run as kv_share slices of group / kv_share heads, each a
    // virtual KV head
    int kv_share = 1;
    int wave_splits = 0;  // > 0: a row's splits are the waves of ws_chunks workgroups per (row, KV head)
    int ws_chunks = 1;
    bool row_major = false;  // the launch runs decode_rows_kernel (one workgroup per item)
    bool need_merge = false, with_tail = false, inline_ok = false;
    size_t kv_bytes = 0;  // algorithmic K/V bytes one launch reads
    RowSplits inline_rows{};  // (first item, splits) per row when rows <= kInlineRows
    WsItems ws_items{};       // wave splits of few items: the items for the kernel arguments
    WorkOrder order{};        // launch order of the items (n == 0: item order)
    // host image
    std::vector<int32_t> h_tables;
    std::vector<int4> h_entries, h_work;
    std::vector<int2> h_items;
    std::vector<int32_t> h_work_blocks;
    // where the device copy lives
    struct Placement {
        const int32_t* tables = nullptr;
        const int4* entries = nullptr;
        const int2* items = nullptr;
        const int4* work = nullptr;
        const int32_t* work_blocks = nullptr;
        float* part_acc = nullptr;
        float* part_ml = nullptr;
        int* row_done = nullptr;
        int* err = nullptr;
    } dev;
    DeviceBuffer region;  // place(): the packed plan (grow-only)
    PinnedBuffer staging;
    PinnedBuffer flag;  // check(): the error flag's host copy, or the flag itself (pinned_err)
    // the kernels set the error flag in pinned host memory (no copy back
    // before a check); plans built by build() use it, the no-allocation path
    // keeps the device flag
    bool pinned_err = false;
    hipStream_t last_stream = nullptr;

    AttnPlan() = default;
    AttnPlan(const AttnPlan&) = delete;
    AttnPlan& operator=(const AttnPlan&) = delete;

    // Builds the plan for rows reading `cached[r]` tokens of `seq_of_row[r]`,
    // followed by the row's uncommitted tail token when tail_rows[r] != 0.
    void compute(DeviceCache* c, const std::vector<uint64_t>& seq_of_row, const std::vector<size_t>& cached,
                 const std::vector<uint8_t>& tail_rows, int heads, size_t split_override);
    // into the plan's own region, one asynchronous copy on the cache's stream
    void place();
    void xcd_balance(int xcds);
    // bytes place_in needs, and the leading part of them it copies
    size_t region_bytes(size_t* copied = nullptr) const;
    // packs the image into `host` (at least the copied bytes; it must stay
    // untouched until the copy on `s` has run) and copies it to `device`
    void place_in(char* device, size_t capacity, hipStream_t s, char* host);
    void build(DeviceCache* c, const std::vector<uint64_t>& seq_of_row, const std::vector<size_t>& cached,
               const std::vector<uint8_t>& tail_rows, int heads, size_t split_override) {
        compute(c, seq_of_row, cached, tail_rows, heads, split_override);
        place();
        use_pinned_error();
    }
    void use_pinned_error();
    void launch(int layer, const float* q, const float* tail_k, const float* tail_v, float* out, hipStream_t s);
    // waits for the last launch's stream; a non-finite score throws
    void check();
    // the same, waiting only for `after` (an event recorded after the last
    // launch) when the kernels write the pinned flag; work queued behind the
    // launch keeps running
    void check_after(hipEvent_t after);
    // the same, with the flag copied to caller-provided host memory (no
    // pinned allocation)
    void check_into(int* host_flag);
    // queues the error flag's copy to pinned host memory on the last launch's
    // stream; after the stream has drained, finish_check() reads it
    void queue_check();
    void finish_check();
};

// Chunked-prefill plan: sequences[i] attends its prompt rows start[i] ..
// start[i] + rows[i] - 1 causally (fused_prompt_attention,
// attention.hpp:85-89).  precision 0 = f32 rows through the decode kernels,
// 1 = the bf16 MFMA tile kernel, 2 = the tile kernel with three products
// per product of split operands (f32 or Q8_0 blocks).  Block tables stay resident, so a plan built
// once per chunk serves every layer.
struct PrefillPlan {
    DeviceCache* cache = nullptr;
    uint64_t epoch = 0;
    int heads = 0, group = 0, count = 0, max_rows = 0, precision = 0;
    int kv_share = 1;  // bf16: GQA groups above eight run as slices (as AttnPlan)
    size_t total_rows = 0;
    AttnPlan rows_plan;
    DeviceBuffer tables, seqs, err;
    // the tile kernels set the error flag in pinned host memory instead
    // (use_pinned_error: no copy back before a check)
    PinnedBuffer flag;
    bool pinned_err = false;
    hipStream_t last_stream = nullptr;
    PrefillPlan() = default;
    PrefillPlan(const PrefillPlan&) = delete;
    PrefillPlan& operator=(const PrefillPlan&) = delete;
    void build(DeviceCache* c, const uint64_t* sequences, size_t count, size_t heads, size_t context,
               const size_t* start, const size_t* rows, int precision);
    void use_pinned_error();
    void launch(int layer, const float* q, float* out, hipStream_t s);
    void check();
    // the same, waiting only for `after` (an event recorded after the last
    // launch) when the flag is pinned
    void check_after(hipEvent_t after);
};

// ModelConfig::validate (model.hpp:13-19), the part attention depends on
void check_attention_config(const DeviceCache& c, size_t heads, size_t context);

// Rows of fused_paged_attention calls (attention.hpp:57-83) for `count`
// sequences: the argument checks of attention.hpp:59-63 and the visible cap.
void attention_rows(const DeviceCache& c, const uint64_t* seqs, size_t count, size_t context, bool tail,
                    const size_t* visible, std::vector<uint64_t>& seq_of_row, std::vector<size_t>& cached,
                    std::vector<uint8_t>& tail_rows);

}  // namespace tvara_amd

// the device cache behind a C ABI handle (capi.cpp); throws for NULL
struct tvara_kv_cache;
namespace tvara_amd {
DeviceCache& device_cache(tvara_kv_cache* handle);
}  // namespace tvara_amd
