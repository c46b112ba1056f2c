// Device half of the paged KV cache: block storage in one HBM allocation,
// every byte movement done by the gfx950 kernels of kv_kernels.hip, and the
// host bookkeeping (pool, tables, append planning) in KvLedger
// (kv_ledger.cpp), which follows core/include/tvara/kv.hpp.
#include "kv_cache.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <limits>
#include <numeric>

namespace tvara_amd {

namespace {
constexpr size_t kMax = std::numeric_limits<size_t>::max();

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

enum Slot { kInitOps = 0, kRowOps = 1, kKeys = 2, kValues = 3, kMisc = 4, kMiscOut = 5 };
}  // namespace

// -------------------------------------------------------------- buffers

void* DeviceBuffer::ensure(size_t n) {
    if (n <= bytes && ptr) return ptr;
    if (ptr) {
        TVARA_HIP(hipDeviceSynchronize());
        TVARA_HIP(hipFree(ptr));
        ptr = nullptr;
        bytes = 0;
    }
    const size_t want = std::max<size_t>(round_up(n, 4096), 4096);
    TVARA_HIP(hipMalloc(&ptr, want));
    bytes = want;
    return ptr;
}

DeviceBuffer::~DeviceBuffer() {
    if (ptr) (void)hipFree(ptr);
}

void* PinnedBuffer::acquire(size_t n) {
    if (done) TVARA_HIP(hipEventSynchronize(done));
    if (n > bytes || !ptr) {
        if (ptr) TVARA_HIP(hipHostFree(ptr));
        ptr = nullptr;
        const size_t want = std::max<size_t>(round_up(n, 4096), 4096);
        TVARA_HIP(hipHostMalloc(&ptr, want, hipHostMallocDefault));
        bytes = want;
    }
    return ptr;
}

void PinnedBuffer::release(hipStream_t s) {
    if (!done) TVARA_HIP(hipEventCreateWithFlags(&done, hipEventDisableTiming));
    TVARA_HIP(hipEventRecord(done, s));
}

PinnedBuffer::~PinnedBuffer() {
    if (done) {
        (void)hipEventSynchronize(done);
        (void)hipEventDestroy(done);
    }
    if (ptr) (void)hipHostFree(ptr);
}

// host vector -> device scratch slot, through pinned memory, on the stream
template <class T>
static T* upload(DeviceCache& c, int slot, const T* data, size_t count) {
    const size_t bytes = count * sizeof(T);
    if (!bytes) return nullptr;
    PinnedBuffer& p = c.pinned(slot);
    void* host = p.acquire(bytes);
    std::memcpy(host, data, bytes);
    void* dev = c.scratch(slot).ensure(bytes);
    TVARA_HIP(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, c.stream()));
    p.release(c.stream());
    return static_cast<T*>(dev);
}

// ------------------------------------------------------- the block store

DeviceCache::DeviceCache(const Geometry& g, int format) : meta_(g), format_(format) {
    const Geometry& geo = meta_.geometry();
    if (format != kF32 && format != kQ8) throw std::invalid_argument("unknown KV format");
    const size_t kvw = geo.kv_width();
    if (format == kQ8 && geo.head_dim % 32) throw std::invalid_argument("Q8_0 KV needs head_dim divisible by 32");
    if (geo.max_blocks > static_cast<size_t>(std::numeric_limits<int32_t>::max()) ||
        kvw > static_cast<size_t>(std::numeric_limits<int32_t>::max() / 16) ||
        geo.layers > 65535 / 2 || geo.tokens_per_block > (1u << 20))
        throw std::invalid_argument("KV geometry outside the device kernels' index range");
    lay_.format = format;
    lay_.layers = static_cast<int>(geo.layers);
    lay_.kv_heads = static_cast<int>(geo.kv_heads);
    lay_.head_dim = static_cast<int>(geo.head_dim);
    lay_.tpb = static_cast<int>(geo.tokens_per_block);
    lay_.kv_width = static_cast<int>(kvw);
    if (format == kF32) {
        lay_.section = geo.tokens_per_block * kvw * sizeof(float);
        lay_.stride = round_up(geo.elements_per_block() * sizeof(float), 256);
    } else {
        lay_.head_bytes =
            round_up(geo.tokens_per_block * geo.head_dim + geo.tokens_per_block * (geo.head_dim / 32) * 2, 16);
        lay_.section = geo.kv_heads * lay_.head_bytes;
        lay_.stride = round_up(2 * geo.layers * lay_.section, 256);
    }
    if (lay_.stride > kMax / geo.max_blocks) throw std::invalid_argument("KV capacity overflow");
    int dev = 0;
    TVARA_HIP(hipGetDevice(&dev));
    TVARA_HIP(hipDeviceGetAttribute(&cus_, hipDeviceAttributeMultiprocessorCount, dev));
    if (hipDeviceGetAttribute(&xcds_, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || xcds_ < 1) xcds_ = 1;
    TVARA_HIP(hipMalloc(&pool_, lay_.stride * geo.max_blocks));
    TVARA_HIP(hipMalloc(&err_, sizeof(int)));
    TVARA_HIP(hipMemset(err_, 0, sizeof(int)));
}

DeviceCache::~DeviceCache() {
    (void)hipStreamSynchronize(stream_);
    for (hipEvent_t e : ordered_)
        if (e) (void)hipEventDestroy(e);
    if (pool_) (void)hipFree(pool_);
    if (err_) (void)hipFree(err_);
}

size_t DeviceCache::canonical_block_bytes() const {
    const size_t elements = geometry().elements_per_block();
    return format_ == kF32 ? elements * sizeof(float) : elements / 32 * 34;
}

void DeviceCache::synchronize() { TVARA_HIP(hipStreamSynchronize(stream_)); }

// BlockPool::allocate's zero-fill (kv.hpp:48), batched over every block handed
// out since the last device access, kInlineOps blocks a launch
void DeviceCache::flush() {
    const std::vector<int64_t> ids = meta_.take_pending_zero_fills();
    for (size_t at = 0; at < ids.size(); at += kInlineOps) {
        const size_t n = std::min<size_t>(kInlineOps, ids.size() - at);
        InlineInitOps ops;
        for (size_t i = 0; i < n; ++i) ops.op[i] = make_int2(static_cast<int>(ids[at + i]), -1);
        launch_block_init_inline(pool_, lay_.stride, ops, static_cast<int>(n), stream_);
    }
}

void DeviceCache::enter(hipStream_t s) {
    if (s == stream_) return;
    if (!ordered_[0]) TVARA_HIP(hipEventCreateWithFlags(&ordered_[0], hipEventDisableTiming));
    TVARA_HIP(hipEventRecord(ordered_[0], stream_));
    TVARA_HIP(hipStreamWaitEvent(s, ordered_[0], 0));
}

void DeviceCache::leave(hipStream_t s) {
    if (s == stream_) return;
    if (!ordered_[1]) TVARA_HIP(hipEventCreateWithFlags(&ordered_[1], hipEventDisableTiming));
    TVARA_HIP(hipEventRecord(ordered_[1], s));
    TVARA_HIP(hipStreamWaitEvent(stream_, ordered_[1], 0));
}

void DeviceCache::block_read(Handle h, void* out, size_t bytes) {
    meta_.check_live(h);
    if (!out || bytes != canonical_block_bytes()) throw std::invalid_argument("block buffer size mismatch");
    flush();
    if (format_ == kF32) {
        TVARA_HIP(hipMemcpyAsync(out, pool_ + h.id * lay_.stride, bytes, hipMemcpyDeviceToHost, stream_));
    } else {
        auto* d = static_cast<uint8_t*>(scratch_[kMiscOut].ensure(bytes));
        launch_q8_to_canonical(pool_, lay_, static_cast<int64_t>(h.id), d, stream_);
        TVARA_HIP(hipMemcpyAsync(out, d, bytes, hipMemcpyDeviceToHost, stream_));
    }
    synchronize();
}

void DeviceCache::block_write(Handle h, size_t offset, const void* data, size_t bytes) {
    meta_.check_live(h);
    const size_t total = canonical_block_bytes();
    if (!data || offset > total || bytes > total - offset) throw std::invalid_argument("write outside block");
    flush();
    if (format_ == kF32) {
        TVARA_HIP(hipMemcpyAsync(pool_ + h.id * lay_.stride + offset, data, bytes, hipMemcpyHostToDevice, stream_));
        synchronize();
        return;
    }
    std::vector<uint8_t> image(total);
    block_read(h, image.data(), total);
    std::memcpy(image.data() + offset, data, bytes);
    auto* d = upload(*this, kMisc, image.data(), image.size());
    launch_canonical_to_q8(pool_, lay_, static_cast<int64_t>(h.id), d, stream_);
    synchronize();
}

void DeviceCache::checksums(const Handle* handles, size_t n, uint64_t* out) {
    std::vector<int64_t> ids(n);
    for (size_t i = 0; i < n; ++i) {
        meta_.check_live(handles[i]);
        ids[i] = static_cast<int64_t>(handles[i].id);
    }
    if (!n) return;
    flush();
    auto* d = upload(*this, kMisc, ids.data(), n);
    auto* o = static_cast<uint64_t*>(scratch_[kMiscOut].ensure(n * sizeof(uint64_t)));
    launch_checksums(pool_, lay_, d, static_cast<int>(n), o, stream_);
    TVARA_HIP(hipMemcpyAsync(out, o, n * sizeof(uint64_t), hipMemcpyDeviceToHost, stream_));
    synchronize();
}

// Appends in order (KvLedger::plan_appends follows PagedCache::append,
// kv.hpp:91-108), then runs the block work of all applied appends as two
// launches: zero-fills and copy-on-write copies first, then the row writes.
size_t DeviceCache::append_batch(const uint64_t* seqs, size_t n, const float* keys, const float* values, bool device,
                                 size_t* applied_out) {
    if (n && (!seqs || !keys || !values)) throw std::invalid_argument("invalid paged KV append dimensions");
    AppendWork w = meta_.plan_appends(seqs, n);
    const size_t applied = w.applied;
    const Geometry& g = meta_.geometry();
    if (applied) {
        run_block_init(w.init);
        const float* k = keys;
        const float* v = values;
        if (!device) {
            const size_t width = g.layers * g.kv_width();
            k = upload(*this, kKeys, keys, applied * width);
            v = upload(*this, kValues, values, applied * width);
        }
        if (format_ == kF32 && w.rows.size() <= static_cast<size_t>(kInlineOps) && g.tokens_per_block <= 32768 &&
            applied <= 65536 && g.kv_width() % 4 == 0 &&
            lay_.stride / 16 <= static_cast<size_t>(std::numeric_limits<int32_t>::max())) {
            InlineRowOps ops;
            for (size_t i = 0; i < w.rows.size(); ++i)
                ops.op[i] = make_int2(w.rows[i].block, (w.rows[i].slot << 16) | w.rows[i].src_row);
            launch_append_rows_inline(pool_, lay_, ops, static_cast<int>(w.rows.size()), k, v, stream_);
        } else {
            auto* d = upload(*this, kRowOps, w.rows.data(), w.rows.size());
            launch_append_rows(pool_, lay_, d, static_cast<int>(w.rows.size()), k, v, stream_);
        }
    }
    if (applied_out) *applied_out = applied;
    if (w.failure) std::rethrow_exception(w.failure);
    return applied;
}

size_t DeviceCache::append_tokens(uint64_t seq, const float* keys, const float* values, size_t count, bool device) {
    std::vector<uint64_t> seqs(count, seq);
    return append_batch(seqs.data(), count, keys, values, device);
}

void DeviceCache::run_block_init(const std::vector<BlockInitOp>& init) {
    flush();
    // small batches pass their ops in the kernel arguments (no upload copy)
    if (!init.empty() && init.size() <= static_cast<size_t>(kInlineOps)) {
        InlineInitOps ops;
        for (size_t i = 0; i < init.size(); ++i)
            ops.op[i] = make_int2(static_cast<int>(init[i].dst), static_cast<int>(init[i].src));
        launch_block_init_inline(pool_, lay_.stride, ops, static_cast<int>(init.size()), stream_);
    } else if (!init.empty()) {
        auto* d = upload(*this, kInitOps, init.data(), init.size());
        launch_block_init(pool_, lay_.stride, d, static_cast<int>(init.size()), stream_);
    }
}

// The ledger half of `count` appends to one sequence (PagedCache::append,
// kv.hpp:91-108, per token), with the rows left to write_layer_rows.
const RowOp* DeviceCache::reserve_tokens(uint64_t seq, size_t count) {
    if (format_ != kF32) throw std::invalid_argument("layer-wise appends need f32 blocks");
    if (!count) return nullptr;
    std::vector<uint64_t> seqs(count, seq);
    AppendWork w = meta_.plan_appends(seqs.data(), count);
    if (w.applied) run_block_init(w.init);
    if (w.failure) std::rethrow_exception(w.failure);
    return upload(*this, kRowOps, w.rows.data(), w.rows.size());
}

void DeviceCache::write_layer_rows(const RowOp* ops, size_t n, int layer, const float* keys, const float* values) {
    if (!n) return;
    if (format_ != kF32 || !ops || !keys || !values || layer < 0 || layer >= lay_.layers ||
        n > static_cast<size_t>(std::numeric_limits<int>::max()))
        throw std::invalid_argument("invalid paged KV append dimensions");
    launch_write_layer_rows(pool_, lay_, ops, static_cast<int>(n), layer, keys, values, stream_);
}

// PagedCache::read (kv.hpp:110-113)
void DeviceCache::read(uint64_t id, size_t layer, size_t position, bool value, float* out) {
    const Handle h = physical_block(id, position);
    if (layer >= geometry().layers) throw std::invalid_argument("KV position outside block");
    meta_.check_live(h);
    flush();
    const int2 row = make_int2(static_cast<int>(h.id), static_cast<int>(position % geometry().tokens_per_block));
    auto* d = upload(*this, kMisc, &row, 1);
    const size_t w = geometry().kv_width();
    auto* o = static_cast<float*>(scratch_[kMiscOut].ensure(w * sizeof(float)));
    launch_gather_rows(pool_, lay_, d, 1, static_cast<int>(layer), value ? 1 : 0, o, stream_);
    TVARA_HIP(hipMemcpyAsync(out, o, w * sizeof(float), hipMemcpyDeviceToHost, stream_));
    synchronize();
}

// PagedCache::read_all (kv.hpp:114-119)
void DeviceCache::read_all(uint64_t id, size_t layer, bool value, float* out, size_t capacity) {
    const Table& t = sequence(id);
    const Geometry& g = geometry();
    if (layer >= g.layers) throw std::invalid_argument("invalid KV layer");
    const size_t w = g.kv_width();
    if (t.length * w > capacity) throw std::invalid_argument("read_all buffer too small");
    if (!t.length) return;
    std::vector<int2> rows(t.length);
    for (size_t p = 0; p < t.length; ++p) {
        const Handle h = t.blocks[p / g.tokens_per_block];
        meta_.check_live(h);
        rows[p] = make_int2(static_cast<int>(h.id), static_cast<int>(p % g.tokens_per_block));
    }
    flush();
    auto* d = upload(*this, kMisc, rows.data(), rows.size());
    auto* o = static_cast<float*>(scratch_[kMiscOut].ensure(t.length * w * sizeof(float)));
    launch_gather_rows(pool_, lay_, d, static_cast<int>(t.length), static_cast<int>(layer), value ? 1 : 0, o, stream_);
    TVARA_HIP(hipMemcpyAsync(out, o, t.length * w * sizeof(float), hipMemcpyDeviceToHost, stream_));
    synchronize();
}

// ------------------------------------------------------------------ plans

void check_attention_config(const DeviceCache& c, size_t heads, size_t context) {
    const Geometry& g = c.geometry();
    if (!heads || !context || heads % g.kv_heads || g.head_dim % 2 || heads > 65535)
        throw std::invalid_argument("invalid native model configuration");
}

void attention_rows(const DeviceCache& c, const uint64_t* seqs, size_t count, size_t context, bool tail,
                    const size_t* visible, std::vector<uint64_t>& seq_of_row, std::vector<size_t>& cached,
                    std::vector<uint8_t>& tail_rows) {
    for (size_t i = 0; i < count; ++i) {
        const size_t length = c.sequence(seqs[i]).length;
        if (length > context || (tail && length == context)) throw std::invalid_argument("invalid fused attention shape");
        const size_t total = length + (tail ? 1 : 0);
        const size_t vis = visible ? std::min(visible[i], total) : total;
        if (!vis) throw std::invalid_argument("empty fused attention");
        if (length > static_cast<size_t>(std::numeric_limits<int32_t>::max()))
            throw std::invalid_argument("sequence too long for the device kernels");
        seq_of_row.push_back(seqs[i]);
        cached.push_back(std::min(vis, length));
        tail_rows.push_back(vis > length ? 1 : 0);
    }
}

void AttnPlan::compute(DeviceCache* c, const std::vector<uint64_t>& seq_of_row, const std::vector<size_t>& cached,
                     const std::vector<uint8_t>& tail_rows, int h, size_t split_override) {
    cache = c;
    epoch = c->epoch();
    heads = h;
    with_tail = false;
    for (uint8_t t : tail_rows) with_tail |= t != 0;
    const Geometry& g = c->geometry();
    group = static_cast<int>(heads / g.kv_heads);
    // slices of at most eight query heads (head_dim 256 and f32 blocks at 96:
    // four, at 80: three, what the fast kernels take there)
    kv_share = 1;
    int max_slice = 8;
    if ((c->format() == kF32 && g.head_dim == 96) || g.head_dim == 256) max_slice = 4;
    if (c->format() == kF32 && g.head_dim == 80) max_slice = 3;
    if (group > max_slice) {
        int slice = max_slice;
        while (group % slice) --slice;
        kv_share = group / slice;
    }
    // the kernels' view: kv_share virtual KV heads per KV head
    const int vkv = static_cast<int>(g.kv_heads) * kv_share, vgroup = group / kv_share;
    rows = static_cast<int>(seq_of_row.size());
    std::map<uint64_t, int32_t> offset;
    std::vector<int32_t>& tab = h_tables;
    tab.clear();
    for (size_t r = 0; r < seq_of_row.size(); ++r) {
        if (offset.count(seq_of_row[r])) continue;
        offset[seq_of_row[r]] = static_cast<int32_t>(tab.size());
        for (const Handle& b : c->sequence(seq_of_row[r]).blocks) tab.push_back(static_cast<int32_t>(b.id));
    }
    if (tab.size() > static_cast<size_t>(std::numeric_limits<int32_t>::max()))
        throw std::invalid_argument("attention batch too large");
    // The decode kernels that stream blocks directly (16-token blocks, and f32
    // blocks of any power of two from 16 to 1,024 tokens) take work items
    // that start on a block, with one id per block in the item's list.
    const int tpb = static_cast<int>(g.tokens_per_block);
    const bool listed = tpb == 16 || (c->format() == kF32 && decode_f32_blocks(tpb));
    const size_t align = listed ? static_cast<size_t>(tpb) : 16;
    // Split length: the shortest (a multiple of 16 from 64 to 1,024 tokens)
    // whose launch fits the workgroup budget of the decode kernel that will
    // run (decode_budget_per_cu, measured on MI355X: the 64-sequence
    // Llama-3.2-1B batch and the 16 x 32,768 Llama-3-8B Q8_0 batch).
    size_t split = split_override;
    if (!split) {
        if (const char* env = std::getenv("TVARA_SPLIT_TOKENS")) split = std::strtoull(env, nullptr, 10);
    }
    // A launch of few (row, KV head) pairs gives every row wave splits: the
    // waves of ws_chunks workgroups per (row, KV head), merged in LDS and
    // across chunks by the merge kernel (wave_split_shape).
    size_t max_n = 0;
    for (size_t n : cached) max_n = std::max(max_n, n);
    const WaveSplitShape ws =
        split ? WaveSplitShape{}
              : wave_split_shape(rows, vkv, vgroup, c->format(), static_cast<int>(g.head_dim),
                                 static_cast<int>(g.tokens_per_block), max_n, c->compute_units());
    wave_splits = ws.waves;
    ws_chunks = ws.waves ? ws.chunks : 1;
    if (wave_splits) split = ws.tokens;
    // The row-major f32 kernel (decode_rows_shape) runs one workgroup per
    // item.  Its split starts from the shortest whose items fit one workgroup
    // per CU and grows in steps of 64 tokens while at least 80% of the CUs
    // still get an item: fewer, longer items stream with less per-item
    // overhead while HBM stays saturated (MI355X, the 64-sequence
    // Llama-3.2-1B batch: 640-token splits, 253 items, 92.1 us; 768, 215
    // items, 90.5 us; 896, 188 items, 93.3 us; 64 x 2,048 tokens at 4 KV
    // heads: 512 and 640 (256 items) 42.6-42.8 us, 704 (192) 43.0 us).  It
    // takes the launch when that is more than kRowMajorMinWorkgroups
    // workgroups (smaller launches merge their splits in the kernel).
    row_major = false;
    auto items_at = [&](size_t sp) {
        size_t n = 0;
        for (size_t len : cached) n += std::max<size_t>(1, (len + sp - 1) / sp);
        return n;
    };
    if (!wave_splits && kv_share == 1 &&
        decode_rows_shape(static_cast<int>(g.kv_heads), group, c->format(), static_cast<int>(g.head_dim),
                          static_cast<int>(g.tokens_per_block))) {
        size_t sp = split;
        if (!sp) {
            const size_t budget = static_cast<size_t>(c->compute_units());
            size_t lo = 4, hi = kMaxSplitTokens / 16;
            while (lo < hi) {
                const size_t mid = (lo + hi) / 2;
                if (items_at(mid * 16) <= budget) hi = mid;
                else lo = mid + 1;
            }
            sp = lo * 16;
            const size_t floor_items = budget * 4 / 5;
            for (size_t wider = round_up(sp + 1, 64); wider <= kMaxSplitTokens; wider += 64) {
                if (items_at(wider) < floor_items) break;
                sp = wider;
            }
        }
        sp = std::min(round_up(std::max<size_t>(sp, 16), align), kMaxSplitTokens);
        if (items_at(sp) > kRowMajorMinWorkgroups) {
            row_major = true;
            split = sp;
        }
    }
    if (!split) {
        const int gd = static_cast<int>(g.head_dim);
        const size_t groups = static_cast<size_t>(decode_slots(vkv, vgroup, c->format(), gd)) /
                              static_cast<size_t>(decode_waves(vkv, vgroup, c->format(), gd));
        const size_t budget = static_cast<size_t>(c->compute_units()) *
                              decode_budget_per_cu(vgroup, c->format(), static_cast<int>(g.head_dim));
        auto workgroups = [&](size_t sp) {
            size_t n = 0;
            for (size_t len : cached) n += std::max<size_t>(1, (len + sp - 1) / sp);
            return n * groups;
        };
        size_t lo = 4, hi = kMaxSplitTokens / 16;  // in units of 16 tokens
        while (lo < hi) {
            const size_t mid = (lo + hi) / 2;
            if (workgroups(mid * 16) <= budget) hi = mid;
            else lo = mid + 1;
        }
        split = lo * 16;
    }
    // the decode kernels keep a split's block ids in one register per lane
    split = std::min(round_up(std::max<size_t>(split, 16), align), kMaxSplitTokens);
    split_tokens = static_cast<int>(split);
    std::vector<int4>& ent = h_entries;
    std::vector<int4>& work = h_work;
    std::vector<int2>& its = h_items;
    std::vector<int32_t>& work_ids = h_work_blocks;
    ent.assign(rows, int4{});
    work.clear();
    its.clear();
    work_ids.clear();
    inline_ok = rows <= kInlineRows;
    need_merge = false;
    kv_bytes = 0;
    const double bytes_per_element = c->format() == kF32 ? 4.0 : 34.0 / 32.0;
    for (int r = 0; r < rows; ++r) {
        const size_t n = cached[r];
        const int tail = tail_rows.empty() ? 0 : (tail_rows[r] ? 1 : 0);
        const int nsplit = wave_splits ? wave_splits * ws_chunks
                                       : static_cast<int>(std::max<size_t>(1, (n + split - 1) / split));
        const int first = static_cast<int>(its.size());
        const int32_t base = offset[seq_of_row[r]];
        ent[r] = make_int4(base, static_cast<int>(n), tail | (nsplit << 1), first);
        // wave splits merge a row's chunks (partials r * chunks ..), not its splits
        if (inline_ok) inline_rows.r[r] = wave_splits ? make_int2(r * ws_chunks, ws_chunks) : make_int2(first, nsplit);
        for (int s = 0; s < nsplit; ++s) {
            its.push_back(make_int2(r, s));
            const int t0 = static_cast<int>(std::min(n, s * split)), t1 = static_cast<int>(std::min(n, (s + 1) * split));
            work.push_back(make_int4(r, t0, t1, ((tail && s == nsplit - 1) ? 1 : 0) | (nsplit << 1)));
            const int nb = listed ? (t1 - t0 + tpb - 1) / tpb : 0;
            for (int j = 0; j < kMaxSplitBlocks; ++j) work_ids.push_back(j < nb ? tab[base + t0 / tpb + j] : 0);
        }
        need_merge |= wave_splits ? ws_chunks > 1 : nsplit > 1;
        kv_bytes += static_cast<size_t>(static_cast<double>(n + tail) * g.kv_width() * 2 * bytes_per_element);
    }
    items = static_cast<int>(its.size());
    ws_items.n = 0;
    if (wave_splits) {
        // item chunk * waves + w goes to slot chunk * kWsInlineWaves + w
        const int per = static_cast<int>((split + tpb - 1) / tpb);
        const int chunks = rows * ws_chunks;
        if (chunks * kWsInlineWaves <= kWsInlineItems && per <= kWsInlinePer && wave_splits <= kWsInlineWaves) {
            for (int ch = 0; ch < chunks; ++ch)
                for (int w = 0; w < wave_splits; ++w) {
                    const int i = ch * wave_splits + w, at = ch * kWsInlineWaves + w;
                    ws_items.item[at] = work[i];
                    for (int j = 0; j < kWsInlinePer; ++j)
                        ws_items.ids[at * kWsInlinePer + j] =
                            j < per ? work_ids[static_cast<size_t>(i) * kMaxSplitBlocks + j] : 0;
                }
            ws_items.n = items;
        }
    }
    order.n = 0;
    const bool one_group = row_major || decode_waves(vkv, vgroup, c->format(), static_cast<int>(g.head_dim)) == vkv;
    if (!wave_splits && one_group && c->format() == kF32 && items <= kOrderedItems && c->xcds() > 1 &&
        items >= c->xcds())
        xcd_balance(c->xcds());
}

// Workgroup s runs on XCD s mod xcds, and every XCD streams from HBM through
// its own L2: the launch order deals the items to the XCDs largest first,
// each to the XCD with the fewest tokens so far that still has a free slot
// (XCD x has ceil((items - x) / xcds) slots), so the XCDs stream about the
// same number of tokens (the 64-sequence Llama-3.2-1B plan: the heaviest XCD
// 7.6% above the mean in item order, 0.1% in this order).
void AttnPlan::xcd_balance(int xcds) {
    const int n = items;
    std::vector<int> tokens(n), idx(n);
    for (int i = 0; i < n; ++i) {
        tokens[i] = h_work[i].z - h_work[i].y;
        idx[i] = i;
    }
    std::stable_sort(idx.begin(), idx.end(), [&](int x, int y) { return tokens[x] > tokens[y]; });
    std::vector<long long> load(xcds, 0);
    std::vector<std::vector<int>> bins(xcds);
    for (int i : idx) {
        int best = -1;
        for (int x = 0; x < xcds; ++x) {
            const int cap = (n - x + xcds - 1) / xcds;
            if (static_cast<int>(bins[x].size()) < cap && (best < 0 || load[x] < load[best])) best = x;
        }
        bins[best].push_back(i);
        load[best] += tokens[i];
    }
    std::vector<uint8_t> seen(n, 0);
    for (int s = 0; s < n; ++s) {
        const int item = bins[s % xcds][s / xcds];
        if (seen[item]) throw std::logic_error("decode launch order is not a permutation");
        seen[item] = 1;
        order.item[s] = static_cast<uint16_t>(item);
    }
    order.n = n;
}

void AttnPlan::place() {
    size_t copied = 0;
    const size_t total = region_bytes(&copied);
    char* device = static_cast<char*>(region.ensure(total));
    char* host = static_cast<char*>(staging.acquire(copied));
    place_in(device, region.bytes, cache->stream(), host);
    staging.release(cache->stream());
}

namespace {
// packed layout of a plan in one region: every section starts on 256 bytes
struct RegionLayout {
    size_t tables, entries, items, work, work_blocks, row_done, err, copied, part_acc, part_ml, total;
};

RegionLayout region_layout(const AttnPlan& p) {
    const Geometry& g = p.cache->geometry();
    RegionLayout r{};
    size_t at = 0;
    auto take = [&](size_t bytes) {
        const size_t here = at;
        at = round_up(at + std::max<size_t>(bytes, 1), 256);
        return here;
    };
    r.tables = take(p.h_tables.size() * sizeof(int32_t));
    r.entries = take(p.h_entries.size() * sizeof(int4));
    r.items = take(p.h_items.size() * sizeof(int2));
    r.work = take(p.h_work.size() * sizeof(int4));
    r.work_blocks = take(p.h_work_blocks.size() * sizeof(int32_t));
    r.row_done = take(static_cast<size_t>(p.rows) * g.kv_heads * p.kv_share * sizeof(int));
    r.err = take(sizeof(int));
    r.copied = at;
    r.part_acc = take(p.need_merge ? static_cast<size_t>(p.items) * p.heads * g.head_dim * sizeof(float) : 0);
    r.part_ml = take(p.need_merge ? static_cast<size_t>(p.items) * p.heads * 2 * sizeof(float) : 0);
    r.total = at;
    return r;
}
}  // namespace

size_t AttnPlan::region_bytes(size_t* copied) const {
    const RegionLayout r = region_layout(*this);
    if (copied) *copied = r.copied;
    return r.total;
}

// One host-to-device copy carries the tables, the work list and zeros for the
// split counters and the error flag, which therefore start cleared whatever
// the region held before.
void AttnPlan::place_in(char* device, size_t capacity, hipStream_t s, char* host) {
    const RegionLayout r = region_layout(*this);
    if (r.total > capacity) throw std::invalid_argument("attention plan exceeds the no-allocation scratch");
    std::memset(host, 0, r.copied);
    auto put = [&](size_t at, const void* data, size_t bytes) {
        if (bytes) std::memcpy(host + at, data, bytes);
        return device + at;
    };
    dev.tables = reinterpret_cast<const int32_t*>(put(r.tables, h_tables.data(), h_tables.size() * sizeof(int32_t)));
    dev.entries = reinterpret_cast<const int4*>(put(r.entries, h_entries.data(), h_entries.size() * sizeof(int4)));
    dev.items = reinterpret_cast<const int2*>(put(r.items, h_items.data(), h_items.size() * sizeof(int2)));
    dev.work = reinterpret_cast<const int4*>(put(r.work, h_work.data(), h_work.size() * sizeof(int4)));
    dev.work_blocks = reinterpret_cast<const int32_t*>(
        put(r.work_blocks, h_work_blocks.data(), h_work_blocks.size() * sizeof(int32_t)));
    dev.row_done = need_merge ? reinterpret_cast<int*>(device + r.row_done) : nullptr;
    dev.err = reinterpret_cast<int*>(device + r.err);
    dev.part_acc = need_merge ? reinterpret_cast<float*>(device + r.part_acc) : nullptr;
    dev.part_ml = need_merge ? reinterpret_cast<float*>(device + r.part_ml) : nullptr;
    TVARA_HIP(hipMemcpyAsync(device, host, r.copied, hipMemcpyHostToDevice, s));
}

void AttnPlan::launch(int layer, const float* q, const float* tail_k, const float* tail_v, float* out, hipStream_t s) {
    if (cache->epoch() != epoch) throw std::invalid_argument("attention plan is stale: the cache changed");
    if (layer < 0 || static_cast<size_t>(layer) >= cache->geometry().layers)
        throw std::invalid_argument("invalid fused attention shape");
    if (with_tail && (!tail_k || !tail_v)) throw std::invalid_argument("plan expects tail K/V");
    if (!dev.tables) throw std::invalid_argument("attention plan is not placed");
    cache->flush();
    cache->enter(s);
    DecodeArgs a{};
    a.pool = cache->pool();
    a.lay = cache->layout();
    a.lay.kv_heads *= kv_share;
    a.kv_share = kv_share;
    a.layer = layer;
    a.heads = heads;
    a.group = group / kv_share;
    a.tables = dev.tables;
    a.entries = dev.entries;
    a.items = dev.items;
    a.split_tokens = split_tokens;
    a.work = dev.work;
    a.work_blocks = dev.work_blocks;
    a.q = q;
    a.tail_k = tail_k;
    a.tail_v = tail_v;
    a.out = out;
    a.part_acc = dev.part_acc;
    a.part_ml = dev.part_ml;
    a.row_done = need_merge ? dev.row_done : nullptr;
    a.wave_splits = wave_splits;
    a.ws_chunks = ws_chunks;
    a.row_major = row_major ? 1 : 0;
    a.qscale = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(cache->geometry().head_dim)));
    a.err = pinned_err ? static_cast<int*>(flag.ptr) : dev.err;
    launch_decode(a, items, rows, need_merge, inline_ok ? &inline_rows : nullptr, order.n ? &order : nullptr, s,
                  ws_items.n ? &ws_items : nullptr);
    cache->leave(s);
    last_stream = s;
}

void AttnPlan::use_pinned_error() {
    if (pinned_err) return;
    *static_cast<volatile int*>(flag.acquire(sizeof(int))) = 0;
    pinned_err = true;
}

void AttnPlan::queue_check() {
    if (pinned_err) return;  // the kernels write the pinned flag themselves
    auto* f = static_cast<int*>(flag.acquire(sizeof(int)));
    TVARA_HIP(hipMemcpyAsync(f, dev.err, sizeof(int), hipMemcpyDeviceToHost, last_stream));
}

void AttnPlan::finish_check() {
    auto* f = static_cast<volatile int*>(flag.ptr);
    if (*f) {
        if (pinned_err) {
            *f = 0;
        } else {
            TVARA_HIP(hipMemsetAsync(dev.err, 0, sizeof(int), last_stream));
            TVARA_HIP(hipStreamSynchronize(last_stream));
        }
        throw std::invalid_argument("invalid online attention input");
    }
}

void AttnPlan::check_into(int* host_flag) {
    TVARA_HIP(hipMemcpyAsync(host_flag, dev.err, sizeof(int), hipMemcpyDeviceToHost, last_stream));
    TVARA_HIP(hipStreamSynchronize(last_stream));
    if (*host_flag) {
        TVARA_HIP(hipMemsetAsync(dev.err, 0, sizeof(int), last_stream));
        TVARA_HIP(hipStreamSynchronize(last_stream));
        throw std::invalid_argument("invalid online attention input");
    }
}

// the flag is (or is copied to) pinned memory, so the call waits for the
// stream once
void AttnPlan::check() {
    queue_check();
    TVARA_HIP(hipStreamSynchronize(last_stream));
    finish_check();
}

void AttnPlan::check_after(hipEvent_t after) {
    if (!pinned_err) {
        check();
        return;
    }
    TVARA_HIP(hipEventSynchronize(after));
    finish_check();
}

void PrefillPlan::build(DeviceCache* c, const uint64_t* sequences, size_t n, size_t h, size_t context,
                        const size_t* start, const size_t* rows, int prec) {
    cache = c;
    const Geometry& g = c->geometry();
    if (!sequences || !start || !rows || !n) throw std::invalid_argument("invalid causal prompt chunk");
    if (prec != 0 && prec != 1 && prec != 2) throw std::invalid_argument("unknown attention precision");
    if (n > static_cast<size_t>(std::numeric_limits<int>::max())) throw std::invalid_argument("attention batch too large");
    heads = static_cast<int>(h);
    group = static_cast<int>(h / g.kv_heads);
    count = static_cast<int>(n);
    precision = prec;
    std::vector<uint64_t> seq_of_row;
    std::vector<size_t> cached;
    total_rows = 0;
    max_rows = 0;
    for (size_t i = 0; i < n; ++i) {
        const size_t length = c->sequence(sequences[i]).length;
        // fused_prompt_attention (attention.hpp:85-87)
        if (!rows[i] || start[i] >= length || rows[i] > length - start[i])
            throw std::invalid_argument("invalid causal prompt chunk");
        if (length > context) throw std::invalid_argument("invalid fused attention shape");
        if (prec == 0) {
            for (size_t j = 0; j < rows[i]; ++j) {
                seq_of_row.push_back(sequences[i]);
                cached.push_back(start[i] + j + 1);
            }
        }
        total_rows += rows[i];
        max_rows = std::max(max_rows, static_cast<int>(std::min<size_t>(rows[i], std::numeric_limits<int>::max())));
    }
    if (total_rows > static_cast<size_t>(std::numeric_limits<int>::max()))
        throw std::invalid_argument("attention batch too large");
    if (prec == 0) {
        rows_plan.build(c, seq_of_row, cached, {}, heads, 0);
        epoch = rows_plan.epoch;
        return;
    }
    // groups above eight: slices of at most eight query heads, each a virtual
    // KV head of the tile kernel
    kv_share = 1;
    if (group > 8) {
        int slice = 8;
        while (group % slice) --slice;
        kv_share = group / slice;
    }
    if (!prefill_bf16_supported(c->layout(), group / kv_share))
        throw std::invalid_argument(
            "bf16 prefill needs f32 or Q8_0 blocks of 16 to 1,024 tokens (a power of two, under 2 GiB) and head_dim "
            "64 or 128");
    std::vector<int32_t> tab;
    std::vector<int4> sq(n);
    size_t row0 = 0;
    for (size_t i = 0; i < n; ++i) {
        sq[i] = make_int4(static_cast<int>(tab.size()), static_cast<int>(start[i]), static_cast<int>(rows[i]),
                          static_cast<int>(row0));
        for (const Handle& b : c->sequence(sequences[i]).blocks) tab.push_back(static_cast<int32_t>(b.id));
        row0 += rows[i];
    }
    if (tab.size() > static_cast<size_t>(std::numeric_limits<int32_t>::max()))
        throw std::invalid_argument("attention batch too large");
    void* pt = tables.ensure(std::max<size_t>(tab.size() * sizeof(int32_t), 16));
    void* ps = seqs.ensure(sq.size() * sizeof(int4));
    void* pe = err.ensure(sizeof(int));
    TVARA_HIP(hipMemcpy(pt, tab.data(), tab.size() * sizeof(int32_t), hipMemcpyHostToDevice));
    TVARA_HIP(hipMemcpy(ps, sq.data(), sq.size() * sizeof(int4), hipMemcpyHostToDevice));
    TVARA_HIP(hipMemset(pe, 0, sizeof(int)));
    epoch = c->epoch();
}

void PrefillPlan::launch(int layer, const float* q, float* out, hipStream_t s) {
    if (layer < 0 || static_cast<size_t>(layer) >= cache->geometry().layers)
        throw std::invalid_argument("invalid fused attention shape");
    if (precision == 0) {
        rows_plan.launch(layer, q, nullptr, nullptr, out, s);
        return;
    }
    if (cache->epoch() != epoch) throw std::invalid_argument("attention plan is stale: the cache changed");
    cache->flush();
    cache->enter(s);
    PrefillArgs a{};
    a.pool = cache->pool();
    a.lay = cache->layout();
    a.lay.kv_heads *= kv_share;
    a.kv_share = kv_share;
    a.layer = layer;
    a.heads = heads;
    a.group = group / kv_share;
    a.tables = static_cast<const int32_t*>(tables.ptr);
    a.seqs = static_cast<const int4*>(seqs.ptr);
    a.q = q;
    a.out = out;
    a.qscale = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(cache->geometry().head_dim)));
    a.err = pinned_err ? static_cast<int*>(flag.ptr) : static_cast<int*>(err.ptr);
    launch_prefill_bf16(a, count, max_rows, s, precision == 2);
    cache->leave(s);
    last_stream = s;
}

void PrefillPlan::use_pinned_error() {
    if (precision == 0) {
        rows_plan.use_pinned_error();
        return;
    }
    if (pinned_err) return;
    *static_cast<volatile int*>(flag.acquire(sizeof(int))) = 0;
    pinned_err = true;
}

void PrefillPlan::check_after(hipEvent_t after) {
    if (precision == 0) {
        rows_plan.check_after(after);
        return;
    }
    if (!pinned_err) {
        check();
        return;
    }
    TVARA_HIP(hipEventSynchronize(after));
    auto* f = static_cast<volatile int*>(flag.ptr);
    if (*f) {
        *f = 0;
        throw std::invalid_argument("invalid online attention input");
    }
}

void PrefillPlan::check() {
    if (precision == 0) {
        rows_plan.check();
        return;
    }
    if (pinned_err) {
        TVARA_HIP(hipStreamSynchronize(last_stream));
        auto* f = static_cast<volatile int*>(flag.ptr);
        if (*f) {
            *f = 0;
            throw std::invalid_argument("invalid online attention input");
        }
        return;
    }
    int bad = 0;
    TVARA_HIP(hipMemcpyAsync(&bad, err.ptr, sizeof(int), hipMemcpyDeviceToHost, last_stream));
    TVARA_HIP(hipStreamSynchronize(last_stream));
    if (bad) {
        TVARA_HIP(hipMemsetAsync(err.ptr, 0, sizeof(int), last_stream));
        TVARA_HIP(hipStreamSynchronize(last_stream));
        throw std::invalid_argument("invalid online attention input");
    }
}

}  // namespace tvara_amd
