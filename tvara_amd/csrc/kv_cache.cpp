// Host side of the device paged KV cache.  The allocator and block tables
// follow the reference's rules exactly (core/include/tvara/kv.hpp): LIFO free
// list handing out 0, 1, 2, ... from a fresh pool, generation-tagged handles,
// zero-on-allocate, copy-on-write of a shared partial tail, truncation that
// keeps stale slots, and CacheExhausted leaving an append unapplied.  Block
// bytes live in HBM and are only touched by the kernels in kv_kernels.hip.
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

// ------------------------------------------------------------- geometry

// CacheGeometry::kv_width (kv.hpp:14-17)
size_t Geometry::kv_width() const {
    if (!kv_heads || !head_dim || kv_heads > kMax / head_dim) throw std::invalid_argument("KV width overflow");
    return kv_heads * head_dim;
}

// CacheGeometry::elements_per_block (kv.hpp:18-23)
size_t Geometry::elements_per_block() const {
    size_t count = kv_width();
    for (size_t dim : {layers, tokens_per_block, size_t(2)}) {
        if (!dim || count > kMax / dim) throw std::invalid_argument("KV block overflow");
        count *= dim;
    }
    return count;
}

// CacheGeometry::validate (kv.hpp:24-28)
void Geometry::validate() const {
    const size_t elements = elements_per_block();
    if (!max_blocks || max_blocks > 1000000 || elements > kMax / sizeof(float) / max_blocks ||
        tokens_per_block > kMax / max_blocks)
        throw std::invalid_argument("KV capacity overflow");
}

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

// -------------------------------------------------------------- the pool

DeviceCache::DeviceCache(const Geometry& g, int format) : g_(g), format_(format) {
    g_.validate();
    if (format != kF32 && format != kQ8) throw std::invalid_argument("unknown KV format");
    const size_t kvw = g_.kv_width();
    if (format == kQ8 && g_.head_dim % 32) throw std::invalid_argument("Q8_0 KV needs head_dim divisible by 32");
    if (g_.max_blocks > static_cast<size_t>(std::numeric_limits<int32_t>::max()) ||
        kvw > static_cast<size_t>(std::numeric_limits<int32_t>::max() / 16) ||
        g_.layers > 65535 / 2 || g_.tokens_per_block > (1u << 20))
        throw std::invalid_argument("KV geometry outside the device kernels' index range");
    lay_.format = format;
    lay_.layers = static_cast<int>(g_.layers);
    lay_.kv_heads = static_cast<int>(g_.kv_heads);
    lay_.head_dim = static_cast<int>(g_.head_dim);
    lay_.tpb = static_cast<int>(g_.tokens_per_block);
    lay_.kv_width = static_cast<int>(kvw);
    if (format == kF32) {
        lay_.section = g_.tokens_per_block * kvw * sizeof(float);
        lay_.stride = round_up(g_.elements_per_block() * sizeof(float), 256);
    } else {
        lay_.head_bytes = round_up(g_.tokens_per_block * g_.head_dim + g_.tokens_per_block * (g_.head_dim / 32) * 2, 16);
        lay_.section = g_.kv_heads * lay_.head_bytes;
        lay_.stride = round_up(2 * g_.layers * lay_.section, 256);
    }
    if (lay_.stride > kMax / g_.max_blocks) throw std::invalid_argument("KV capacity overflow");
    int dev = 0;
    TVARA_HIP(hipGetDevice(&dev));
    TVARA_HIP(hipDeviceGetAttribute(&cus_, hipDeviceAttributeMultiprocessorCount, dev));
    TVARA_HIP(hipMalloc(&pool_, lay_.stride * g_.max_blocks));
    TVARA_HIP(hipMalloc(&err_, sizeof(int)));
    TVARA_HIP(hipMemset(err_, 0, sizeof(int)));
    refs_.assign(g_.max_blocks, 0);
    gens_.assign(g_.max_blocks, 0);
    zero_pending_.assign(g_.max_blocks, 0);
    free_.reserve(g_.max_blocks);
    for (size_t i = g_.max_blocks; i > 0; --i) free_.push_back(i - 1);  // kv.hpp:42
}

DeviceCache::~DeviceCache() {
    (void)hipStreamSynchronize(stream_);
    if (pool_) (void)hipFree(pool_);
    if (err_) (void)hipFree(err_);
}

size_t DeviceCache::canonical_block_bytes() const {
    const size_t elements = g_.elements_per_block();
    return format_ == kF32 ? elements * sizeof(float) : elements / 32 * 34;
}

void DeviceCache::synchronize() { TVARA_HIP(hipStreamSynchronize(stream_)); }

// BlockPool::validated (kv.hpp:68-72)
const Handle& DeviceCache::validated(Handle h) const {
    static thread_local Handle out;
    if (h.id >= g_.max_blocks || !refs_[h.id] || gens_[h.id] != h.generation)
        throw std::invalid_argument("stale or invalid KV handle");
    out = h;
    return out;
}

// BlockPool::allocate (kv.hpp:44-50) without the zero-fill
Handle DeviceCache::take_free() {
    if (free_.empty()) throw CacheExhausted();
    const size_t id = free_.back();
    if (gens_[id] == std::numeric_limits<uint64_t>::max()) throw std::runtime_error("KV generation exhausted");
    free_.pop_back();
    refs_[id] = 1;
    ++gens_[id];
    zero_pending_[id] = 0;
    ++epoch_;
    return {id, gens_[id]};
}

// BlockPool::allocate (kv.hpp:44-50).  The zero-fill is queued and runs, batched,
// before the next device access of the cache.
Handle DeviceCache::allocate() {
    Handle h = take_free();
    zero_pending_[h.id] = 1;
    zero_list_.push_back(h.id);
    return h;
}

void DeviceCache::flush() {
    if (zero_list_.empty()) return;
    std::vector<BlockInitOp> ops;
    for (size_t id : zero_list_)
        if (zero_pending_[id] && refs_[id]) {
            ops.push_back({static_cast<int64_t>(id), -1});
            zero_pending_[id] = 0;
        }
    zero_list_.clear();
    if (ops.empty()) return;
    auto* d = upload(*this, kInitOps, ops.data(), ops.size());
    launch_block_init(pool_, lay_.stride, d, static_cast<int>(ops.size()), stream_);
}

// BlockPool::retain (kv.hpp:56)
void DeviceCache::retain(Handle h) {
    validated(h);
    if (refs_[h.id] == kMax) throw std::runtime_error("KV reference overflow");
    ++refs_[h.id];
    ++epoch_;
}

// BlockPool::release (kv.hpp:57)
void DeviceCache::release(Handle h) {
    validated(h);
    if (--refs_[h.id] == 0) free_.push_back(h.id);
    ++epoch_;
}

// BlockPool::references (kv.hpp:58)
size_t DeviceCache::references(Handle h) const {
    validated(h);
    return refs_[h.id];
}

// BlockPool::references_by_id (kv.hpp:59): blocks_.at() throws out_of_range
size_t DeviceCache::references_by_id(size_t id) const {
    if (id >= g_.max_blocks) throw std::out_of_range("KV block id out of range");
    return refs_[id];
}

// BlockPool::audit (kv.hpp:61-64)
void DeviceCache::pool_audit() const {
    std::vector<bool> seen(g_.max_blocks);
    for (size_t id : free_) {
        if (id >= g_.max_blocks || seen[id] || refs_[id]) throw std::logic_error("KV free-list invariant");
        seen[id] = true;
    }
    for (size_t i = 0; i < g_.max_blocks; ++i)
        if (seen[i] != (refs_[i] == 0)) throw std::logic_error("KV allocation invariant");
}

void DeviceCache::pool_state(size_t* refs, uint64_t* generations, size_t* free_pop_order, size_t* free_count) const {
    if (refs) std::copy(refs_.begin(), refs_.end(), refs);
    if (generations) std::copy(gens_.begin(), gens_.end(), generations);
    if (free_pop_order) std::copy(free_.rbegin(), free_.rend(), free_pop_order);
    if (free_count) *free_count = free_.size();
}

void DeviceCache::block_read(Handle h, void* out, size_t bytes) {
    validated(h);
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
    validated(h);
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
    for (size_t i = 0; i < n; ++i) ids[i] = static_cast<int64_t>(validated(handles[i]).id);
    if (!n) return;
    flush();
    auto* d = upload(*this, kMisc, ids.data(), n);
    auto* o = static_cast<uint64_t*>(scratch_[kMiscOut].ensure(n * sizeof(uint64_t)));
    launch_checksums(pool_, lay_, d, static_cast<int>(n), o, stream_);
    TVARA_HIP(hipMemcpyAsync(out, o, n * sizeof(uint64_t), hipMemcpyDeviceToHost, stream_));
    synchronize();
}

// ------------------------------------------------------------ the tables

// PagedCache::create_sequence (kv.hpp:81)
uint64_t DeviceCache::create_sequence() {
    if (next_ == std::numeric_limits<uint64_t>::max()) throw std::runtime_error("sequence ID exhausted");
    const uint64_t id = ++next_;
    sequences_.emplace(id, Table{});
    ++epoch_;
    return id;
}

// PagedCache::sequence (kv.hpp:82-84)
const Table& DeviceCache::sequence(uint64_t id) const {
    auto it = sequences_.find(id);
    if (it == sequences_.end()) throw std::invalid_argument("unknown KV sequence");
    return it->second;
}

Table& DeviceCache::mutable_sequence(uint64_t id) { return const_cast<Table&>(sequence(id)); }

std::vector<uint64_t> DeviceCache::sequence_ids() const {
    std::vector<uint64_t> ids;
    ids.reserve(sequences_.size());
    for (auto& kv : sequences_) ids.push_back(kv.first);
    return ids;
}

// PagedCache::physical_block (kv.hpp:85-87)
Handle DeviceCache::physical_block(uint64_t id, size_t position) const {
    const auto& t = sequence(id);
    if (position >= t.length) throw std::invalid_argument("KV position beyond sequence");
    return t.blocks.at(position / g_.tokens_per_block);
}

// Appends in order, each following PagedCache::append (kv.hpp:91-108) on the
// host metadata, then runs the block work of all applied appends as two
// launches: zero-fills and copy-on-write copies first, then the row writes.
// Within one call no append writes a block another append copies from: a block
// is written in place only when its reference count is 1, and reference counts
// never grow during appends.
size_t DeviceCache::append_batch(const uint64_t* seqs, size_t n, const float* keys, const float* values, bool device,
                                 size_t* applied_out) {
    if (n && (!seqs || !keys || !values)) throw std::invalid_argument("invalid paged KV append dimensions");
    std::vector<BlockInitOp> init;
    std::vector<RowOp> rows;
    std::exception_ptr failure;
    size_t applied = 0;
    for (; applied < n; ++applied) {
        try {
            Table& t = mutable_sequence(seqs[applied]);
            if (t.length >= g_.max_blocks * g_.tokens_per_block)
                throw std::invalid_argument("invalid paged KV append dimensions");
            const size_t slot = t.length % g_.tokens_per_block;
            if (slot == 0) {  // kv.hpp:96
                Handle h = take_free();
                try {
                    t.blocks.push_back(h);
                } catch (...) {
                    release(h);
                    throw;
                }
                init.push_back({static_cast<int64_t>(h.id), -1});
            } else if (refs_[t.blocks.back().id] > 1) {  // kv.hpp:97-101
                const Handle original = t.blocks.back();
                const Handle replacement = take_free();
                init.push_back({static_cast<int64_t>(replacement.id), static_cast<int64_t>(original.id)});
                t.blocks.back() = replacement;
                release(original);
            }
            rows.push_back({static_cast<int32_t>(t.blocks.back().id), static_cast<int32_t>(slot),
                            static_cast<int32_t>(applied), 0});
            ++t.length;
            ++epoch_;
        } catch (...) {
            failure = std::current_exception();
            break;
        }
    }
    if (applied) {
        flush();
        // small batches pass their ops in the kernel arguments (no upload copy)
        if (!init.empty() && init.size() <= static_cast<size_t>(kInlineOps) &&
            g_.max_blocks <= static_cast<size_t>(std::numeric_limits<int32_t>::max())) {
            InlineInitOps ops;
            for (size_t i = 0; i < init.size(); ++i)
                ops.op[i] = make_int2(static_cast<int>(init[i].dst), static_cast<int>(init[i].src));
            launch_block_init_inline(pool_, lay_.stride, ops, static_cast<int>(init.size()), stream_);
        } else if (!init.empty()) {
            auto* d = upload(*this, kInitOps, init.data(), init.size());
            launch_block_init(pool_, lay_.stride, d, static_cast<int>(init.size()), stream_);
        }
        const float* k = keys;
        const float* v = values;
        if (!device) {
            const size_t w = g_.layers * g_.kv_width();
            k = upload(*this, kKeys, keys, applied * w);
            v = upload(*this, kValues, values, applied * w);
        }
        if (format_ == kF32 && rows.size() <= static_cast<size_t>(kInlineOps) && g_.tokens_per_block <= 32768 &&
            applied <= 65536 && g_.kv_width() % 4 == 0 &&
            lay_.stride / 16 <= static_cast<size_t>(std::numeric_limits<int32_t>::max())) {
            InlineRowOps ops;
            for (size_t i = 0; i < rows.size(); ++i)
                ops.op[i] = make_int2(rows[i].block, (rows[i].slot << 16) | rows[i].src_row);
            launch_append_rows_inline(pool_, lay_, ops, static_cast<int>(rows.size()), k, v, stream_);
        } else {
            auto* d = upload(*this, kRowOps, rows.data(), rows.size());
            launch_append_rows(pool_, lay_, d, static_cast<int>(rows.size()), k, v, stream_);
        }
    }
    if (applied_out) *applied_out = applied;
    if (failure) std::rethrow_exception(failure);
    return applied;
}

size_t DeviceCache::append_tokens(uint64_t seq, const float* keys, const float* values, size_t count, bool device) {
    std::vector<uint64_t> seqs(count, seq);
    return append_batch(seqs.data(), count, keys, values, device);
}

// PagedCache::read (kv.hpp:110-113)
void DeviceCache::read(uint64_t id, size_t layer, size_t position, bool value, float* out) {
    const Handle h = physical_block(id, position);
    if (layer >= g_.layers) throw std::invalid_argument("KV position outside block");
    validated(h);
    flush();
    const int2 row = make_int2(static_cast<int>(h.id), static_cast<int>(position % g_.tokens_per_block));
    auto* d = upload(*this, kMisc, &row, 1);
    const size_t w = g_.kv_width();
    auto* o = static_cast<float*>(scratch_[kMiscOut].ensure(w * sizeof(float)));
    launch_gather_rows(pool_, lay_, d, 1, static_cast<int>(layer), value ? 1 : 0, o, stream_);
    TVARA_HIP(hipMemcpyAsync(out, o, w * sizeof(float), hipMemcpyDeviceToHost, stream_));
    synchronize();
}

// PagedCache::read_all (kv.hpp:114-119)
void DeviceCache::read_all(uint64_t id, size_t layer, bool value, float* out, size_t capacity) {
    const Table& t = sequence(id);
    if (layer >= g_.layers) throw std::invalid_argument("invalid KV layer");
    const size_t w = g_.kv_width();
    if (t.length * w > capacity) throw std::invalid_argument("read_all buffer too small");
    if (!t.length) return;
    std::vector<int2> rows(t.length);
    for (size_t p = 0; p < t.length; ++p) {
        const Handle h = t.blocks[p / g_.tokens_per_block];
        validated(h);
        rows[p] = make_int2(static_cast<int>(h.id), static_cast<int>(p % g_.tokens_per_block));
    }
    flush();
    auto* d = upload(*this, kMisc, rows.data(), rows.size());
    auto* o = static_cast<float*>(scratch_[kMiscOut].ensure(t.length * w * sizeof(float)));
    launch_gather_rows(pool_, lay_, d, static_cast<int>(t.length), static_cast<int>(layer), value ? 1 : 0, o, stream_);
    TVARA_HIP(hipMemcpyAsync(out, o, t.length * w * sizeof(float), hipMemcpyDeviceToHost, stream_));
    synchronize();
}

// PagedCache::drop (kv.hpp:121)
void DeviceCache::drop(uint64_t id) {
    Table& t = mutable_sequence(id);
    for (const Handle& h : t.blocks) release(h);
    sequences_.erase(id);
    ++epoch_;
}

// shared tail of fork (kv.hpp:123-129) and import_sequence (kv.hpp:149-159)
uint64_t DeviceCache::publish(const Handle* blocks, size_t count, size_t length) {
    size_t retained = 0;
    try {
        for (; retained < count; ++retained) retain(blocks[retained]);
        if (next_ == std::numeric_limits<uint64_t>::max()) throw std::runtime_error("sequence ID exhausted");
        Table t;
        t.blocks.assign(blocks, blocks + count);
        t.length = length;
        const uint64_t id = next_ + 1;
        sequences_.emplace(id, std::move(t));
        next_ = id;
        ++epoch_;
        return id;
    } catch (...) {
        for (size_t i = 0; i < retained; ++i) release(blocks[i]);
        throw;
    }
}

uint64_t DeviceCache::fork(uint64_t id) {
    const Table copy = sequence(id);
    return publish(copy.blocks.data(), copy.blocks.size(), copy.length);
}

// PagedCache::truncate (kv.hpp:131-136): released pages only; stale slots stay
void DeviceCache::truncate(uint64_t id, size_t length) {
    Table& t = mutable_sequence(id);
    if (length > t.length) throw std::invalid_argument("cannot extend KV by truncating");
    const size_t tpb = g_.tokens_per_block;
    const size_t keep = length / tpb + (length % tpb ? 1 : 0);
    for (size_t i = keep; i < t.blocks.size(); ++i) release(t.blocks[i]);
    t.blocks.resize(keep);
    t.length = length;
    ++epoch_;
}

// PagedCache::audit (kv.hpp:138-146)
void DeviceCache::audit(const size_t* external, size_t count) const {
    pool_audit();
    std::vector<size_t> counts(g_.max_blocks);
    if (count && count != counts.size()) throw std::invalid_argument("external reference counts mismatch");
    const size_t tpb = g_.tokens_per_block;
    for (const auto& [id, t] : sequences_) {
        (void)id;
        const size_t expected = t.length / tpb + (t.length % tpb ? 1 : 0);
        if (t.blocks.size() != expected) throw std::logic_error("KV block table length invariant");
        for (const Handle& h : t.blocks) {
            validated(h);
            ++counts.at(h.id);
        }
    }
    for (size_t i = 0; i < counts.size(); ++i)
        if (counts[i] + (count ? external[i] : 0) != refs_[i]) throw std::logic_error("KV reference invariant");
}

// PagedCache::import_sequence (kv.hpp:149-159)
uint64_t DeviceCache::import_sequence(const Handle* blocks, size_t count, size_t source_length, size_t length) {
    if (length > source_length) throw std::invalid_argument("prefix exceeds snapshot");
    const size_t tpb = g_.tokens_per_block;
    const size_t need = length / tpb + (length % tpb ? 1 : 0);
    if (count < need) throw std::invalid_argument("invalid prefix snapshot");
    std::vector<Handle> prefix(blocks, blocks + need);
    return publish(prefix.data(), prefix.size(), length);
}

// ------------------------------------------------------------------ plans

void AttnPlan::build(DeviceCache* c, const std::vector<uint64_t>& seq_of_row, const std::vector<size_t>& cached,
                     const std::vector<uint8_t>& tail_rows, int h, size_t split_override) {
    cache = c;
    epoch = c->epoch();
    heads = h;
    with_tail = false;
    for (uint8_t t : tail_rows) with_tail |= t != 0;
    const Geometry& g = c->geometry();
    group = static_cast<int>(heads / g.kv_heads);
    rows = static_cast<int>(seq_of_row.size());
    std::map<uint64_t, int32_t> offset;
    std::vector<int32_t> tab;
    size_t total = 0;
    for (size_t r = 0; r < seq_of_row.size(); ++r) {
        total += cached[r];
        if (offset.count(seq_of_row[r])) continue;
        offset[seq_of_row[r]] = static_cast<int32_t>(tab.size());
        for (const Handle& b : c->sequence(seq_of_row[r]).blocks) tab.push_back(static_cast<int32_t>(b.id));
    }
    if (tab.size() > static_cast<size_t>(std::numeric_limits<int32_t>::max()))
        throw std::invalid_argument("attention batch too large");
    // Split length: the shortest (a multiple of 16 from 64 to 1,024 tokens)
    // whose launch fits the workgroup budget of the decode kernel that will
    // run (decode_budget_per_cu, measured on MI355X: the 64-sequence
    // Llama-3.2-1B batch and the 16 x 32,768 Llama-3-8B Q8_0 batch).
    size_t split = split_override;
    if (!split) {
        if (const char* env = std::getenv("TVARA_SPLIT_TOKENS")) split = std::strtoull(env, nullptr, 10);
    }
    // A launch too small to fill the GPU gives every row one split per wave of
    // a workgroup per (row, KV head), merged in LDS (wave_split_waves).
    size_t max_n = 0;
    for (size_t n : cached) max_n = std::max(max_n, n);
    wave_splits = split ? 0
                        : wave_split_waves(rows, static_cast<int>(g.kv_heads), group, c->format(),
                                           static_cast<int>(g.head_dim), static_cast<int>(g.tokens_per_block), max_n);
    if (wave_splits) split = round_up((max_n + wave_splits - 1) / wave_splits, 16);
    if (!split) {
        const int gw = static_cast<int>(g.kv_heads), gd = static_cast<int>(g.head_dim);
        const size_t groups = static_cast<size_t>(decode_slots(gw, group, c->format(), gd)) /
                              static_cast<size_t>(decode_waves(gw, group, c->format(), gd));
        const size_t budget = static_cast<size_t>(c->compute_units()) *
                              decode_budget_per_cu(group, c->format(), static_cast<int>(g.head_dim));
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
    split = std::min(round_up(std::max<size_t>(split, 16), 16), kMaxSplitTokens);
    split_tokens = static_cast<int>(split);
    std::vector<int4> ent(rows), work;
    std::vector<int2> its;
    std::vector<int32_t> work_ids;
    const bool blocks16 = g.tokens_per_block == 16;
    inline_ok = rows <= kInlineRows;
    need_merge = false;
    kv_bytes = 0;
    const double bytes_per_element = c->format() == kF32 ? 4.0 : 34.0 / 32.0;
    for (int r = 0; r < rows; ++r) {
        const size_t n = cached[r];
        const int tail = tail_rows.empty() ? 0 : (tail_rows[r] ? 1 : 0);
        const int nsplit = wave_splits ? wave_splits : static_cast<int>(std::max<size_t>(1, (n + split - 1) / split));
        const int first = static_cast<int>(its.size());
        const int32_t base = offset[seq_of_row[r]];
        ent[r] = make_int4(base, static_cast<int>(n), tail | (nsplit << 1), first);
        if (inline_ok) inline_rows.r[r] = make_int2(first, nsplit);
        for (int s = 0; s < nsplit; ++s) {
            its.push_back(make_int2(r, s));
            const int t0 = static_cast<int>(std::min(n, s * split)), t1 = static_cast<int>(std::min(n, (s + 1) * split));
            work.push_back(make_int4(r, t0, t1, ((tail && s == nsplit - 1) ? 1 : 0) | (nsplit << 1)));
            const int nb = blocks16 ? (t1 - t0 + 15) / 16 : 0;
            for (int j = 0; j < kMaxSplitBlocks; ++j) work_ids.push_back(j < nb ? tab[base + t0 / 16 + j] : 0);
        }
        need_merge |= nsplit > 1 && !wave_splits;
        kv_bytes += static_cast<size_t>(static_cast<double>(n + tail) * g.kv_width() * 2 * bytes_per_element);
    }
    items = static_cast<int>(its.size());
    auto put = [&](DeviceBuffer& b, const void* data, size_t bytes) {
        void* d = b.ensure(std::max<size_t>(bytes, 16));
        if (bytes) TVARA_HIP(hipMemcpy(d, data, bytes, hipMemcpyHostToDevice));
    };
    put(tables, tab.data(), tab.size() * sizeof(int32_t));
    put(entries, ent.data(), ent.size() * sizeof(int4));
    put(items_buf, its.data(), its.size() * sizeof(int2));
    put(work_buf, work.data(), work.size() * sizeof(int4));
    put(work_blocks, work_ids.data(), work_ids.size() * sizeof(int32_t));
    if (need_merge) {
        part_acc.ensure(static_cast<size_t>(items) * heads * g.head_dim * sizeof(float));
        part_ml.ensure(static_cast<size_t>(items) * heads * 2 * sizeof(float));
        // split counters of the in-kernel merge, one per (row, KV head) at
        // most; every launch that counts leaves them at zero again, so only a
        // new allocation is cleared
        const size_t bytes = static_cast<size_t>(rows) * g.kv_heads * sizeof(int);
        if (!row_done.ptr || row_done.bytes < bytes) {
            row_done.ensure(bytes);
            TVARA_HIP(hipMemset(row_done.ptr, 0, row_done.bytes));
        }
    }
    err.ensure(sizeof(int));
    TVARA_HIP(hipMemset(err.ptr, 0, sizeof(int)));
}

void AttnPlan::launch(int layer, const float* q, const float* tail_k, const float* tail_v, float* out, hipStream_t s) {
    if (cache->epoch() != epoch) throw std::invalid_argument("attention plan is stale: the cache changed");
    if (layer < 0 || static_cast<size_t>(layer) >= cache->geometry().layers)
        throw std::invalid_argument("invalid fused attention shape");
    if (with_tail && (!tail_k || !tail_v)) throw std::invalid_argument("plan expects tail K/V");
    cache->flush();
    DecodeArgs a{};
    a.pool = cache->pool();
    a.lay = cache->layout();
    a.layer = layer;
    a.heads = heads;
    a.group = group;
    a.tables = static_cast<const int32_t*>(tables.ptr);
    a.entries = static_cast<const int4*>(entries.ptr);
    a.items = static_cast<const int2*>(items_buf.ptr);
    a.split_tokens = split_tokens;
    a.work = static_cast<const int4*>(work_buf.ptr);
    a.work_blocks = static_cast<const int32_t*>(work_blocks.ptr);
    a.q = q;
    a.tail_k = tail_k;
    a.tail_v = tail_v;
    a.out = out;
    a.part_acc = static_cast<float*>(part_acc.ptr);
    a.part_ml = static_cast<float*>(part_ml.ptr);
    a.row_done = need_merge ? static_cast<int*>(row_done.ptr) : nullptr;
    a.wave_splits = wave_splits;
    a.qscale = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(cache->geometry().head_dim)));
    a.err = static_cast<int*>(err.ptr);
    launch_decode(a, items, rows, need_merge, inline_ok ? &inline_rows : nullptr, s);
}

void AttnPlan::check() {
    int flag = 0;
    TVARA_HIP(hipDeviceSynchronize());
    TVARA_HIP(hipMemcpy(&flag, err.ptr, sizeof(int), hipMemcpyDeviceToHost));
    if (flag) {
        TVARA_HIP(hipMemset(err.ptr, 0, sizeof(int)));
        throw std::invalid_argument("invalid online attention input");
    }
}

void PrefillPlan::build(DeviceCache* c, const uint64_t* sequences, size_t n, size_t h, size_t context,
                        const size_t* start, const size_t* rows, int prec) {
    cache = c;
    const Geometry& g = c->geometry();
    if (!sequences || !start || !rows || !n) throw std::invalid_argument("invalid causal prompt chunk");
    if (prec != 0 && prec != 1) throw std::invalid_argument("unknown attention precision");
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
    if (!prefill_bf16_supported(c->layout(), group))
        throw std::invalid_argument("bf16 prefill needs f32 blocks of 16 tokens, head_dim 64, GQA group 1/2/4/8");
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
    PrefillArgs a{};
    a.pool = cache->pool();
    a.lay = cache->layout();
    a.layer = layer;
    a.heads = heads;
    a.group = group;
    a.tables = static_cast<const int32_t*>(tables.ptr);
    a.seqs = static_cast<const int4*>(seqs.ptr);
    a.q = q;
    a.out = out;
    a.qscale = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(cache->geometry().head_dim)));
    a.err = static_cast<int*>(err.ptr);
    launch_prefill_bf16(a, count, max_rows, s);
}

void PrefillPlan::check() {
    if (precision == 0) {
        rows_plan.check();
        return;
    }
    int flag = 0;
    TVARA_HIP(hipDeviceSynchronize());
    TVARA_HIP(hipMemcpy(&flag, err.ptr, sizeof(int), hipMemcpyDeviceToHost));
    if (flag) {
        TVARA_HIP(hipMemset(err.ptr, 0, sizeof(int)));
        throw std::invalid_argument("invalid online attention input");
    }
}

}  // namespace tvara_amd
