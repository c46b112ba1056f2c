// Host bookkeeping of the paged KV cache (see kv_ledger.hpp).  The rules are
// the reference's (core/include/tvara/kv.hpp): a LIFO free list that hands out
// 0, 1, 2, ... from a fresh pool, generation-tagged handles, zero-on-allocate,
// copy-on-write of a shared partial tail, truncation that keeps stale slots,
// and CacheExhausted leaving an append unapplied.
#include "kv_ledger.hpp"

#include <algorithm>
#include <limits>

namespace tvara_amd {

namespace {
constexpr size_t kMax = std::numeric_limits<size_t>::max();

size_t blocks_for(size_t tokens, size_t tpb) { return tokens / tpb + (tokens % tpb ? 1 : 0); }
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

// ------------------------------------------------------- the sequence map

Table* SequenceMap::find(uint64_t id) const {
    const size_t mask = keys_.size() - 1;
    for (size_t i = home(id);; i = (i + 1) & mask) {
        if (keys_[i] == id) return vals_[i].get();
        if (keys_[i] == kEmpty) return nullptr;
    }
}

Table& SequenceMap::insert(uint64_t id, Table&& t) {
    if (id == kEmpty || id == kErased) throw std::invalid_argument("invalid KV sequence id");
    if (2 * (used_ + 1) > keys_.size()) rehash(4 * (size_ + 1) > keys_.size() ? 2 * keys_.size() : keys_.size());
    auto table = std::make_unique<Table>(std::move(t));
    const size_t mask = keys_.size() - 1;
    size_t i = home(id);
    while (keys_[i] != kEmpty && keys_[i] != kErased) i = (i + 1) & mask;
    if (keys_[i] == kEmpty) ++used_;
    keys_[i] = id;
    vals_[i] = std::move(table);
    ++size_;
    return *vals_[i];
}

bool SequenceMap::erase(uint64_t id) {
    const size_t mask = keys_.size() - 1;
    for (size_t i = home(id);; i = (i + 1) & mask) {
        if (keys_[i] == kEmpty) return false;
        if (keys_[i] == id) {
            keys_[i] = kErased;
            vals_[i].reset();
            --size_;
            return true;
        }
    }
}

// capacity: a power of two of at least 2 * (size_ + 1) slots
void SequenceMap::rehash(size_t capacity) {
    std::vector<uint64_t> keys(capacity, kEmpty);
    std::vector<std::unique_ptr<Table>> vals(capacity);
    int shift = 64;
    for (size_t c = capacity; c > 1; c >>= 1) --shift;
    const size_t mask = capacity - 1;
    for (size_t j = 0; j < keys_.size(); ++j) {
        if (keys_[j] == kEmpty || keys_[j] == kErased) continue;
        size_t i = static_cast<size_t>((keys_[j] * 0x9E3779B97F4A7C15ull) >> shift);
        while (keys[i] != kEmpty) i = (i + 1) & mask;
        keys[i] = keys_[j];
        vals[i] = std::move(vals_[j]);
    }
    keys_.swap(keys);
    vals_.swap(vals);
    shift_ = shift;
    used_ = size_;
}

// -------------------------------------------------------------- the pool

KvLedger::KvLedger(const Geometry& g) : g_(g) {
    g_.validate();
    if ((g_.tokens_per_block & (g_.tokens_per_block - 1)) == 0) slot_mask_ = g_.tokens_per_block - 1;
    max_tokens_ = g_.max_blocks * g_.tokens_per_block;
    refs_.assign(g_.max_blocks, 0);
    gens_.assign(g_.max_blocks, 0);
    zero_pending_.assign(g_.max_blocks, 0);
    free_.reserve(g_.max_blocks);
    for (size_t i = g_.max_blocks; i > 0; --i) free_.push_back(i - 1);  // kv.hpp:42
}

// BlockPool::validated (kv.hpp:68-72)
void KvLedger::check_live(Handle h) const {
    if (h.id >= g_.max_blocks || !refs_[h.id] || gens_[h.id] != h.generation)
        throw std::invalid_argument("stale or invalid KV handle");
}

// BlockPool::allocate (kv.hpp:44-50) without the zero-fill
Handle KvLedger::take_free() {
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

Handle KvLedger::allocate() {
    // room first, so that nothing can fail once the block is taken
    if (zero_list_.size() == zero_list_.capacity()) zero_list_.reserve(2 * zero_list_.size() + 16);
    Handle h = take_free();
    zero_pending_[h.id] = 1;
    zero_list_.push_back(h.id);
    return h;
}

std::vector<int64_t> KvLedger::take_pending_zero_fills() {
    std::vector<int64_t> ids;
    ids.reserve(zero_list_.size());
    for (size_t id : zero_list_)
        if (zero_pending_[id] && refs_[id]) {
            ids.push_back(static_cast<int64_t>(id));
            zero_pending_[id] = 0;
        }
    zero_list_.clear();
    return ids;
}

// BlockPool::retain (kv.hpp:56)
void KvLedger::retain(Handle h) {
    check_live(h);
    if (refs_[h.id] == kMax) throw std::runtime_error("KV reference overflow");
    ++refs_[h.id];
    ++epoch_;
}

// BlockPool::release (kv.hpp:57); the free list has room for every block
void KvLedger::release(Handle h) {
    check_live(h);
    if (--refs_[h.id] == 0) free_.push_back(h.id);
    ++epoch_;
}

// BlockPool::references (kv.hpp:58)
size_t KvLedger::references(Handle h) const {
    check_live(h);
    return refs_[h.id];
}

// BlockPool::references_by_id (kv.hpp:59): blocks_.at() throws out_of_range
size_t KvLedger::references_by_id(size_t id) const {
    if (id >= g_.max_blocks) throw std::out_of_range("KV block id out of range");
    return refs_[id];
}

// BlockPool::audit (kv.hpp:61-64)
void KvLedger::pool_audit() const {
    std::vector<bool> seen(g_.max_blocks);
    for (size_t id : free_) {
        if (id >= g_.max_blocks || seen[id] || refs_[id]) throw std::logic_error("KV free-list invariant");
        seen[id] = true;
    }
    for (size_t i = 0; i < g_.max_blocks; ++i)
        if (seen[i] != (refs_[i] == 0)) throw std::logic_error("KV allocation invariant");
}

void KvLedger::pool_state(size_t* refs, uint64_t* generations, size_t* free_pop_order, size_t* free_count) const {
    if (refs)
        for (size_t i = 0; i < refs_.size(); ++i) refs[i] = refs_[i];
    if (generations)
        for (size_t i = 0; i < gens_.size(); ++i) generations[i] = gens_[i];
    if (free_pop_order)
        for (size_t i = 0; i < free_.size(); ++i) free_pop_order[i] = free_[free_.size() - 1 - i];
    if (free_count) *free_count = free_.size();
}

// ------------------------------------------------------------ the tables

// PagedCache::create_sequence (kv.hpp:81)
uint64_t KvLedger::create_sequence() {
    if (next_ == std::numeric_limits<uint64_t>::max()) throw std::runtime_error("sequence ID exhausted");
    sequences_.insert(next_ + 1, Table{});
    ++next_;
    ++epoch_;
    return next_;
}

// PagedCache::sequence (kv.hpp:82-84)
const Table& KvLedger::sequence(uint64_t id) const {
    const Table* t = sequences_.find(id);
    if (!t) throw std::invalid_argument("unknown KV sequence");
    return *t;
}

Table& KvLedger::mutable_sequence(uint64_t id) { return const_cast<Table&>(sequence(id)); }

std::vector<uint64_t> KvLedger::sequence_ids() const {
    std::vector<uint64_t> ids;
    ids.reserve(sequences_.size());
    sequences_.for_each([&](uint64_t id, const Table&) { ids.push_back(id); });
    std::sort(ids.begin(), ids.end());
    return ids;
}

// PagedCache::physical_block (kv.hpp:85-87)
Handle KvLedger::physical_block(uint64_t id, size_t position) const {
    const Table& t = sequence(id);
    if (position >= t.length) throw std::invalid_argument("KV position beyond sequence");
    return t.blocks.at(position / g_.tokens_per_block);
}

// PagedCache::append (kv.hpp:91-108), once per listed sequence.  Within one
// batch no append writes a block another append copies from: a block is
// written in place only while its reference count is 1, and appends never
// raise a count.
AppendWork KvLedger::plan_appends(const uint64_t* seqs, size_t n) {
    AppendWork w;
    if (n && !seqs) throw std::invalid_argument("invalid paged KV append dimensions");
    w.rows.reserve(n);
    w.init.reserve(n);  // at most one block op per append
    for (; w.applied < n; ++w.applied) {
        try {
            Table& t = mutable_sequence(seqs[w.applied]);
            if (t.length >= max_tokens_) throw std::invalid_argument("invalid paged KV append dimensions");
            const size_t slot = slot_mask_ ? t.length & slot_mask_ : t.length % g_.tokens_per_block;
            if (slot == 0) {  // kv.hpp:96: a fresh, zeroed block
                if (t.blocks.size() == t.blocks.capacity()) t.blocks.reserve(2 * t.blocks.size() + 4);
                const Handle h = take_free();
                t.blocks.push_back(h);
                w.init.push_back({static_cast<int64_t>(h.id), -1});
            } else if (refs_[t.blocks.back().id] > 1) {  // kv.hpp:97-101: copy-on-write
                const Handle original = t.blocks.back();
                const Handle replacement = take_free();
                w.init.push_back({static_cast<int64_t>(replacement.id), static_cast<int64_t>(original.id)});
                t.blocks.back() = replacement;
                release(original);
            }
            w.rows.push_back({static_cast<int32_t>(t.blocks.back().id), static_cast<int32_t>(slot),
                              static_cast<int32_t>(w.applied), 0});
            ++t.length;
            ++epoch_;
        } catch (...) {
            w.failure = std::current_exception();
            break;
        }
    }
    return w;
}

// PagedCache::drop (kv.hpp:121)
void KvLedger::drop(uint64_t id) {
    Table& t = mutable_sequence(id);
    for (const Handle& h : t.blocks) release(h);
    sequences_.erase(id);
    ++epoch_;
}

// shared tail of fork (kv.hpp:123-129) and import_sequence (kv.hpp:149-159):
// every retain is undone if the new table cannot be stored
uint64_t KvLedger::publish(const Handle* blocks, size_t count, size_t length) {
    size_t retained = 0;
    try {
        for (; retained < count; ++retained) retain(blocks[retained]);
        if (next_ == std::numeric_limits<uint64_t>::max()) throw std::runtime_error("sequence ID exhausted");
        Table t;
        t.blocks.assign(blocks, blocks + count);
        t.length = length;
        sequences_.insert(next_ + 1, std::move(t));
        ++next_;
        ++epoch_;
        return next_;
    } catch (...) {
        for (size_t i = 0; i < retained; ++i) release(blocks[i]);
        throw;
    }
}

uint64_t KvLedger::fork(uint64_t id) {
    const Table copy = sequence(id);
    return publish(copy.blocks.data(), copy.blocks.size(), copy.length);
}

// PagedCache::truncate (kv.hpp:131-136): released pages only; stale slots stay
void KvLedger::truncate(uint64_t id, size_t length) {
    Table& t = mutable_sequence(id);
    if (length > t.length) throw std::invalid_argument("cannot extend KV by truncating");
    const size_t keep = blocks_for(length, g_.tokens_per_block);
    for (size_t i = keep; i < t.blocks.size(); ++i) release(t.blocks[i]);
    t.blocks.resize(keep);
    t.length = length;
    ++epoch_;
}

// PagedCache::audit (kv.hpp:138-146)
void KvLedger::audit(const size_t* external, size_t count) const {
    pool_audit();
    std::vector<size_t> counts(g_.max_blocks);
    if (count && count != counts.size()) throw std::invalid_argument("external reference counts mismatch");
    sequences_.for_each([&](uint64_t, const Table& t) {
        if (t.blocks.size() != blocks_for(t.length, g_.tokens_per_block))
            throw std::logic_error("KV block table length invariant");
        for (const Handle& h : t.blocks) {
            check_live(h);
            ++counts.at(h.id);
        }
    });
    for (size_t i = 0; i < counts.size(); ++i)
        if (counts[i] + (count ? external[i] : 0) != refs_[i]) throw std::logic_error("KV reference invariant");
}

// PagedCache::import_sequence (kv.hpp:149-159)
uint64_t KvLedger::import_sequence(const Handle* blocks, size_t count, size_t source_length, size_t length) {
    if (length > source_length) throw std::invalid_argument("prefix exceeds snapshot");
    const size_t need = blocks_for(length, g_.tokens_per_block);
    if (count < need) throw std::invalid_argument("invalid prefix snapshot");
    return publish(blocks, need, length);
}

}  // namespace tvara_amd
