// Exports that touch only a cache's bookkeeping, never its block bytes: the
// pool (BlockPool, kv.hpp:36-75), the tables (PagedCache, kv.hpp:78-165) and
// the prefix cache (RadixCache, radix.hpp:17-131).  No device code, so the
// sanitizer and failure-injection tests build this file unchanged.
#include <algorithm>
#include <cstdint>
#include <memory>
#include <vector>

#include "abi.hpp"
#include "radix.hpp"

using tvara_amd::Handle;
using tvara_amd::KvLedger;
using tvara_amd::PrefixTree;
using tvara_amd::abi::exported;
using tvara_amd::abi::guard;
using tvara_amd::abi::handle;
using tvara_amd::abi::ledger_of;

struct tvara_radix {
    std::unique_ptr<PrefixTree> tree;
};

namespace {
PrefixTree& tree(tvara_radix* r) {
    if (!r) throw std::invalid_argument("closed prefix cache");
    return *r->tree;
}

void check_tokens(const int32_t* tokens, size_t count) {
    if (!tokens && count) throw std::invalid_argument("invalid prefix tokens");
}
}  // namespace

extern "C" {

// ---------------------------------------------------------------- the pool

int tvara_kv_pool_allocate(tvara_kv_cache* cache, tvara_kv_handle* out) {
    return guard([&] {
        if (!out) throw std::invalid_argument("null handle output");
        *out = exported(ledger_of(cache).allocate());
    });
}

int tvara_kv_pool_retain(tvara_kv_cache* cache, tvara_kv_handle h) {
    return guard([&] { ledger_of(cache).retain(handle(h)); });
}

int tvara_kv_pool_release(tvara_kv_cache* cache, tvara_kv_handle h) {
    return guard([&] { ledger_of(cache).release(handle(h)); });
}

int tvara_kv_pool_references(tvara_kv_cache* cache, tvara_kv_handle h, size_t* out) {
    return guard([&] {
        const size_t n = ledger_of(cache).references(handle(h));
        if (out) *out = n;
    });
}

int tvara_kv_pool_references_by_id(tvara_kv_cache* cache, size_t id, size_t* out) {
    return guard([&] {
        const size_t n = ledger_of(cache).references_by_id(id);
        if (out) *out = n;
    });
}

size_t tvara_kv_pool_available(tvara_kv_cache* cache) {
    size_t n = 0;
    guard([&] { n = ledger_of(cache).available(); });
    return n;
}

int tvara_kv_pool_audit(tvara_kv_cache* cache) {
    return guard([&] { ledger_of(cache).pool_audit(); });
}

int tvara_kv_pool_state(tvara_kv_cache* cache, size_t* refs, uint64_t* generations, size_t* free_pop_order,
                        size_t* free_count) {
    return guard([&] { ledger_of(cache).pool_state(refs, generations, free_pop_order, free_count); });
}

// -------------------------------------------------------------- the tables

uint64_t tvara_kv_sequence_create(tvara_kv_cache* cache) {
    uint64_t id = 0;
    guard([&] { id = ledger_of(cache).create_sequence(); });
    return id;
}

int tvara_kv_sequence(tvara_kv_cache* cache, uint64_t sequence, size_t* length, tvara_kv_handle* blocks,
                      size_t capacity, size_t* count) {
    return guard([&] {
        const tvara_amd::Table& t = ledger_of(cache).sequence(sequence);
        if (blocks && capacity < t.blocks.size()) throw std::invalid_argument("block list buffer too small");
        if (length) *length = t.length;
        if (count) *count = t.blocks.size();
        if (blocks)
            for (size_t i = 0; i < t.blocks.size(); ++i) blocks[i] = exported(t.blocks[i]);
    });
}

int tvara_kv_sequence_ids(tvara_kv_cache* cache, uint64_t* ids, size_t capacity, size_t* count) {
    return guard([&] {
        const std::vector<uint64_t> v = ledger_of(cache).sequence_ids();
        if (ids && capacity < v.size()) throw std::invalid_argument("id buffer too small");
        if (count) *count = v.size();
        if (ids) std::copy(v.begin(), v.end(), ids);
    });
}

int tvara_kv_physical_block(tvara_kv_cache* cache, uint64_t sequence, size_t position, tvara_kv_handle* out) {
    return guard([&] {
        const Handle h = ledger_of(cache).physical_block(sequence, position);
        if (out) *out = exported(h);
    });
}

int tvara_kv_drop(tvara_kv_cache* cache, uint64_t sequence) {
    return guard([&] { ledger_of(cache).drop(sequence); });
}

uint64_t tvara_kv_fork(tvara_kv_cache* cache, uint64_t sequence) {
    uint64_t id = 0;
    guard([&] { id = ledger_of(cache).fork(sequence); });
    return id;
}

int tvara_kv_truncate(tvara_kv_cache* cache, uint64_t sequence, size_t length) {
    return guard([&] { ledger_of(cache).truncate(sequence, length); });
}

// PagedCache::truncate (kv.hpp:131-136) over a list, in order; a failure at
// entry k leaves entries 0..k-1 applied and reports k in *applied
int tvara_kv_truncate_batch(tvara_kv_cache* cache, const uint64_t* sequences, const size_t* lengths, size_t count,
                            size_t* applied) {
    size_t done = 0;
    const int rc = guard([&] {
        if (count && (!sequences || !lengths)) throw std::invalid_argument("null truncation batch");
        KvLedger& ledger = ledger_of(cache);
        for (; done < count; ++done) ledger.truncate(sequences[done], lengths[done]);
    });
    if (applied) *applied = done;
    return rc;
}

int tvara_kv_audit(tvara_kv_cache* cache, const size_t* external, size_t count) {
    return guard([&] { ledger_of(cache).audit(external, external ? count : 0); });
}

uint64_t tvara_kv_import_sequence(tvara_kv_cache* cache, const tvara_kv_handle* blocks, size_t block_count,
                                  size_t source_length, size_t length) {
    uint64_t id = 0;
    guard([&] {
        if (block_count && !blocks) throw std::invalid_argument("null snapshot blocks");
        std::vector<Handle> hs(block_count);
        for (size_t i = 0; i < block_count; ++i) hs[i] = handle(blocks[i]);
        id = ledger_of(cache).import_sequence(hs.data(), block_count, source_length, length);
    });
    return id;
}

// ------------------------------------------------------------ prefix cache

tvara_radix* tvara_radix_create(tvara_kv_cache* cache, const char* isolation) {
    tvara_radix* out = nullptr;
    guard([&] {
        auto r = std::make_unique<tvara_radix>();
        r->tree = std::make_unique<PrefixTree>(ledger_of(cache), isolation ? isolation : "");
        out = r.release();
    });
    return out;
}

void tvara_radix_destroy(tvara_radix* radix) { delete radix; }

int tvara_radix_insert(tvara_radix* radix, const int32_t* tokens, size_t count, uint64_t* node) {
    return guard([&] {
        check_tokens(tokens, count);
        const uint64_t id = tree(radix).insert(tokens, count);
        if (node) *node = id;
    });
}

int tvara_radix_lookup(tvara_radix* radix, const int32_t* tokens, size_t count, uint64_t* node, size_t* matched) {
    return guard([&] {
        check_tokens(tokens, count);
        const auto m = tree(radix).lookup(tokens, count);
        if (node) *node = m.first;
        if (matched) *matched = m.second;
    });
}

int tvara_radix_attach(tvara_radix* radix, uint64_t node, uint64_t sequence) {
    return guard([&] { tree(radix).attach(node, sequence); });
}

int tvara_radix_reuse(tvara_radix* radix, const int32_t* tokens, size_t count, int partial, uint64_t* sequence,
                      size_t* length) {
    return guard([&] {
        check_tokens(tokens, count);
        const auto r = tree(radix).reuse(tokens, count, partial != 0);
        if (sequence) *sequence = r.first;
        if (length) *length = r.second;
    });
}

int tvara_radix_pin(tvara_radix* radix, uint64_t node) { return guard([&] { tree(radix).pin(node); }); }
int tvara_radix_unpin(tvara_radix* radix, uint64_t node) { return guard([&] { tree(radix).unpin(node); }); }
int tvara_radix_touch(tvara_radix* radix, uint64_t node) { return guard([&] { tree(radix).touch(node); }); }

int tvara_radix_eviction_candidate(tvara_radix* radix, uint64_t* node) {
    return guard([&] {
        const auto c = tree(radix).eviction_candidate();
        if (node) *node = c.value_or(0);
    });
}

int tvara_radix_evict_one(tvara_radix* radix, int* evicted) {
    return guard([&] {
        const bool e = tree(radix).evict_one();
        if (evicted) *evicted = e ? 1 : 0;
    });
}

int tvara_radix_reset(tvara_radix* radix) { return guard([&] { tree(radix).reset(); }); }

int tvara_radix_size(tvara_radix* radix, size_t* size) {
    return guard([&] {
        const size_t n = tree(radix).size();
        if (size) *size = n;
    });
}

int tvara_radix_node(tvara_radix* radix, uint64_t id, uint64_t* parent, int32_t* edge, size_t edge_capacity,
                     size_t* edge_length, size_t* pins, uint64_t* accessed, size_t* kv_length, size_t* kv_blocks,
                     size_t* children) {
    return guard([&] {
        const PrefixTree::NodeInfo n = tree(radix).node(id);
        if (parent) *parent = n.parent;
        if (edge_length) *edge_length = n.edge_length;
        if (edge) std::copy(n.edge, n.edge + std::min(edge_capacity, n.edge_length), edge);
        if (pins) *pins = n.pins;
        if (accessed) *accessed = n.accessed;
        if (kv_length) *kv_length = n.kv ? n.kv->length : 0;
        if (kv_blocks) *kv_blocks = n.kv ? n.kv->blocks.size() : static_cast<size_t>(-1);
        if (children) *children = n.children;
    });
}

int tvara_radix_external_references(tvara_radix* radix, size_t* counts, size_t capacity) {
    return guard([&] {
        const std::vector<size_t> c = tree(radix).external_references();
        if (!counts || capacity < c.size()) throw std::invalid_argument("reference count buffer too small");
        std::copy(c.begin(), c.end(), counts);
    });
}

}  // extern "C"
