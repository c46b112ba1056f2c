// Test harness, not product code: the block-byte exports of libtvara_capi
// (create, append, read, read_all, block_read) over host memory instead of
// HBM, linked with the library's own HIP-free sources -- the pool and tables
// (kv_ledger.cpp), the prefix tree (radix.cpp), the ledger and prefix-cache
// exports (ledger_capi.cpp) and the error convention (abi.cpp) -- into
// libtvara_host.so.  The CPU tests drive it through the same Python classes
// as the GPU library and compare every result, node and pool state with the
// reference's own classes (built from core/include/tvara/kv.hpp and radix.hpp
// into oracle/_ref).  Byte movement follows PagedCache::append (kv.hpp:91-108)
// through the block work KvLedger::plan_appends lists: zero-fills and
// copy-on-write copies first, then the row writes.  f32 blocks only.
#include <algorithm>
#include <cstring>
#include <memory>
#include <vector>

#include "abi.hpp"

using tvara_amd::AppendWork;
using tvara_amd::Geometry;
using tvara_amd::Handle;
using tvara_amd::KvLedger;
using tvara_amd::abi::guard;
using tvara_amd::abi::handle;

struct tvara_kv_cache {
    KvLedger ledger;
    std::vector<float> blocks;
    size_t block_floats;
    explicit tvara_kv_cache(const Geometry& g)
        : ledger(g), blocks(g.max_blocks * g.elements_per_block()), block_floats(g.elements_per_block()) {}

    float* block(size_t id) { return blocks.data() + id * block_floats; }
    // kv_offset (kv.hpp:30-33)
    size_t offset(size_t layer, size_t kind, size_t slot) const {
        const Geometry& g = ledger.geometry();
        return ((layer * 2 + kind) * g.tokens_per_block + slot) * g.kv_width();
    }
    void zero_fills() {
        for (int64_t id : ledger.take_pending_zero_fills()) std::fill_n(block(static_cast<size_t>(id)), block_floats, 0.f);
    }
};

tvara_amd::KvLedger& tvara_amd::abi::ledger_of(tvara_kv_cache* cache) {
    if (!cache) throw std::invalid_argument("closed KV cache");
    return cache->ledger;
}

namespace {
tvara_kv_cache& live(tvara_kv_cache* c) {
    if (!c) throw std::invalid_argument("closed KV cache");
    return *c;
}

void append(tvara_kv_cache& c, const uint64_t* seqs, size_t n, const float* keys, const float* values,
            size_t* applied) {
    if (n && (!seqs || !keys || !values)) throw std::invalid_argument("invalid paged KV append dimensions");
    AppendWork w = c.ledger.plan_appends(seqs, n);
    if (applied) *applied = w.applied;
    c.zero_fills();
    for (const auto& op : w.init) {
        float* dst = c.block(static_cast<size_t>(op.dst));
        if (op.src < 0) std::fill_n(dst, c.block_floats, 0.f);
        else std::copy_n(c.block(static_cast<size_t>(op.src)), c.block_floats, dst);
    }
    const Geometry& g = c.ledger.geometry();
    const size_t kvw = g.kv_width(), width = g.layers * kvw;
    for (const auto& r : w.rows) {
        float* b = c.block(static_cast<size_t>(r.block));
        const size_t src = static_cast<size_t>(r.src_row) * width;
        for (size_t layer = 0; layer < g.layers; ++layer) {
            std::copy_n(keys + src + layer * kvw, kvw, b + c.offset(layer, 0, static_cast<size_t>(r.slot)));
            std::copy_n(values + src + layer * kvw, kvw, b + c.offset(layer, 1, static_cast<size_t>(r.slot)));
        }
    }
    if (w.failure) std::rethrow_exception(w.failure);
}
}  // namespace

extern "C" {

tvara_kv_cache* tvara_kv_cache_create(size_t layers, size_t kv_heads, size_t head_dim, size_t tokens_per_block,
                                      size_t max_blocks, int format) {
    tvara_kv_cache* out = nullptr;
    guard([&] {
        if (format != TVARA_KV_F32) throw std::invalid_argument("the host harness stores f32 blocks only");
        out = new tvara_kv_cache(Geometry{layers, kv_heads, head_dim, tokens_per_block, max_blocks});
    });
    return out;
}

void tvara_kv_cache_destroy(tvara_kv_cache* cache) { delete cache; }

size_t tvara_kv_block_bytes(tvara_kv_cache* cache) {
    size_t n = 0;
    guard([&] { n = live(cache).block_floats * sizeof(float); });
    return n;
}

int tvara_kv_set_stream(tvara_kv_cache* cache, void*) {
    return guard([&] { live(cache); });
}

int tvara_kv_synchronize(tvara_kv_cache* cache) {
    return guard([&] { live(cache).zero_fills(); });
}

int tvara_kv_block_read(tvara_kv_cache* cache, tvara_kv_handle h, void* out, size_t bytes) {
    return guard([&] {
        tvara_kv_cache& c = live(cache);
        c.ledger.check_live(handle(h));
        if (!out || bytes != c.block_floats * sizeof(float)) throw std::invalid_argument("block buffer size mismatch");
        c.zero_fills();
        std::memcpy(out, c.block(static_cast<size_t>(h.id)), bytes);
    });
}

int tvara_kv_block_write(tvara_kv_cache* cache, tvara_kv_handle h, size_t offset, const void* data, size_t bytes) {
    return guard([&] {
        tvara_kv_cache& c = live(cache);
        c.ledger.check_live(handle(h));
        const size_t total = c.block_floats * sizeof(float);
        if (!data || offset > total || bytes > total - offset) throw std::invalid_argument("write outside block");
        c.zero_fills();
        std::memcpy(reinterpret_cast<char*>(c.block(static_cast<size_t>(h.id))) + offset, data, bytes);
    });
}

int tvara_kv_append(tvara_kv_cache* cache, uint64_t sequence, const float* keys, const float* values) {
    return guard([&] { append(live(cache), &sequence, 1, keys, values, nullptr); });
}

int tvara_kv_append_batch(tvara_kv_cache* cache, const uint64_t* sequences, size_t count, const float* keys,
                          const float* values, int device_ptrs, size_t* applied) {
    size_t done = 0;
    const int rc = guard([&] {
        if (device_ptrs) throw std::invalid_argument("the host harness has no device memory");
        append(live(cache), sequences, count, keys, values, &done);
    });
    if (applied) *applied = done;
    return rc;
}

int tvara_kv_append_tokens(tvara_kv_cache* cache, uint64_t sequence, const float* keys, const float* values,
                           size_t count, int device_ptrs, size_t* applied) {
    return tvara_kv_append_batch(cache, std::vector<uint64_t>(count, sequence).data(), count, keys, values,
                                 device_ptrs, applied);
}

// PagedCache::read (kv.hpp:110-113)
int tvara_kv_read(tvara_kv_cache* cache, uint64_t sequence, size_t layer, size_t position, int value, float* out) {
    return guard([&] {
        tvara_kv_cache& c = live(cache);
        if (!out) throw std::invalid_argument("null output");
        const Handle h = c.ledger.physical_block(sequence, position);
        const Geometry& g = c.ledger.geometry();
        if (layer >= g.layers) throw std::invalid_argument("KV position outside block");
        c.zero_fills();
        std::copy_n(c.block(h.id) + c.offset(layer, value ? 1 : 0, position % g.tokens_per_block), g.kv_width(), out);
    });
}

// PagedCache::read_all (kv.hpp:114-119)
int tvara_kv_read_all(tvara_kv_cache* cache, uint64_t sequence, size_t layer, int value, float* out,
                      size_t capacity) {
    return guard([&] {
        tvara_kv_cache& c = live(cache);
        const tvara_amd::Table& t = c.ledger.sequence(sequence);
        const Geometry& g = c.ledger.geometry();
        if (layer >= g.layers) throw std::invalid_argument("invalid KV layer");
        const size_t w = g.kv_width();
        if (!out || t.length * w > capacity) {
            if (t.length) throw std::invalid_argument("read_all buffer too small");
            return;
        }
        c.zero_fills();
        for (size_t p = 0; p < t.length; ++p) {
            const Handle h = t.blocks[p / g.tokens_per_block];
            c.ledger.check_live(h);
            std::copy_n(c.block(h.id) + c.offset(layer, value ? 1 : 0, p % g.tokens_per_block), w, out + p * w);
        }
    });
}

}  // extern "C"
