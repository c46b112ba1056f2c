// ref_shim.cpp -- a C ABI over the reference's own header-only KV cache and
// attention code, compiled from the reference sources where they lie
// (oracle/Makefile, target `ref`, output oracle/_ref/libtvara_ref.so).
//
// TEST INFRASTRUCTURE ONLY.  It exists to validate the C restatement in
// tvara_oracle.c, to write the golden fixtures under tests/golden/, and to time
// the reference CPU path as bench.py's cpu_baseline.  Nothing in the product
// library links or loads it.  No reference source is copied: this file only
// includes the reference headers and forwards calls to them.
#include "tvara/attention.hpp"
#include "tvara/kv.hpp"
#include "tvara/quant.hpp"
#include "tvara/radix.hpp"

#include <algorithm>
#include <atomic>
#include <functional>
#include <mutex>
#include <stdexcept>
#include <chrono>
#include <cstring>
#include <span>
#include <new>
#include <string>
#include <thread>
#include <vector>

namespace {
thread_local std::string last_error;

template <class F>
int guard(F&& f) {
    last_error.clear();
    try {
        f();
        return 0;
    } catch (const tvara::CacheExhausted& e) {
        last_error = e.what();
        return -3;
    } catch (const std::invalid_argument& e) {
        last_error = e.what();
        return -2;
    } catch (const std::logic_error& e) {
        last_error = e.what();
        return -4;
    } catch (const std::bad_alloc& e) {
        last_error = e.what();
        return -5;
    } catch (const std::exception& e) {
        last_error = e.what();
        return -1;
    }
}

tvara::ModelConfig config(const tvara::PagedCache& cache, std::size_t heads, std::size_t context) {
    const auto& g = cache.geometry();
    return tvara::ModelConfig{1, heads * g.head_dim, 1, g.layers, heads, g.kv_heads, context};
}
}  // namespace

struct tvr_cache {
    tvara::PagedCache cache;
    explicit tvr_cache(tvara::CacheGeometry g) : cache(g) {}
};

extern "C" {
const char* tvr_last_error(void) { return last_error.c_str(); }

tvr_cache* tvr_cache_create(std::size_t layers, std::size_t kv_heads, std::size_t head_dim, std::size_t tpb,
                            std::size_t max_blocks) {
    tvr_cache* out = nullptr;
    guard([&] { out = new tvr_cache(tvara::CacheGeometry{layers, kv_heads, head_dim, tpb, max_blocks}); });
    return out;
}

void tvr_cache_destroy(tvr_cache* c) { delete c; }

int tvr_pool_allocate(tvr_cache* c, std::uint64_t* id, std::uint64_t* gen) {
    return guard([&] {
        auto h = c->cache.pool().allocate();
        *id = h.id;
        *gen = h.generation;
    });
}
int tvr_pool_retain(tvr_cache* c, std::uint64_t id, std::uint64_t gen) {
    return guard([&] { c->cache.pool().retain({id, gen}); });
}
int tvr_pool_release(tvr_cache* c, std::uint64_t id, std::uint64_t gen) {
    return guard([&] { c->cache.pool().release({id, gen}); });
}
int tvr_pool_references(tvr_cache* c, std::uint64_t id, std::uint64_t gen, std::size_t* out) {
    return guard([&] { *out = c->cache.pool().references({id, gen}); });
}
std::size_t tvr_pool_available(tvr_cache* c) { return c->cache.pool().available(); }

std::uint64_t tvr_create_sequence(tvr_cache* c) {
    std::uint64_t id = 0;
    guard([&] { id = c->cache.create_sequence(); });
    return id;
}

int tvr_append(tvr_cache* c, std::uint64_t seq, const float* keys, const float* values) {
    return guard([&] {
        const auto& g = c->cache.geometry();
        const std::size_t n = g.layers * g.kv_width();
        c->cache.append(seq, std::span<const float>(keys, n), std::span<const float>(values, n));
    });
}

// n consecutive appends of rows laid out [n][layers*kv_width]
int tvr_append_many(tvr_cache* c, std::uint64_t seq, const float* keys, const float* values, std::size_t n) {
    return guard([&] {
        const auto& g = c->cache.geometry();
        const std::size_t w = g.layers * g.kv_width();
        for (std::size_t i = 0; i < n; ++i)
            c->cache.append(seq, std::span<const float>(keys + i * w, w), std::span<const float>(values + i * w, w));
    });
}

int tvr_read_all(tvr_cache* c, std::uint64_t seq, std::size_t layer, int value, float* out, std::size_t capacity) {
    return guard([&] {
        auto v = c->cache.read_all(seq, layer, value != 0);
        if (v.size() > capacity) throw std::invalid_argument("buffer too small");
        std::memcpy(out, v.data(), v.size() * sizeof(float));
    });
}

int tvr_read(tvr_cache* c, std::uint64_t seq, std::size_t layer, std::size_t position, int value, float* out) {
    return guard([&] {
        auto v = c->cache.read(seq, layer, position, value != 0);
        std::memcpy(out, v.data(), v.size() * sizeof(float));
    });
}

int tvr_kv_offset(tvr_cache* c, std::size_t layer, std::size_t kind, std::size_t slot, std::size_t* out) {
    return guard([&] { *out = tvara::kv_offset(c->cache.geometry(), layer, kind, slot); });
}

int tvr_drop(tvr_cache* c, std::uint64_t seq) { return guard([&] { c->cache.drop(seq); }); }

std::uint64_t tvr_fork(tvr_cache* c, std::uint64_t seq) {
    std::uint64_t id = 0;
    guard([&] { id = c->cache.fork(seq); });
    return id;
}

int tvr_truncate(tvr_cache* c, std::uint64_t seq, std::size_t length) {
    return guard([&] { c->cache.truncate(seq, length); });
}

int tvr_audit(tvr_cache* c, const std::size_t* external, std::size_t count) {
    return guard([&] { c->cache.audit(std::span<const std::size_t>(external, count)); });
}

// import_sequence of a prefix of an existing sequence's table (the pattern of
// RadixCache::reuse, radix.hpp:90-96)
std::uint64_t tvr_import(tvr_cache* c, std::uint64_t source, std::size_t length) {
    std::uint64_t id = 0;
    guard([&] {
        const auto snapshot = c->cache.sequence(source);
        id = c->cache.import_sequence(snapshot, length);
    });
    return id;
}

// import_sequence of an explicit snapshot (a RadixNode's BlockTable, radix.hpp:12)
std::uint64_t tvr_import_blocks(tvr_cache* c, const std::uint64_t* ids, const std::uint64_t* gens, std::size_t count,
                                std::size_t source_length, std::size_t length) {
    std::uint64_t id = 0;
    guard([&] {
        tvara::BlockTable snapshot;
        snapshot.length = source_length;
        for (std::size_t i = 0; i < count; ++i) snapshot.blocks.push_back({ids[i], gens[i]});
        id = c->cache.import_sequence(snapshot, length);
    });
    return id;
}

int tvr_sequence(tvr_cache* c, std::uint64_t seq, std::size_t* length, std::uint64_t* ids, std::uint64_t* gens,
                 std::size_t capacity, std::size_t* count) {
    return guard([&] {
        const auto& t = c->cache.sequence(seq);
        *length = t.length;
        *count = t.blocks.size();
        if (ids) {
            if (capacity < t.blocks.size()) throw std::invalid_argument("buffer too small");
            for (std::size_t i = 0; i < t.blocks.size(); ++i) {
                ids[i] = t.blocks[i].id;
                gens[i] = t.blocks[i].generation;
            }
        }
    });
}

// refs and generations of every block plus the free list in pop order.  The
// pool keeps generations and the free list private, so they are observed: live
// generations by probing handles, free ones by draining a copy of the cache.
int tvr_pool_state(tvr_cache* c, std::size_t* refs, std::uint64_t* gens, std::size_t* free_pop_order,
                   std::size_t* free_count, std::uint64_t max_generation) {
    return guard([&] {
        const std::size_t n = c->cache.geometry().max_blocks;
        for (std::size_t i = 0; i < n; ++i) {
            refs[i] = c->cache.pool().references_by_id(i);
            gens[i] = 0;
            if (refs[i]) {
                for (std::uint64_t g = 1; g <= max_generation; ++g) {
                    try {
                        (void)c->cache.pool().references({i, g});
                        gens[i] = g;
                        break;
                    } catch (const std::invalid_argument&) {
                    }
                }
            }
        }
        tvara::PagedCache copy = c->cache;
        std::size_t k = 0;
        while (copy.pool().available()) {
            auto h = copy.pool().allocate();
            free_pop_order[k++] = h.id;
            gens[h.id] = h.generation - 1;
        }
        *free_count = k;
    });
}

int tvr_block_data(tvr_cache* c, std::uint64_t id, std::uint64_t gen, float* out, std::size_t capacity) {
    return guard([&] {
        auto d = c->cache.pool().data({id, gen});
        if (d.size() > capacity) throw std::invalid_argument("buffer too small");
        std::memcpy(out, d.data(), d.size() * sizeof(float));
    });
}

int tvr_block_write(tvr_cache* c, std::uint64_t id, std::uint64_t gen, std::size_t offset, const float* in,
                    std::size_t count) {
    return guard([&] {
        auto d = c->cache.pool().data({id, gen});
        if (offset > d.size() || count > d.size() - offset) throw std::invalid_argument("write outside block");
        std::memcpy(d.data() + offset, in, count * sizeof(float));
    });
}

int tvr_fused_paged_attention(tvr_cache* c, std::uint64_t seq, std::size_t layer, std::size_t heads,
                              std::size_t context, const float* q, const float* tail_key, const float* tail_value,
                              std::size_t visible, int scalar, float* out) {
    return guard([&] {
        const auto cfg = config(c->cache, heads, context);
        const std::size_t w = c->cache.geometry().kv_width();
        std::span<const float> tk, tv;
        if (tail_key) {
            tk = std::span<const float>(tail_key, w);
            tv = std::span<const float>(tail_value, w);
        }
        auto o = tvara::fused_paged_attention(std::span<const float>(q, cfg.hidden), c->cache, seq, layer, cfg, tk,
                                              tv, visible, scalar != 0);
        std::memcpy(out, o.data(), o.size() * sizeof(float));
    });
}

int tvr_fused_prompt_attention(tvr_cache* c, std::uint64_t seq, std::size_t layer, std::size_t heads,
                               std::size_t context, std::size_t start, std::size_t count, const float* queries,
                               float* out) {
    return guard([&] {
        const auto cfg = config(c->cache, heads, context);
        auto o = tvara::fused_prompt_attention(std::span<const float>(queries, count * cfg.hidden), c->cache, seq,
                                               layer, start, count, cfg);
        std::memcpy(out, o.data(), o.size() * sizeof(float));
    });
}

// grouped_attention (model.hpp:86-107), the contiguous two-pass comparator
int tvr_grouped_attention(const float* q, const float* keys, const float* values, std::size_t positions,
                          std::size_t heads, std::size_t kv_heads, std::size_t head_dim, std::size_t context,
                          float* out) {
    return guard([&] {
        tvara::ModelConfig cfg{1, heads * head_dim, 1, 1, heads, kv_heads, context};
        const std::size_t n = positions * kv_heads * head_dim;
        auto o = tvara::grouped_attention(std::span<const float>(q, cfg.hidden), std::span<const float>(keys, n),
                                          std::span<const float>(values, n), positions, cfg);
        std::memcpy(out, o.data(), o.size() * sizeof(float));
    });
}

// ---- RadixCache (radix.hpp) over a reference cache
struct tvr_radix {
    tvara::RadixCache tree;
    tvr_radix(tvara::PagedCache& c, const char* iso) : tree(c, iso) {}
};

tvr_radix* tvr_radix_create(tvr_cache* c, const char* isolation) {
    tvr_radix* out = nullptr;
    guard([&] { out = new tvr_radix(c->cache, isolation ? isolation : ""); });
    return out;
}
void tvr_radix_destroy(tvr_radix* r) { delete r; }
int tvr_radix_insert(tvr_radix* r, const std::int32_t* t, std::size_t n, std::uint64_t* node) {
    return guard([&] { *node = r->tree.insert(std::span<const std::int32_t>(t, n)); });
}
int tvr_radix_lookup(tvr_radix* r, const std::int32_t* t, std::size_t n, std::uint64_t* node, std::size_t* matched) {
    return guard([&] {
        auto m = r->tree.lookup(std::span<const std::int32_t>(t, n));
        *node = m.node;
        *matched = m.tokens;
    });
}
int tvr_radix_attach(tvr_radix* r, std::uint64_t node, std::uint64_t seq) {
    return guard([&] { r->tree.attach(node, seq); });
}
int tvr_radix_reuse(tvr_radix* r, const std::int32_t* t, std::size_t n, int partial, std::uint64_t* seq,
                    std::size_t* length) {
    return guard([&] {
        auto x = r->tree.reuse(std::span<const std::int32_t>(t, n), partial != 0);
        *seq = x.first;
        *length = x.second;
    });
}
int tvr_radix_pin(tvr_radix* r, std::uint64_t node) { return guard([&] { r->tree.pin(node); }); }
int tvr_radix_unpin(tvr_radix* r, std::uint64_t node) { return guard([&] { r->tree.unpin(node); }); }
int tvr_radix_touch(tvr_radix* r, std::uint64_t node) { return guard([&] { r->tree.touch(node); }); }
int tvr_radix_eviction_candidate(tvr_radix* r, std::uint64_t* node) {
    return guard([&] {
        auto c = r->tree.eviction_candidate();
        *node = c ? *c : 0;
    });
}
int tvr_radix_evict_one(tvr_radix* r, int* evicted) { return guard([&] { *evicted = r->tree.evict_one() ? 1 : 0; }); }
int tvr_radix_reset(tvr_radix* r) { return guard([&] { r->tree.reset(); }); }
int tvr_radix_size(tvr_radix* r, std::size_t* n) { return guard([&] { *n = r->tree.size(); }); }
int tvr_radix_node(tvr_radix* r, std::uint64_t id, std::uint64_t* parent, std::int32_t* edge, std::size_t cap,
                   std::size_t* edge_len, std::size_t* pins, std::uint64_t* accessed, std::size_t* kv_length,
                   std::size_t* kv_blocks, std::size_t* children) {
    return guard([&] {
        const auto& n = r->tree.node(id);
        *parent = n.parent;
        *edge_len = n.edge.size();
        std::copy(n.edge.begin(), n.edge.begin() + std::min(cap, n.edge.size()), edge);
        *pins = n.pins;
        *accessed = n.accessed;
        *kv_length = n.kv ? n.kv->length : 0;
        *kv_blocks = n.kv ? n.kv->blocks.size() : static_cast<std::size_t>(-1);
        *children = n.children.size();
    });
}
int tvr_radix_external_references(tvr_radix* r, std::size_t* counts, std::size_t cap) {
    return guard([&] {
        auto c = r->tree.external_references();
        if (cap < c.size()) throw std::invalid_argument("reference count buffer too small");
        std::copy(c.begin(), c.end(), counts);
    });
}

// ---- CPU-baseline runners (bench.py): the reference's own functions over a
// batch, on `threads` std::threads taking work units from a shared counter.

static void run_parallel(std::size_t units, int threads, const std::function<void(std::size_t)>& body) {
    std::atomic<std::size_t> next{0};
    std::atomic<bool> failed{false};
    std::string error;
    std::mutex lock;
    auto worker = [&] {
        for (std::size_t u; !failed && (u = next++) < units;) {
            try {
                body(u);
            } catch (const std::exception& e) {
                std::lock_guard<std::mutex> hold(lock);
                failed = true;
                error = e.what();
            }
        }
    };
    std::vector<std::thread> pool;
    for (int t = 1; t < threads; ++t) pool.emplace_back(worker);
    worker();
    for (auto& t : pool) t.join();
    if (failed) throw std::runtime_error(error);
}

// fused_paged_attention (attention.hpp:57-83) for every listed sequence, one
// sequence a work unit; q and out are [count][heads * head_dim]
int tvr_fused_batch(tvr_cache* c, const std::uint64_t* seqs, std::size_t count, std::size_t layer,
                    std::size_t heads, std::size_t context, const float* q, float* out, int threads) {
    return guard([&] {
        const auto cfg = config(c->cache, heads, context);
        run_parallel(count, threads, [&](std::size_t i) {
            auto o = tvara::fused_paged_attention(std::span<const float>(q + i * cfg.hidden, cfg.hidden), c->cache,
                                                  seqs[i], layer, cfg);
            std::memcpy(out + i * cfg.hidden, o.data(), o.size() * sizeof(float));
        });
    });
}

// fused_prompt_attention (attention.hpp:85-89) over rows start .. start+count-1
// of one sequence, in runs of `rows_per_unit` rows a work unit (each run is a
// call of the reference function on its own rows)
int tvr_prompt_batch(tvr_cache* c, std::uint64_t seq, std::size_t layer, std::size_t heads, std::size_t context,
                     std::size_t start, std::size_t count, const float* queries, float* out,
                     std::size_t rows_per_unit, int threads) {
    return guard([&] {
        const auto cfg = config(c->cache, heads, context);
        const std::size_t units = (count + rows_per_unit - 1) / rows_per_unit;
        run_parallel(units, threads, [&](std::size_t u) {
            const std::size_t a = u * rows_per_unit, n = std::min(rows_per_unit, count - a);
            auto o = tvara::fused_prompt_attention(std::span<const float>(queries + a * cfg.hidden, n * cfg.hidden),
                                                   c->cache, seq, layer, start + a, n, cfg);
            std::memcpy(out + a * cfg.hidden, o.data(), o.size() * sizeof(float));
        });
    });
}

// whether the reference's attention dot takes its AVX2 path here (simd.hpp:14-17)
int tvr_use_avx2(void) { return tvara::use_avx2() ? 1 : 0; }

// STREAM-style triad a = b + s*c over n doubles per array on `threads` threads
// (each its own contiguous share), best of `reps`: bytes moved (3 x 8 x n) per
// second.  The host's memory bandwidth, measured before any CPU fraction is
// quoted.
double tvr_host_triad(std::size_t n, int threads, int reps) {
    std::vector<double> a(n), b(n, 1.0), c(n, 2.0);
    double best = 0;
    for (int r = 0; r < reps; ++r) {
        const auto t0 = std::chrono::steady_clock::now();
        std::vector<std::thread> pool;
        for (int t = 0; t < threads; ++t)
            pool.emplace_back([&, t] {
                const std::size_t lo = n * t / threads, hi = n * (t + 1) / threads;
                for (std::size_t i = lo; i < hi; ++i) a[i] = b[i] + 3.0 * c[i];
            });
        for (auto& th : pool) th.join();
        const double s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        best = std::max(best, 24.0 * static_cast<double>(n) / s);
    }
    volatile double sink = a[n / 2];
    (void)sink;
    return best;
}

float tvr_half_to_float(std::uint16_t h) { return tvara::quant::half_to_float(h); }

int tvr_dequantize_q8_0(const std::uint8_t* bytes, std::size_t nbytes, float* out, std::size_t count) {
    return guard([&] {
        tvara::quant::dequantize_q8_0(std::span<const std::byte>(reinterpret_cast<const std::byte*>(bytes), nbytes),
                                      std::span<float>(out, count));
    });
}
}
