// Test driver, not product code: the library's HIP-free host sources --
// KvLedger (kv_ledger.cpp), PrefixTree (radix.cpp) and the GGUF reader
// (gguf.cpp) -- built with -fsanitize=address,undefined (the reference's
// TVARA_SANITIZERS option, CMakeLists.txt:6,13-19) and driven three ways:
//
//   ledger_faults churn       random pool / table / prefix-tree operations,
//                             every invariant audited after every step;
//   ledger_faults faults      every allocation inside every mutating
//                             operation made to fail in turn (operator new
//                             throws on the k-th call, as in
//                             tests/core/test_core_regressions.cpp:10-58 for
//                             snapshot publication): a failed call must leave
//                             the pool, the tables and the tree exactly as
//                             they were, with no reference leaked;
//   ledger_faults gguf F...   parse each file as tvara_model_open does and
//                             print "ok" or the rejection message.
//
// Exit status 0 and the line "passed" mean every check held.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <chrono>
#include <functional>
#include <map>
#include <new>
#include <string>
#include <vector>

#include "gguf.hpp"
#include "kv_ledger.hpp"
#include "radix.hpp"

using tvara_amd::Geometry;
using tvara_amd::Handle;
using tvara_amd::KvLedger;
using tvara_amd::PrefixTree;

// ------------------------------------------------------ failure injection

static long g_countdown = 0;  // > 0: the allocation that brings it to 0 fails
static long g_allocations = 0;

[[gnu::noinline]] void* operator new(std::size_t size) {
    ++g_allocations;
    if (g_countdown > 0 && --g_countdown == 0) throw std::bad_alloc();
    if (void* p = std::malloc(size ? size : 1)) return p;
    throw std::bad_alloc();
}
[[gnu::noinline]] void* operator new[](std::size_t size) { return ::operator new(size); }
[[gnu::noinline]] void* operator new(std::size_t size, const std::nothrow_t&) noexcept {
    try {
        return ::operator new(size);
    } catch (...) {
        return nullptr;
    }
}
[[gnu::noinline]] void operator delete(void* p) noexcept { std::free(p); }
[[gnu::noinline]] void operator delete[](void* p) noexcept { std::free(p); }
[[gnu::noinline]] void operator delete(void* p, std::size_t) noexcept { std::free(p); }
[[gnu::noinline]] void operator delete[](void* p, std::size_t) noexcept { std::free(p); }
[[gnu::noinline]] void operator delete(void* p, const std::nothrow_t&) noexcept { std::free(p); }

static void check(bool ok, const char* what, long detail = -1) {
    if (ok) return;
    std::fprintf(stderr, "check failed: %s (%ld)\n", what, detail);
    std::exit(1);
}

// counter-based splitmix64, the test inputs' generator
static uint64_t mix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
struct Rng {
    uint64_t s;
    uint64_t below(uint64_t n) { return mix(s++) % n; }
};

// ----------------------------------------------------------- a whole state

struct World {
    KvLedger kv;
    PrefixTree tree;
    std::vector<uint64_t> seqs;
    explicit World(const Geometry& g) : kv(g), tree(kv, "faults/tenant") {}
};

// Everything observable: allocator arrays, every table, every node.
static std::string dump(World& w) {
    const size_t n = w.kv.geometry().max_blocks;
    std::vector<size_t> refs(n), order(n);
    std::vector<uint64_t> gens(n);
    size_t nfree = 0;
    w.kv.pool_state(refs.data(), gens.data(), order.data(), &nfree);
    std::string s;
    auto put = [&](uint64_t v) { s += std::to_string(v) + ","; };
    for (size_t i = 0; i < n; ++i) {
        put(refs[i]);
        put(gens[i]);
    }
    s += "|";
    for (size_t i = 0; i < nfree; ++i) put(order[i]);
    s += "|";
    for (uint64_t id : w.kv.sequence_ids()) {
        const auto& t = w.kv.sequence(id);
        put(id);
        put(t.length);
        for (const Handle& h : t.blocks) {
            put(h.id);
            put(h.generation);
        }
        s += ";";
    }
    s += "|" + std::to_string(w.tree.size()) + "|";
    for (uint64_t id = 0; id < 512; ++id) {
        try {
            const auto info = w.tree.node(id);
            put(id);
            put(info.parent);
            put(info.pins);
            put(info.accessed);
            put(info.children);
            for (size_t i = 0; i < info.edge_length; ++i) put(static_cast<uint32_t>(info.edge[i]));
            put(info.kv ? info.kv->length : 999999);
            if (info.kv)
                for (const Handle& h : info.kv->blocks) put(h.id);
            s += ";";
        } catch (const std::out_of_range&) {
        }
    }
    const auto cand = w.tree.eviction_candidate();
    s += "|" + std::to_string(cand ? *cand : 0);
    return s;
}

static void audit(World& w) {
    const auto ext = w.tree.external_references();
    w.kv.audit(ext.data(), ext.size());
}

// ------------------------------------------------------------- operations

static std::vector<int32_t> tokens(Rng& r, size_t min_len, size_t max_len, int alphabet) {
    std::vector<int32_t> t(min_len + r.below(max_len - min_len + 1));
    for (auto& x : t) x = static_cast<int32_t>(r.below(static_cast<uint64_t>(alphabet)));
    return t;
}

static uint64_t grow(World& w, size_t length) {
    const uint64_t s = w.kv.create_sequence();
    std::vector<uint64_t> ids(length, s);
    auto work = w.kv.plan_appends(ids.data(), ids.size());
    if (work.failure) std::rethrow_exception(work.failure);
    return s;
}

// one mutation of a random kind; errors other than bad_alloc are part of the
// contract and ignored here
static void random_op(World& w, Rng& r) {
    const uint64_t node = r.below(24);
    auto t = tokens(r, 1, 6, 3);
    try {
        switch (r.below(12)) {
            case 0:
            case 1: w.tree.insert(t.data(), t.size()); break;
            case 2: {  // a length that mostly mismatches the node's depth
                const uint64_t s = grow(w, r.below(8));
                try {
                    w.tree.attach(node, s);
                } catch (const std::exception&) {
                }
                w.kv.drop(s);
                break;
            }
            case 3: {
                const auto m = w.tree.lookup(t.data(), t.size());
                size_t depth = 0;
                for (uint64_t c = m.first; c; c = w.tree.node(c).parent) depth += w.tree.node(c).edge_length;
                const uint64_t s = grow(w, depth);
                w.tree.attach(m.first, s);
                w.kv.drop(s);
                break;
            }
            case 4: w.seqs.push_back(w.tree.reuse(t.data(), t.size(), r.below(2)).first); break;
            case 5: w.tree.pin(node); break;
            case 6: w.tree.unpin(node); break;
            case 7: w.tree.touch(node); break;
            case 8: w.tree.evict_one(); break;
            case 9:
                if (!w.seqs.empty()) {
                    const uint64_t s = w.seqs[r.below(w.seqs.size())];
                    auto work = w.kv.plan_appends(&s, 1);
                    if (work.failure) std::rethrow_exception(work.failure);
                }
                break;
            case 10:
                if (!w.seqs.empty()) {
                    const size_t i = r.below(w.seqs.size());
                    if (r.below(2)) {
                        w.kv.drop(w.seqs[i]);
                        w.seqs.erase(w.seqs.begin() + static_cast<std::ptrdiff_t>(i));
                    } else {
                        w.seqs.push_back(w.kv.fork(w.seqs[i]));
                    }
                }
                break;
            default:
                if (r.below(4) == 0) w.tree.reset();
                else if (!w.seqs.empty())
                    w.kv.truncate(w.seqs[r.below(w.seqs.size())], r.below(3));
                break;
        }
    } catch (const std::bad_alloc&) {
        throw;
    } catch (const std::exception&) {
    }
}

static Geometry small() { return Geometry{1, 1, 2, 3, 40}; }

static void churn() {
    int emptied = 0;
    for (uint64_t seed = 1; seed <= 8; ++seed) {
        World w(small());
        Rng r{seed * 1000003};
        for (int step = 0; step < 3000; ++step) {
            random_op(w, r);
            audit(w);
        }
        // Undo pins deepest first (a pin counts on a whole path, and an
        // ancestor may already have been unpinned below a descendant's count,
        // which then stays pinned), drop every sequence and reset: with no
        // pin left the whole pool is free again.
        std::vector<std::pair<size_t, uint64_t>> by_depth;
        for (uint64_t id = 1; id <= 100000; ++id) {
            try {
                size_t d = 0;
                for (uint64_t c = id; c; c = w.tree.node(c).parent) ++d;
                by_depth.emplace_back(d, id);
            } catch (const std::out_of_range&) {
            }
        }
        std::sort(by_depth.rbegin(), by_depth.rend());
        for (const auto& e : by_depth) {
            try {
                while (w.tree.node(e.second).pins) w.tree.unpin(e.second);
            } catch (const std::invalid_argument&) {
            }
        }
        for (uint64_t s : w.kv.sequence_ids()) w.kv.drop(s);
        bool pinned = false;
        try {
            w.tree.reset();
        } catch (const std::logic_error&) {
            pinned = true;
        }
        audit(w);
        if (!pinned) {
            check(w.kv.available() == w.kv.geometry().max_blocks, "blocks leaked after churn", static_cast<long>(seed));
            ++emptied;
        }
    }
    std::printf("churn: 8 x 3000 operations audited, %d pools emptied to the last block\n", emptied);
    check(emptied > 0, "no churn run could be torn down");
}

// One case: `prepare` runs with allocation working, then `act` makes exactly
// one mutating call with every allocation in turn made to fail.
struct Case {
    const char* name;
    std::function<void(World&, Rng&)> prepare;
    std::function<void(World&)> act;
};

// Sets a world up by a fixed prefix of random operations, prepares the case,
// then fails the k-th allocation of its call for k = 1, 2, ... until the call
// goes through.
static int sweep(const Case& c, uint64_t seed, int setup_steps) {
    int failures = 0;
    for (long k = 1;; ++k) {
        World w(small());
        Rng r{seed};
        for (int i = 0; i < setup_steps; ++i) random_op(w, r);
        Rng rp{seed ^ 0xABCDEF};
        c.prepare(w, rp);
        const std::string before = dump(w);
        g_countdown = k;
        bool failed = false;
        try {
            c.act(w);
        } catch (const std::bad_alloc&) {
            failed = true;
        } catch (const std::exception&) {
        }
        g_countdown = 0;
        if (!failed) break;
        ++failures;
        if (dump(w) != before) {
            std::fprintf(stderr, "%s: allocation %ld failed and the state changed\n", c.name, k);
            std::exit(1);
        }
        audit(w);
        check(k < 100000, "allocation sweep does not end");
    }
    return failures;
}

static void faults() {
    // arguments the prepare step leaves for the call
    static std::vector<int32_t> t;
    static uint64_t node = 0, seq = 0;
    static bool partial = false;
    auto some_seq = [](World& w) -> uint64_t {
        const auto ids = w.kv.sequence_ids();
        return ids.empty() ? w.kv.create_sequence() : ids[ids.size() / 2];
    };
    const std::vector<Case> cases = {
        {"insert (split and leaf)", [](World&, Rng& r) { t = tokens(r, 2, 7, 3); },
         [](World& w) { w.tree.insert(t.data(), t.size()); }},
        {"attach (snapshot publication)",
         [](World& w, Rng& r) {
             t = tokens(r, 1, 6, 3);
             node = w.tree.insert(t.data(), t.size());
             seq = grow(w, t.size());
         },
         [](World& w) { w.tree.attach(node, seq); }},
        {"reuse (import_sequence)",
         [](World&, Rng& r) {
             t = tokens(r, 1, 6, 3);
             partial = r.below(2);
         },
         [](World& w) { w.tree.reuse(t.data(), t.size(), partial); }},
        {"pin", [](World&, Rng& r) { node = r.below(16); }, [](World& w) { w.tree.pin(node); }},
        {"unpin",
         [](World& w, Rng& r) {
             node = r.below(16);
             try {
                 w.tree.pin(node);
             } catch (const std::exception&) {
             }
         },
         [](World& w) { w.tree.unpin(node); }},
        {"touch", [](World&, Rng& r) { node = r.below(16); }, [](World& w) { w.tree.touch(node); }},
        {"evict_one", [](World&, Rng&) {}, [](World& w) { w.tree.evict_one(); }},
        {"reset", [](World&, Rng&) {}, [](World& w) { w.tree.reset(); }},
        {"fork", [some_seq](World& w, Rng&) { seq = some_seq(w); }, [](World& w) { w.kv.fork(seq); }},
        {"append (new block or copy-on-write)",
         [some_seq](World& w, Rng& r) {
             seq = some_seq(w);
             if (r.below(2)) seq = w.kv.fork(seq);
         },
         [](World& w) {
             auto work = w.kv.plan_appends(&seq, 1);
             if (work.failure) std::rethrow_exception(work.failure);
         }},
        {"truncate", [some_seq](World& w, Rng&) { seq = some_seq(w); }, [](World& w) { w.kv.truncate(seq, 0); }},
        {"drop", [some_seq](World& w, Rng&) { seq = some_seq(w); }, [](World& w) { w.kv.drop(seq); }},
        {"create_sequence", [](World&, Rng&) {}, [](World& w) { w.kv.create_sequence(); }},
    };
    int total = 0;
    for (const Case& c : cases) {
        int n = 0;
        for (uint64_t seed = 1; seed <= 12; ++seed) n += sweep(c, seed * 7919, static_cast<int>(20 * seed));
        std::printf("%s: %d injected failures, state unchanged after each\n", c.name, n);
        total += n;
    }
    check(total > 0, "no allocation was ever failed");
}

// The sequence map against std::map: random inserts and erases over a small
// id range (many erased slots, repeated growth and same-size rehashes), every
// id looked up after every step, the live set compared by for_each.
static void sequence_map() {
    for (uint64_t seed = 1; seed <= 4; ++seed) {
        tvara_amd::SequenceMap m;
        std::map<uint64_t, size_t> model;
        Rng r{seed * 7777};
        const uint64_t range = seed == 4 ? 5000 : 200;
        for (int step = 0; step < 20000; ++step) {
            const uint64_t id = 1 + r.below(range);
            if (model.count(id)) {
                check(m.erase(id), "erase of a live id failed", step);
                model.erase(id);
            } else {
                tvara_amd::Table t;
                t.length = static_cast<size_t>(step);
                m.insert(id, std::move(t));
                model[id] = static_cast<size_t>(step);
            }
            check(m.size() == model.size(), "sequence map size", step);
            if (step % 97 == 0 || range <= 200) {
                for (uint64_t k = 1; k <= range; k += (range <= 200 ? 1 : 13)) {
                    const tvara_amd::Table* t = m.find(k);
                    const auto it = model.find(k);
                    check((t != nullptr) == (it != model.end()), "sequence map membership", static_cast<long>(k));
                    if (t) check(t->length == it->second, "sequence map value", static_cast<long>(k));
                }
            }
        }
        size_t seen = 0;
        m.for_each([&](uint64_t id, const tvara_amd::Table& t) {
            check(model.count(id) && model[id] == t.length, "for_each entry", static_cast<long>(id));
            ++seen;
        });
        check(seen == model.size(), "for_each count");
        check(!m.erase(range + 1), "erase of an absent id");
    }
    std::printf("sequence map: 4 x 20000 random inserts and erases matched std::map\n");
}

// evict_one on a victim whose snapshot holds a handle released outside the
// tree: the release throws, the victim stays, and its parent (which would
// have become a leaf) must not be listed as evictable, or a later eviction
// would remove an interior node.
static void stale_eviction() {
    World w(Geometry{1, 1, 2, 2, 8});
    const int32_t a[] = {5, 6}, b[] = {5, 6, 7};
    const uint64_t parent = w.tree.insert(a, 2);
    const uint64_t leaf = w.tree.insert(b, 3);
    const uint64_t s = grow(w, 3);
    w.tree.attach(leaf, s);
    w.kv.drop(s);
    const Handle stale = w.tree.node(leaf).kv->blocks[1];
    w.kv.release(stale);  // the snapshot's only reference: the block is freed
    check(w.tree.eviction_candidate() == leaf, "the leaf is the eviction candidate");
    bool threw = false;
    try {
        w.tree.evict_one();
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    check(threw, "evict_one releases a stale handle without error");
    check(w.tree.size() == 2, "the victim left the tree after a failed release", static_cast<long>(w.tree.size()));
    check(w.tree.eviction_candidate() == leaf, "the failed eviction changed the candidate",
          static_cast<long>(w.tree.eviction_candidate().value_or(0)));
    check(w.tree.node(parent).children == 1, "the parent lost its child");
    std::printf("stale eviction: the victim and the eviction index are unchanged\n");
}

// Many inserts into one tree: each reserves arena room only when it is short,
// so building n nodes costs O(n log n), not O(n^2).  80,000 leaves under one
// root took 143 s with a reserve on every insert; the bound here is loose
// enough for a sanitized build on a slow host.
static void insert_scaling() {
    World w(Geometry{1, 1, 2, 2, 8});
    const auto t0 = std::chrono::steady_clock::now();
    const int n = 50000;
    for (int i = 0; i < n; ++i) {
        const int32_t t[] = {i % 97, i, 1};
        w.tree.insert(t, 3);
    }
    const double s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    check(w.tree.size() == static_cast<size_t>(n + 97), "tree size after the inserts", static_cast<long>(w.tree.size()));
    check(s < 20.0, "50,000 inserts took over 20 s", static_cast<long>(s));
    std::printf("insert scaling: %d inserts in %.2f s\n", n, s);
}

static void gguf_files(int argc, char** argv) {
    for (int i = 2; i < argc; ++i) {
        try {
            tvara_amd::gguf::ModelFile file(argv[i]);
            const auto shape = tvara_amd::gguf::llama_shape(file.document());
            tvara_amd::gguf::validate_llama_tensors(file.document(), shape);
            (void)tvara_amd::gguf::metadata_json(file.document());
            std::printf("ok\n");
        } catch (const std::exception& e) {
            std::printf("error: %s\n", e.what());
        }
    }
}

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "all";
    if (mode == "gguf") {
        gguf_files(argc, argv);
        return 0;
    }
    if (mode == "all" || mode == "churn") {
        sequence_map();
        churn();
    }
    if (mode == "all" || mode == "faults") {
        faults();
        stale_eviction();
        insert_scaling();
    }
    std::printf("passed (%ld allocations)\n", g_allocations);
    return 0;
}
