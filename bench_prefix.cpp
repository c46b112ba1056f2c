// Prefix-cache lookup-and-restore timing for bench.py (the `prefix` line).
//
// Replays the reference's own radix benchmark (bench/radix_prefix.cpp): a
// cache of one layer, one KV head, head_dim 1 and 4-token blocks (128 of
// them); an 8-token prefix appended to a sequence, inserted and attached;
// then 10,000 requests, every fourth with its first token changed (a miss),
// each restored with reuse() (whole blocks) and its sequence dropped.  The
// time of the 10,000 requests is taken with steady_clock, as the reference
// takes it, over a C ABI loaded with dlopen:
//
//   bench_prefix tvara LIB   this library's exports (tvara_kv_*, tvara_radix_*)
//   bench_prefix ref LIB     the reference's PagedCache and RadixCache built
//                            from its headers (the tvr_* exports of the test
//                            build), the CPU baseline
//
// Prints one JSON object per run: {"runs": [ns, ...], "hits", "saved", ...}.
#include <dlfcn.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace {

struct Api {
    void* (*cache_create)(size_t, size_t, size_t, size_t, size_t);              // tvr_cache_create
    void* (*cache_create_fmt)(size_t, size_t, size_t, size_t, size_t, int);     // tvara_kv_cache_create (f32 = 0)
    void (*cache_destroy)(void*);
    uint64_t (*create_sequence)(void*);
    int (*append)(void*, uint64_t, const float*, const float*);
    int (*drop)(void*, uint64_t);
    void* (*radix_create)(void*, const char*);
    void (*radix_destroy)(void*);
    int (*insert)(void*, const int32_t*, size_t, uint64_t*);
    int (*attach)(void*, uint64_t, uint64_t);
    int (*reuse)(void*, const int32_t*, size_t, int, uint64_t*, size_t*);
};

template <class F>
bool bind(void* lib, const char* name, F& f) {
    f = reinterpret_cast<F>(dlsym(lib, name));
    if (!f) std::fprintf(stderr, "missing export %s\n", name);
    return f != nullptr;
}

bool load(const std::string& kind, void* lib, Api& a) {
    const bool t = kind == "tvara";
    bool ok = true;
    if (t)
        ok &= bind(lib, "tvara_kv_cache_create", a.cache_create_fmt);
    else
        ok &= bind(lib, "tvr_cache_create", a.cache_create);
    ok &= bind(lib, t ? "tvara_kv_cache_destroy" : "tvr_cache_destroy", a.cache_destroy);
    ok &= bind(lib, t ? "tvara_kv_sequence_create" : "tvr_create_sequence", a.create_sequence);
    ok &= bind(lib, t ? "tvara_kv_append" : "tvr_append", a.append);
    ok &= bind(lib, t ? "tvara_kv_drop" : "tvr_drop", a.drop);
    ok &= bind(lib, t ? "tvara_radix_create" : "tvr_radix_create", a.radix_create);
    ok &= bind(lib, t ? "tvara_radix_destroy" : "tvr_radix_destroy", a.radix_destroy);
    ok &= bind(lib, t ? "tvara_radix_insert" : "tvr_radix_insert", a.insert);
    ok &= bind(lib, t ? "tvara_radix_attach" : "tvr_radix_attach", a.attach);
    ok &= bind(lib, t ? "tvara_radix_reuse" : "tvr_radix_reuse", a.reuse);
    return ok;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 3 && argc != 4) {
        std::fprintf(stderr, "usage: bench_prefix tvara|ref LIBRARY [RUNS]\n");
        return 2;
    }
    const std::string kind = argv[1];
    const int runs = argc == 4 ? std::max(1, std::atoi(argv[3])) : 9;
    void* lib = dlopen(argv[2], RTLD_NOW | RTLD_LOCAL);
    if (!lib) {
        std::fprintf(stderr, "dlopen: %s\n", dlerror());
        return 2;
    }
    Api a{};
    if (!load(kind, lib, a)) return 2;

    void* cache = kind == "tvara" ? a.cache_create_fmt(1, 1, 1, 4, 128, 0) : a.cache_create(1, 1, 1, 4, 128);
    if (!cache) return 3;
    void* tree = a.radix_create(cache, "benchmark-fixture");
    if (!tree) return 3;
    const std::vector<int32_t> prefix{1, 2, 3, 4, 5, 6, 7, 8};
    const uint64_t s = a.create_sequence(cache);
    const float one = 1.f;
    for (size_t i = 0; i < prefix.size(); ++i)
        if (a.append(cache, s, &one, &one)) return 3;
    uint64_t node = 0;
    if (a.insert(tree, prefix.data(), prefix.size(), &node) || a.attach(tree, node, s)) return 3;

    std::vector<long long> times;
    size_t hits = 0, saved = 0, total = 0;
    for (int r = 0; r < runs + 1; ++r) {  // the first run warms the caches and is not reported
        hits = saved = total = 0;
        std::vector<int32_t> query(prefix.size());
        const auto begin = std::chrono::steady_clock::now();
        for (int i = 0; i < 10000; ++i) {
            std::copy(prefix.begin(), prefix.end(), query.begin());
            if (i % 4 == 0) query[0] = 99;
            uint64_t seq = 0;
            size_t length = 0;
            if (a.reuse(tree, query.data(), query.size(), 0, &seq, &length)) return 4;
            hits += length != 0;
            saved += length;
            total += query.size();
            if (a.drop(cache, seq)) return 4;
        }
        const long long ns =
            std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - begin).count();
        if (r) times.push_back(ns);
    }
    std::printf("{\"kind\": \"%s\", \"requests\": 10000, \"hits\": %zu, \"saved_prefill_tokens\": %zu, "
                "\"requested_tokens\": %zu, \"runs_ns\": [",
                kind.c_str(), hits, saved, total);
    for (size_t i = 0; i < times.size(); ++i) std::printf("%s%lld", i ? ", " : "", times[i]);
    std::printf("]}\n");
    a.drop(cache, s);
    a.radix_destroy(tree);
    a.cache_destroy(cache);
    return 0;
}
