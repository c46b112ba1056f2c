// Prefix cache over the device KV pool: RadixCache (core/include/tvara/radix.hpp
// :17-131) restated over DeviceCache.  The tree is host metadata; a node's
// KV snapshot is a retained copy of a sequence's block table, and reuse
// imports it as a new sequence that shares those blocks (copy-on-write on
// append).  Node ids, eviction order, errors and messages are the
// reference's.
#pragma once

#include <cstdint>
#include <map>
#include <optional>
#include <string>
#include <utility>
#include <vector>

#include "kv_cache.hpp"

namespace tvara_amd {

struct RadixNode {
    uint64_t id = 0, parent = 0;
    std::vector<int32_t> edge;
    std::map<int32_t, uint64_t> children;
    std::optional<Table> kv;
    size_t pins = 0;
    uint64_t accessed = 0;
};

class RadixCache {
public:
    RadixCache(DeviceCache& cache, std::string isolation);
    ~RadixCache();
    RadixCache(const RadixCache&) = delete;
    RadixCache& operator=(const RadixCache&) = delete;

    const RadixNode& node(uint64_t id) const;
    size_t size() const { return nodes_.size() - 1; }
    const std::string& isolation() const { return isolation_; }
    // (deepest node on the path, tokens matched)
    std::pair<uint64_t, size_t> lookup(const int32_t* tokens, size_t n) const;
    uint64_t insert(const int32_t* tokens, size_t n);
    void attach(uint64_t id, uint64_t sequence);
    std::vector<size_t> external_references() const;
    // (new sequence, tokens it starts with)
    std::pair<uint64_t, size_t> reuse(const int32_t* tokens, size_t n, bool partial);
    void pin(uint64_t id);
    void unpin(uint64_t id);
    void touch(uint64_t id);
    std::optional<uint64_t> eviction_candidate() const;
    bool evict_one();
    void reset();

private:
    void release_kv(RadixNode& n);
    DeviceCache& cache_;
    std::string isolation_;
    std::map<uint64_t, RadixNode> nodes_;
    uint64_t next_ = 0, clock_ = 0;
};

}  // namespace tvara_amd
