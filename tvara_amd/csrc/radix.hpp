// Prefix cache over the paged KV pool: the contract of RadixCache
// (core/include/tvara/radix.hpp:17-131) on this library's KvLedger.  The tree
// is host metadata; a node's KV is a retained snapshot of a sequence's block
// table, and reuse imports it as a new sequence sharing those blocks (the
// first append to a shared partial block copies it).
//
// Storage, unlike a map of nodes each owning its edge and child map:
//  * nodes live in one arena ordered by id (ids only grow, so appending keeps
//    the order); a lookup by id is a binary search, a removed node is a
//    tombstone until the arena is compacted;
//  * every edge is a slice of one token store, so splitting an edge moves no
//    tokens: the two halves are two slices of the same run;
//  * children are found through one hash map keyed by (parent id, first token
//    of the edge); a node keeps only its child count;
//  * a node records its depth (tokens from the root to the end of its edge),
//    which a split does not change, so attach checks lengths in O(1);
//  * the nodes that may be evicted (unpinned leaves other than the root) sit
//    in an ordered index by (last access stamp, id): the eviction candidate is
//    its first entry.
// What callers observe is the reference's: node ids, which node a split
// leaves the pins on, the eviction order, the order blocks are released in
// (which fixes the pool's free list), errors and messages.
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>
#include <set>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "kv_ledger.hpp"

namespace tvara_amd {

class PrefixTree {
public:
    // what tvara_radix_node reports of one node
    struct NodeInfo {
        uint64_t parent = 0;
        const int32_t* edge = nullptr;
        size_t edge_length = 0;
        size_t pins = 0;
        uint64_t accessed = 0;
        const Table* kv = nullptr;  // null when no snapshot is attached
        size_t children = 0;
    };

    PrefixTree(KvLedger& kv, std::string isolation);
    ~PrefixTree();
    PrefixTree(const PrefixTree&) = delete;
    PrefixTree& operator=(const PrefixTree&) = delete;

    const std::string& isolation() const { return isolation_; }
    size_t size() const { return live_ - 1; }  // the root is not counted
    NodeInfo node(uint64_t id) const;
    // deepest node on the path of `tokens` and how many tokens matched
    std::pair<uint64_t, size_t> lookup(const int32_t* tokens, size_t n) const;
    // the node ending exactly at `tokens`, made by splitting an edge and / or
    // adding a leaf when needed
    uint64_t insert(const int32_t* tokens, size_t n);
    // the node keeps a retained copy of `sequence`'s block table
    void attach(uint64_t id, uint64_t sequence);
    // retained count per block id over every attached snapshot
    std::vector<size_t> external_references() const;
    // a new sequence holding the longest cached prefix of `tokens` (whole
    // blocks unless `partial`) and its length
    std::pair<uint64_t, size_t> reuse(const int32_t* tokens, size_t n, bool partial);
    void pin(uint64_t id);
    void unpin(uint64_t id);
    void touch(uint64_t id);
    std::optional<uint64_t> eviction_candidate() const;
    bool evict_one();
    void reset();

private:
    struct Node {
        uint64_t id = 0, parent = 0;
        size_t edge_at = 0, edge_len = 0;  // slice of tokens_
        size_t depth = 0;
        size_t children = 0;
        size_t pins = 0;
        uint64_t stamp = 0;
        bool dead = false;
        std::optional<Table> kv;
    };
    struct EdgeKey {
        uint64_t parent;
        int32_t token;
        bool operator==(const EdgeKey& o) const { return parent == o.parent && token == o.token; }
    };
    struct EdgeHash {
        size_t operator()(const EdgeKey& k) const;
    };
    // where a walk of `tokens` from the root stops: `at` is the deepest node
    // whose whole edge matched, after `consumed` tokens; `into` is the child
    // of `at` whose edge matched only its first `shared` tokens (0 if none)
    struct Stop {
        uint64_t at = 0;
        size_t consumed = 0;
        uint64_t into = 0;
        size_t shared = 0;
    };

    Stop walk(const int32_t* tokens, size_t n) const;
    Node* find(uint64_t id);
    const Node* find(uint64_t id) const;
    Node& at(uint64_t id);  // out_of_range("map::at") for an absent id, as nodes_.at
    const Node& at(uint64_t id) const;
    Node& add_node(Node n);  // appends to the arena (capacity reserved first)
    bool evictable(const Node& n) const { return n.id && !n.children && !n.pins; }
    void index_out(const Node& n);  // leave the eviction index
    void release_snapshot(Node& n);
    void compact();

    KvLedger& kv_;
    std::string isolation_;
    std::vector<Node> arena_;  // ascending ids; arena_[0] is the root while any node lives
    std::vector<int32_t> tokens_;
    std::unordered_map<EdgeKey, uint64_t, EdgeHash> edges_;
    std::set<std::pair<uint64_t, uint64_t>> idle_;  // (stamp, id) of evictable nodes
    size_t live_ = 0, live_tokens_ = 0;
    uint64_t last_id_ = 0, clock_ = 0;
};

}  // namespace tvara_amd
