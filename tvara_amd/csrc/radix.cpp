// Prefix cache over the paged KV pool (the storage design is described in
// radix.hpp).  Every mutation does the steps that can fail (id exhaustion,
// memory for the edge map, the eviction index or the arena) before it changes
// anything, so a failed call leaves the tree and the pool as they were.
#include "radix.hpp"

#include <algorithm>
#include <limits>
#include <stdexcept>

namespace tvara_amd {

size_t PrefixTree::EdgeHash::operator()(const EdgeKey& k) const {
    uint64_t x = k.parent * 0x9E3779B97F4A7C15ull ^ static_cast<uint32_t>(k.token);
    x ^= x >> 31;
    x *= 0xBF58476D1CE4E5B9ull;
    return static_cast<size_t>(x ^ (x >> 29));
}

PrefixTree::PrefixTree(KvLedger& kv, std::string isolation) : kv_(kv), isolation_(std::move(isolation)) {
    if (isolation_.empty()) throw std::invalid_argument("prefix isolation key is required");
    arena_.emplace_back();  // the root: id 0, empty edge
    live_ = 1;
}

PrefixTree::~PrefixTree() {
    for (Node& n : arena_) {
        if (n.dead) continue;
        try {
            release_snapshot(n);
        } catch (...) {
        }
    }
}

// ------------------------------------------------------------- the arena

PrefixTree::Node* PrefixTree::find(uint64_t id) {
    auto it = std::lower_bound(arena_.begin(), arena_.end(), id, [](const Node& n, uint64_t v) { return n.id < v; });
    return it != arena_.end() && it->id == id && !it->dead ? &*it : nullptr;
}

const PrefixTree::Node* PrefixTree::find(uint64_t id) const { return const_cast<PrefixTree*>(this)->find(id); }

PrefixTree::Node& PrefixTree::at(uint64_t id) {
    Node* n = find(id);
    if (!n) throw std::out_of_range("map::at");
    return *n;
}

const PrefixTree::Node& PrefixTree::at(uint64_t id) const { return const_cast<PrefixTree*>(this)->at(id); }

PrefixTree::Node& PrefixTree::add_node(Node n) {
    arena_.push_back(std::move(n));  // capacity reserved by the caller: cannot throw
    last_id_ = arena_.back().id;
    ++live_;
    return arena_.back();
}

void PrefixTree::index_out(const Node& n) { idle_.erase({n.stamp, n.id}); }

void PrefixTree::release_snapshot(Node& n) {
    if (!n.kv) return;
    for (const Handle& b : n.kv->blocks) kv_.release(b);
    n.kv.reset();
}

// Drops tombstones once they outnumber the live nodes, and rewrites the token
// store once most of it belongs to removed edges.  Optional work: a failed
// allocation leaves everything as it was.
void PrefixTree::compact() {
    const size_t dead = arena_.size() - live_;
    if (dead > 64 && dead > live_) std::erase_if(arena_, [](const Node& n) { return n.dead; });
    if (tokens_.size() <= 4096 || tokens_.size() <= 2 * live_tokens_) return;
    try {
        std::vector<int32_t> packed;
        packed.reserve(live_tokens_);
        std::vector<size_t> moved(arena_.size());
        for (size_t i = 0; i < arena_.size(); ++i) {
            const Node& n = arena_[i];
            if (n.dead || !n.edge_len) continue;
            moved[i] = packed.size();
            packed.insert(packed.end(), tokens_.begin() + static_cast<std::ptrdiff_t>(n.edge_at),
                          tokens_.begin() + static_cast<std::ptrdiff_t>(n.edge_at + n.edge_len));
        }
        for (size_t i = 0; i < arena_.size(); ++i)
            if (!arena_[i].dead && arena_[i].edge_len) arena_[i].edge_at = moved[i];
        tokens_.swap(packed);
    } catch (...) {
    }
}

// ----------------------------------------------------------------- paths

PrefixTree::Stop PrefixTree::walk(const int32_t* tokens, size_t n) const {
    Stop s;
    while (s.consumed < n) {
        auto e = edges_.find({s.at, tokens[s.consumed]});
        if (e == edges_.end()) break;
        const Node& child = at(e->second);
        const int32_t* edge = tokens_.data() + child.edge_at;
        size_t k = 1;  // the edge map matched its first token
        while (k < child.edge_len && s.consumed + k < n && edge[k] == tokens[s.consumed + k]) ++k;
        if (k < child.edge_len) {
            s.into = child.id;
            s.shared = k;
            break;
        }
        s.at = child.id;
        s.consumed += k;
    }
    return s;
}

// radix.hpp:29-42: a match that ends inside an edge names that edge's node
std::pair<uint64_t, size_t> PrefixTree::lookup(const int32_t* tokens, size_t n) const {
    const Stop s = walk(tokens, n);
    if (s.into) return {s.into, s.consumed + s.shared};
    return {s.at, s.consumed};
}

// radix.hpp:44-69: split the edge the path leaves inside (if any) and hang
// the unmatched rest of the tokens below as one leaf.  The split's new node
// takes the id before the leaf's.  Every allocation (both edge-map entries,
// the leaf's eviction-index entry, arena and token capacity) happens before
// the tree changes.
uint64_t PrefixTree::insert(const int32_t* tokens, size_t n) {
    if (!n) throw std::invalid_argument("cannot cache empty prefix");
    const Stop s = walk(tokens, n);
    const size_t done = s.consumed + s.shared;
    if (!s.into && done == n) return s.at;
    uint64_t next = last_id_;
    auto mint = [&] {
        if (next == std::numeric_limits<uint64_t>::max()) throw std::overflow_error("radix ID exhausted");
        return ++next;
    };
    const uint64_t inner = s.into ? mint() : 0;
    const uint64_t leaf = done < n ? mint() : 0;
    const uint64_t leaf_parent = inner ? inner : s.at;

    // room for the two nodes this call may add; growth is geometric, so a
    // long run of inserts reallocates the arena O(log n) times
    if (arena_.capacity() - arena_.size() < 2) arena_.reserve(arena_.size() + 2 + arena_.size() / 2);
    if (leaf && tokens_.capacity() - tokens_.size() < n - done)
        tokens_.reserve(std::max(2 * tokens_.capacity(), tokens_.size() + n - done));
    EdgeKey added[2];
    int count = 0;
    try {
        if (inner) {
            const Node& c = at(s.into);
            added[count] = EdgeKey{inner, tokens_[c.edge_at + s.shared]};
            edges_.emplace(added[count], s.into);
            ++count;
        }
        if (leaf) {
            added[count] = EdgeKey{leaf_parent, tokens[done]};
            edges_.emplace(added[count], leaf);
            ++count;
            idle_.emplace(0, leaf);  // a new leaf is unpinned and never touched
        }
    } catch (...) {
        for (int i = 0; i < count; ++i) edges_.erase(added[i]);
        throw;
    }
    if (inner) {
        // The first `shared` tokens of the child's edge become the inner
        // node.  It takes the child's pins (radix.hpp:60): every pin counted
        // on the child was counted along the whole path above it.
        const Node& c = at(s.into);
        const int32_t first = tokens_[c.edge_at];
        Node mid;
        mid.id = inner;
        mid.parent = s.at;
        mid.edge_at = c.edge_at;
        mid.edge_len = s.shared;
        mid.depth = c.depth - c.edge_len + s.shared;
        mid.children = 1;
        mid.pins = c.pins;
        add_node(std::move(mid));
        Node& moved = at(s.into);
        moved.parent = inner;
        moved.edge_at += s.shared;
        moved.edge_len -= s.shared;
        edges_.find({s.at, first})->second = inner;
    }
    if (!leaf) return inner;
    Node tip;
    tip.id = leaf;
    tip.parent = leaf_parent;
    tip.edge_at = tokens_.size();
    tip.edge_len = n - done;
    tokens_.insert(tokens_.end(), tokens + done, tokens + n);
    Node& p = at(leaf_parent);
    tip.depth = p.depth + tip.edge_len;
    index_out(p);
    ++p.children;
    live_tokens_ += tip.edge_len;
    add_node(std::move(tip));
    return leaf;
}

// ------------------------------------------------------------- snapshots

// radix.hpp:72-81: every block of the new snapshot is retained before the old
// one is released; a failed retain releases the ones taken
void PrefixTree::attach(uint64_t id, uint64_t sequence) {
    Node& entry = at(id);
    const Table& source = kv_.sequence(sequence);
    if (source.length != entry.depth) throw std::invalid_argument("token and KV prefix lengths differ");
    Table snapshot = source;
    size_t retained = 0;
    try {
        for (; retained < snapshot.blocks.size(); ++retained) kv_.retain(snapshot.blocks[retained]);
    } catch (...) {
        for (size_t i = 0; i < retained; ++i) kv_.release(snapshot.blocks[i]);
        throw;
    }
    release_snapshot(entry);
    entry.kv = std::move(snapshot);
}

std::vector<size_t> PrefixTree::external_references() const {
    std::vector<size_t> counts(kv_.geometry().max_blocks);
    for (const Node& n : arena_)
        if (!n.dead && n.kv)
            for (const Handle& b : n.kv->blocks) ++counts.at(b.id);
    return counts;
}

// radix.hpp:90-96
std::pair<uint64_t, size_t> PrefixTree::reuse(const int32_t* tokens, size_t n, bool partial) {
    const auto [id, matched] = lookup(tokens, n);
    const Node* hit = id ? find(id) : nullptr;
    if (!hit || !hit->kv) return {kv_.create_sequence(), 0};
    const size_t length = partial ? matched : matched - matched % kv_.geometry().tokens_per_block;
    const Table& kv = *hit->kv;
    return {kv_.import_sequence(kv.blocks.data(), kv.blocks.size(), kv.length, length), length};
}

// ------------------------------------------------------- pins and access

// radix.hpp:99: a pin counts on the node and every ancestor but the root
void PrefixTree::pin(uint64_t id) {
    std::vector<Node*> path;
    for (uint64_t c = id; c;) {
        Node& n = at(c);
        if (n.pins == std::numeric_limits<size_t>::max()) throw std::overflow_error("prefix pin overflow");
        path.push_back(&n);
        c = n.parent;
    }
    if (!path.empty()) index_out(*path.front());  // only the start can be a leaf
    for (Node* n : path) ++n->pins;
}

// radix.hpp:100
void PrefixTree::unpin(uint64_t id) {
    std::vector<Node*> path;
    for (uint64_t c = id; c;) {
        Node& n = at(c);
        path.push_back(&n);
        c = n.parent;
    }
    for (Node* n : path)
        if (!n->pins) throw std::invalid_argument("prefix pin underflow");
    if (!path.empty() && path.front()->pins == 1 && !path.front()->children)
        idle_.emplace(path.front()->stamp, path.front()->id);
    for (Node* n : path) --n->pins;
}

// radix.hpp:103
void PrefixTree::touch(uint64_t id) {
    Node& n = at(id);
    if (clock_ == std::numeric_limits<uint64_t>::max()) throw std::overflow_error("prefix access clock exhausted");
    const uint64_t stamp = clock_ + 1;
    if (evictable(n)) {
        idle_.emplace(stamp, n.id);
        idle_.erase({n.stamp, n.id});
    }
    n.stamp = stamp;
    clock_ = stamp;
}

// ------------------------------------------------------------ eviction

// radix.hpp:106-110: the least recently touched unpinned leaf, the lowest id
// among equal stamps -- the first entry of the (stamp, id) index
std::optional<uint64_t> PrefixTree::eviction_candidate() const {
    if (idle_.empty()) return std::nullopt;
    return idle_.begin()->second;
}

// radix.hpp:113-117
bool PrefixTree::evict_one() {
    if (idle_.empty()) return false;
    Node& victim = at(idle_.begin()->second);
    Node& parent = at(victim.parent);
    // the parent becomes a leaf: its index entry is made first (the only
    // allocation here) and taken back if the victim's snapshot cannot be
    // released (a handle gone stale outside the tree), which leaves the
    // victim in place as the reference does
    const bool parent_idle = parent.id && parent.children == 1 && !parent.pins;
    if (parent_idle) idle_.emplace(parent.stamp, parent.id);
    try {
        release_snapshot(victim);
    } catch (...) {
        if (parent_idle) idle_.erase({parent.stamp, parent.id});
        throw;
    }
    edges_.erase({victim.parent, tokens_[victim.edge_at]});
    index_out(victim);
    --parent.children;
    victim.dead = true;
    --live_;
    live_tokens_ -= victim.edge_len;
    compact();
    return true;
}

// radix.hpp:119-123: snapshots are released in ascending node id order; ids
// keep counting from where they were
void PrefixTree::reset() {
    for (const Node& n : arena_)
        if (!n.dead && n.id && n.pins) throw std::logic_error("cannot reset pinned prefix nodes");
    for (Node& n : arena_)
        if (!n.dead) release_snapshot(n);
    arena_.erase(arena_.begin() + 1, arena_.end());
    arena_.front().children = 0;
    arena_.front().stamp = 0;
    tokens_.clear();
    edges_.clear();
    idle_.clear();
    live_ = 1;
    live_tokens_ = 0;
    clock_ = 0;
}

// --------------------------------------------------------------- queries

PrefixTree::NodeInfo PrefixTree::node(uint64_t id) const {
    const Node& n = at(id);
    NodeInfo info;
    info.parent = n.parent;
    info.edge = tokens_.data() + n.edge_at;
    info.edge_length = n.edge_len;
    info.pins = n.pins;
    info.accessed = n.stamp;
    info.kv = n.kv ? &*n.kv : nullptr;
    info.children = n.children;
    return info;
}

}  // namespace tvara_amd
