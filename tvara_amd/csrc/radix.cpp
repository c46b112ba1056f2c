// Prefix cache over the device KV pool (see radix.hpp).
#include "radix.hpp"

#include <limits>
#include <stdexcept>

namespace tvara_amd {

namespace {
size_t common_prefix(const std::vector<int32_t>& edge, const int32_t* tokens, size_t n) {
    size_t k = 0;
    while (k < edge.size() && k < n && edge[k] == tokens[k]) ++k;
    return k;
}
}  // namespace

RadixCache::RadixCache(DeviceCache& cache, std::string isolation) : cache_(cache), isolation_(std::move(isolation)) {
    if (isolation_.empty()) throw std::invalid_argument("prefix isolation key is required");
    nodes_.emplace(0, RadixNode{});
}

RadixCache::~RadixCache() {
    for (auto& [id, n] : nodes_) {
        (void)id;
        try {
            release_kv(n);
        } catch (...) {
        }
    }
}

const RadixNode& RadixCache::node(uint64_t id) const { return nodes_.at(id); }

void RadixCache::release_kv(RadixNode& n) {
    if (n.kv)
        for (const Handle& b : n.kv->blocks) cache_.release(b);
}

// radix.hpp:29-42: follow matching edges; a match that ends inside an edge
// still names that edge's node
std::pair<uint64_t, size_t> RadixCache::lookup(const int32_t* tokens, size_t n) const {
    uint64_t current = 0;
    size_t offset = 0;
    std::pair<uint64_t, size_t> result{0, 0};
    while (offset < n) {
        const RadixNode& parent = nodes_.at(current);
        auto it = parent.children.find(tokens[offset]);
        if (it == parent.children.end()) break;
        const RadixNode& child = nodes_.at(it->second);
        const size_t k = common_prefix(child.edge, tokens + offset, n - offset);
        offset += k;
        result = {child.id, offset};
        if (k != child.edge.size()) break;
        current = child.id;
    }
    return result;
}

// radix.hpp:44-69: a new leaf for an unmatched suffix; an edge matched only
// in part is split at the divergence (the new inner node takes the child's pins)
uint64_t RadixCache::insert(const int32_t* tokens, size_t n) {
    if (!n) throw std::invalid_argument("cannot cache empty prefix");
    uint64_t current = 0;
    size_t offset = 0;
    while (offset < n) {
        RadixNode& parent = nodes_.at(current);
        auto found = parent.children.find(tokens[offset]);
        if (found == parent.children.end()) {
            if (next_ == std::numeric_limits<uint64_t>::max()) throw std::overflow_error("radix ID exhausted");
            const uint64_t id = ++next_;
            RadixNode leaf;
            leaf.id = id;
            leaf.parent = current;
            leaf.edge.assign(tokens + offset, tokens + n);
            nodes_.emplace(id, std::move(leaf));
            parent.children.emplace(tokens[offset], id);
            return id;
        }
        RadixNode& child = nodes_.at(found->second);
        const size_t k = common_prefix(child.edge, tokens + offset, n - offset);
        if (k != child.edge.size()) {
            if (next_ == std::numeric_limits<uint64_t>::max()) throw std::overflow_error("radix ID exhausted");
            const uint64_t split = ++next_;
            RadixNode inner;
            inner.id = split;
            inner.parent = current;
            inner.pins = child.pins;
            inner.edge.assign(child.edge.begin(), child.edge.begin() + static_cast<std::ptrdiff_t>(k));
            child.edge.erase(child.edge.begin(), child.edge.begin() + static_cast<std::ptrdiff_t>(k));
            inner.children.emplace(child.edge.front(), child.id);
            child.parent = split;
            parent.children[tokens[offset]] = split;
            nodes_.emplace(split, std::move(inner));
            current = split;
            offset += k;
            continue;
        }
        current = child.id;
        offset += k;
    }
    return current;
}

// radix.hpp:72-81: the node keeps a retained snapshot of the sequence's table
void RadixCache::attach(uint64_t id, uint64_t sequence) {
    RadixNode& entry = nodes_.at(id);
    Table source = cache_.sequence(sequence);
    size_t depth = 0;
    for (uint64_t c = id; c; c = nodes_.at(c).parent) depth += nodes_.at(c).edge.size();
    if (source.length != depth) throw std::invalid_argument("token and KV prefix lengths differ");
    size_t retained = 0;
    try {
        for (const Handle& b : source.blocks) {
            cache_.retain(b);
            ++retained;
        }
    } catch (...) {
        for (size_t i = 0; i < retained; ++i) cache_.release(source.blocks[i]);
        throw;
    }
    release_kv(entry);
    entry.kv = std::move(source);
}

std::vector<size_t> RadixCache::external_references() const {
    std::vector<size_t> counts(cache_.geometry().max_blocks);
    for (const auto& [id, n] : nodes_) {
        (void)id;
        if (n.kv)
            for (const Handle& b : n.kv->blocks) ++counts.at(b.id);
    }
    return counts;
}

// radix.hpp:90-96: import the matched prefix (whole blocks unless partial)
std::pair<uint64_t, size_t> RadixCache::reuse(const int32_t* tokens, size_t n, bool partial) {
    const auto match = lookup(tokens, n);
    if (!match.first || !nodes_.at(match.first).kv) return {cache_.create_sequence(), 0};
    size_t length = match.second;
    if (!partial) length -= length % cache_.geometry().tokens_per_block;
    const Table& kv = *nodes_.at(match.first).kv;
    return {cache_.import_sequence(kv.blocks.data(), kv.blocks.size(), kv.length, length), length};
}

void RadixCache::pin(uint64_t id) {
    for (uint64_t c = id; c; c = nodes_.at(c).parent)
        if (nodes_.at(c).pins == std::numeric_limits<size_t>::max()) throw std::overflow_error("prefix pin overflow");
    for (uint64_t c = id; c; c = nodes_.at(c).parent) ++nodes_.at(c).pins;
}

void RadixCache::unpin(uint64_t id) {
    for (uint64_t c = id; c; c = nodes_.at(c).parent)
        if (!nodes_.at(c).pins) throw std::invalid_argument("prefix pin underflow");
    for (uint64_t c = id; c; c = nodes_.at(c).parent) --nodes_.at(c).pins;
}

void RadixCache::touch(uint64_t id) {
    RadixNode& entry = nodes_.at(id);
    if (clock_ == std::numeric_limits<uint64_t>::max()) throw std::overflow_error("prefix access clock exhausted");
    entry.accessed = ++clock_;
}

// least recently touched unpinned leaf; the lowest id among equals
std::optional<uint64_t> RadixCache::eviction_candidate() const {
    std::optional<uint64_t> best;
    for (const auto& [id, n] : nodes_)
        if (id && n.children.empty() && !n.pins && (!best || n.accessed < nodes_.at(*best).accessed)) best = id;
    return best;
}

bool RadixCache::evict_one() {
    const auto c = eviction_candidate();
    if (!c) return false;
    RadixNode& entry = nodes_.at(*c);
    release_kv(entry);
    nodes_.at(entry.parent).children.erase(entry.edge.front());
    nodes_.erase(*c);
    return true;
}

void RadixCache::reset() {
    for (const auto& [id, n] : nodes_)
        if (id && n.pins) throw std::logic_error("cannot reset pinned prefix nodes");
    for (auto& [id, n] : nodes_) {
        (void)id;
        release_kv(n);
    }
    nodes_.clear();
    nodes_.emplace(0, RadixNode{});
    clock_ = 0;
}

}  // namespace tvara_amd
