// Host bookkeeping of the paged KV cache, with no device code: the block
// pool's free list, reference counts and generations (BlockPool,
// core/include/tvara/kv.hpp:36-75) and the sequences' block tables
// (PagedCache, kv.hpp:78-165).  An append is planned here as a list of block
// operations (zero-fill, whole-block copy, row write) that the device cache
// then runs as kernels; nothing in this file touches block bytes, so it builds
// with any C++20 compiler (the sanitizer and failure-injection tests build it
// with g++).
#pragma once

#include <cstddef>
#include <cstdint>
#include <exception>
#include <memory>
#include <stdexcept>
#include <vector>

namespace tvara_amd {

// tvara::CacheExhausted (kv.hpp:34)
struct CacheExhausted : std::runtime_error {
    CacheExhausted() : std::runtime_error("KV cache exhausted") {}
};

// CacheGeometry (kv.hpp:12-29)
struct Geometry {
    size_t layers = 1, kv_heads = 1, head_dim = 4, tokens_per_block = 16, max_blocks = 64;
    size_t kv_width() const;
    size_t elements_per_block() const;
    void validate() const;
};

// BlockHandle (kv.hpp:35)
struct Handle {
    size_t id = 0;
    uint64_t generation = 0;
};

// BlockTable (kv.hpp:77)
struct Table {
    std::vector<Handle> blocks;
    size_t length = 0;
};

// Sequence id -> block table.  An append batch looks up every listed
// sequence, so this is open addressing with linear probing over a power-of-two
// array and a multiplicative hash (no division per lookup).  Ids are never 0
// (the first is 1) nor ~0 (an exhausted counter throws first), which mark
// empty and erased slots.  Tables sit behind unique_ptr, so a reference stays
// valid while other sequences are added or erased.
class SequenceMap {
public:
    SequenceMap() { rehash(64); }
    Table* find(uint64_t id) const;
    Table& insert(uint64_t id, Table&& t);  // id must not be present
    bool erase(uint64_t id);
    size_t size() const { return size_; }
    template <class F>
    void for_each(F&& f) const {
        for (size_t i = 0; i < keys_.size(); ++i)
            if (keys_[i] != kEmpty && keys_[i] != kErased) f(keys_[i], *vals_[i]);
    }

private:
    static constexpr uint64_t kEmpty = 0, kErased = ~uint64_t(0);
    size_t home(uint64_t id) const { return static_cast<size_t>((id * 0x9E3779B97F4A7C15ull) >> shift_); }
    void rehash(size_t capacity);

    std::vector<uint64_t> keys_;
    std::vector<std::unique_ptr<Table>> vals_;
    size_t size_ = 0, used_ = 0;  // live slots; live + erased slots
    int shift_ = 64;
};

// Block initialisation: zero-fill (src < 0, BlockPool::allocate, kv.hpp:48)
// or whole-block copy (copy-on-write, kv.hpp:99).
struct BlockInitOp {
    int64_t dst;
    int64_t src;
};

// One appended token: destination block, slot and the row of the input.
struct RowOp {
    int32_t block;
    int32_t slot;
    int32_t src_row;
    int32_t pad;
};

// The block work of a batch of appends, in the order it must run: every
// init op (zero-fills of new blocks, copy-on-write copies) before every row
// write.  `applied` appends took effect; `failure` is the error of the next
// one, which changed nothing.
struct AppendWork {
    std::vector<BlockInitOp> init;
    std::vector<RowOp> rows;
    size_t applied = 0;
    std::exception_ptr failure;
};

class KvLedger {
public:
    explicit KvLedger(const Geometry& g);

    const Geometry& geometry() const { return g_; }
    // bumped by every change of the pool or the tables; plans built against
    // one value are stale once it moves
    uint64_t epoch() const { return epoch_; }

    // ---- BlockPool (kv.hpp:36-75)
    Handle allocate();  // take_free() plus a queued zero-fill (kv.hpp:48)
    void retain(Handle h);
    void release(Handle h);
    size_t references(Handle h) const;
    size_t references_by_id(size_t id) const;
    size_t available() const { return free_.size(); }
    void pool_audit() const;
    void pool_state(size_t* refs, uint64_t* generations, size_t* free_pop_order, size_t* free_count) const;
    // BlockPool::data's handle check (kv.hpp:68-72)
    void check_live(Handle h) const;
    // blocks handed out by allocate() whose zero-fill has not run and that are
    // still live; the queue is emptied
    std::vector<int64_t> take_pending_zero_fills();

    // ---- PagedCache (kv.hpp:78-165)
    uint64_t create_sequence();
    const Table& sequence(uint64_t id) const;
    std::vector<uint64_t> sequence_ids() const;
    Handle physical_block(uint64_t id, size_t position) const;
    // appends one token to each listed sequence in order (append,
    // kv.hpp:91-108), stopping at the first that fails
    AppendWork plan_appends(const uint64_t* seqs, size_t n);
    void drop(uint64_t id);
    uint64_t fork(uint64_t id);
    void truncate(uint64_t id, size_t length);
    void audit(const size_t* external, size_t count) const;
    uint64_t import_sequence(const Handle* blocks, size_t count, size_t source_length, size_t length);

private:
    Handle take_free();  // pop the free list: refs = 1, ++generation
    Table& mutable_sequence(uint64_t id);
    uint64_t publish(const Handle* blocks, size_t count, size_t length);

    Geometry g_;
    uint64_t epoch_ = 0;
    std::vector<size_t> refs_;
    std::vector<uint64_t> gens_;
    std::vector<size_t> free_;  // popped from the back
    std::vector<uint8_t> zero_pending_;
    std::vector<size_t> zero_list_;
    size_t slot_mask_ = 0;  // tokens_per_block - 1 when it is a power of two
    size_t max_tokens_ = 0;
    SequenceMap sequences_;  // sequence_ids() sorts: the reference's std::map order
    uint64_t next_ = 0;
};

}  // namespace tvara_amd
