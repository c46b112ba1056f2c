// Exported C ABI of libtvara_capi (declared in include/tvara_capi.h).  Error
// convention of core/src/c_api.cpp:66-107: each call clears a thread-local
// message, catches every exception and returns a status naming its class.
#include "tvara_capi.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "abi.hpp"
#include "host_copy.hpp"
#include "kv_cache.hpp"
#include "model.hpp"

using tvara_amd::AttnPlan;
using tvara_amd::DeviceCache;
using tvara_amd::Geometry;
using tvara_amd::Handle;

// a cache handle either owns its DeviceCache (tvara_kv_cache_create) or lends
// a model's (tvara_model_cache; destroying that handle does nothing)
struct tvara_kv_cache {
    std::unique_ptr<DeviceCache> owned;
    DeviceCache* cache = nullptr;
    // The synchronous attention calls keep their last plan and reuse it while
    // the cache and the call's rows are unchanged (a model's layers share one
    // batch), and stage host buffers through pinned memory into grow-only
    // device buffers: no allocation and no device-wide wait per call.
    std::vector<uint64_t> decode_key, prefill_key;
    AttnPlan decode_plan;
    tvara_amd::PrefillPlan prefill_plan;
    tvara_amd::DeviceBuffer io;
    tvara_amd::PinnedBuffer io_in, io_out;
    tvara_kv_cache(const Geometry& g, int format)
        : owned(std::make_unique<DeviceCache>(g, format)), cache(owned.get()) {}
    explicit tvara_kv_cache(DeviceCache* lent) : cache(lent) {}
};

struct tvara_attn_plan {
    AttnPlan plan;
    size_t context = 0;
};

// the handle of the model-level exports (c_api.cpp:6-13): the executor and one
// mutex held for every call that touches sequences
struct tvara_model {
    std::unique_ptr<tvara_amd::DeviceModel> model;
    std::unique_ptr<tvara_kv_cache> kv;  // the model's cache, lent as a KV handle
    std::mutex mutex;
};

struct tvara_prefill_plan {
    tvara_amd::PrefillPlan plan;
};

namespace tvara_amd {
void profile_enable(bool on);
void profile_read(const char* prefix, double* ms, size_t* launches);
void profile_reset();
}  // namespace tvara_amd

using tvara_amd::abi::exported;
using tvara_amd::abi::failed;
using tvara_amd::abi::guard;
using tvara_amd::abi::handle;

namespace {
DeviceCache& live(tvara_kv_cache* c) {
    if (!c) throw std::invalid_argument("closed KV cache");
    return *c->cache;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// the identity of a synchronous attention call's plan: the cache's mutation
// count and every argument the plan depends on
std::vector<uint64_t> plan_key(const DeviceCache& c, std::initializer_list<uint64_t> scalars, const uint64_t* seqs,
                               size_t count, const size_t* a, const size_t* b) {
    std::vector<uint64_t> key{c.epoch(), count};
    key.insert(key.end(), scalars);
    key.insert(key.end(), seqs, seqs + count);
    key.push_back(a ? 1 : 0);
    if (a) key.insert(key.end(), a, a + count);
    if (b) key.insert(key.end(), b, b + count);
    return key;
}
}  // namespace

tvara_amd::KvLedger& tvara_amd::abi::ledger_of(tvara_kv_cache* cache) { return live(cache).ledger(); }
tvara_amd::DeviceCache& tvara_amd::device_cache(tvara_kv_cache* cache) { return live(cache); }

extern "C" {

tvara_kv_cache* tvara_kv_cache_create(size_t layers, size_t kv_heads, size_t head_dim, size_t tokens_per_block,
                                      size_t max_blocks, int format) {
    tvara_kv_cache* out = nullptr;
    guard([&] {
        Geometry g{layers, kv_heads, head_dim, tokens_per_block, max_blocks};
        out = new tvara_kv_cache(g, format);
    });
    return out;
}

void tvara_kv_cache_destroy(tvara_kv_cache* cache) {
    if (cache && cache->owned) delete cache;  // a lent handle belongs to its model
}

size_t tvara_kv_block_bytes(tvara_kv_cache* cache) {
    size_t n = 0;
    guard([&] { n = live(cache).canonical_block_bytes(); });
    return n;
}

int tvara_kv_set_stream(tvara_kv_cache* cache, void* stream) {
    return guard([&] { live(cache).set_stream(static_cast<hipStream_t>(stream)); });
}

int tvara_kv_synchronize(tvara_kv_cache* cache) {
    return guard([&] {
        live(cache).flush();
        live(cache).synchronize();
    });
}

int tvara_kv_block_read(tvara_kv_cache* cache, tvara_kv_handle h, void* out, size_t bytes) {
    return guard([&] { live(cache).block_read(handle(h), out, bytes); });
}

int tvara_kv_block_write(tvara_kv_cache* cache, tvara_kv_handle h, size_t offset, const void* data, size_t bytes) {
    return guard([&] { live(cache).block_write(handle(h), offset, data, bytes); });
}

int tvara_kv_block_checksums(tvara_kv_cache* cache, const tvara_kv_handle* handles, size_t count, uint64_t* out) {
    return guard([&] {
        if (count && (!handles || !out)) throw std::invalid_argument("null checksum buffers");
        std::vector<Handle> hs(count);
        for (size_t i = 0; i < count; ++i) hs[i] = handle(handles[i]);
        live(cache).checksums(hs.data(), count, out);
    });
}

int tvara_kv_append(tvara_kv_cache* cache, uint64_t sequence, const float* keys, const float* values) {
    return guard([&] { live(cache).append_batch(&sequence, 1, keys, values, false); });
}

int tvara_kv_append_batch(tvara_kv_cache* cache, const uint64_t* sequences, size_t count, const float* keys,
                          const float* values, int device_ptrs, size_t* applied) {
    size_t done = 0;
    const int rc = guard([&] { live(cache).append_batch(sequences, count, keys, values, device_ptrs != 0, &done); });
    if (applied) *applied = done;
    return rc;
}

int tvara_kv_append_tokens(tvara_kv_cache* cache, uint64_t sequence, const float* keys, const float* values,
                           size_t count, int device_ptrs, size_t* applied) {
    return tvara_kv_append_batch(cache, std::vector<uint64_t>(count, sequence).data(), count, keys, values,
                                 device_ptrs, applied);
}

int tvara_kv_read(tvara_kv_cache* cache, uint64_t sequence, size_t layer, size_t position, int value, float* out) {
    return guard([&] {
        if (!out) throw std::invalid_argument("null output");
        live(cache).read(sequence, layer, position, value != 0, out);
    });
}

int tvara_kv_read_all(tvara_kv_cache* cache, uint64_t sequence, size_t layer, int value, float* out,
                      size_t capacity) {
    return guard([&] { live(cache).read_all(sequence, layer, value != 0, out, out ? capacity : 0); });
}

int tvara_attn_decode(tvara_kv_cache* cache, const uint64_t* sequences, size_t count, size_t layer, size_t heads,
                      size_t context, const float* q, const float* tail_keys, const float* tail_values,
                      const size_t* visible, float* out, int device_ptrs) {
    return guard([&] {
        auto& c = live(cache);
        tvara_amd::check_attention_config(c, heads, context);
        if (!count) return;
        if (!sequences || !q || !out || (tail_keys == nullptr) != (tail_values == nullptr))
            throw std::invalid_argument("invalid fused attention shape");
        if (layer >= c.geometry().layers) throw std::invalid_argument("invalid fused attention shape");
        const bool tail = tail_keys != nullptr;
        std::vector<uint64_t> seq_of_row;
        std::vector<size_t> cached;
        std::vector<uint8_t> tails;
        tvara_amd::attention_rows(c, sequences, count, context, tail, visible, seq_of_row, cached, tails);
        AttnPlan& plan = cache->decode_plan;
        std::vector<uint64_t> key = plan_key(c, {heads, tail ? 1u : 0u}, sequences, count, visible, nullptr);
        if (key != cache->decode_key || plan.cache != &c) {
            cache->decode_key.clear();
            plan.build(&c, seq_of_row, cached, tails, static_cast<int>(heads), 0);
            cache->decode_key = std::move(key);
        }
        const size_t hidden = heads * c.geometry().head_dim, kvw = c.geometry().kv_width();
        hipStream_t s = c.stream();
        if (device_ptrs) {
            if (!aligned16(q) || !aligned16(out) || (tail && (!aligned16(tail_keys) || !aligned16(tail_values))))
                throw std::invalid_argument("device buffers must be 16-byte aligned");
            plan.launch(static_cast<int>(layer), q, tail_keys, tail_values, out, s);
            plan.check();
            return;
        }
        // q | tail keys | tail values in one pinned buffer and one copy in;
        // the kernels write the output (and the error flag) straight into
        // pinned host memory, so the call waits for the stream once and no
        // copy comes back
        const size_t nq = count * hidden, nt = tail ? count * kvw : 0;
        tvara_amd::HostCopier& copier = tvara_amd::HostCopier::shared();
        std::lock_guard<std::mutex> hold(copier.lock());
        auto* in = static_cast<float*>(cache->io_in.acquire((nq + 2 * nt) * sizeof(float)));
        auto stage = [&](float* to, const float* from, size_t n) {
            copier.parallel_copy(reinterpret_cast<char*>(to), reinterpret_cast<const char*>(from), n * sizeof(float));
        };
        stage(in, q, nq);
        if (tail) {
            stage(in + nq, tail_keys, nt);
            stage(in + nq + nt, tail_values, nt);
        }
        auto* d = static_cast<float*>(cache->io.ensure((nq + 2 * nt) * sizeof(float)));
        TVARA_HIP(hipMemcpyAsync(d, in, (nq + 2 * nt) * sizeof(float), hipMemcpyHostToDevice, s));
        cache->io_in.release(s);
        auto* back = static_cast<float*>(cache->io_out.acquire(nq * sizeof(float)));
        plan.launch(static_cast<int>(layer), d, tail ? d + nq : nullptr, tail ? d + nq + nt : nullptr, back, s);
        plan.queue_check();
        TVARA_HIP(hipStreamSynchronize(s));
        plan.finish_check();
        stage(out, back, nq);
    });
}

int tvara_attn_prefill(tvara_kv_cache* cache, const uint64_t* sequences, size_t count, size_t layer, size_t heads,
                       size_t context, const size_t* start, const size_t* rows, const float* queries, float* out,
                       int precision, int device_ptrs) {
    return guard([&] {
        auto& c = live(cache);
        tvara_amd::check_attention_config(c, heads, context);
        if (!count) return;
        if (!sequences || !start || !rows || !queries || !out) throw std::invalid_argument("invalid causal prompt chunk");
        if (layer >= c.geometry().layers) throw std::invalid_argument("invalid fused attention shape");
        if (precision != TVARA_ATTN_F32 && precision != TVARA_ATTN_BF16 && precision != TVARA_ATTN_F32X3)
            throw std::invalid_argument("unknown attention precision");
        tvara_amd::PrefillPlan& plan = cache->prefill_plan;
        std::vector<uint64_t> key =
            plan_key(c, {heads, context, static_cast<uint64_t>(precision)}, sequences, count, start, rows);
        if (key != cache->prefill_key || plan.cache != &c) {
            cache->prefill_key.clear();
            plan.build(&c, sequences, count, heads, context, start, rows, precision);
            cache->prefill_key = std::move(key);
        }
        const size_t n = plan.total_rows * heads * c.geometry().head_dim;
        hipStream_t s = c.stream();
        if (device_ptrs) {
            if (!aligned16(queries) || !aligned16(out)) throw std::invalid_argument("device buffers must be 16-byte aligned");
            plan.launch(static_cast<int>(layer), queries, out, s);
            plan.check();
            return;
        }
        tvara_amd::HostCopier& copier = tvara_amd::HostCopier::shared();
        std::lock_guard<std::mutex> hold(copier.lock());
        auto* in = static_cast<float*>(cache->io_in.acquire(n * sizeof(float)));
        copier.parallel_copy(reinterpret_cast<char*>(in), reinterpret_cast<const char*>(queries), n * sizeof(float));
        const size_t out_at = (n + 3) / 4 * 4;
        auto* d = static_cast<float*>(cache->io.ensure((out_at + n) * sizeof(float)));
        TVARA_HIP(hipMemcpyAsync(d, in, n * sizeof(float), hipMemcpyHostToDevice, s));
        cache->io_in.release(s);
        plan.launch(static_cast<int>(layer), d, d + out_at, s);
        auto* back = static_cast<float*>(cache->io_out.acquire(n * sizeof(float)));
        TVARA_HIP(hipMemcpyAsync(back, d + out_at, n * sizeof(float), hipMemcpyDeviceToHost, s));
        plan.check();
        copier.parallel_copy(reinterpret_cast<char*>(out), reinterpret_cast<const char*>(back), n * sizeof(float));
    });
}

tvara_attn_plan* tvara_attn_plan_create(tvara_kv_cache* cache, const uint64_t* sequences, size_t count, size_t heads,
                                        size_t context, const size_t* visible, int with_tail) {
    tvara_attn_plan* out = nullptr;
    guard([&] {
        auto& c = live(cache);
        tvara_amd::check_attention_config(c, heads, context);
        if (!count || !sequences) throw std::invalid_argument("empty attention plan");
        std::vector<uint64_t> seq_of_row;
        std::vector<size_t> cached;
        std::vector<uint8_t> tails;
        tvara_amd::attention_rows(c, sequences, count, context, with_tail != 0, visible, seq_of_row, cached, tails);
        auto p = std::make_unique<tvara_attn_plan>();
        p->context = context;
        p->plan.build(&c, seq_of_row, cached, tails, static_cast<int>(heads), 0);
        out = p.release();
    });
    return out;
}

int tvara_attn_plan_decode(tvara_attn_plan* plan, size_t layer, const float* q, const float* tail_keys,
                           const float* tail_values, float* out, void* stream) {
    return guard([&] {
        if (!plan) throw std::invalid_argument("null attention plan");
        if (!q || !out || !aligned16(q) || !aligned16(out)) throw std::invalid_argument("device buffers must be 16-byte aligned");
        if ((tail_keys && !aligned16(tail_keys)) || (tail_values && !aligned16(tail_values)))
            throw std::invalid_argument("device buffers must be 16-byte aligned");
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : plan->plan.cache->stream();
        plan->plan.launch(static_cast<int>(layer), q, tail_keys, tail_values, out, s);
    });
}

int tvara_attn_plan_check(tvara_attn_plan* plan) {
    return guard([&] {
        if (!plan) throw std::invalid_argument("null attention plan");
        plan->plan.check();
    });
}

int tvara_attn_plan_info(tvara_attn_plan* plan, size_t* split_tokens, size_t* items, size_t* kv_bytes) {
    return guard([&] {
        if (!plan) throw std::invalid_argument("null attention plan");
        if (split_tokens) *split_tokens = static_cast<size_t>(plan->plan.split_tokens);
        if (items) *items = static_cast<size_t>(plan->plan.items);
        if (kv_bytes) *kv_bytes = plan->plan.kv_bytes;
    });
}

void tvara_attn_plan_destroy(tvara_attn_plan* plan) { delete plan; }

tvara_prefill_plan* tvara_prefill_plan_create(tvara_kv_cache* cache, const uint64_t* sequences, size_t count,
                                              size_t heads, size_t context, const size_t* start, const size_t* rows,
                                              int precision) {
    tvara_prefill_plan* out = nullptr;
    guard([&] {
        auto& c = live(cache);
        tvara_amd::check_attention_config(c, heads, context);
        auto p = std::make_unique<tvara_prefill_plan>();
        p->plan.build(&c, sequences, count, heads, context, start, rows, precision);
        out = p.release();
    });
    return out;
}

int tvara_prefill_plan_launch(tvara_prefill_plan* plan, size_t layer, const float* queries, float* out, void* stream) {
    return guard([&] {
        if (!plan) throw std::invalid_argument("null attention plan");
        if (!queries || !out || !aligned16(queries) || !aligned16(out))
            throw std::invalid_argument("device buffers must be 16-byte aligned");
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : plan->plan.cache->stream();
        plan->plan.launch(static_cast<int>(layer), queries, out, s);
    });
}

int tvara_prefill_plan_check(tvara_prefill_plan* plan) {
    return guard([&] {
        if (!plan) throw std::invalid_argument("null attention plan");
        plan->plan.check();
    });
}

void tvara_prefill_plan_destroy(tvara_prefill_plan* plan) { delete plan; }

// ------------------------------------------------------- model-level exports
// c_api.cpp:35-78: return conventions (nullptr / 0 / -1), messages and the
// per-handle lock are the reference's.

tvara_model* tvara_model_open(const char* path, size_t blocks, size_t tokens) {
    tvara_amd::abi::clear();
    try {
        if (!path || !*path) throw std::invalid_argument("empty model path");
        auto m = std::make_unique<tvara_model>();
        m->model = std::make_unique<tvara_amd::DeviceModel>(path, blocks, tokens);
        m->kv = std::make_unique<tvara_kv_cache>(&m->model->cache());
        return m.release();
    } catch (const std::exception& e) {
        failed(TVARA_ERROR, e.what());
        return nullptr;
    } catch (...) {
        failed(TVARA_ERROR, "unknown native error");
        return nullptr;
    }
}

void tvara_model_close(tvara_model* model) { delete model; }

size_t tvara_model_vocab_size(tvara_model* model) {
    if (!model) {
        failed(TVARA_ERROR, "closed model");
        return 0;
    }
    return model->model->config().vocab;
}

size_t tvara_model_context_size(tvara_model* model) {
    if (!model) {
        failed(TVARA_ERROR, "closed model");
        return 0;
    }
    return model->model->config().context;
}

const char* tvara_model_metadata(tvara_model* model) {
    if (!model) {
        failed(TVARA_ERROR, "closed model");
        return nullptr;
    }
    return model->model->metadata().c_str();
}

uint64_t tvara_sequence_create(tvara_model* model) {
    tvara_amd::abi::clear();
    try {
        if (!model) throw std::invalid_argument("closed model");
        std::lock_guard<std::mutex> lock(model->mutex);
        return model->model->cache().create_sequence();
    } catch (const std::exception& e) {
        failed(TVARA_ERROR, e.what());
        return 0;
    } catch (...) {
        failed(TVARA_ERROR, "unknown native error");
        return 0;
    }
}

int tvara_sequence_decode(tvara_model* model, uint64_t sequence, uint32_t token, float* logits, size_t count) {
    tvara_amd::abi::clear();
    try {
        if (!model || !logits || count != model->model->config().vocab)
            throw std::invalid_argument("invalid logit output buffer");
        std::lock_guard<std::mutex> lock(model->mutex);
        model->model->decode(sequence, token, logits);
        return 0;
    } catch (const std::exception& e) {
        failed(TVARA_ERROR, e.what());
        return -1;
    } catch (...) {
        failed(TVARA_ERROR, "unknown native error");
        return -1;
    }
}

int tvara_sequence_drop(tvara_model* model, uint64_t sequence) {
    tvara_amd::abi::clear();
    try {
        if (!model) throw std::invalid_argument("closed model");
        std::lock_guard<std::mutex> lock(model->mutex);
        model->model->cache().drop(sequence);
        return 0;
    } catch (const std::exception& e) {
        failed(TVARA_ERROR, e.what());
        return -1;
    } catch (...) {
        failed(TVARA_ERROR, "unknown native error");
        return -1;
    }
}

int tvara_sequence_decode_batch(tvara_model* model, uint64_t sequence, const uint32_t* tokens, size_t token_count,
                                float* logits, size_t count) {
    tvara_amd::abi::clear();
    try {
        if (!model || (!tokens && token_count) || (!logits && count)) throw std::invalid_argument("invalid batch buffers");
        const size_t vocab = model->model->config().vocab;
        if (token_count > std::numeric_limits<size_t>::max() / vocab || count != token_count * vocab)
            throw std::invalid_argument("invalid batch dimensions");
        std::lock_guard<std::mutex> lock(model->mutex);
        auto& cache = model->model->cache();
        const size_t length = cache.sequence(sequence).length;
        if (token_count > model->model->config().context - length) throw std::invalid_argument("batch exceeds context");
        for (size_t i = 0; i < token_count; ++i)
            if (tokens[i] >= vocab) throw std::invalid_argument("invalid batch token");
        // the reference decodes token by token (c_api.cpp:68); the chunk pass
        // gives the same logits with every weight row read once per chunk
        try {
            model->model->decode_chunk(sequence, tokens, token_count, logits, false);
        } catch (...) {
            cache.truncate(sequence, length);  // no partial batch stays in the cache (c_api.cpp:68-70)
            throw;
        }
        return 0;
    } catch (const std::exception& e) {
        failed(TVARA_ERROR, e.what());
        return -1;
    } catch (...) {
        failed(TVARA_ERROR, "unknown batch error");
        return -1;
    }
}

int tvara_sequence_prefill(tvara_model* model, uint64_t sequence, const uint32_t* tokens, size_t token_count,
                           float* logits, size_t count) {
    tvara_amd::abi::clear();
    try {
        if (!model || (!tokens && token_count) || !logits) throw std::invalid_argument("invalid batch buffers");
        const size_t vocab = model->model->config().vocab;
        if (!token_count || count != vocab) throw std::invalid_argument("invalid batch dimensions");
        std::lock_guard<std::mutex> lock(model->mutex);
        auto& cache = model->model->cache();
        const size_t length = cache.sequence(sequence).length;
        if (token_count > model->model->config().context - length) throw std::invalid_argument("batch exceeds context");
        for (size_t i = 0; i < token_count; ++i)
            if (tokens[i] >= vocab) throw std::invalid_argument("invalid batch token");
        try {
            model->model->decode_chunk(sequence, tokens, token_count, logits, true);
        } catch (...) {
            cache.truncate(sequence, length);
            throw;
        }
        return 0;
    } catch (const std::exception& e) {
        failed(TVARA_ERROR, e.what());
        return -1;
    } catch (...) {
        failed(TVARA_ERROR, "unknown batch error");
        return -1;
    }
}

int tvara_sequence_truncate(tvara_model* model, uint64_t sequence, size_t length) {
    tvara_amd::abi::clear();
    try {
        if (!model) throw std::invalid_argument("closed model");
        std::lock_guard<std::mutex> lock(model->mutex);
        model->model->cache().truncate(sequence, length);
        return 0;
    } catch (const std::exception& e) {
        failed(TVARA_ERROR, e.what());
        return -1;
    } catch (...) {
        failed(TVARA_ERROR, "unknown truncate error");
        return -1;
    }
}

int tvara_sequences_decode(tvara_model* model, const uint64_t* sequences, const uint32_t* tokens, size_t count,
                           float* logits, size_t logits_count) {
    tvara_amd::abi::clear();
    try {
        if (!model || (count && (!sequences || !tokens || !logits))) throw std::invalid_argument("invalid batch buffers");
        const size_t vocab = model->model->config().vocab;
        if (count > std::numeric_limits<size_t>::max() / vocab || logits_count != count * vocab)
            throw std::invalid_argument("invalid batch dimensions");
        std::lock_guard<std::mutex> lock(model->mutex);
        if (count == 1)
            model->model->decode(sequences[0], tokens[0], logits);
        else
            model->model->decode_many(sequences, tokens, count, logits);
        return 0;
    } catch (const std::exception& e) {
        failed(TVARA_ERROR, e.what());
        return -1;
    } catch (...) {
        failed(TVARA_ERROR, "unknown batch error");
        return -1;
    }
}

tvara_kv_cache* tvara_model_cache(tvara_model* model) {
    if (!model) {
        failed(TVARA_INVALID, "closed model");
        return nullptr;
    }
    return model->kv.get();
}

int tvara_profile_enable(int enabled) {
    return guard([&] { tvara_amd::profile_enable(enabled != 0); });
}

int tvara_profile_read(const char* kernel, double* milliseconds, size_t* launches) {
    return guard([&] {
        double ms = 0;
        size_t n = 0;
        tvara_amd::profile_read(kernel, &ms, &n);
        if (milliseconds) *milliseconds = ms;
        if (launches) *launches = n;
    });
}

int tvara_profile_reset(void) {
    return guard([&] { tvara_amd::profile_reset(); });
}

}  // extern "C"
