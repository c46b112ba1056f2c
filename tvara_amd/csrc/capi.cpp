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

// ModelConfig::validate (model.hpp:13-19), the part attention depends on
void check_config(const DeviceCache& c, size_t heads, size_t context) {
    const Geometry& g = c.geometry();
    if (!heads || !context || heads % g.kv_heads || g.head_dim % 2 || heads > 65535)
        throw std::invalid_argument("invalid native model configuration");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Rows of fused_paged_attention calls (attention.hpp:57-83) for `count`
// sequences: the argument checks of attention.hpp:59-63 and the visible cap.
void decode_rows(const DeviceCache& c, const uint64_t* seqs, size_t count, size_t context, bool tail,
                 const size_t* visible, std::vector<uint64_t>& seq_of_row, std::vector<size_t>& cached,
                 std::vector<uint8_t>& tail_rows) {
    for (size_t i = 0; i < count; ++i) {
        const size_t length = c.sequence(seqs[i]).length;
        if (length > context || (tail && length == context)) throw std::invalid_argument("invalid fused attention shape");
        const size_t total = length + (tail ? 1 : 0);
        const size_t vis = visible ? std::min(visible[i], total) : total;
        if (!vis) throw std::invalid_argument("empty fused attention");
        if (length > static_cast<size_t>(std::numeric_limits<int32_t>::max()))
            throw std::invalid_argument("sequence too long for the device kernels");
        seq_of_row.push_back(seqs[i]);
        cached.push_back(std::min(vis, length));
        tail_rows.push_back(vis > length ? 1 : 0);
    }
}

// device copies of host arrays for the synchronous attention entry points
struct Staged {
    std::vector<void*> owned;
    ~Staged() {
        for (void* p : owned) (void)hipFree(p);
    }
    const float* in(const float* host, size_t n) {
        if (!host) return nullptr;
        void* d = nullptr;
        TVARA_HIP(hipMalloc(&d, std::max<size_t>(n, 1) * sizeof(float)));
        owned.push_back(d);
        TVARA_HIP(hipMemcpy(d, host, n * sizeof(float), hipMemcpyHostToDevice));
        return static_cast<const float*>(d);
    }
    float* out(size_t n) {
        void* d = nullptr;
        TVARA_HIP(hipMalloc(&d, std::max<size_t>(n, 1) * sizeof(float)));
        owned.push_back(d);
        return static_cast<float*>(d);
    }
};
}  // namespace

tvara_amd::KvLedger& tvara_amd::abi::ledger_of(tvara_kv_cache* cache) { return live(cache).ledger(); }

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
        check_config(c, heads, context);
        if (!count) return;
        if (!sequences || !q || !out || (tail_keys == nullptr) != (tail_values == nullptr))
            throw std::invalid_argument("invalid fused attention shape");
        if (layer >= c.geometry().layers) throw std::invalid_argument("invalid fused attention shape");
        const bool tail = tail_keys != nullptr;
        std::vector<uint64_t> seq_of_row;
        std::vector<size_t> cached;
        std::vector<uint8_t> tails;
        decode_rows(c, sequences, count, context, tail, visible, seq_of_row, cached, tails);
        AttnPlan plan;
        plan.build(&c, seq_of_row, cached, tails, static_cast<int>(heads), 0);
        const size_t hidden = heads * c.geometry().head_dim, kvw = c.geometry().kv_width();
        if (device_ptrs) {
            if (!aligned16(q) || !aligned16(out) || (tail && (!aligned16(tail_keys) || !aligned16(tail_values))))
                throw std::invalid_argument("device buffers must be 16-byte aligned");
            plan.launch(static_cast<int>(layer), q, tail_keys, tail_values, out, c.stream());
            plan.check();
            return;
        }
        Staged st;
        const float* dq = st.in(q, count * hidden);
        const float* dk = st.in(tail_keys, count * kvw);
        const float* dv = st.in(tail_values, count * kvw);
        float* dout = st.out(count * hidden);
        plan.launch(static_cast<int>(layer), dq, dk, dv, dout, c.stream());
        plan.check();
        TVARA_HIP(hipMemcpy(out, dout, count * hidden * sizeof(float), hipMemcpyDeviceToHost));
    });
}

int tvara_attn_prefill(tvara_kv_cache* cache, const uint64_t* sequences, size_t count, size_t layer, size_t heads,
                       size_t context, const size_t* start, const size_t* rows, const float* queries, float* out,
                       int precision, int device_ptrs) {
    return guard([&] {
        auto& c = live(cache);
        check_config(c, heads, context);
        if (!count) return;
        if (!sequences || !start || !rows || !queries || !out) throw std::invalid_argument("invalid causal prompt chunk");
        if (layer >= c.geometry().layers) throw std::invalid_argument("invalid fused attention shape");
        if (precision != TVARA_ATTN_F32 && precision != TVARA_ATTN_BF16)
            throw std::invalid_argument("unknown attention precision");
        tvara_amd::PrefillPlan plan;
        plan.build(&c, sequences, count, heads, context, start, rows, precision);
        const size_t total_rows = plan.total_rows;
        const size_t hidden = heads * c.geometry().head_dim;
        if (device_ptrs && (!aligned16(queries) || !aligned16(out)))
            throw std::invalid_argument("device buffers must be 16-byte aligned");
        Staged st;
        const float* dq = device_ptrs ? queries : st.in(queries, total_rows * hidden);
        float* dout = device_ptrs ? out : st.out(total_rows * hidden);
        plan.launch(static_cast<int>(layer), dq, dout, c.stream());
        plan.check();
        if (!device_ptrs)
            TVARA_HIP(hipMemcpy(out, dout, total_rows * hidden * sizeof(float), hipMemcpyDeviceToHost));
        else
            c.synchronize();
    });
}

tvara_attn_plan* tvara_attn_plan_create(tvara_kv_cache* cache, const uint64_t* sequences, size_t count, size_t heads,
                                        size_t context, const size_t* visible, int with_tail) {
    tvara_attn_plan* out = nullptr;
    guard([&] {
        auto& c = live(cache);
        check_config(c, heads, context);
        if (!count || !sequences) throw std::invalid_argument("empty attention plan");
        std::vector<uint64_t> seq_of_row;
        std::vector<size_t> cached;
        std::vector<uint8_t> tails;
        decode_rows(c, sequences, count, context, with_tail != 0, visible, seq_of_row, cached, tails);
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
        check_config(c, heads, context);
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
        try {
            for (size_t i = 0; i < token_count; ++i) model->model->decode(sequence, tokens[i], logits + i * vocab);
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
