/*
 * tvara_capi.h -- C ABI of the MI355X paged KV cache and paged attention
 * library (libtvara_capi.so, hand-written HIP for gfx950).
 *
 * The reference exposes this path only through its in-process C++ API
 * (core/include/tvara/kv.hpp, core/include/tvara/attention.hpp); its C ABI
 * (core/include/tvara/c_api.h:13-24) reaches it through the model executor.
 * The entry points below are the additive exports that a Tvara build binds for
 * the path itself: each one names the reference interface it replaces.
 *
 * Conventions (mirroring core/src/c_api.cpp:66-107):
 *   - every call clears a thread-local message; on failure it returns a
 *     negative status (or NULL / 0 for constructors and id-returning calls)
 *     and tvara_last_error() describes it;
 *   - the status distinguishes the reference's exception classes;
 *   - host pointers passed in are consumed before the call returns unless a
 *     call says otherwise; device pointers are HBM addresses on the current
 *     HIP device;
 *   - a cache handle is single-owner, like PagedCache (docs/kv-cache.md): the
 *     caller serialises calls on one handle;
 *   - device work is issued on the handle's stream (the null stream unless
 *     tvara_kv_set_stream was called); calls that return host data
 *     synchronise that stream.
 */
#ifndef TVARA_CAPI_H
#define TVARA_CAPI_H
#include <stddef.h>
#include <stdint.h>

#define TVARA_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define TVARA_OK 0
#define TVARA_ERROR (-1)     /* std::runtime_error or a HIP failure */
#define TVARA_INVALID (-2)   /* std::invalid_argument */
#define TVARA_EXHAUSTED (-3) /* tvara::CacheExhausted (kv.hpp:34) */
#define TVARA_LOGIC (-4)     /* std::logic_error (audit invariants, kv.hpp:61-64, 138-146) */

/* KV storage formats of a cache */
#define TVARA_KV_F32 0  /* f32 blocks, byte-identical to the reference block layout (kv.hpp:30-33) */
#define TVARA_KV_Q8_0 1 /* Q8_0 groups (quant.hpp:40-49) of the same element order */

/* attention precisions for tvara_attn_prefill */
#define TVARA_ATTN_F32 0  /* reference semantics: one fused_paged_attention per row */
#define TVARA_ATTN_BF16 1 /* bf16 MFMA tiles, f32 accumulation */
/* MFMA tiles on f32 inputs split as hi + lo, three products each
 * (hi*hi + hi*lo + lo*hi): queries and keys as fp16 parts (about 2^-22
 * relative error per score term; a key beyond the fp16 range, 65,504, or a
 * query beyond it once multiplied by log2(e)/sqrt(head_dim) makes the call
 * fail as a non-finite input does), values and probabilities as bf16
 * parts (about 2^-16 per output term); the bf16 tiles' blocks (f32 or Q8_0,
 * dequantised as d * q when staged) */
#define TVARA_ATTN_F32X3 2

typedef struct tvara_model tvara_model;
typedef struct tvara_kv_cache tvara_kv_cache;
typedef struct tvara_attn_plan tvara_attn_plan;
typedef struct tvara_prefill_plan tvara_prefill_plan;
typedef struct tvara_radix tvara_radix;

/* BlockHandle (kv.hpp:35) */
typedef struct {
    uint64_t id;
    uint64_t generation;
} tvara_kv_handle;

/* c_api.h:17 -- thread-local message of the last failed call */
TVARA_API const char* tvara_last_error(void);

/* ---- model-level exports: the reference's 11 (c_api.h:13-24), same
 * signatures, return conventions (NULL / 0 / -1 with tvara_last_error set),
 * messages and per-handle lock (c_api.cpp:35-78).  The model runs on the GPU:
 * Q8_0 weight matrices stay quantised in HBM (34 bytes per 32 weights,
 * repacked into MFMA operand order), other GGUF types are dequantised to f32
 * at load, every layer of a token runs on device, and the KV cache lives in
 * this library's paged pool. */

/* tvara_model_open (c_api.cpp:36-40): load a Llama GGUF file; the KV pool holds
 * max_blocks blocks of block_tokens tokens */
TVARA_API tvara_model* tvara_model_open(const char* utf8_path, size_t max_blocks, size_t block_tokens);
/* c_api.cpp:42 */
TVARA_API void tvara_model_close(tvara_model* model);
/* c_api.cpp:43-44: 0 and "closed model" for a NULL handle */
TVARA_API size_t tvara_model_vocab_size(tvara_model* model);
TVARA_API size_t tvara_model_context_size(tvara_model* model);
/* c_api.cpp:46: the GGUF metadata as one JSON object, owned by the handle */
TVARA_API const char* tvara_model_metadata(tvara_model* model);
/* c_api.cpp:47-50: a new empty sequence (ids from 1), 0 on failure */
TVARA_API uint64_t tvara_sequence_create(tvara_model* model);
/* c_api.cpp:51-55 (PagedModelExecutor::decode, paged_model.hpp:12-28): logits
 * (count == vocab) of `token` at the end of `sequence`; its K/V are appended
 * only when every layer succeeded */
TVARA_API int tvara_sequence_decode(tvara_model* model, uint64_t sequence, uint32_t token, float* logits,
                                    size_t count);
/* c_api.cpp:56-59 */
TVARA_API int tvara_sequence_drop(tvara_model* model, uint64_t sequence);
/* c_api.cpp:61-73: token_count decodes (count == token_count * vocab); all
 * tokens are checked first and a failure truncates back to the entry length.
 * The tokens run as one pass per chunk of up to 512: batched products (each
 * weight row read once per chunk), each layer's K/V written into the cache,
 * then the chunk's causal attention over it; the logits are those of
 * token_count single decodes (f32 arithmetic throughout). */
TVARA_API int tvara_sequence_decode_batch(tvara_model* model, uint64_t sequence, const uint32_t* tokens,
                                          size_t token_count, float* logits, size_t count);
/* A prompt: tvara_sequence_decode_batch with only the last token's logits
 * returned (count == vocab, token_count >= 1), the same checks, messages and
 * rollback.  Replaces the per-token loop of NativeSchedulerBackend.prefill
 * (python/tvara/scheduler.py:197-199), which keeps the last token's logits;
 * no counterpart in the reference ABI. */
TVARA_API int tvara_sequence_prefill(tvara_model* model, uint64_t sequence, const uint32_t* tokens,
                                     size_t token_count, float* logits, size_t count);
/* c_api.cpp:76-78 (PagedCache::truncate, kv.hpp:131-136) */
TVARA_API int tvara_sequence_truncate(tvara_model* model, uint64_t sequence, size_t length);

/* One decode step for `count` distinct sequences at once: tokens[i] is decoded
 * at the end of sequences[i] and logits[i*vocab ...] receives its logits, as
 * tvara_sequence_decode(sequences[i], tokens[i]) would give them (the batched
 * matvecs accumulate in f32).  Every weight row is read once for the whole
 * batch.  All or nothing: on failure no sequence changes.  Returns 0 / -1.
 * Replaces the per-sequence loop of NativeSchedulerBackend.decode_batch
 * (python/tvara/scheduler.py:201-210); no counterpart in the reference ABI. */
TVARA_API int tvara_sequences_decode(tvara_model* model, const uint64_t* sequences, const uint32_t* tokens,
                                     size_t count, float* logits, size_t logits_count);

/* The model's KV cache as a tvara_kv_cache handle owned by the model (the
 * in-process PagedModelExecutor::cache(), paged_model.hpp:10), so every
 * tvara_kv_* call -- fork (kv.hpp:123-129), snapshots, retain / release,
 * import_sequence, audit -- and the prefix cache below work on the model's
 * sequences.  tvara_kv_cache_destroy on it does nothing; it lives until
 * tvara_model_close.  The caller serialises it with the model's calls.  No
 * counterpart in the reference ABI, which has no fork
 * (docs/architecture.md:110). */
TVARA_API tvara_kv_cache* tvara_model_cache(tvara_model* model);

/* ---- prefix cache: RadixCache (radix.hpp:17-131) over a cache handle, with
 * its node ids, eviction order and messages.  The tree is host metadata; a
 * node's KV is a retained snapshot of a sequence's blocks, and reuse imports
 * it as a new sequence sharing those blocks.  Destroy the tree before its
 * cache.  Additive: the reference keeps RadixCache in process. */
/* RadixCache(cache, isolation) (radix.hpp:19-23); isolation must be non-empty */
TVARA_API tvara_radix* tvara_radix_create(tvara_kv_cache* cache, const char* isolation);
TVARA_API void tvara_radix_destroy(tvara_radix* radix);
/* insert (radix.hpp:44-69): the node ending the path, created or split as needed */
TVARA_API int tvara_radix_insert(tvara_radix* radix, const int32_t* tokens, size_t count, uint64_t* node);
/* lookup (radix.hpp:29-42): deepest node reached and tokens matched */
TVARA_API int tvara_radix_lookup(tvara_radix* radix, const int32_t* tokens, size_t count, uint64_t* node,
                                 size_t* matched);
/* attach (radix.hpp:72-81): retain `sequence`'s blocks as the node's KV */
TVARA_API int tvara_radix_attach(tvara_radix* radix, uint64_t node, uint64_t sequence);
/* reuse (radix.hpp:90-96): a new sequence holding the matched prefix (whole
 * blocks unless partial) and its length */
TVARA_API int tvara_radix_reuse(tvara_radix* radix, const int32_t* tokens, size_t count, int partial,
                                uint64_t* sequence, size_t* length);
/* pin / unpin / touch (radix.hpp:99-103) */
TVARA_API int tvara_radix_pin(tvara_radix* radix, uint64_t node);
TVARA_API int tvara_radix_unpin(tvara_radix* radix, uint64_t node);
TVARA_API int tvara_radix_touch(tvara_radix* radix, uint64_t node);
/* eviction_candidate (radix.hpp:106-110): 0 when there is none */
TVARA_API int tvara_radix_eviction_candidate(tvara_radix* radix, uint64_t* node);
/* evict_one (radix.hpp:113-117) */
TVARA_API int tvara_radix_evict_one(tvara_radix* radix, int* evicted);
/* reset (radix.hpp:119-123) */
TVARA_API int tvara_radix_reset(tvara_radix* radix);
/* size (radix.hpp:26) */
TVARA_API int tvara_radix_size(tvara_radix* radix, size_t* size);
/* node(id) (radix.hpp:25): parent, edge tokens, pins, access stamp, KV
 * length and block count (kv_blocks = SIZE_MAX when none is attached),
 * children */
TVARA_API int tvara_radix_node(tvara_radix* radix, uint64_t id, uint64_t* parent, int32_t* edge, size_t edge_capacity,
                               size_t* edge_length, size_t* pins, uint64_t* accessed, size_t* kv_length,
                               size_t* kv_blocks, size_t* children);
/* external_references (radix.hpp:83-87): retained count per block id */
TVARA_API int tvara_radix_external_references(tvara_radix* radix, size_t* counts, size_t capacity);
/* Status of the last failed call on this thread (TVARA_OK after a success);
 * lets callers of the NULL- or 0-returning entry points tell the exception
 * classes apart.  No reference counterpart: the reference throws in C++. */
TVARA_API int tvara_last_status(void);

/* ------------------------------------------------------------------ caches */

/* PagedCache(CacheGeometry) (kv.hpp:80) with BlockPool's constructor
 * (kv.hpp:39-43) and CacheGeometry::validate (kv.hpp:24-28).  The block pool
 * is one HBM allocation.  format: TVARA_KV_F32 or TVARA_KV_Q8_0 (head_dim a
 * multiple of 32).  NULL on failure. */
TVARA_API tvara_kv_cache* tvara_kv_cache_create(size_t layers, size_t kv_heads, size_t head_dim,
                                                size_t tokens_per_block, size_t max_blocks, int format);
TVARA_API void tvara_kv_cache_destroy(tvara_kv_cache* cache);
/* Bytes of one block in the reference's element order: f32 blocks are
 * CacheGeometry::elements_per_block (kv.hpp:18-23) floats; Q8_0 blocks are 34
 * bytes per 32 elements. */
TVARA_API size_t tvara_kv_block_bytes(tvara_kv_cache* cache);
/* Issue device work on `stream` (a hipStream_t; NULL = null stream). */
TVARA_API int tvara_kv_set_stream(tvara_kv_cache* cache, void* stream);
/* Wait for the handle's stream. */
TVARA_API int tvara_kv_synchronize(tvara_kv_cache* cache);

/* ---------------------------------------------------------------- the pool */

/* BlockPool::allocate (kv.hpp:44-50): LIFO free list, refs=1, ++generation,
 * the block reads as zeros. */
TVARA_API int tvara_kv_pool_allocate(tvara_kv_cache* cache, tvara_kv_handle* out);
/* BlockPool::retain (kv.hpp:56) */
TVARA_API int tvara_kv_pool_retain(tvara_kv_cache* cache, tvara_kv_handle handle);
/* BlockPool::release and BlockPool::free (kv.hpp:51, 57) */
TVARA_API int tvara_kv_pool_release(tvara_kv_cache* cache, tvara_kv_handle handle);
/* BlockPool::references (kv.hpp:58) */
TVARA_API int tvara_kv_pool_references(tvara_kv_cache* cache, tvara_kv_handle handle, size_t* out);
/* BlockPool::references_by_id (kv.hpp:59) */
TVARA_API int tvara_kv_pool_references_by_id(tvara_kv_cache* cache, size_t id, size_t* out);
/* BlockPool::available (kv.hpp:55); 0 for a null handle */
TVARA_API size_t tvara_kv_pool_available(tvara_kv_cache* cache);
/* BlockPool::audit (kv.hpp:61-64) */
TVARA_API int tvara_kv_pool_audit(tvara_kv_cache* cache);
/* Exact allocator state (no reference counterpart: the pool keeps it private):
 * refs[max_blocks], generations[max_blocks] and the free list in the order
 * allocate() would pop it.  Any pointer may be NULL. */
TVARA_API int tvara_kv_pool_state(tvara_kv_cache* cache, size_t* refs, uint64_t* generations,
                                  size_t* free_pop_order, size_t* free_count);
/* BlockPool::data (kv.hpp:52-53): copy a live block out, `bytes` must equal
 * tvara_kv_block_bytes.  Q8_0 blocks come out as canonical 34-byte groups
 * (little-endian fp16 d, 32 int8). */
TVARA_API int tvara_kv_block_read(tvara_kv_cache* cache, tvara_kv_handle handle, void* out, size_t bytes);
/* Writes through BlockPool::data's mutable span (kv.hpp:52), as the
 * reference's tests do (tests/core/prefill_t173.cpp:6, prefill_t174.cpp:5);
 * byte range of the canonical block image. */
TVARA_API int tvara_kv_block_write(tvara_kv_cache* cache, tvara_kv_handle handle, size_t offset,
                                   const void* data, size_t bytes);
/* On-device 64-bit checksums of live blocks' canonical images:
 * sum over 32-bit words w_i of mix64(i << 32 | w_i) mod 2^64, mix64 being the
 * splitmix64 finaliser.  No reference counterpart; used to compare whole pools. */
TVARA_API int tvara_kv_block_checksums(tvara_kv_cache* cache, const tvara_kv_handle* handles, size_t count,
                                       uint64_t* out);

/* -------------------------------------------------------------- the tables */

/* PagedCache::create_sequence (kv.hpp:81); 0 on failure */
TVARA_API uint64_t tvara_kv_sequence_create(tvara_kv_cache* cache);
/* PagedCache::sequence (kv.hpp:82-84): length and block handles; `blocks` may
 * be NULL to query the count. */
TVARA_API int tvara_kv_sequence(tvara_kv_cache* cache, uint64_t sequence, size_t* length, tvara_kv_handle* blocks,
                                size_t capacity, size_t* count);
/* Live sequence ids in ascending order (the keys of PagedCache::sequences_). */
TVARA_API int tvara_kv_sequence_ids(tvara_kv_cache* cache, uint64_t* ids, size_t capacity, size_t* count);
/* PagedCache::physical_block (kv.hpp:85-87) */
TVARA_API int tvara_kv_physical_block(tvara_kv_cache* cache, uint64_t sequence, size_t position,
                                      tvara_kv_handle* out);
/* PagedCache::append (kv.hpp:91-108): keys and values are host f32
 * [layers * kv_width]; copy-on-write of a shared partial tail block. */
TVARA_API int tvara_kv_append(tvara_kv_cache* cache, uint64_t sequence, const float* keys, const float* values);
/* `count` appends, in order, one token per listed sequence:
 * keys/values are f32 [count][layers * kv_width] (device pointers when
 * `device_ptrs` is nonzero); a sequence may appear more than once.  On
 * failure of append k, appends 0..k-1 stay applied (as a loop over
 * PagedCache::append would leave them), append k changes nothing, and
 * *applied = k. */
TVARA_API int tvara_kv_append_batch(tvara_kv_cache* cache, const uint64_t* sequences, size_t count,
                                    const float* keys, const float* values, int device_ptrs, size_t* applied);
/* `count` consecutive appends to one sequence (a prompt's K/V) */
TVARA_API int tvara_kv_append_tokens(tvara_kv_cache* cache, uint64_t sequence, const float* keys,
                                     const float* values, size_t count, int device_ptrs, size_t* applied);
/* PagedCache::read (kv.hpp:110-113): kv_width floats of one position */
TVARA_API int tvara_kv_read(tvara_kv_cache* cache, uint64_t sequence, size_t layer, size_t position, int value,
                            float* out);
/* PagedCache::read_all (kv.hpp:114-119): [length][kv_width] floats */
TVARA_API int tvara_kv_read_all(tvara_kv_cache* cache, uint64_t sequence, size_t layer, int value, float* out,
                                size_t capacity);
/* PagedCache::drop (kv.hpp:121) */
TVARA_API int tvara_kv_drop(tvara_kv_cache* cache, uint64_t sequence);
/* PagedCache::fork (kv.hpp:123-129); 0 on failure */
TVARA_API uint64_t tvara_kv_fork(tvara_kv_cache* cache, uint64_t sequence);
/* PagedCache::truncate (kv.hpp:131-136) */
TVARA_API int tvara_kv_truncate(tvara_kv_cache* cache, uint64_t sequence, size_t length);
/* `count` truncations, in order: sequence i to lengths[i] tokens, as a loop
 * over PagedCache::truncate (kv.hpp:131-136) would apply them (a batch's
 * speculative rollback in one call).  On failure of truncation k, 0..k-1
 * stay applied, k changes nothing, and *applied = k. */
TVARA_API int tvara_kv_truncate_batch(tvara_kv_cache* cache, const uint64_t* sequences, const size_t* lengths,
                                      size_t count, size_t* applied);
/* PagedCache::audit (kv.hpp:138-146); external may be NULL (count 0) */
TVARA_API int tvara_kv_audit(tvara_kv_cache* cache, const size_t* external, size_t count);
/* PagedCache::import_sequence (kv.hpp:149-159) from a snapshot's handles; 0 on failure */
TVARA_API uint64_t tvara_kv_import_sequence(tvara_kv_cache* cache, const tvara_kv_handle* blocks,
                                            size_t block_count, size_t source_length, size_t length);

/* --------------------------------------------------------------- attention */

/* `count` calls of fused_paged_attention (attention.hpp:57-83), one per listed
 * sequence, in one launch: q f32 [count][heads * head_dim]; tail_keys /
 * tail_values f32 [count][kv_width] or both NULL (the current token's
 * uncommitted K/V, paged_model.hpp:22); visible [count] or NULL (no cap);
 * out f32 [count][heads * head_dim].  `context` is ModelConfig::context.
 * Synchronous; a non-finite score fails with TVARA_INVALID as
 * OnlineAttention::update does (attention.hpp:11). */
TVARA_API int tvara_attn_decode(tvara_kv_cache* cache, const uint64_t* sequences, size_t count, size_t layer,
                                size_t heads, size_t context, const float* q, const float* tail_keys,
                                const float* tail_values, const size_t* visible, float* out, int device_ptrs);
/* `count` calls of fused_prompt_attention (attention.hpp:85-89): queries for
 * sequence i are rows start[i] .. start[i]+rows[i]-1, packed one sequence
 * after the other, f32 [sum rows][heads * head_dim]; out likewise.
 * precision TVARA_ATTN_F32 keeps the reference's semantics; TVARA_ATTN_BF16
 * runs the causal tiles on MFMA with bf16 operands and f32 accumulation (f32 or
 * Q8_0 blocks of a power of two from 16 to 1,024 tokens and head_dim 64 or
 * 128, any number of query heads per KV head; other shapes fail with
 * TVARA_INVALID); TVARA_ATTN_F32X3 runs the same tiles with every operand as a
 * hi/lo pair (the same blocks; keys, and scaled queries, within the fp16
 * range). */
TVARA_API int tvara_attn_prefill(tvara_kv_cache* cache, const uint64_t* sequences, size_t count, size_t layer,
                                 size_t heads, size_t context, const size_t* start, const size_t* rows,
                                 const float* queries, float* out, int precision, int device_ptrs);

/* tvara_attn_decode with device pointers that allocates nothing: no
 * hipMalloc, hipFree or allocating library call.  No counterpart in the
 * reference; it is for callers that cannot allocate device memory (serving
 * loops, harnesses that forbid hipMalloc).  It is not for graph capture: the
 * call copies its plan from host memory and waits for its own work, so it
 * must not be called while the cache's stream is capturing.  The
 * plan (block ids, rows, work items, split counters, error flag) and the
 * split partials live in a fixed per-GPU device array of
 * tvara_attn_decode_noalloc_limit() bytes (32 MiB, held until the process
 * ends); a batch needing more fails with TVARA_INVALID.  Same arguments,
 * kernels and results as tvara_attn_decode(..., device_ptrs = 1): q, the
 * optional tails and out are 16-byte aligned device buffers; synchronous on
 * the cache's stream.  Calls on one GPU share the array: the library
 * serialises them and each waits for its own work, so none overlap on it. */
TVARA_API int tvara_attn_decode_noalloc(tvara_kv_cache* cache, const uint64_t* sequences, size_t count, size_t layer,
                                        size_t heads, size_t context, const float* q, const float* tail_keys,
                                        const float* tail_values, const size_t* visible, float* out);
TVARA_API size_t tvara_attn_decode_noalloc_limit(void);

/* A decode plan keeps the listed sequences' block tables resident in HBM so
 * that repeated launches (the same batch over several layers, or timing)
 * upload nothing.  It records the cache's mutation count; launching it after
 * the cache changed fails with TVARA_INVALID. */
TVARA_API tvara_attn_plan* tvara_attn_plan_create(tvara_kv_cache* cache, const uint64_t* sequences, size_t count,
                                                  size_t heads, size_t context, const size_t* visible,
                                                  int with_tail);
/* Asynchronous decode over device buffers (q, optional tails, out) on `stream`
 * (NULL = the cache's stream). */
TVARA_API int tvara_attn_plan_decode(tvara_attn_plan* plan, size_t layer, const float* q, const float* tail_keys,
                                     const float* tail_values, float* out, void* stream);
/* Synchronise the plan's last launch and report a non-finite score. */
TVARA_API int tvara_attn_plan_check(tvara_attn_plan* plan);
/* Work decomposition of the plan: split length in tokens, work items, KV bytes
 * one launch reads (algorithmic). */
TVARA_API int tvara_attn_plan_info(tvara_attn_plan* plan, size_t* split_tokens, size_t* items, size_t* kv_bytes);
TVARA_API void tvara_attn_plan_destroy(tvara_attn_plan* plan);

/* A chunked-prefill plan: tvara_attn_prefill's work (fused_prompt_attention,
 * attention.hpp:85-89, for each sequence's rows start[i] .. start[i]+rows[i]-1)
 * with the block tables resident, so one plan per prompt chunk serves every
 * layer.  Launches take device pointers, run asynchronously on `stream` (NULL:
 * the cache's stream) and fail with TVARA_INVALID once the cache has changed
 * since the plan was made.  No counterpart in the reference, which recomputes
 * the block walk per call. */
TVARA_API tvara_prefill_plan* tvara_prefill_plan_create(tvara_kv_cache* cache, const uint64_t* sequences,
                                                        size_t count, size_t heads, size_t context,
                                                        const size_t* start, const size_t* rows, int precision);
TVARA_API int tvara_prefill_plan_launch(tvara_prefill_plan* plan, size_t layer, const float* queries, float* out,
                                        void* stream);
/* Synchronise the plan's last launch and report a non-finite score. */
TVARA_API int tvara_prefill_plan_check(tvara_prefill_plan* plan);
TVARA_API void tvara_prefill_plan_destroy(tvara_prefill_plan* plan);

/* ----------------------------------------------------------------- timing */

/* When enabled, every kernel launch of the library is bracketed by HIP events
 * on its stream; tvara_profile_read synchronises and returns, per kernel name
 * prefix, the summed milliseconds and launch count since the last reset. */
TVARA_API int tvara_profile_enable(int enabled);
TVARA_API int tvara_profile_read(const char* kernel, double* milliseconds, size_t* launches);
TVARA_API int tvara_profile_reset(void);

#ifdef __cplusplus
}
#endif
#endif
