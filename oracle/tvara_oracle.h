/*
 * tvara_oracle.h -- CPU restatement of Tvara's paged KV cache, fused paged
 * attention and Q8_0 block format, in plain C11.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py may load it; the product library (libtvara_capi.so) never
 * links, loads or calls it.
 *
 * Every function restates one reference function; the citation is given as
 * file:line relative to the reference repository root.  The restatement keeps
 * the reference's loop order and its FP64 arithmetic so that it can be timed as
 * the CPU baseline.
 *
 * Pinning (how each part is checked independently of this file):
 *   - pool / cache state machine: known-answer checks restated from
 *     tests/core/test_kv.cpp:7-46 and tests/core/test_radix.cpp, plus exact
 *     state comparison against the reference headers compiled in oracle/_ref
 *     (tests/test_oracle_vs_ref.py) and committed golden traces.
 *   - fused paged attention: float64 brute-force two-pass softmax in numpy,
 *     known answers (q=0 gives mean of V, one position gives V, huge scores stay
 *     finite), and the committed golden outputs produced by the reference.
 *   - half_to_float / dequantize_q8_0: tests/core/test_quant.cpp:16-29,135-138
 *     known answers, and exhaustive comparison with numpy float16 for all 65536
 *     bit patterns.
 *   - Q8_0 encoder: numpy float32/float16 library rounding on the expression of
 *     tools/make_api_fixture.py:131-137 (the same expression, evaluated by
 *     numpy's IEEE routines), including round-half-even ties and zero blocks.
 */
#ifndef TVARA_ORACLE_H
#define TVARA_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: the reference throws; the oracle returns the exception class. */
enum {
    TVO_OK = 0,
    TVO_EINVAL = -2,     /* std::invalid_argument */
    TVO_EXHAUSTED = -3,  /* tvara::CacheExhausted */
    TVO_ERUNTIME = -1,   /* std::runtime_error */
    TVO_ELOGIC = -4,     /* std::logic_error */
    TVO_ENOMEM = -5
};

typedef struct {
    size_t layers, kv_heads, head_dim, tokens_per_block, max_blocks;
} tvo_geometry;

typedef struct {
    size_t id;
    uint64_t generation;
} tvo_handle;

typedef struct tvo_cache tvo_cache;

const char* tvo_last_error(void);

/* CacheGeometry (core/include/tvara/kv.hpp:12-29) */
int tvo_geometry_validate(const tvo_geometry* g);
size_t tvo_elements_per_block(const tvo_geometry* g);
/* kv_offset (kv.hpp:30-33); returns (size_t)-1 and sets the error when outside */
size_t tvo_kv_offset(const tvo_geometry* g, size_t layer, size_t kind, size_t slot);

/* PagedCache + BlockPool (kv.hpp:36-165) */
tvo_cache* tvo_cache_create(const tvo_geometry* g);
void tvo_cache_destroy(tvo_cache* c);
tvo_cache* tvo_cache_clone(const tvo_cache* c);

int tvo_pool_allocate(tvo_cache* c, tvo_handle* out);
int tvo_pool_retain(tvo_cache* c, tvo_handle h);
int tvo_pool_release(tvo_cache* c, tvo_handle h);
int tvo_pool_references(const tvo_cache* c, tvo_handle h, size_t* out);
size_t tvo_pool_references_by_id(const tvo_cache* c, size_t id);
size_t tvo_pool_available(const tvo_cache* c);
int tvo_pool_audit(const tvo_cache* c);
/* pool_.data(handle) (kv.hpp:52-53, validated 68-72) */
int tvo_pool_data(tvo_cache* c, tvo_handle h, float** out);

uint64_t tvo_create_sequence(tvo_cache* c);               /* 0 on error */
int tvo_sequence_length(const tvo_cache* c, uint64_t seq, size_t* length);
int tvo_sequence_blocks(const tvo_cache* c, uint64_t seq, tvo_handle* out, size_t capacity, size_t* count);
int tvo_physical_block(const tvo_cache* c, uint64_t seq, size_t position, tvo_handle* out);
int tvo_append(tvo_cache* c, uint64_t seq, const float* keys, const float* values);
int tvo_read(const tvo_cache* c, uint64_t seq, size_t layer, size_t position, int value, float* out);
int tvo_read_all(const tvo_cache* c, uint64_t seq, size_t layer, int value, float* out, size_t capacity);
int tvo_drop(tvo_cache* c, uint64_t seq);
uint64_t tvo_fork(tvo_cache* c, uint64_t seq);           /* 0 on error */
int tvo_truncate(tvo_cache* c, uint64_t seq, size_t length);
int tvo_audit(const tvo_cache* c, const size_t* external, size_t external_count);
uint64_t tvo_import_sequence(tvo_cache* c, const tvo_handle* blocks, size_t block_count,
                             size_t source_length, size_t length); /* 0 on error */

/* State dump used for exact comparison: refs[max_blocks], generations[max_blocks],
 * free list in pop order (last pushed first), sequence ids in ascending order. */
int tvo_pool_state(const tvo_cache* c, size_t* refs, uint64_t* generations, size_t* free_pop_order,
                   size_t* free_count);
size_t tvo_sequence_count(const tvo_cache* c);
int tvo_sequence_ids(const tvo_cache* c, uint64_t* ids, size_t capacity);
/* 64-bit order-sensitive checksum of a block's 32-bit words (same definition as
 * the device checksum kernel): sum over i of mix64(word_i | i<<32) modulo 2^64. */
uint64_t tvo_checksum_words(const uint32_t* words, size_t count);

/* Attention (core/include/tvara/attention.hpp) */
double tvo_attention_dot(const float* a, const float* b, size_t n);   /* attention.hpp:203-205 */
int tvo_fused_paged_attention(const tvo_cache* c, uint64_t seq, size_t layer, size_t heads, size_t context,
                              const float* q, const float* tail_key, const float* tail_value,
                              size_t visible, float* out);             /* attention.hpp:57-83 */
int tvo_fused_prompt_attention(const tvo_cache* c, uint64_t seq, size_t layer, size_t heads, size_t context,
                               size_t start, size_t count, const float* queries, float* out); /* :85-89 */
/* 0: scalar double dot (attention.hpp:203-205); 1: the AVX2 summation order
 * (attention.hpp:197-201: four double lanes, lanes summed left to right, tail). */
void tvo_set_dot_mode(int mode);

/* Q8_0 (core/include/tvara/quant.hpp:14-49, tools/make_api_fixture.py:131-137) */
float tvo_half_to_float(uint16_t h);
uint16_t tvo_double_to_half(double x);
int tvo_dequantize_q8_0(const uint8_t* bytes, size_t nbytes, float* out, size_t count);
void tvo_quantize_q8_0_block(const float* x32, uint8_t* out34);
void tvo_quantize_q8_0(const float* x, size_t groups, uint8_t* out);

#ifdef __cplusplus
}
#endif
#endif
