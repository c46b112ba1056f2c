/*
 * tvara_oracle.c -- CPU restatement of Tvara's paged KV cache and fused paged
 * attention (plain C11).  TEST INFRASTRUCTURE ONLY: see tvara_oracle.h for who
 * may load it and how each part is pinned.
 *
 * Citations are file:line in the reference repository:
 *   kv.hpp        = core/include/tvara/kv.hpp
 *   attention.hpp = core/include/tvara/attention.hpp
 *   quant.hpp     = core/include/tvara/quant.hpp
 *   fixture.py    = tools/make_api_fixture.py
 */
#include "tvara_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static _Thread_local char g_error[256];

static int fail(int code, const char* message) {
    snprintf(g_error, sizeof g_error, "%s", message);
    return code;
}

const char* tvo_last_error(void) { return g_error; }

/* ------------------------------------------------------------------ geometry */

/* CacheGeometry::kv_width (kv.hpp:14-17) */
static int kv_width(const tvo_geometry* g, size_t* out) {
    if (!g->kv_heads || !g->head_dim || g->kv_heads > SIZE_MAX / g->head_dim)
        return fail(TVO_EINVAL, "KV width overflow");
    *out = g->kv_heads * g->head_dim;
    return TVO_OK;
}

/* CacheGeometry::elements_per_block (kv.hpp:18-23) */
static int elements_per_block(const tvo_geometry* g, size_t* out) {
    size_t count;
    int rc = kv_width(g, &count);
    if (rc) return rc;
    const size_t dims[3] = {g->layers, g->tokens_per_block, 2};
    for (int i = 0; i < 3; ++i) {
        if (!dims[i] || count > SIZE_MAX / dims[i]) return fail(TVO_EINVAL, "KV block overflow");
        count *= dims[i];
    }
    *out = count;
    return TVO_OK;
}

size_t tvo_elements_per_block(const tvo_geometry* g) {
    size_t n = 0;
    return elements_per_block(g, &n) ? 0 : n;
}

/* CacheGeometry::validate (kv.hpp:24-28) */
int tvo_geometry_validate(const tvo_geometry* g) {
    size_t elements;
    int rc = elements_per_block(g, &elements);
    if (rc) return rc;
    if (!g->max_blocks || g->max_blocks > 1000000 ||
        elements > SIZE_MAX / sizeof(float) / g->max_blocks ||
        g->tokens_per_block > SIZE_MAX / g->max_blocks)
        return fail(TVO_EINVAL, "KV capacity overflow");
    return TVO_OK;
}

/* kv_offset (kv.hpp:30-33) */
size_t tvo_kv_offset(const tvo_geometry* g, size_t layer, size_t kind, size_t slot) {
    if (layer >= g->layers || kind > 1 || slot >= g->tokens_per_block) {
        fail(TVO_EINVAL, "KV position outside block");
        return (size_t)-1;
    }
    return ((layer * 2 + kind) * g->tokens_per_block + slot) * (g->kv_heads * g->head_dim);
}

/* ----------------------------------------------------------------- the pool */

typedef struct {
    uint64_t id;
    tvo_handle* blocks;
    size_t nblocks, cap;
    size_t length;
} table_t;

struct tvo_cache {
    tvo_geometry g;
    size_t elements;   /* floats per block */
    float* values;     /* max_blocks * elements, zero-initialised */
    size_t* refs;
    uint64_t* gens;
    size_t* free_ids;  /* stack; back = next allocation */
    size_t free_count;
    table_t* seqs;     /* sorted by id */
    size_t nseq, seqcap;
    uint64_t next;
};

/* BlockPool::BlockPool (kv.hpp:39-43): every block zeroed, free list
 * max_blocks-1 ... 0 so that a fresh pool hands out 0, 1, 2, ... */
tvo_cache* tvo_cache_create(const tvo_geometry* g) {
    if (tvo_geometry_validate(g)) return NULL;
    tvo_cache* c = calloc(1, sizeof *c);
    if (!c) return NULL;
    c->g = *g;
    elements_per_block(g, &c->elements);
    c->values = calloc(g->max_blocks * c->elements, sizeof(float));
    c->refs = calloc(g->max_blocks, sizeof(size_t));
    c->gens = calloc(g->max_blocks, sizeof(uint64_t));
    c->free_ids = malloc(g->max_blocks * sizeof(size_t));
    if (!c->values || !c->refs || !c->gens || !c->free_ids) {
        tvo_cache_destroy(c);
        fail(TVO_ENOMEM, "out of memory");
        return NULL;
    }
    for (size_t i = g->max_blocks; i > 0; --i) c->free_ids[c->free_count++] = i - 1;
    return c;
}

void tvo_cache_destroy(tvo_cache* c) {
    if (!c) return;
    for (size_t i = 0; i < c->nseq; ++i) free(c->seqs[i].blocks);
    free(c->seqs);
    free(c->values);
    free(c->refs);
    free(c->gens);
    free(c->free_ids);
    free(c);
}

tvo_cache* tvo_cache_clone(const tvo_cache* c) {
    tvo_cache* d = tvo_cache_create(&c->g);
    if (!d) return NULL;
    memcpy(d->values, c->values, c->g.max_blocks * c->elements * sizeof(float));
    memcpy(d->refs, c->refs, c->g.max_blocks * sizeof(size_t));
    memcpy(d->gens, c->gens, c->g.max_blocks * sizeof(uint64_t));
    memcpy(d->free_ids, c->free_ids, c->free_count * sizeof(size_t));
    d->free_count = c->free_count;
    d->next = c->next;
    d->seqs = calloc(c->nseq ? c->nseq : 1, sizeof(table_t));
    d->seqcap = c->nseq ? c->nseq : 1;
    for (size_t i = 0; i < c->nseq; ++i) {
        d->seqs[i] = c->seqs[i];
        d->seqs[i].cap = c->seqs[i].nblocks ? c->seqs[i].nblocks : 1;
        d->seqs[i].blocks = malloc(d->seqs[i].cap * sizeof(tvo_handle));
        memcpy(d->seqs[i].blocks, c->seqs[i].blocks, c->seqs[i].nblocks * sizeof(tvo_handle));
    }
    d->nseq = c->nseq;
    return d;
}

/* BlockPool::validated (kv.hpp:68-72) */
static int validated(const tvo_cache* c, tvo_handle h) {
    if (h.id >= c->g.max_blocks || !c->refs[h.id] || c->gens[h.id] != h.generation)
        return fail(TVO_EINVAL, "stale or invalid KV handle");
    return TVO_OK;
}

/* BlockPool::allocate (kv.hpp:44-50) */
int tvo_pool_allocate(tvo_cache* c, tvo_handle* out) {
    if (!c->free_count) return fail(TVO_EXHAUSTED, "KV cache exhausted");
    const size_t id = c->free_ids[c->free_count - 1];
    if (c->gens[id] == UINT64_MAX) return fail(TVO_ERUNTIME, "KV generation exhausted");
    c->free_count--;
    c->refs[id] = 1;
    ++c->gens[id];
    memset(c->values + id * c->elements, 0, c->elements * sizeof(float));
    out->id = id;
    out->generation = c->gens[id];
    return TVO_OK;
}

/* BlockPool::retain (kv.hpp:56) */
int tvo_pool_retain(tvo_cache* c, tvo_handle h) {
    int rc = validated(c, h);
    if (rc) return rc;
    if (c->refs[h.id] == SIZE_MAX) return fail(TVO_ERUNTIME, "KV reference overflow");
    ++c->refs[h.id];
    return TVO_OK;
}

/* BlockPool::release (kv.hpp:57) */
int tvo_pool_release(tvo_cache* c, tvo_handle h) {
    int rc = validated(c, h);
    if (rc) return rc;
    if (--c->refs[h.id] == 0) c->free_ids[c->free_count++] = h.id;
    return TVO_OK;
}

/* BlockPool::references (kv.hpp:58) */
int tvo_pool_references(const tvo_cache* c, tvo_handle h, size_t* out) {
    int rc = validated(c, h);
    if (rc) return rc;
    *out = c->refs[h.id];
    return TVO_OK;
}

/* BlockPool::references_by_id (kv.hpp:59); blocks_.at() throws out_of_range */
size_t tvo_pool_references_by_id(const tvo_cache* c, size_t id) {
    if (id >= c->g.max_blocks) {
        fail(TVO_ELOGIC, "block id out of range");
        return SIZE_MAX;
    }
    return c->refs[id];
}

/* BlockPool::available (kv.hpp:55) */
size_t tvo_pool_available(const tvo_cache* c) { return c->free_count; }

/* BlockPool::data (kv.hpp:52-53) */
int tvo_pool_data(tvo_cache* c, tvo_handle h, float** out) {
    int rc = validated(c, h);
    if (rc) return rc;
    *out = c->values + h.id * c->elements;
    return TVO_OK;
}

/* BlockPool::audit (kv.hpp:61-64) */
int tvo_pool_audit(const tvo_cache* c) {
    const size_t n = c->g.max_blocks;
    unsigned char* seen = calloc(n ? n : 1, 1);
    int rc = TVO_OK;
    for (size_t i = 0; i < c->free_count && !rc; ++i) {
        const size_t id = c->free_ids[i];
        if (id >= n || seen[id] || c->refs[id]) rc = fail(TVO_ELOGIC, "KV free-list invariant");
        else seen[id] = 1;
    }
    for (size_t i = 0; i < n && !rc; ++i)
        if ((seen[i] != 0) != (c->refs[i] == 0)) rc = fail(TVO_ELOGIC, "KV allocation invariant");
    free(seen);
    return rc;
}

/* ---------------------------------------------------------------- the cache */

/* std::map lookup in PagedCache::sequence (kv.hpp:82-84) */
static table_t* find(const tvo_cache* c, uint64_t id) {
    size_t lo = 0, hi = c->nseq;
    while (lo < hi) {
        size_t mid = (lo + hi) / 2;
        if (c->seqs[mid].id < id) lo = mid + 1;
        else hi = mid;
    }
    if (lo < c->nseq && c->seqs[lo].id == id) return &c->seqs[lo];
    fail(TVO_EINVAL, "unknown KV sequence");
    return NULL;
}

static int push_handle(table_t* t, tvo_handle h) {
    if (t->nblocks == t->cap) {
        size_t cap = t->cap ? 2 * t->cap : 8;
        tvo_handle* b = realloc(t->blocks, cap * sizeof *b);
        if (!b) return fail(TVO_ENOMEM, "out of memory");
        t->blocks = b;
        t->cap = cap;
    }
    t->blocks[t->nblocks++] = h;
    return TVO_OK;
}

/* sequences_.emplace with ids that only grow, so appending keeps the order */
static int emplace(tvo_cache* c, table_t t) {
    if (c->nseq == c->seqcap) {
        size_t cap = c->seqcap ? 2 * c->seqcap : 16;
        table_t* s = realloc(c->seqs, cap * sizeof *s);
        if (!s) return fail(TVO_ENOMEM, "out of memory");
        c->seqs = s;
        c->seqcap = cap;
    }
    c->seqs[c->nseq++] = t;
    return TVO_OK;
}

/* PagedCache::create_sequence (kv.hpp:81) */
uint64_t tvo_create_sequence(tvo_cache* c) {
    if (c->next == UINT64_MAX) {
        fail(TVO_ERUNTIME, "sequence ID exhausted");
        return 0;
    }
    table_t t = {0};
    t.id = c->next + 1;
    if (emplace(c, t)) return 0;
    return ++c->next;
}

int tvo_sequence_length(const tvo_cache* c, uint64_t seq, size_t* length) {
    const table_t* t = find(c, seq);
    if (!t) return TVO_EINVAL;
    *length = t->length;
    return TVO_OK;
}

int tvo_sequence_blocks(const tvo_cache* c, uint64_t seq, tvo_handle* out, size_t capacity, size_t* count) {
    const table_t* t = find(c, seq);
    if (!t) return TVO_EINVAL;
    *count = t->nblocks;
    if (out) {
        if (capacity < t->nblocks) return fail(TVO_EINVAL, "block list buffer too small");
        memcpy(out, t->blocks, t->nblocks * sizeof(tvo_handle));
    }
    return TVO_OK;
}

/* PagedCache::physical_block (kv.hpp:85-87) */
int tvo_physical_block(const tvo_cache* c, uint64_t seq, size_t position, tvo_handle* out) {
    const table_t* t = find(c, seq);
    if (!t) return TVO_EINVAL;
    if (position >= t->length) return fail(TVO_EINVAL, "KV position beyond sequence");
    *out = t->blocks[position / c->g.tokens_per_block];
    return TVO_OK;
}

/* PagedCache::append (kv.hpp:91-108) */
int tvo_append(tvo_cache* c, uint64_t seq, const float* keys, const float* values) {
    table_t* t = find(c, seq);
    if (!t) return TVO_EINVAL;
    const tvo_geometry* g = &c->g;
    const size_t width = g->kv_heads * g->head_dim;
    if (!keys || !values || t->length >= g->max_blocks * g->tokens_per_block)
        return fail(TVO_EINVAL, "invalid paged KV append dimensions");
    const size_t slot = t->length % g->tokens_per_block;
    if (slot == 0) {                                   /* kv.hpp:96 */
        tvo_handle h;
        int rc = tvo_pool_allocate(c, &h);
        if (rc) return rc;
        rc = push_handle(t, h);
        if (rc) {
            tvo_pool_release(c, h);
            return rc;
        }
    }
    if (slot != 0 && c->refs[t->blocks[t->nblocks - 1].id] > 1) { /* kv.hpp:97-101 copy-on-write */
        const tvo_handle original = t->blocks[t->nblocks - 1];
        tvo_handle replacement;
        int rc = tvo_pool_allocate(c, &replacement);
        if (rc) return rc;
        memcpy(c->values + replacement.id * c->elements, c->values + original.id * c->elements,
               c->elements * sizeof(float));
        t->blocks[t->nblocks - 1] = replacement;
        tvo_pool_release(c, original);
    }
    float* block = c->values + t->blocks[t->nblocks - 1].id * c->elements;
    for (size_t layer = 0; layer < g->layers; ++layer) {    /* kv.hpp:103-106 */
        memcpy(block + tvo_kv_offset(g, layer, 0, slot), keys + layer * width, width * sizeof(float));
        memcpy(block + tvo_kv_offset(g, layer, 1, slot), values + layer * width, width * sizeof(float));
    }
    ++t->length;
    return TVO_OK;
}

/* PagedCache::read (kv.hpp:110-113) */
int tvo_read(const tvo_cache* c, uint64_t seq, size_t layer, size_t position, int value, float* out) {
    tvo_handle h;
    int rc = tvo_physical_block(c, seq, position, &h);
    if (rc) return rc;
    const size_t offset = tvo_kv_offset(&c->g, layer, value ? 1 : 0, position % c->g.tokens_per_block);
    if (offset == (size_t)-1) return TVO_EINVAL;
    rc = validated(c, h);
    if (rc) return rc;
    memcpy(out, c->values + h.id * c->elements + offset, c->g.kv_heads * c->g.head_dim * sizeof(float));
    return TVO_OK;
}

/* PagedCache::read_all (kv.hpp:114-119) */
int tvo_read_all(const tvo_cache* c, uint64_t seq, size_t layer, int value, float* out, size_t capacity) {
    const table_t* t = find(c, seq);
    if (!t) return TVO_EINVAL;
    if (layer >= c->g.layers) return fail(TVO_EINVAL, "invalid KV layer");
    const size_t width = c->g.kv_heads * c->g.head_dim;
    if (capacity < t->length * width) return fail(TVO_EINVAL, "read_all buffer too small");
    for (size_t p = 0; p < t->length; ++p) {
        int rc = tvo_read(c, seq, layer, p, value, out + p * width);
        if (rc) return rc;
    }
    return TVO_OK;
}

/* PagedCache::drop (kv.hpp:121) */
int tvo_drop(tvo_cache* c, uint64_t seq) {
    table_t* t = find(c, seq);
    if (!t) return TVO_EINVAL;
    for (size_t i = 0; i < t->nblocks; ++i) {
        int rc = tvo_pool_release(c, t->blocks[i]);
        if (rc) return rc;
    }
    free(t->blocks);
    const size_t index = (size_t)(t - c->seqs);
    memmove(c->seqs + index, c->seqs + index + 1, (c->nseq - index - 1) * sizeof(table_t));
    c->nseq--;
    return TVO_OK;
}

/* shared tail of fork and import_sequence: publish a table under ++next_ */
static uint64_t publish(tvo_cache* c, const tvo_handle* blocks, size_t count, size_t length) {
    size_t retained = 0;
    int rc = TVO_OK;
    for (; retained < count; ++retained) {
        rc = tvo_pool_retain(c, blocks[retained]);
        if (rc) break;
    }
    if (!rc && c->next == UINT64_MAX) rc = fail(TVO_ERUNTIME, "sequence ID exhausted");
    table_t t = {0};
    if (!rc) {
        t.id = c->next + 1;
        t.length = length;
        t.cap = count ? count : 1;
        t.blocks = malloc(t.cap * sizeof(tvo_handle));
        if (!t.blocks) rc = fail(TVO_ENOMEM, "out of memory");
        else {
            memcpy(t.blocks, blocks, count * sizeof(tvo_handle));
            t.nblocks = count;
            rc = emplace(c, t);
            if (rc) free(t.blocks);
        }
    }
    if (rc) { /* roll the retains back (kv.hpp:128, kv.hpp:158) */
        char saved[sizeof g_error];
        memcpy(saved, g_error, sizeof saved);
        for (size_t i = 0; i < retained; ++i) tvo_pool_release(c, blocks[i]);
        memcpy(g_error, saved, sizeof saved);
        return 0;
    }
    return ++c->next;
}

/* PagedCache::fork (kv.hpp:123-129) */
uint64_t tvo_fork(tvo_cache* c, uint64_t seq) {
    const table_t* t = find(c, seq);
    if (!t) return 0;
    /* copy first: emplace may move the table array */
    tvo_handle* copy = malloc((t->nblocks ? t->nblocks : 1) * sizeof(tvo_handle));
    if (!copy) return fail(TVO_ENOMEM, "out of memory"), 0;
    memcpy(copy, t->blocks, t->nblocks * sizeof(tvo_handle));
    const size_t n = t->nblocks, length = t->length;
    uint64_t id = publish(c, copy, n, length);
    free(copy);
    return id;
}

/* PagedCache::truncate (kv.hpp:131-136): stale slots are not cleared */
int tvo_truncate(tvo_cache* c, uint64_t seq, size_t length) {
    table_t* t = find(c, seq);
    if (!t) return TVO_EINVAL;
    if (length > t->length) return fail(TVO_EINVAL, "cannot extend KV by truncating");
    const size_t tpb = c->g.tokens_per_block;
    const size_t keep = length / tpb + (length % tpb ? 1 : 0);
    for (size_t i = keep; i < t->nblocks; ++i) {
        int rc = tvo_pool_release(c, t->blocks[i]);
        if (rc) return rc;
    }
    if (keep < t->nblocks) t->nblocks = keep;
    t->length = length;
    return TVO_OK;
}

/* PagedCache::audit (kv.hpp:138-146) */
int tvo_audit(const tvo_cache* c, const size_t* external, size_t external_count) {
    int rc = tvo_pool_audit(c);
    if (rc) return rc;
    const size_t n = c->g.max_blocks, tpb = c->g.tokens_per_block;
    if (external_count && external_count != n) return fail(TVO_EINVAL, "external reference counts mismatch");
    size_t* counts = calloc(n ? n : 1, sizeof(size_t));
    for (size_t s = 0; s < c->nseq && !rc; ++s) {
        const table_t* t = &c->seqs[s];
        const size_t expected = t->length / tpb + (t->length % tpb ? 1 : 0);
        if (t->nblocks != expected) rc = fail(TVO_ELOGIC, "KV block table length invariant");
        for (size_t b = 0; b < t->nblocks && !rc; ++b) {
            rc = validated(c, t->blocks[b]);
            if (!rc) ++counts[t->blocks[b].id];
        }
    }
    for (size_t i = 0; i < n && !rc; ++i)
        if (counts[i] + (external_count ? external[i] : 0) != c->refs[i])
            rc = fail(TVO_ELOGIC, "KV reference invariant");
    free(counts);
    return rc;
}

/* PagedCache::import_sequence (kv.hpp:149-159) */
uint64_t tvo_import_sequence(tvo_cache* c, const tvo_handle* blocks, size_t block_count,
                             size_t source_length, size_t length) {
    if (length > source_length) return fail(TVO_EINVAL, "prefix exceeds snapshot"), 0;
    const size_t tpb = c->g.tokens_per_block;
    const size_t count = length / tpb + (length % tpb ? 1 : 0);
    if (block_count < count) return fail(TVO_EINVAL, "invalid prefix snapshot"), 0;
    return publish(c, blocks, count, length);
}

int tvo_pool_state(const tvo_cache* c, size_t* refs, uint64_t* generations, size_t* free_pop_order,
                   size_t* free_count) {
    const size_t n = c->g.max_blocks;
    if (refs) memcpy(refs, c->refs, n * sizeof(size_t));
    if (generations) memcpy(generations, c->gens, n * sizeof(uint64_t));
    if (free_pop_order)
        for (size_t i = 0; i < c->free_count; ++i) free_pop_order[i] = c->free_ids[c->free_count - 1 - i];
    if (free_count) *free_count = c->free_count;
    return TVO_OK;
}

size_t tvo_sequence_count(const tvo_cache* c) { return c->nseq; }

int tvo_sequence_ids(const tvo_cache* c, uint64_t* ids, size_t capacity) {
    if (capacity < c->nseq) return fail(TVO_EINVAL, "id buffer too small");
    for (size_t i = 0; i < c->nseq; ++i) ids[i] = c->seqs[i].id;
    return TVO_OK;
}

static uint64_t mix64(uint64_t z) {
    z ^= z >> 30;
    z *= 0xBF58476D1CE4E5B9ULL;
    z ^= z >> 27;
    z *= 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t tvo_checksum_words(const uint32_t* words, size_t count) {
    uint64_t h = 0;
    for (size_t i = 0; i < count; ++i) h += mix64(((uint64_t)i << 32) | words[i]);
    return h;
}

/* ---------------------------------------------------------------- attention */

static int g_dot_mode = 0;
void tvo_set_dot_mode(int mode) { g_dot_mode = mode; }

/* attention_dot_scalar (attention.hpp:203-205) */
static double dot_scalar(const float* a, const float* b, size_t n) {
    double sum = 0;
    for (size_t i = 0; i < n; ++i) sum += (double)a[i] * (double)b[i];
    return sum;
}

/* attention_dot_avx2 summation order (attention.hpp:197-201) */
static double dot_avx2_order(const float* a, const float* b, size_t n) {
    double lane[4] = {0, 0, 0, 0};
    size_t i = 0;
    for (; i + 4 <= n; i += 4)
        for (int j = 0; j < 4; ++j) lane[j] = lane[j] + (double)a[i + j] * (double)b[i + j];
    double sum = lane[0] + lane[1] + lane[2] + lane[3];
    for (; i < n; ++i) sum += (double)a[i] * (double)b[i];
    return sum;
}

double tvo_attention_dot(const float* a, const float* b, size_t n) {
    return g_dot_mode ? dot_avx2_order(a, b, n) : dot_scalar(a, b, n);
}

/* OnlineAttention (attention.hpp:6-16), FP64 state */
typedef struct {
    double maximum, normalizer;
    double* sum;
    size_t dim;
} online_t;

static int online_update(online_t* s, double score, const float* value) {
    if (!isfinite(score)) return fail(TVO_EINVAL, "invalid online attention input");
    const double next = s->maximum > score ? s->maximum : score;
    const double old = exp(s->maximum - next), weight = exp(score - next);
    s->normalizer = s->normalizer * old + weight;
    for (size_t i = 0; i < s->dim; ++i) s->sum[i] = s->sum[i] * old + weight * (double)value[i];
    s->maximum = next;
    return TVO_OK;
}

static int online_finish(const online_t* s, float* out) {
    if (!(s->normalizer > 0)) return fail(TVO_EINVAL, "empty attention");
    for (size_t i = 0; i < s->dim; ++i) out[i] = (float)(s->sum[i] / s->normalizer);
    return TVO_OK;
}

/* ModelConfig::validate (model.hpp:13-19) restricted to what attention reads */
static int check_config(const tvo_geometry* g, size_t heads, size_t context) {
    if (!heads || !context || !g->kv_heads || heads % g->kv_heads || g->head_dim % 2)
        return fail(TVO_EINVAL, "invalid native model configuration");
    return TVO_OK;
}

/* fused_paged_attention (attention.hpp:57-83) */
int tvo_fused_paged_attention(const tvo_cache* c, uint64_t seq, size_t layer, size_t heads, size_t context,
                              const float* q, const float* tail_key, const float* tail_value,
                              size_t visible, float* out) {
    const tvo_geometry* g = &c->g;
    int rc = check_config(g, heads, context);
    if (rc) return rc;
    const table_t* t = find(c, seq);
    if (!t) return TVO_EINVAL;
    const size_t dim = g->head_dim, width = g->kv_heads * dim, tpb = g->tokens_per_block;
    const int tail = tail_key != NULL;
    if (layer >= g->layers || (tail_key == NULL) != (tail_value == NULL) || t->length > context ||
        (tail && t->length == context))
        return fail(TVO_EINVAL, "invalid fused attention shape");
    const size_t total = t->length + (tail ? 1 : 0);
    if (visible > total) visible = total;
    if (!visible) return fail(TVO_EINVAL, "empty fused attention");
    const size_t cached = visible < t->length ? visible : t->length;
    const double root = sqrt((double)dim);
    online_t state = {0};
    state.dim = dim;
    state.sum = malloc(dim * sizeof(double));
    for (size_t h = 0; h < heads && !rc; ++h) {
        state.maximum = -INFINITY;
        state.normalizer = 0;
        for (size_t i = 0; i < dim; ++i) state.sum[i] = 0;
        const size_t kh = h / (heads / g->kv_heads);
        const float* query = q + h * dim;
        for (size_t b = 0; b < t->nblocks && b * tpb < cached && !rc; ++b) {
            rc = validated(c, t->blocks[b]);
            if (rc) break;
            const float* data = c->values + t->blocks[b].id * c->elements;
            const size_t count = tpb < cached - b * tpb ? tpb : cached - b * tpb;
            for (size_t slot = 0; slot < count && !rc; ++slot) {
                const float* key = data + ((layer * 2 + 0) * tpb + slot) * width + kh * dim;
                const float* value = data + ((layer * 2 + 1) * tpb + slot) * width + kh * dim;
                const double score = tvo_attention_dot(query, key, dim);
                rc = online_update(&state, score / root, value);
            }
        }
        if (!rc && visible > t->length) {
            const double score = tvo_attention_dot(query, tail_key + kh * dim, dim);
            rc = online_update(&state, score / root, tail_value + kh * dim);
        }
        if (!rc) rc = online_finish(&state, out + h * dim);
    }
    free(state.sum);
    return rc;
}

/* fused_prompt_attention (attention.hpp:85-89) */
int tvo_fused_prompt_attention(const tvo_cache* c, uint64_t seq, size_t layer, size_t heads, size_t context,
                               size_t start, size_t count, const float* queries, float* out) {
    int rc = check_config(&c->g, heads, context);
    if (rc) return rc;
    const table_t* t = find(c, seq);
    if (!t) return TVO_EINVAL;
    const size_t length = t->length, hidden = heads * c->g.head_dim;
    if (!count || start >= length || count > length - start)
        return fail(TVO_EINVAL, "invalid causal prompt chunk");
    for (size_t i = 0; i < count && !rc; ++i)
        rc = tvo_fused_paged_attention(c, seq, layer, heads, context, queries + i * hidden, NULL, NULL,
                                       start + i + 1, out + i * hidden);
    return rc;
}

/* --------------------------------------------------------------------- Q8_0 */

/* half_to_float (quant.hpp:14-29) */
float tvo_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t exponent = (h >> 10) & 31, mantissa = h & 1023, bits;
    if (exponent == 0) {
        if (!mantissa) bits = sign;
        else {
            int e = -14;
            while ((mantissa & 1024) == 0) {
                mantissa <<= 1;
                --e;
            }
            bits = sign | ((uint32_t)(e + 127) << 23) | ((mantissa & 1023) << 13);
        }
    } else if (exponent == 31) bits = sign | 0x7f800000u | (mantissa << 13);
    else bits = sign | ((exponent + 112) << 23) | (mantissa << 13);
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* float64 -> float16, round to nearest even (what numpy's '<f2' cast does for
 * the scale in fixture.py:137) */
uint16_t tvo_double_to_half(double x) {
    uint64_t b;
    memcpy(&b, &x, sizeof b);
    const uint16_t sign = (uint16_t)((b >> 48) & 0x8000);
    const int biased = (int)((b >> 52) & 0x7ff);
    const uint64_t mant = b & 0xfffffffffffffULL;
    if (biased == 0x7ff) return (uint16_t)(sign | 0x7c00 | (mant ? 0x200 | (uint16_t)(mant >> 42) : 0));
    const int e = biased - 1023;
    if (e > 15) return (uint16_t)(sign | 0x7c00);
    if (e >= -14) {
        uint32_t h = ((uint32_t)(e + 15) << 10) | (uint32_t)(mant >> 42);
        const uint64_t rem = mant & ((1ULL << 42) - 1), half = 1ULL << 41;
        if (rem > half || (rem == half && (h & 1))) h += 1;
        return (uint16_t)(sign | h);
    }
    if (e < -25 || biased == 0) return sign;
    const uint64_t full = mant | (1ULL << 52);
    const int shift = 28 - e; /* 43 .. 53 */
    uint64_t hm = full >> shift;
    const uint64_t rem = full & ((1ULL << shift) - 1), half = 1ULL << (shift - 1);
    if (rem > half || (rem == half && (hm & 1))) hm += 1;
    return (uint16_t)(sign | hm);
}

/* dequantize_q8_0 (quant.hpp:40-49): x = half_to_float(d) * float(q), f32 */
int tvo_dequantize_q8_0(const uint8_t* bytes, size_t nbytes, float* out, size_t count) {
    if (nbytes % 34 || out == NULL || count != nbytes / 34 * 32)
        return fail(TVO_EINVAL, "quantized storage/output size mismatch");
    for (size_t b = 0; b < nbytes / 34; ++b) {
        const float scale = tvo_half_to_float((uint16_t)(bytes[b * 34] | (bytes[b * 34 + 1] << 8)));
        for (size_t i = 0; i < 32; ++i) out[b * 32 + i] = scale * (float)(int8_t)bytes[b * 34 + 2 + i];
    }
    return TVO_OK;
}

/* Q8_0 encoder of fixture.py:131-137:
 *   scale = float(max|x|) / 127            (float64)
 *   q = clip(round(x / scale), -127, 127)  (x is float32 and the scale a weak
 *                                           Python float, so the division and
 *                                           the half-to-even rounding are f32)
 *   d = float16(scale)                     (float64 -> float16, nearest even)
 * An all-zero block stores q = 0. */
void tvo_quantize_q8_0_block(const float* x, uint8_t* out) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        const float a = fabsf(x[i]);
        if (a > amax || isnan(a)) amax = a;
    }
    const double scale = (double)amax / 127.0;
    const uint16_t d = tvo_double_to_half(scale);
    out[0] = (uint8_t)(d & 0xff);
    out[1] = (uint8_t)(d >> 8);
    if (scale == 0) {
        memset(out + 2, 0, 32);
        return;
    }
    const float s = (float)scale;
    for (int i = 0; i < 32; ++i) {
        float r = nearbyintf(x[i] / s);
        if (r < -127.0f) r = -127.0f;
        if (r > 127.0f) r = 127.0f;
        out[2 + i] = (uint8_t)(int8_t)r;
    }
}

/* tvo_quantize_q8_0_block over `groups` consecutive groups of 32 floats. */
void tvo_quantize_q8_0(const float* x, size_t groups, uint8_t* out) {
    for (size_t g = 0; g < groups; ++g) tvo_quantize_q8_0_block(x + 32 * g, out + 34 * g);
}
