/*
 * oracle.c -- CPU restatement of dlm's paged KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP product
 * (dlm_amd/, libdlmk.so) is compared against.  Only tests/, the smoke() entry
 * in __graft_entry__.py and bench.py's cpu_baseline leg may load it.  The
 * product never links, calls or falls back to anything here.
 *
 * Reference: vedantnimbarte/dlm (Rust).  The reference cannot be built in this
 * image (no Rust toolchain), so oracle/_ref is empty and this restatement is
 * pinned by the reference's own known-answer tests, closed forms and f64
 * brute force (tests/test_oracle_*.py).  Each function below cites the
 * reference code it follows.
 *
 * Arithmetic rules kept from the reference (compile with -ffp-contract=off):
 *   - dot products are a sequential f32 sum of rounded f32 products
 *     (Iterator::sum over a.map(|(a,b)| a*b), src/forward/cpu.rs:806);
 *   - V accumulation is `o += w * v`, a rounded multiply then a rounded add
 *     (src/forward/cpu.rs:829-831);
 *   - softmax is max -> exp(x-max) -> running sum -> divide when sum > 0
 *     (src/forward/cpu.rs:945-957), exp = libm expf as Rust's f32::exp.
 *
 * Parts with no reference counterpart (physical paging, f16 KV, free-order
 * injection, truncate, fork, block copy, swap gather/scatter, multi-query
 * causal verify) are defined here by the contract "paged result == the
 * reference's contiguous result on the same logical sequence".
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_F32 0
#define ORC_F16 1
#define ORC_BF16 2

#define ORC_OK 0
#define ORC_ERR_INVALID -1
#define ORC_ERR_EXHAUSTED -2
#define ORC_ERR_UNKNOWN_SEQ -5

/* ------------------------------------------------------------------------ */
/* Seeded RNG: SplitMix64 as in tests/gpu_parity.rs:30-52.                   */
/* ------------------------------------------------------------------------ */

uint64_t orc_rng_seed(uint64_t seed) { return seed ^ 0x9E3779B97F4A7C15ull; }

uint64_t orc_rng_next(uint64_t *state) {
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Rng::vec (tests/gpu_parity.rs:44-51): uniform in [-scale, scale) from the top
 * 24 bits. */
void orc_rng_uniform(uint64_t seed, float scale, float *out, int64_t n) {
    uint64_t s = orc_rng_seed(seed);
    for (int64_t i = 0; i < n; ++i) {
        float u = (float)(orc_rng_next(&s) >> 40) / (float)(1u << 24);
        out[i] = (u * 2.0f - 1.0f) * scale;
    }
}

/* ------------------------------------------------------------------------ */
/* f16 -> f32, exact: src/storage/safetensors.rs:87-108.                     */
/* ------------------------------------------------------------------------ */

float orc_f16_to_f32(uint16_t h) {
    unsigned sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    float val;
    if (ex == 0)
        val = (float)mant * ldexpf(1.0f, -24);
    else if (ex == 0x1f)
        val = mant == 0 ? INFINITY : NAN;
    else
        val = (1.0f + (float)mant / 1024.0f) * ldexpf(1.0f, (int)ex - 15);
    return sign ? -val : val;
}

/* bf16 -> f32 is a 16-bit shift (the bf16 pattern is the high half of f32). */
static float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float load_elem(const void *base, int64_t idx, int dtype) {
    if (dtype == ORC_F32) return ((const float *)base)[idx];
    if (dtype == ORC_F16) return orc_f16_to_f32(((const uint16_t *)base)[idx]);
    return bf16_to_f32(((const uint16_t *)base)[idx]);
}

static int elem_bytes(int dtype) { return dtype == ORC_F32 ? 4 : 2; }

/* ------------------------------------------------------------------------ */
/* Block geometry: src/cache/paged.rs:23-71.                                 */
/* ------------------------------------------------------------------------ */

typedef struct {
    uint32_t num_layers, num_kv_heads, head_dim, block_size;
} orc_cache_config;

/* KV_DTYPE_BYTES = 2 (paged.rs:26): the budget math always assumes fp16. */
uint64_t orc_bytes_per_token(const orc_cache_config *c) {
    return 2ull * c->num_kv_heads * c->head_dim * 2ull * c->num_layers;
}
uint64_t orc_bytes_per_block(const orc_cache_config *c) {
    return orc_bytes_per_token(c) * c->block_size;
}
uint64_t orc_blocks_for_tokens(const orc_cache_config *c, uint64_t tokens) {
    uint64_t bs = c->block_size;
    return (tokens + bs - 1) / bs; /* u64::div_ceil */
}

/* ------------------------------------------------------------------------ */
/* PagedKvCache bookkeeping: src/cache/paged.rs:106-227.                     */
/* ------------------------------------------------------------------------ */

typedef struct {
    uint64_t id, length;
    uint32_t *blocks;
    uint32_t nblocks, cap;
} orc_seq;

typedef struct {
    orc_cache_config cfg;
    uint32_t total_blocks;
    uint32_t *free; /* LIFO stack; top = free[nfree-1] */
    uint32_t nfree;
    orc_seq *seqs; /* unordered; BTreeMap order is never observable here */
    uint32_t nseqs, seqcap;
} orc_cache;

/* PagedKvCache::new (paged.rs:116-126): free = (0..n).rev(), so popping from
 * the back hands out 0, 1, 2, ... */
orc_cache *orc_cache_new(const orc_cache_config *cfg, uint32_t total_blocks) {
    orc_cache *c = (orc_cache *)calloc(1, sizeof(orc_cache));
    c->cfg = *cfg;
    if (c->cfg.block_size == 0) c->cfg.block_size = 1; /* block_size.max(1), :46 */
    c->total_blocks = total_blocks;
    c->free = (uint32_t *)malloc(sizeof(uint32_t) * (total_blocks ? total_blocks : 1));
    for (uint32_t i = 0; i < total_blocks; ++i) c->free[i] = total_blocks - 1 - i;
    c->nfree = total_blocks;
    return c;
}

/* Extension (no reference counterpart): blocks are handed out in the order
 * `order[0], order[1], ...`, i.e. the stack is `order` reversed.  With
 * order = 0..n it is identical to orc_cache_new. */
orc_cache *orc_cache_new_with_free_order(const orc_cache_config *cfg, const uint32_t *order,
                                         uint32_t n) {
    orc_cache *c = orc_cache_new(cfg, n);
    for (uint32_t i = 0; i < n; ++i) c->free[i] = order[n - 1 - i];
    return c;
}

/* with_budget (paged.rs:130-134). */
orc_cache *orc_cache_with_budget(const orc_cache_config *cfg, uint64_t budget) {
    orc_cache_config c2 = *cfg;
    if (c2.block_size == 0) c2.block_size = 1;
    uint64_t per = orc_bytes_per_block(&c2);
    if (per == 0) per = 1;
    uint64_t n = budget / per;
    if (n > 0xffffffffull) n = 0xffffffffull;
    return orc_cache_new(cfg, (uint32_t)n);
}

void orc_cache_destroy(orc_cache *c) {
    if (!c) return;
    for (uint32_t i = 0; i < c->nseqs; ++i) free(c->seqs[i].blocks);
    free(c->seqs);
    free(c->free);
    free(c);
}

static orc_seq *find_seq(orc_cache *c, uint64_t id) {
    for (uint32_t i = 0; i < c->nseqs; ++i)
        if (c->seqs[i].id == id) return &c->seqs[i];
    return NULL;
}

static orc_seq *insert_seq(orc_cache *c, uint64_t id) {
    if (c->nseqs == c->seqcap) {
        c->seqcap = c->seqcap ? 2 * c->seqcap : 8;
        c->seqs = (orc_seq *)realloc(c->seqs, sizeof(orc_seq) * c->seqcap);
    }
    orc_seq *s = &c->seqs[c->nseqs++];
    memset(s, 0, sizeof(*s));
    s->id = id;
    return s;
}

static void seq_push(orc_seq *s, uint32_t b) {
    if (s->nblocks == s->cap) {
        s->cap = s->cap ? 2 * s->cap : 8;
        s->blocks = (uint32_t *)realloc(s->blocks, sizeof(uint32_t) * s->cap);
    }
    s->blocks[s->nblocks++] = b;
}

/* append_tokens (paged.rs:164-190): check first, then commit; the error carries
 * {requested = to_alloc (saturated to u32), free, total}. */
int orc_cache_append_tokens(orc_cache *c, uint64_t seq_id, uint64_t n, uint32_t err[3]) {
    orc_seq *s = find_seq(c, seq_id);
    uint64_t cur_len = s ? s->length : 0, cur_blocks = s ? s->nblocks : 0;
    uint64_t new_len = cur_len + n;
    uint64_t needed = orc_blocks_for_tokens(&c->cfg, new_len);
    uint64_t to_alloc = needed > cur_blocks ? needed - cur_blocks : 0;
    if (to_alloc > c->nfree) {
        if (err) {
            err[0] = to_alloc > 0xffffffffull ? 0xffffffffu : (uint32_t)to_alloc;
            err[1] = c->nfree;
            err[2] = c->total_blocks;
        }
        return ORC_ERR_EXHAUSTED;
    }
    if (!s) s = insert_seq(c, seq_id);
    for (uint64_t i = 0; i < to_alloc; ++i) seq_push(s, c->free[--c->nfree]);
    s->length = new_len;
    return ORC_OK;
}

static void remove_seq(orc_cache *c, orc_seq *s) {
    free(s->blocks);
    *s = c->seqs[--c->nseqs];
}

/* free_sequence (paged.rs:193-197): blocks go back onto the stack in table
 * order (Vec::extend), so the last block of the table is handed out next. */
void orc_cache_free_sequence(orc_cache *c, uint64_t seq_id) {
    orc_seq *s = find_seq(c, seq_id);
    if (!s) return;
    for (uint32_t i = 0; i < s->nblocks; ++i) c->free[c->nfree++] = s->blocks[i];
    remove_seq(c, s);
}

/* Extension: roll a sequence back to `new_len` tokens (speculative rejection).
 * Whole blocks beyond blocks_for_tokens(new_len) return to the stack from the
 * table's tail backwards, so re-appending the same number of tokens pops the
 * same physical blocks into the same table slots.  new_len >= len is a no-op. */
int orc_cache_truncate_sequence(orc_cache *c, uint64_t seq_id, uint64_t new_len) {
    orc_seq *s = find_seq(c, seq_id);
    if (!s) return ORC_ERR_UNKNOWN_SEQ;
    if (new_len >= s->length) return ORC_OK;
    uint64_t keep = orc_blocks_for_tokens(&c->cfg, new_len);
    while (s->nblocks > keep) c->free[c->nfree++] = s->blocks[--s->nblocks];
    s->length = new_len;
    return ORC_OK;
}

/* Extension: fork `src` into a new sequence `dst` holding a private copy of
 * every block (the paged form of KvSnapshot clone + resume,
 * src/forward/orchestrator.rs:73-105).  Atomic like append_tokens.  Writes
 * (src_block, dst_block) pairs for the device block copy.  dst must be new. */
int orc_cache_fork_sequence(orc_cache *c, uint64_t src, uint64_t dst, int32_t *pairs,
                            uint32_t cap, uint32_t *npairs, uint32_t err[3]) {
    orc_seq *s = find_seq(c, src);
    if (!s) return ORC_ERR_UNKNOWN_SEQ;
    if (find_seq(c, dst)) return ORC_ERR_INVALID;
    uint32_t need = s->nblocks;
    if (need > cap) return ORC_ERR_INVALID;
    if (need > c->nfree) {
        if (err) {
            err[0] = need;
            err[1] = c->nfree;
            err[2] = c->total_blocks;
        }
        return ORC_ERR_EXHAUSTED;
    }
    uint64_t len = s->length;
    uint32_t sidx = (uint32_t)(s - c->seqs);
    orc_seq *d = insert_seq(c, dst); /* may realloc c->seqs */
    s = &c->seqs[sidx];
    for (uint32_t i = 0; i < need; ++i) {
        uint32_t b = c->free[--c->nfree];
        seq_push(d, b);
        pairs[2 * i] = (int32_t)s->blocks[i];
        pairs[2 * i + 1] = (int32_t)b;
    }
    d->length = len;
    *npairs = need;
    return ORC_OK;
}

uint64_t orc_cache_sequence_len(orc_cache *c, uint64_t id) {
    orc_seq *s = find_seq(c, id);
    return s ? s->length : 0;
}

/* block_table (paged.rs:205-207); returns -1 for an unknown sequence. */
int64_t orc_cache_block_table(orc_cache *c, uint64_t id, uint32_t *out, uint64_t cap) {
    orc_seq *s = find_seq(c, id);
    if (!s) return -1;
    for (uint32_t i = 0; i < s->nblocks && i < cap; ++i) out[i] = s->blocks[i];
    return s->nblocks;
}

uint32_t orc_cache_total_blocks(orc_cache *c) { return c->total_blocks; }
uint32_t orc_cache_free_blocks(orc_cache *c) { return c->nfree; }
uint32_t orc_cache_used_blocks(orc_cache *c) { return c->total_blocks - c->nfree; }
uint64_t orc_cache_capacity_tokens(orc_cache *c) {
    return (uint64_t)c->total_blocks * c->cfg.block_size;
}
uint64_t orc_cache_num_sequences(orc_cache *c) { return c->nseqs; }
uint64_t orc_cache_used_tokens(orc_cache *c) {
    uint64_t t = 0;
    for (uint32_t i = 0; i < c->nseqs; ++i) t += c->seqs[i].length;
    return t;
}
/* The free stack, bottom to top, for exact-order comparisons. */
uint32_t orc_cache_free_list(orc_cache *c, uint32_t *out) {
    memcpy(out, c->free, sizeof(uint32_t) * c->nfree);
    return c->nfree;
}

/* ------------------------------------------------------------------------ */
/* Contiguous attention: src/forward/cpu.rs:1126-1151 with softmax_inplace   */
/* (:945-957), key_head_dot / value_head_accumulate for the f32 store        */
/* (:798-846).  keys/values are the KvLayerCache layout [pos][kv_head][d].   */
/* ------------------------------------------------------------------------ */

static void softmax_inplace(float *v, int64_t n) {
    float mx = -INFINITY;
    for (int64_t i = 0; i < n; ++i) mx = fmaxf(mx, v[i]);
    float sum = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        v[i] = expf(v[i] - mx);
        sum += v[i];
    }
    if (sum > 0.0f)
        for (int64_t i = 0; i < n; ++i) v[i] /= sum;
}

/* `scale` is passed in; dlm computes it as 1.0f / sqrtf((float)d) (:1128). */
void orc_attention(const float *q, const float *keys, const float *values, int64_t positions,
                   int num_heads, int num_kv_heads, int head_dim, float scale, float *ctx) {
    int d = head_dim, group = num_heads / num_kv_heads;
    int64_t kv_dim = (int64_t)num_kv_heads * d;
    float *scores = (float *)malloc(sizeof(float) * (positions ? positions : 1));
    for (int h = 0; h < num_heads; ++h) {
        int kvh = h / group;
        const float *qh = q + (int64_t)h * d;
        for (int64_t p = 0; p < positions; ++p) {
            const float *k = keys + p * kv_dim + (int64_t)kvh * d;
            float dot = 0.0f;
            for (int j = 0; j < d; ++j) dot += qh[j] * k[j];
            scores[p] = dot * scale;
        }
        softmax_inplace(scores, positions);
        float *out = ctx + (int64_t)h * d;
        for (int j = 0; j < d; ++j) out[j] = 0.0f;
        for (int64_t p = 0; p < positions; ++p) {
            const float *v = values + p * kv_dim + (int64_t)kvh * d;
            float w = scores[p];
            for (int j = 0; j < d; ++j) out[j] += w * v[j];
        }
    }
    free(scores);
}

/* ------------------------------------------------------------------------ */
/* Physical paging (no reference counterpart; see header).                   */
/*                                                                           */
/* Per-layer pools, one for K and one for V, each [num_blocks][Hkv][tile]:   */
/*   K tile = [d / X][block_size][X]  with X = 16 / elem_bytes (16-byte      */
/*            chunks of X consecutive dims, token-minor inside a chunk row)  */
/*   V tile = [d][block_size]         (dims outer, tokens contiguous)        */
/* The logical view is dlm's [pos][kv_head][d].                              */
/* ------------------------------------------------------------------------ */

static int64_t k_index(int64_t blk, int kvh, int t, int j, int Hkv, int d, int bs, int X) {
    return ((blk * Hkv + kvh) * (int64_t)d * bs) + ((int64_t)(j / X) * bs + t) * X + (j % X);
}
static int64_t v_index(int64_t blk, int kvh, int t, int j, int Hkv, int d, int bs) {
    return ((blk * Hkv + kvh) * (int64_t)d * bs) + (int64_t)j * bs + t;
}

/* Paged append (the physical form of KvLayerCache::append, cpu.rs:765-795 for
 * the f32 store, where extend_from_slice is a bit copy).  src is
 * [n_tok][Hkv][d]; slot = block*bs + offset; a negative slot, or one beyond
 * the pool, is skipped.  Elements are copied as raw bits. */
void orc_paged_append(void *k_pool, void *v_pool, const void *k_src, const void *v_src,
                      const int64_t *slots, int64_t n_tok, int Hkv, int d, int bs, int dtype,
                      int64_t num_blocks) {
    int eb = elem_bytes(dtype), X = 16 / eb;
    for (int64_t i = 0; i < n_tok; ++i) {
        int64_t slot = slots[i];
        if (slot < 0 || slot >= num_blocks * bs) continue;
        int64_t blk = slot / bs;
        int t = (int)(slot % bs);
        for (int h = 0; h < Hkv; ++h)
            for (int j = 0; j < d; ++j) {
                int64_t s = (i * Hkv + h) * (int64_t)d + j;
                memcpy((char *)k_pool + k_index(blk, h, t, j, Hkv, d, bs, X) * eb,
                       (const char *)k_src + s * eb, eb);
                memcpy((char *)v_pool + v_index(blk, h, t, j, Hkv, d, bs) * eb,
                       (const char *)v_src + s * eb, eb);
            }
    }
}

/* Logical view of the first `ctx` tokens of a sequence as f32 [pos][Hkv][d]
 * (exact f16/bf16 widening). */
void orc_paged_gather_logical(const void *k_pool, const void *v_pool, const int32_t *table,
                              int64_t ctx, int Hkv, int d, int bs, int dtype, float *keys,
                              float *values) {
    int X = 16 / elem_bytes(dtype);
    for (int64_t p = 0; p < ctx; ++p) {
        int64_t blk = table[p / bs];
        int t = (int)(p % bs);
        for (int h = 0; h < Hkv; ++h)
            for (int j = 0; j < d; ++j) {
                int64_t o = (p * Hkv + h) * (int64_t)d + j;
                keys[o] = load_elem(k_pool, k_index(blk, h, t, j, Hkv, d, bs, X), dtype);
                values[o] = load_elem(v_pool, v_index(blk, h, t, j, Hkv, d, bs), dtype);
            }
    }
}

/* Paged GQA attention: attention() (cpu.rs:1126-1151) with key_head_dot /
 * value_head_accumulate (:798-846) reading through the block table instead
 * of a contiguous Vec; same arithmetic order, elements widened exactly to f32.
 *
 * q is [B][nq][Hq][d] in `dtype`; out is [B][nq][Hq][d] f32.
 * Multi-query verify: query j of sequence s attends to the first
 * ctx_lens[s] - nq + j + 1 tokens (causal over the nq appended drafts).
 * A query with no visible token gets zeros (softmax of an empty vector). */
void orc_paged_attention(float *out, const void *q, const void *k_pool, const void *v_pool,
                         int dtype, const int32_t *tables, const int32_t *ctx_lens, int B,
                         int nq, int Hq, int Hkv, int d, int bs, int max_blocks, float scale) {
    int X = 16 / elem_bytes(dtype), group = Hq / Hkv;
    int64_t maxctx = 0;
    for (int s = 0; s < B; ++s)
        if (ctx_lens[s] > maxctx) maxctx = ctx_lens[s];
    float *scores = (float *)malloc(sizeof(float) * (maxctx ? maxctx : 1));
    float *qh = (float *)malloc(sizeof(float) * d);
    for (int s = 0; s < B; ++s) {
        const int32_t *table = tables + (int64_t)s * max_blocks;
        for (int qi = 0; qi < nq; ++qi) {
            int64_t positions = (int64_t)ctx_lens[s] - nq + qi + 1;
            if (positions < 0) positions = 0;
            for (int h = 0; h < Hq; ++h) {
                int kvh = h / group;
                int64_t row = ((int64_t)s * nq + qi) * Hq + h;
                for (int j = 0; j < d; ++j) qh[j] = load_elem(q, row * d + j, dtype);
                for (int64_t p = 0; p < positions; ++p) {
                    int64_t blk = table[p / bs];
                    int t = (int)(p % bs);
                    float dot = 0.0f;
                    for (int j = 0; j < d; ++j)
                        dot += qh[j] *
                               load_elem(k_pool, k_index(blk, kvh, t, j, Hkv, d, bs, X), dtype);
                    scores[p] = dot * scale;
                }
                softmax_inplace(scores, positions);
                float *o = out + row * d;
                for (int j = 0; j < d; ++j) o[j] = 0.0f;
                for (int64_t p = 0; p < positions; ++p) {
                    int64_t blk = table[p / bs];
                    int t = (int)(p % bs);
                    float w = scores[p];
                    for (int j = 0; j < d; ++j)
                        o[j] += w * load_elem(v_pool, v_index(blk, kvh, t, j, Hkv, d, bs), dtype);
                }
            }
        }
    }
    free(qh);
    free(scores);
}

/* Block copy for fork: for each (src, dst) pair, the dst block of both pools
 * becomes a byte copy of the src block.  Pairs are applied in order. */
void orc_copy_blocks(void *k_pool, void *v_pool, const int32_t *pairs, int64_t n,
                     int64_t block_bytes) {
    for (int64_t i = 0; i < n; ++i) {
        int64_t s = pairs[2 * i], d = pairs[2 * i + 1];
        memmove((char *)k_pool + d * block_bytes, (char *)k_pool + s * block_bytes, block_bytes);
        memmove((char *)v_pool + d * block_bytes, (char *)v_pool + s * block_bytes, block_bytes);
    }
}

/* Swap-out gather: staging is [n][2][block_bytes] (K block then V block). */
void orc_gather_blocks(void *staging, const void *k_pool, const void *v_pool,
                       const int32_t *ids, int64_t n, int64_t block_bytes) {
    for (int64_t i = 0; i < n; ++i) {
        memcpy((char *)staging + (2 * i) * block_bytes, (const char *)k_pool + ids[i] * block_bytes,
               block_bytes);
        memcpy((char *)staging + (2 * i + 1) * block_bytes,
               (const char *)v_pool + ids[i] * block_bytes, block_bytes);
    }
}

/* Swap-in scatter: inverse of orc_gather_blocks. */
void orc_scatter_blocks(void *k_pool, void *v_pool, const void *staging, const int32_t *ids,
                        int64_t n, int64_t block_bytes) {
    for (int64_t i = 0; i < n; ++i) {
        memcpy((char *)k_pool + ids[i] * block_bytes, (const char *)staging + (2 * i) * block_bytes,
               block_bytes);
        memcpy((char *)v_pool + ids[i] * block_bytes,
               (const char *)staging + (2 * i + 1) * block_bytes, block_bytes);
    }
}

/* ------------------------------------------------------------------------ */
/* Per-token KV quantization: src/forward/cpu.rs:667-711.                    */
/* ------------------------------------------------------------------------ */

/* `(v / scale).round().clamp(-qmax, qmax) as i8` (:680, :696): round half
 * away from zero, clamp, and Rust's saturating float->int cast, which sends NaN
 * (from inf / inf, or a NaN element) to 0. */
static int saturating_code(float r, float qmax) {
    r = roundf(r);
    if (r != r) return 0;
    return (int)fminf(fmaxf(r, -qmax), qmax);
}

/* quantize_i8 (:667-680): scale = max|x| / 127; q = round(x/scale) clamped. */
float orc_quantize_i8(const float *x, int64_t n, int8_t *q) {
    float mx = 0.0f;
    for (int64_t i = 0; i < n; ++i) mx = fmaxf(mx, fabsf(x[i]));
    float scale = mx / 127.0f;
    if (!(scale > 0.0f)) {
        memset(q, 0, n);
        return 0.0f;
    }
    for (int64_t i = 0; i < n; ++i) q[i] = (int8_t)saturating_code(x[i] / scale, 127.0f);
    return scale;
}

/* quantize_i4 (:685-700): scale = max|x| / 7; nibbles two per byte, element i
 * in byte i/2, low nibble for even i. */
float orc_quantize_i4(const float *x, int64_t n, uint8_t *packed) {
    memset(packed, 0, (n + 1) / 2);
    float mx = 0.0f;
    for (int64_t i = 0; i < n; ++i) mx = fmaxf(mx, fabsf(x[i]));
    float scale = mx / 7.0f;
    if (!(scale > 0.0f)) return 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        int8_t q = (int8_t)saturating_code(x[i] / scale, 7.0f);
        uint8_t nib = (uint8_t)q & 0x0f;
        packed[i / 2] |= (i % 2 == 0) ? nib : (uint8_t)(nib << 4);
    }
    return scale;
}

/* read_i4 (:706-711). */
float orc_read_i4(const uint8_t *packed, int64_t base, int64_t i) {
    uint8_t byte = packed[base + i / 2];
    uint8_t nib = (i % 2 == 0) ? (byte & 0x0f) : (byte >> 4);
    int code = nib >= 8 ? (int)nib - 16 : (int)nib;
    return (float)code;
}

/* ------------------------------------------------------------------------ */
/* Quantized KV store (KvStore::Int8 / Int4, src/forward/cpu.rs:641-661) and */
/* its attention (key_head_dot / value_head_accumulate, :798-846).           */
/* Contiguous reference layout: int8 codes [pos][kv_dim]; int4 codes packed  */
/* [pos][ceil(kv_dim/2)] (element i in byte i/2, low nibble for even i);     */
/* one f32 scale per position for K and one for V.                           */
/* ------------------------------------------------------------------------ */

#define ORC_I8 3
#define ORC_I4 4

static float quant_code(const void *codes, int64_t row_base, int64_t i, int quant) {
    if (quant == ORC_I8) return (float)((const int8_t *)codes)[row_base + i];
    return orc_read_i4((const uint8_t *)codes, row_base, i);
}

static int64_t quant_row_bytes(int64_t kv_dim, int quant) {
    return quant == ORC_I8 ? kv_dim : (kv_dim + 1) / 2;
}

/* attention() over a quantized history: a * (code * s) per key element
 * (:808-818) and o += w * (code * s) per value element (:833-845). */
void orc_attention_quant(const float *q, const void *kcodes, const float *kscales,
                         const void *vcodes, const float *vscales, int64_t positions,
                         int num_heads, int num_kv_heads, int head_dim, float scale, int quant,
                         float *ctx) {
    int d = head_dim, group = num_heads / num_kv_heads;
    int64_t kv_dim = (int64_t)num_kv_heads * d, rb = quant_row_bytes(kv_dim, quant);
    float *scores = (float *)malloc(sizeof(float) * (positions ? positions : 1));
    for (int h = 0; h < num_heads; ++h) {
        int kvh = h / group;
        const float *qh = q + (int64_t)h * d;
        for (int64_t p = 0; p < positions; ++p) {
            float s = kscales[p], dot = 0.0f;
            for (int j = 0; j < d; ++j)
                dot += qh[j] * (quant_code(kcodes, p * rb, (int64_t)kvh * d + j, quant) * s);
            scores[p] = dot * scale;
        }
        softmax_inplace(scores, positions);
        float *out = ctx + (int64_t)h * d;
        for (int j = 0; j < d; ++j) out[j] = 0.0f;
        for (int64_t p = 0; p < positions; ++p) {
            float s = vscales[p], w = scores[p];
            for (int j = 0; j < d; ++j)
                out[j] += w * (quant_code(vcodes, p * rb, (int64_t)kvh * d + j, quant) * s);
        }
    }
    free(scores);
}

/* KvLayerCache::append for the quantized stores (:780-793): quantize each
 * token's K and V over the whole kv_dim; codes go to the contiguous layout. */
void orc_quantize_tokens(const float *src, int64_t n_tok, int64_t kv_dim, int quant, void *codes,
                         float *scales) {
    int64_t rb = quant_row_bytes(kv_dim, quant);
    for (int64_t i = 0; i < n_tok; ++i) {
        if (quant == ORC_I8)
            scales[i] = orc_quantize_i8(src + i * kv_dim, kv_dim, (int8_t *)codes + i * rb);
        else
            scales[i] = orc_quantize_i4(src + i * kv_dim, kv_dim, (uint8_t *)codes + i * rb);
    }
}

/* Paged quantized pools (layout of this build, no reference counterpart).
 * head_dim d is a multiple of 64.  Elements are 8-bit codes (int8) or 4-bit
 * codes two to a byte (int4, low nibble the even element), stored offset
 * binary: the byte c + 128, the nibble c + 8.
 *   K tile of one (block, kv head): [d/KG][16 tokens][KG dims], KG = 16
 *     (int8) or, for int4, 32 when d % 128 == 0 else 16 -- one token's KG
 *     consecutive dims fill 16 bytes (8 for int4 at d = 64).
 *   V tile: [d/(16 VG)][4 token quads][16 dim groups][VG dims][4 tokens],
 *     VG = 4 (int8) or, for int4, 8 when d % 128 == 0 else 4; an int4 byte
 *     holds one token's dims 2p, 2p + 1 (low nibble 2p), so a byte never
 *     mixes tokens and appends never share one.
 *   scales: K and V f32 [nb][16], one per token (shared by all heads). */
static void put_nibble(uint8_t *b, int hi, int code) {
    uint8_t nib = (uint8_t)code & 0x0f;
    *b = hi ? (uint8_t)((*b & 0x0f) | (nib << 4)) : (uint8_t)((*b & 0xf0) | nib);
}
/* Pool codes are offset binary: int8 code c is the byte c + 128, int4 code c
 * the nibble c + 8 (the contiguous reference rows stay two's complement). */
static void pool_put(void *pool, int64_t off, int hi, int code, int quant) {
    if (quant == ORC_I8) {
        ((uint8_t *)pool)[off] = (uint8_t)(code + 128);
        return;
    }
    uint8_t *b = (uint8_t *)pool + off, nib = (uint8_t)(code + 8) & 0x0f;
    *b = hi ? (uint8_t)((*b & 0x0f) | (nib << 4)) : (uint8_t)((*b & 0xf0) | nib);
}
static int pool_get(const void *pool, int64_t off, int hi, int quant) {
    const uint8_t b = ((const uint8_t *)pool)[off];
    if (quant == ORC_I8) return (int)b - 128;
    return (int)(hi ? (b >> 4) : (b & 0x0f)) - 8;
}

int orc_quant_k_group(int d, int quant) { return quant == ORC_I8 ? 16 : (d % 128 == 0 ? 32 : 16); }
int orc_quant_v_group(int d, int quant) { return quant == ORC_I8 ? 4 : (d % 128 == 0 ? 8 : 4); }

/* Byte offset of element (token t, dim j) of kv head h in block blk; for int4
 * the element is nibble j % 2 of that byte. */
static int64_t qk_off(int64_t blk, int h, int t, int j, int Hkv, int d, int quant) {
    int64_t tile = (blk * Hkv + h) * (int64_t)d * 16 * (quant == ORC_I8 ? 2 : 1) / 2;
    int kg = orc_quant_k_group(d, quant);
    int64_t el = ((int64_t)(j / kg) * 16 + t) * kg + (j % kg);
    return tile + (quant == ORC_I8 ? el : el / 2);
}
static int64_t qv_off(int64_t blk, int h, int t, int j, int Hkv, int d, int quant) {
    int64_t tile = (blk * Hkv + h) * (int64_t)d * 16 * (quant == ORC_I8 ? 2 : 1) / 2;
    int vg = orc_quant_v_group(d, quant), per = 16 * vg;
    int q = j / per, r = j % per, n = r / vg, kk = r % vg;
    int lane_bytes = quant == ORC_I8 ? 4 * vg : 2 * vg;
    int word = quant == ORC_I8 ? kk : kk / 2;
    return tile + ((int64_t)(q * 4 + t / 4) * 16 + n) * lane_bytes + word * 4 + t % 4;
}

/* Quantize n_tok tokens (src [n][Hkv][d] f32) and scatter codes + scales. */
void orc_paged_append_quant(void *k_pool, void *v_pool, float *k_scales, float *v_scales,
                            const float *k_src, const float *v_src, const int64_t *slots,
                            int64_t n_tok, int Hkv, int d, int bs, int quant, int64_t num_blocks) {
    int64_t kv_dim = (int64_t)Hkv * d, rb = quant_row_bytes(kv_dim, quant);
    void *kc = malloc(rb), *vc = malloc(rb);
    for (int64_t i = 0; i < n_tok; ++i) {
        int64_t slot = slots[i];
        if (slot < 0 || slot >= num_blocks * bs) continue;
        int64_t blk = slot / bs;
        int t = (int)(slot % bs);
        float ks, vs;
        orc_quantize_tokens(k_src + i * kv_dim, 1, kv_dim, quant, kc, &ks);
        orc_quantize_tokens(v_src + i * kv_dim, 1, kv_dim, quant, vc, &vs);
        k_scales[slot] = ks;
        v_scales[slot] = vs;
        for (int h = 0; h < Hkv; ++h)
            for (int j = 0; j < d; ++j) {
                int e = h * d + j;
                int kq = (int)quant_code(kc, 0, e, quant), vq = (int)quant_code(vc, 0, e, quant);
                int64_t ko = qk_off(blk, h, t, j, Hkv, d, quant);
                int64_t vo = qv_off(blk, h, t, j, Hkv, d, quant);
                pool_put(k_pool, ko, j % 2, kq, quant);
                pool_put(v_pool, vo, j % 2, vq, quant);
            }
    }
    free(kc);
    free(vc);
}

/* Logical view of a paged quantized sequence in the reference's contiguous
 * layout (codes + per-position scales). */
void orc_paged_gather_quant(const void *k_pool, const void *v_pool, const float *k_scales,
                            const float *v_scales, const int32_t *table, int64_t ctx, int Hkv,
                            int d, int bs, int quant, void *kcodes, float *ks, void *vcodes,
                            float *vs) {
    int64_t kv_dim = (int64_t)Hkv * d, rb = quant_row_bytes(kv_dim, quant);
    memset(kcodes, 0, rb * ctx);
    memset(vcodes, 0, rb * ctx);
    for (int64_t p = 0; p < ctx; ++p) {
        int64_t blk = table[p / bs];
        int t = (int)(p % bs);
        ks[p] = k_scales[blk * bs + t];
        vs[p] = v_scales[blk * bs + t];
        for (int h = 0; h < Hkv; ++h)
            for (int j = 0; j < d; ++j) {
                int64_t e = (int64_t)h * d + j;
                int64_t ko = qk_off(blk, h, t, j, Hkv, d, quant);
                int64_t vo = qv_off(blk, h, t, j, Hkv, d, quant);
                if (quant == ORC_I8) {
                    ((int8_t *)kcodes)[p * rb + e] = (int8_t)pool_get(k_pool, ko, 0, quant);
                    ((int8_t *)vcodes)[p * rb + e] = (int8_t)pool_get(v_pool, vo, 0, quant);
                } else {
                    uint8_t *kb = (uint8_t *)kcodes + p * rb + e / 2;
                    uint8_t *vb = (uint8_t *)vcodes + p * rb + e / 2;
                    put_nibble(kb, (int)(e % 2), pool_get(k_pool, ko, j % 2, quant));
                    put_nibble(vb, (int)(e % 2), pool_get(v_pool, vo, j % 2, quant));
                }
            }
    }
}

/* Paged quantized attention: gather each sequence's logical history, then
 * orc_attention_quant per query (causal over the nq newest tokens).  q is f32
 * [B][nq][Hq][d]; out f32 [B][nq][Hq][d]. */
void orc_paged_attention_quant(float *out, const float *q, const void *k_pool, const void *v_pool,
                               const float *k_scales, const float *v_scales, int quant,
                               const int32_t *tables, const int32_t *ctx_lens, int B, int nq,
                               int Hq, int Hkv, int d, int bs, int max_blocks, float scale) {
    int64_t kv_dim = (int64_t)Hkv * d, rb = quant_row_bytes(kv_dim, quant);
    for (int s = 0; s < B; ++s) {
        int64_t ctx = ctx_lens[s] > 0 ? ctx_lens[s] : 0;
        void *kc = malloc(rb * (ctx ? ctx : 1)), *vc = malloc(rb * (ctx ? ctx : 1));
        float *ks = (float *)malloc(sizeof(float) * (ctx ? ctx : 1));
        float *vs = (float *)malloc(sizeof(float) * (ctx ? ctx : 1));
        orc_paged_gather_quant(k_pool, v_pool, k_scales, v_scales, tables + (int64_t)s * max_blocks,
                               ctx, Hkv, d, bs, quant, kc, ks, vc, vs);
        for (int qi = 0; qi < nq; ++qi) {
            int64_t positions = ctx - nq + qi + 1;
            if (positions < 0) positions = 0;
            int64_t row = (int64_t)s * nq + qi;
            orc_attention_quant(q + row * Hq * d, kc, ks, vc, vs, positions, Hq, Hkv, d, scale,
                                quant, out + row * Hq * d);
        }
        free(kc);
        free(vc);
        free(ks);
        free(vs);
    }
}

/* ======================================================================== */
/* One decode block (the caller of the paged path): decode_block,           */
/* src/forward/cpu.rs:1156-1219, with its KvLayerCache replaced by a paged  */
/* f32 pool and a block table.                                              */
/* ======================================================================== */

#define ORC_W_F32 0
#define ORC_W_BF16 1
#define ORC_W_F16 2
#define ORC_W_INT4 3
#define ORC_W_INT8 4

/* QuantLayout (src/forward/cpu.rs:132-159): [codes][pad to 4][scales g x f32]
 * [zeros g x f32], g = ceil(n / group_size). */
typedef struct {
    int64_t scales_off, zeros_off, num_groups, total_bytes;
} orc_qlayout;

static orc_qlayout qlayout(int dtype, int64_t n, int64_t group_size) {
    orc_qlayout L;
    int64_t code_bytes = dtype == ORC_W_INT4 ? (n + 1) / 2 : n;
    L.scales_off = (code_bytes + 3) / 4 * 4;
    L.num_groups = (n + (group_size > 0 ? group_size : 1) - 1) / (group_size > 0 ? group_size : 1);
    L.zeros_off = L.scales_off + L.num_groups * 4;
    L.total_bytes = L.zeros_off + L.num_groups * 4;
    return L;
}

int64_t orc_quant_blob_bytes(int dtype, int64_t n, int64_t group_size) {
    return qlayout(dtype, n, group_size).total_bytes;
}

static float blob_f32(const uint8_t *blob, int64_t off) {
    float f;
    memcpy(&f, blob + off, 4);
    return f;
}

/* Weights::get (src/forward/cpu.rs:204-217): element i as f32.  bf16 is the
 * high half of an f32 (:171-174); f16 via the exact decoder above; int4 /
 * int8 per int4_get / int8_get (:321-347): (code - zero) * scale of the
 * element's group, codes low-nibble-first. */
float orc_weight_get(const void *w, int dtype, int64_t n, int64_t group_size, int64_t i) {
    const uint8_t *b = (const uint8_t *)w;
    switch (dtype) {
        case ORC_W_F32: return ((const float *)w)[i];
        case ORC_W_BF16: return bf16_to_f32(((const uint16_t *)w)[i]);
        case ORC_W_F16: return orc_f16_to_f32(((const uint16_t *)w)[i]);
        default: {
            orc_qlayout L = qlayout(dtype, n, group_size);
            float code = dtype == ORC_W_INT4 ? (float)((i % 2 == 0) ? (b[i / 2] & 0x0F) : (b[i / 2] >> 4))
                                             : (float)b[i];
            int64_t g = i / group_size;
            return (code - blob_f32(b, L.zeros_off + g * 4)) * blob_f32(b, L.scales_off + g * 4);
        }
    }
}

/* quantize_groups (src/quant/dequant.rs:200-236) packed into the blob layout
 * by Weights::quantize_int4 / quantize_int8 (src/forward/cpu.rs:237-305):
 * per group, scale = (max - min) / levels (1 when max - min < f32::EPSILON),
 * zero = -min / scale, code = round((v - min) / scale) clamped to [0, levels]
 * (f32::round: half away from zero, C roundf).  blob must hold
 * orc_quant_blob_bytes(dtype, n, group_size) bytes. */
int orc_quantize_weights(const float *values, int64_t n, int64_t group_size, int dtype,
                         uint8_t *blob) {
    if (group_size <= 0 || (dtype != ORC_W_INT4 && dtype != ORC_W_INT8)) return ORC_ERR_INVALID;
    orc_qlayout L = qlayout(dtype, n, group_size);
    float levels = dtype == ORC_W_INT4 ? 15.0f : 255.0f;
    memset(blob, 0, (size_t)L.total_bytes);
    for (int64_t g = 0; g < L.num_groups; ++g) {
        int64_t start = g * group_size, end = start + group_size < n ? start + group_size : n;
        float mn = INFINITY, mx = -INFINITY;
        for (int64_t i = start; i < end; ++i) {
            mn = fminf(mn, values[i]);
            mx = fmaxf(mx, values[i]);
        }
        float scale = fabsf(mx - mn) < 1.1920929e-7f ? 1.0f : (mx - mn) / levels;
        float zero = -mn / scale;
        for (int64_t i = start; i < end; ++i) {
            float c = roundf((values[i] - mn) / scale);
            c = c < 0.0f ? 0.0f : (c > levels ? levels : c);
            uint8_t code = (uint8_t)c;
            if (dtype == ORC_W_INT8)
                blob[i] = code;
            else
                blob[i / 2] |= (uint8_t)((code & 0x0F) << (i % 2 ? 4 : 0));
        }
        memcpy(blob + L.scales_off + g * 4, &scale, 4);
        memcpy(blob + L.zeros_off + g * 4, &zero, 4);
    }
    return ORC_OK;
}

/* matvec / matvec_native (src/forward/cpu.rs:852-903): y[o] is the sequential
 * f32 sum over j of get(o * in_dim + j) * x[j] (Iterator::sum).  `n` is the
 * matrix's element count, for the quantized layouts. */
void orc_matvec(const void *w, int dtype, int64_t group_size, const float *x, int64_t out_dim,
                int64_t in_dim, float *y) {
    int64_t n = out_dim * in_dim;
    for (int64_t o = 0; o < out_dim; ++o) {
        float s = 0.0f;
        for (int64_t j = 0; j < in_dim; ++j)
            s += orc_weight_get(w, dtype, n, group_size, o * in_dim + j) * x[j];
        y[o] = s;
    }
}

/* rmsnorm (src/forward/cpu.rs:934-943): mean of squares (sequential sum / n),
 * inv = 1 / sqrt(mean + eps), out = v * inv * w. */
void orc_rmsnorm(const float *x, const float *w, int64_t n, float eps, float *out) {
    float ss = 0.0f;
    for (int64_t i = 0; i < n; ++i) ss += x[i] * x[i];
    float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] * inv * w[i];
}

/* silu (src/forward/cpu.rs:960-962). */
float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* rope_inv_freqs (src/forward/cpu.rs:1057-1092).  scaling: 0 none, 1 linear
 * (factor), 2 llama3 (factor, low_freq_factor, high_freq_factor,
 * original_max_position). */
void orc_rope_inv_freqs(int head_dim, float theta, int scaling, float factor, float low_ff,
                        float high_ff, float orig_max, float *out) {
    for (int i = 0; i < head_dim / 2; ++i) {
        float base = powf(theta, -2.0f * (float)i / (float)head_dim);
        float f = base;
        if (scaling == 1) {
            f = base / factor;
        } else if (scaling == 2) {
            float wavelen = 2.0f * 3.14159265358979323846f / base;
            float low_wavelen = orig_max / low_ff, high_wavelen = orig_max / high_ff;
            if (wavelen > low_wavelen) {
                f = base / factor;
            } else if (wavelen < high_wavelen) {
                f = base;
            } else {
                float smooth = (orig_max / wavelen - low_ff) / (high_ff - low_ff);
                f = (1.0f - smooth) * base / factor + smooth * base;
            }
        }
        out[i] = f;
    }
}

/* rope_inplace (src/forward/cpu.rs:1094-1114): NeoX split-half rotation of
 * each head's (i, i + d/2) pair by position * inv_freq[i]. */
void orc_rope(float *v, int num_heads, int head_dim, int64_t position, const float *inv_freq) {
    int half = head_dim / 2;
    for (int h = 0; h < num_heads; ++h) {
        int64_t base = (int64_t)h * head_dim;
        for (int i = 0; i < half; ++i) {
            float angle = (float)position * inv_freq[i];
            float s = sinf(angle), c = cosf(angle);
            float a = v[base + i], b = v[base + i + half];
            v[base + i] = a * c - b * s;
            v[base + i + half] = a * s + b * c;
        }
    }
}

typedef struct {
    int hidden_size, num_heads, num_kv_heads, head_dim, inter;
    float rms_eps;
    int w_dtype;
    int64_t w_group_size;
} orc_block_config;

/* decode_block (src/forward/cpu.rs:1156-1219), dense SwiGLU FFN, with the KV
 * history in a paged f32 pool: the token goes to position num_positions of
 * the sequence (slot table[p / bs] * bs + p % bs), then attention runs over
 * positions 0..num_positions through the table.  Biases may be NULL.  x is
 * the hidden state, updated in place. */
int orc_decode_block_paged(const orc_block_config *c, const void *q_proj, const void *k_proj,
                           const void *v_proj, const void *o_proj, const void *gate_proj,
                           const void *up_proj, const void *down_proj, const float *in_norm,
                           const float *post_norm, const float *q_bias, const float *k_bias,
                           const float *v_bias, const float *inv_freq, float *x, void *k_pool,
                           void *v_pool, const int32_t *table, int max_blocks, int64_t num_blocks,
                           int bs, int64_t num_positions, int64_t position) {
    int H = c->hidden_size, Hq = c->num_heads, Hkv = c->num_kv_heads, d = c->head_dim;
    int qd = Hq * d, kvd = Hkv * d, I = c->inter, dt = c->w_dtype;
    int64_t gs = c->w_group_size;
    if ((num_positions + 1 + bs - 1) / bs > max_blocks) return ORC_ERR_INVALID;
    float *normed = malloc(sizeof(float) * H), *q = malloc(sizeof(float) * qd);
    float *k = malloc(sizeof(float) * kvd), *v = malloc(sizeof(float) * kvd);
    float *ctx = malloc(sizeof(float) * qd), *attn = malloc(sizeof(float) * H);
    float *gate = malloc(sizeof(float) * I), *up = malloc(sizeof(float) * I);
    float *down = malloc(sizeof(float) * H);

    orc_rmsnorm(x, in_norm, H, c->rms_eps, normed);
    orc_matvec(q_proj, dt, gs, normed, qd, H, q);
    orc_matvec(k_proj, dt, gs, normed, kvd, H, k);
    orc_matvec(v_proj, dt, gs, normed, kvd, H, v);
    if (q_bias) for (int i = 0; i < qd; ++i) q[i] += q_bias[i];
    if (k_bias) for (int i = 0; i < kvd; ++i) k[i] += k_bias[i];
    if (v_bias) for (int i = 0; i < kvd; ++i) v[i] += v_bias[i];
    orc_rope(q, Hq, d, position, inv_freq);
    orc_rope(k, Hkv, d, position, inv_freq);

    int64_t slot = (int64_t)table[num_positions / bs] * bs + num_positions % bs;
    orc_paged_append(k_pool, v_pool, k, v, &slot, 1, Hkv, d, bs, ORC_F32, num_blocks);
    int32_t ctx_len = (int32_t)(num_positions + 1);
    orc_paged_attention(ctx, q, k_pool, v_pool, ORC_F32, table, &ctx_len, 1, 1, Hq, Hkv, d, bs,
                        max_blocks, 1.0f / sqrtf((float)d));
    orc_matvec(o_proj, dt, gs, ctx, H, qd, attn);
    for (int i = 0; i < H; ++i) x[i] = x[i] + attn[i];

    orc_rmsnorm(x, post_norm, H, c->rms_eps, normed);
    orc_matvec(gate_proj, dt, gs, normed, I, H, gate);
    orc_matvec(up_proj, dt, gs, normed, I, H, up);
    for (int i = 0; i < I; ++i) gate[i] = orc_silu(gate[i]) * up[i];
    orc_matvec(down_proj, dt, gs, gate, H, I, down);
    for (int i = 0; i < H; ++i) x[i] += down[i];

    free(normed); free(q); free(k); free(v); free(ctx); free(attn);
    free(gate); free(up); free(down);
    return ORC_OK;
}
