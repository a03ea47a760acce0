// Block-table KV store: host bookkeeping behind the dlmk_cache_* C ABI.
//
// Follows PagedKvCache (src/cache/paged.rs:106-227): a LIFO stack of free
// block ids, an ordered map of per-sequence {length, block table}, and an
// append that checks capacity before committing anything.  Extensions for the
// paged hot path: an injectable free order (seeded shuffled pools), truncate
// (speculative rollback), fork by block copy (KvSnapshot clone) and fork by
// shared blocks (prefix cache without copying), and the device-side views
// (slot mappings, padded block tables).
//
// Shared blocks carry a reference count (one per table that lists them); a
// block returns to the free list when its count drops to zero.  Only the
// block holding position `length` can be written (appends go to the end), so
// the one rule sharing needs is that a sequence never appends into a shared
// partially-filled last block: dlmk_cache_append_tokens refuses that case and
// dlmk_cache_append_tokens_cow first gives the sequence a private copy of the
// block (returning the copy for the caller to run on the device).

#include <cstring>
#include <map>
#include <new>
#include <vector>

#include "dlmk.h"
#include "dlmk_internal.h"

struct dlmk_kv_cache {
    dlmk_kv_cache_config cfg;
    uint32_t total_blocks = 0;
    std::vector<uint32_t> free;  // top of stack = back()
    std::vector<uint32_t> refs;  // per block: number of tables listing it (0 = free)
    struct Seq {
        uint64_t length = 0;
        std::vector<uint32_t> blocks;
    };
    std::map<uint64_t, Seq> seqs;
};

namespace {

dlmk_kv_cache_config normalized(const dlmk_kv_cache_config *cfg) {
    dlmk_kv_cache_config c = *cfg;
    if (c.block_size == 0) c.block_size = 1;  // block_size.max(1), paged.rs:46
    return c;
}

// Drop one reference to block b; a block nobody lists goes back on the stack.
void release(dlmk_kv_cache *c, uint32_t b) {
    if (--c->refs[b] == 0) c->free.push_back(b);
}

uint32_t take_free(dlmk_kv_cache *c) {
    uint32_t b = c->free.back();
    c->free.pop_back();
    c->refs[b] = 1;
    return b;
}

// True when the sequence's last block is partially filled and listed by
// another table too: the next append would write into another sequence's
// tokens' block.
bool shared_partial_tail(const dlmk_kv_cache *c, const dlmk_kv_cache::Seq &s) {
    return !s.blocks.empty() && s.length % c->cfg.block_size != 0 && c->refs[s.blocks.back()] > 1;
}

void set_exhausted(dlmk_kv_exhausted *err, uint64_t requested, uint32_t free, uint32_t total) {
    if (!err) return;
    err->requested = requested > 0xffffffffull ? 0xffffffffu : (uint32_t)requested;
    err->free = free;
    err->total = total;
}

// Append n tokens to seq_id; with cow, first replace a shared partial last
// block by a private copy (pair = {shared, private}).  Capacity for both is
// checked before anything changes (paged.rs:164-190: check, then commit).
int append_impl(dlmk_kv_cache *c, uint64_t seq_id, uint64_t n, bool cow, int32_t *pair,
                uint32_t *n_pairs, dlmk_kv_exhausted *err, const char *who) {
    auto it = c->seqs.find(seq_id);
    const bool exists = it != c->seqs.end();
    uint64_t cur_len = exists ? it->second.length : 0;
    uint64_t cur_blocks = exists ? it->second.blocks.size() : 0;
    const bool must_copy = exists && n > 0 && shared_partial_tail(c, it->second);
    if (must_copy && !cow)
        return dlmk::fail(DLMK_ERR_INVALID_ARG,
                          "%s: sequence %llu ends in a shared partially-filled block; append "
                          "with dlmk_cache_append_tokens_cow", who, (unsigned long long)seq_id);
    uint64_t new_len = cur_len + n;
    uint64_t needed = dlmk_blocks_for_tokens(&c->cfg, new_len);
    uint64_t to_alloc = (needed > cur_blocks ? needed - cur_blocks : 0) + (must_copy ? 1 : 0);
    if (to_alloc > c->free.size()) {
        set_exhausted(err, to_alloc, (uint32_t)c->free.size(), c->total_blocks);
        return dlmk::fail(DLMK_ERR_KV_EXHAUSTED, "KV cache pool exhausted: need %llu more block(s), %u free of %u",
                          (unsigned long long)to_alloc, (unsigned)c->free.size(), c->total_blocks);
    }
    auto &seq = c->seqs[seq_id];
    if (n_pairs) *n_pairs = 0;
    if (must_copy) {
        const uint32_t shared = seq.blocks.back();
        const uint32_t mine = take_free(c);
        release(c, shared);  // still listed elsewhere: count stays >= 1
        seq.blocks.back() = mine;
        pair[0] = (int32_t)shared;
        pair[1] = (int32_t)mine;
        *n_pairs = 1;
    }
    while (seq.blocks.size() < needed) seq.blocks.push_back(take_free(c));
    seq.length = new_len;
    return DLMK_OK;
}

}  // namespace

extern "C" {

uint64_t dlmk_bytes_per_token(const dlmk_kv_cache_config *cfg) {
    // 2 (K,V) x heads x dim x 2 bytes x layers (paged.rs:52-58).
    return 2ull * cfg->num_kv_heads * cfg->head_dim * 2ull * cfg->num_layers;
}

uint64_t dlmk_bytes_per_block(const dlmk_kv_cache_config *cfg) {
    dlmk_kv_cache_config c = normalized(cfg);
    return dlmk_bytes_per_token(&c) * c.block_size;
}

uint64_t dlmk_blocks_for_tokens(const dlmk_kv_cache_config *cfg, uint64_t tokens) {
    uint64_t bs = cfg->block_size ? cfg->block_size : 1;
    return tokens / bs + (tokens % bs != 0);
}

dlmk_kv_cache *dlmk_cache_new(const dlmk_kv_cache_config *cfg, uint32_t total_blocks) {
    if (!cfg) {
        dlmk::set_error("dlmk_cache_new: null config");
        return nullptr;
    }
    auto *c = new (std::nothrow) dlmk_kv_cache;
    if (!c) return nullptr;
    c->cfg = normalized(cfg);
    c->total_blocks = total_blocks;
    // Low ids first: the stack holds n-1 ... 0 (paged.rs:118-119).
    c->free.resize(total_blocks);
    for (uint32_t i = 0; i < total_blocks; ++i) c->free[i] = total_blocks - 1 - i;
    c->refs.assign(total_blocks, 0);
    return c;
}

dlmk_kv_cache *dlmk_cache_with_budget(const dlmk_kv_cache_config *cfg, uint64_t budget_bytes) {
    if (!cfg) return nullptr;
    uint64_t per = dlmk_bytes_per_block(cfg);
    if (per == 0) per = 1;
    uint64_t n = budget_bytes / per;
    if (n > 0xffffffffull) n = 0xffffffffull;
    return dlmk_cache_new(cfg, (uint32_t)n);
}

dlmk_kv_cache *dlmk_cache_new_with_free_order(const dlmk_kv_cache_config *cfg,
                                              const uint32_t *order, uint32_t n) {
    if (!cfg || (n && !order)) {
        dlmk::set_error("dlmk_cache_new_with_free_order: null argument");
        return nullptr;
    }
    std::vector<char> seen(n, 0);
    for (uint32_t i = 0; i < n; ++i) {
        if (order[i] >= n || seen[order[i]]) {
            dlmk::set_error("dlmk_cache_new_with_free_order: order is not a permutation of 0..n");
            return nullptr;
        }
        seen[order[i]] = 1;
    }
    dlmk_kv_cache *c = dlmk_cache_new(cfg, n);
    if (!c) return nullptr;
    for (uint32_t i = 0; i < n; ++i) c->free[i] = order[n - 1 - i];
    return c;
}

void dlmk_cache_destroy(dlmk_kv_cache *cache) { delete cache; }

int dlmk_cache_append_tokens(dlmk_kv_cache *c, uint64_t seq_id, uint64_t n,
                             dlmk_kv_exhausted *err) {
    if (!c) return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_cache_append_tokens: null cache");
    return append_impl(c, seq_id, n, false, nullptr, nullptr, err, "dlmk_cache_append_tokens");
}

int dlmk_cache_append_tokens_cow(dlmk_kv_cache *c, uint64_t seq_id, uint64_t n,
                                 int32_t *cow_pair, uint32_t *n_pairs, dlmk_kv_exhausted *err) {
    if (!c || !cow_pair || !n_pairs)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_cache_append_tokens_cow: null argument");
    return append_impl(c, seq_id, n, true, cow_pair, n_pairs, err, "dlmk_cache_append_tokens_cow");
}

void dlmk_cache_free_sequence(dlmk_kv_cache *c, uint64_t seq_id) {
    if (!c) return;
    auto it = c->seqs.find(seq_id);
    if (it == c->seqs.end()) return;
    // Table order (paged.rs:195); shared blocks stay until their last table goes.
    for (uint32_t b : it->second.blocks) release(c, b);
    c->seqs.erase(it);
}

int dlmk_cache_truncate_sequence(dlmk_kv_cache *c, uint64_t seq_id, uint64_t new_len) {
    if (!c) return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_cache_truncate_sequence: null cache");
    auto it = c->seqs.find(seq_id);
    if (it == c->seqs.end())
        return dlmk::fail(DLMK_ERR_UNKNOWN_SEQ, "truncate: unknown sequence %llu",
                          (unsigned long long)seq_id);
    auto &seq = it->second;
    if (new_len >= seq.length) return DLMK_OK;
    uint64_t keep = dlmk_blocks_for_tokens(&c->cfg, new_len);
    while (seq.blocks.size() > keep) {
        release(c, seq.blocks.back());
        seq.blocks.pop_back();
    }
    seq.length = new_len;
    return DLMK_OK;
}

int dlmk_cache_fork_sequence(dlmk_kv_cache *c, uint64_t src_seq, uint64_t dst_seq,
                             int32_t *pairs, uint32_t pairs_capacity, uint32_t *n_pairs,
                             dlmk_kv_exhausted *err) {
    if (!c || !n_pairs) return dlmk::fail(DLMK_ERR_INVALID_ARG, "fork: null argument");
    auto it = c->seqs.find(src_seq);
    if (it == c->seqs.end())
        return dlmk::fail(DLMK_ERR_UNKNOWN_SEQ, "fork: unknown source sequence %llu",
                          (unsigned long long)src_seq);
    if (c->seqs.count(dst_seq))
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "fork: destination sequence %llu exists",
                          (unsigned long long)dst_seq);
    const uint64_t need = it->second.blocks.size();
    if (need > pairs_capacity || (need && !pairs))
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "fork: pairs buffer holds %u, need %llu",
                          pairs_capacity, (unsigned long long)need);
    if (need > c->free.size()) {
        set_exhausted(err, need, (uint32_t)c->free.size(), c->total_blocks);
        return dlmk::fail(DLMK_ERR_KV_EXHAUSTED, "fork: KV cache pool exhausted");
    }
    const uint64_t len = it->second.length;
    std::vector<uint32_t> src_blocks = it->second.blocks;
    auto &dst = c->seqs[dst_seq];
    for (uint64_t i = 0; i < need; ++i) {
        uint32_t b = take_free(c);
        dst.blocks.push_back(b);
        pairs[2 * i] = (int32_t)src_blocks[i];
        pairs[2 * i + 1] = (int32_t)b;
    }
    dst.length = len;
    *n_pairs = (uint32_t)need;
    return DLMK_OK;
}

int dlmk_cache_fork_sequence_shared(dlmk_kv_cache *c, uint64_t src_seq, uint64_t dst_seq) {
    if (!c) return dlmk::fail(DLMK_ERR_INVALID_ARG, "fork_shared: null cache");
    auto it = c->seqs.find(src_seq);
    if (it == c->seqs.end())
        return dlmk::fail(DLMK_ERR_UNKNOWN_SEQ, "fork_shared: unknown source sequence %llu",
                          (unsigned long long)src_seq);
    if (c->seqs.count(dst_seq))
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "fork_shared: destination sequence %llu exists",
                          (unsigned long long)dst_seq);
    dlmk_kv_cache::Seq copy = it->second;
    for (uint32_t b : copy.blocks) ++c->refs[b];
    c->seqs.emplace(dst_seq, std::move(copy));
    return DLMK_OK;
}

uint32_t dlmk_cache_block_refcount(const dlmk_kv_cache *c, uint32_t block) {
    return c && block < c->total_blocks ? c->refs[block] : 0;
}

uint64_t dlmk_cache_sequence_len(const dlmk_kv_cache *c, uint64_t seq_id) {
    if (!c) return 0;
    auto it = c->seqs.find(seq_id);
    return it == c->seqs.end() ? 0 : it->second.length;
}

int64_t dlmk_cache_block_table(const dlmk_kv_cache *c, uint64_t seq_id, uint32_t *out,
                               uint64_t cap) {
    if (!c) return -1;
    auto it = c->seqs.find(seq_id);
    if (it == c->seqs.end()) return -1;
    const auto &b = it->second.blocks;
    if (out)
        for (uint64_t i = 0; i < b.size() && i < cap; ++i) out[i] = b[i];
    return (int64_t)b.size();
}

uint64_t dlmk_cache_num_sequences(const dlmk_kv_cache *c) { return c ? c->seqs.size() : 0; }

void dlmk_cache_stats(const dlmk_kv_cache *c, dlmk_kv_cache_stats *out) {
    if (!c || !out) return;
    std::memset(out, 0, sizeof(*out));
    out->total_blocks = c->total_blocks;
    out->free_blocks = (uint32_t)c->free.size();
    out->used_blocks = c->total_blocks - out->free_blocks;
    out->num_sequences = c->seqs.size();
    for (const auto &kv : c->seqs) out->used_tokens += kv.second.length;
    out->capacity_tokens = (uint64_t)c->total_blocks * c->cfg.block_size;
    out->bytes_per_block = dlmk_bytes_per_block(&c->cfg);
}

uint32_t dlmk_cache_free_list(const dlmk_kv_cache *c, uint32_t *out, uint32_t cap) {
    if (!c) return 0;
    if (out)
        for (uint32_t i = 0; i < c->free.size() && i < cap; ++i) out[i] = c->free[i];
    return (uint32_t)c->free.size();
}

int dlmk_cache_slot_mapping(const dlmk_kv_cache *c, uint64_t seq_id, uint64_t start_pos,
                            uint64_t n, int64_t *slot_mapping) {
    if (!c || (n && !slot_mapping)) return dlmk::fail(DLMK_ERR_INVALID_ARG, "slot_mapping: null argument");
    auto it = c->seqs.find(seq_id);
    if (it == c->seqs.end())
        return dlmk::fail(DLMK_ERR_UNKNOWN_SEQ, "slot_mapping: unknown sequence %llu",
                          (unsigned long long)seq_id);
    const auto &seq = it->second;
    if (start_pos + n > seq.length)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "slot_mapping: tokens [%llu, %llu) beyond length %llu",
                          (unsigned long long)start_pos, (unsigned long long)(start_pos + n),
                          (unsigned long long)seq.length);
    const uint64_t bs = c->cfg.block_size;
    for (uint64_t i = 0; i < n; ++i) {
        uint64_t p = start_pos + i;
        slot_mapping[i] = (int64_t)seq.blocks[p / bs] * (int64_t)bs + (int64_t)(p % bs);
    }
    return DLMK_OK;
}

int dlmk_cache_fill_block_tables(const dlmk_kv_cache *c, const uint64_t *seq_ids,
                                 uint32_t n_seqs, uint32_t max_blocks, int32_t *block_tables,
                                 int32_t *ctx_lens) {
    if (!c || (n_seqs && (!seq_ids || !block_tables || !ctx_lens)))
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "fill_block_tables: null argument");
    for (uint32_t s = 0; s < n_seqs; ++s) {
        int32_t *row = block_tables + (size_t)s * max_blocks;
        auto it = c->seqs.find(seq_ids[s]);
        if (it == c->seqs.end()) {
            std::memset(row, 0, sizeof(int32_t) * max_blocks);
            ctx_lens[s] = 0;
            continue;
        }
        const auto &seq = it->second;
        if (seq.blocks.size() > max_blocks || seq.length > 0x7fffffffull)
            return dlmk::fail(DLMK_ERR_INVALID_ARG, "fill_block_tables: sequence %llu has %zu blocks > max %u",
                              (unsigned long long)seq_ids[s], seq.blocks.size(), max_blocks);
        for (uint32_t i = 0; i < max_blocks; ++i)
            row[i] = i < seq.blocks.size() ? (int32_t)seq.blocks[i] : 0;
        ctx_lens[s] = (int32_t)seq.length;
    }
    return DLMK_OK;
}

}  // extern "C"
