/*
 * dlmk.h -- C ABI of the MI355X (gfx950) paged KV-cache library, libdlmk.so.
 *
 * Drop-in for dlm's paged KV-cache path (vedantnimbarte/dlm).  The reference
 * keeps KV bookkeeping in Rust (src/cache/paged.rs) and reaches the GPU through
 * one extern "C" entry, dlm_decode_block (src/gpu/kernels.cu:313-392, declared
 * in src/forward/gpu.rs:34-64), whose KV part is a contiguous copy_kernel append
 * (kernels.cu:361-363) and attention_kernel (kernels.cu:365-366).  This header
 * replaces those with paged equivalents plus the block-table store itself.
 *
 * Conventions (following dlm_decode_block, kernels.cu:378-391):
 *   - every function returns int: 0 on success, a positive hipError_t from the
 *     HIP runtime, or a negative DLMK_ERR_* code for an argument/state error;
 *     dlmk_get_last_error_string() describes the last failure on this thread;
 *   - device entry points take an explicit hipStream_t (passed as void*; NULL is
 *     the null stream), only enqueue work, and never synchronise;
 *   - every buffer is caller-owned; pointers named *_pool, q, out, slot_mapping,
 *     block_tables, ctx_lens, pairs, block_ids, workspace and staging are device
 *     pointers; host_* pointers are pinned host memory;
 *   - no torch types appear anywhere: plain pointers and sizes.
 *
 * Physical layout of one layer's pools (both pools hold num_blocks blocks):
 *   K pool: [num_blocks][num_kv_heads][head_dim / X][block_size][X]
 *   V pool: [num_blocks][num_kv_heads][head_dim][block_size]
 * with X = 16 / element bytes (8 for f16/bf16, 4 for f32), so every K row of a
 * block is a run of 16-byte chunks and one (block, kv head) tile is contiguous.
 * The logical view is dlm's KvLayerCache layout [pos][kv_head][head_dim]
 * (src/forward/cpu.rs:802): token p of a sequence lives in block
 * table[p / block_size] at offset p % block_size.
 */
#ifndef DLMK_H
#define DLMK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DLMK_ABI_VERSION 1

/* Element types of K/V pools, queries and outputs; DLMK_I8 / DLMK_I4 are the
 * quantized pool formats (dlm's KvQuant::Int8 / Int4, src/forward/cpu.rs:627-639). */
enum dlmk_dtype { DLMK_F32 = 0, DLMK_F16 = 1, DLMK_BF16 = 2, DLMK_I8 = 3, DLMK_I4 = 4 };

/* Projection weight dtypes of dlmk_decode_block_paged: dlm's DLM_W_* tags
 * (src/gpu/kernels.cu:61-65, Weights::dtype_code at src/forward/cpu.rs:307-317),
 * same values.  INT4 / INT8 are dlm's group-affine blobs: codes (int4 two a
 * byte, low nibble first), padded to 4 bytes, then ceil(n / group) f32 scales,
 * then as many f32 zero-points; element = (code - zero) * scale (QuantLayout,
 * src/forward/cpu.rs:132-159). */
enum dlmk_wdtype { DLMK_W_F32 = 0, DLMK_W_BF16 = 1, DLMK_W_F16 = 2, DLMK_W_INT4 = 3, DLMK_W_INT8 = 4 };

/* Negative status codes (positive values are hipError_t). */
#define DLMK_OK 0
#define DLMK_ERR_INVALID_ARG -1 /* DlmError::ShapeMismatch / InvalidConfig analogue */
#define DLMK_ERR_KV_EXHAUSTED -2 /* DlmError::KvCacheExhausted, src/error.rs:70-75 */
#define DLMK_ERR_UNSUPPORTED -3 /* shape/dtype combination with no kernel */
#define DLMK_ERR_WORKSPACE -4 /* workspace or staging buffer too small */
#define DLMK_ERR_UNKNOWN_SEQ -5 /* sequence id not present */

/* Library identity and last error (thread-local). */
int dlmk_abi_version(void);
const char *dlmk_get_last_error_string(void);

/* ======================================================================== */
/* Block-table KV store (host bookkeeping).                                 */
/* Replaces PagedKvCache, src/cache/paged.rs:106-227, with the same LIFO    */
/* free list, atomic append and error payload, plus an injectable free      */
/* order, truncate (speculative rollback) and fork (block-copy prefix        */
/* sharing).  Not thread-safe: one thread drives a cache at a time, as dlm's */
/* engine thread does (src/forward/gpu.rs:196-200).                         */
/* ======================================================================== */

/* KvCacheConfig, src/cache/paged.rs:30-40. */
typedef struct dlmk_kv_cache_config {
    uint32_t num_layers;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t block_size;
} dlmk_kv_cache_config;

/* KvCacheStats, src/cache/paged.rs:83-92. */
typedef struct dlmk_kv_cache_stats {
    uint32_t total_blocks;
    uint32_t used_blocks;
    uint32_t free_blocks;
    uint32_t _pad;
    uint64_t num_sequences;
    uint64_t used_tokens;
    uint64_t capacity_tokens;
    uint64_t bytes_per_block;
} dlmk_kv_cache_stats;

/* Payload of DLMK_ERR_KV_EXHAUSTED (DlmError::KvCacheExhausted, error.rs:70-75). */
typedef struct dlmk_kv_exhausted {
    uint32_t requested;
    uint32_t free;
    uint32_t total;
} dlmk_kv_exhausted;

typedef struct dlmk_kv_cache dlmk_kv_cache;

/* KvCacheConfig::{bytes_per_token, bytes_per_block, blocks_for_tokens},
 * src/cache/paged.rs:52-71 (bytes assume 2-byte elements, paged.rs:26). */
uint64_t dlmk_bytes_per_token(const dlmk_kv_cache_config *cfg);
uint64_t dlmk_bytes_per_block(const dlmk_kv_cache_config *cfg);
uint64_t dlmk_blocks_for_tokens(const dlmk_kv_cache_config *cfg, uint64_t tokens);

/* PagedKvCache::new, paged.rs:116-126 (ids handed out 0, 1, 2, ...). */
dlmk_kv_cache *dlmk_cache_new(const dlmk_kv_cache_config *cfg, uint32_t total_blocks);
/* PagedKvCache::with_budget, paged.rs:130-134. */
dlmk_kv_cache *dlmk_cache_with_budget(const dlmk_kv_cache_config *cfg, uint64_t budget_bytes);
/* Extension: a pool of n blocks handed out in the order order[0], order[1], ...
 * (a seeded shuffle of the pool); each id in [0, n) exactly once. NULL on error. */
dlmk_kv_cache *dlmk_cache_new_with_free_order(const dlmk_kv_cache_config *cfg,
                                              const uint32_t *order, uint32_t n);
void dlmk_cache_destroy(dlmk_kv_cache *cache);

/* append_tokens, paged.rs:164-190.  Atomic: on DLMK_ERR_KV_EXHAUSTED nothing
 * changes and *err (if non-NULL) holds {requested, free, total}.  A sequence
 * whose partially-filled last block is shared (dlmk_cache_fork_sequence_shared)
 * gets DLMK_ERR_INVALID_ARG: append it with dlmk_cache_append_tokens_cow. */
int dlmk_cache_append_tokens(dlmk_kv_cache *cache, uint64_t seq_id, uint64_t n,
                             dlmk_kv_exhausted *err);
/* free_sequence, paged.rs:193-197 (blocks return in table order; no-op if
 * unknown).  A shared block returns when the last table listing it goes. */
void dlmk_cache_free_sequence(dlmk_kv_cache *cache, uint64_t seq_id);
/* Extension: roll back to new_len tokens; freed tail blocks return last-first,
 * so re-appending pops the same blocks.  new_len >= len is a no-op. */
int dlmk_cache_truncate_sequence(dlmk_kv_cache *cache, uint64_t seq_id, uint64_t new_len);
/* Extension: new sequence dst with a private copy of src's blocks (paged
 * KvSnapshot clone, src/forward/orchestrator.rs:73-105).  Writes n (src, dst)
 * block pairs (host int32[n][2]) for dlmk_copy_blocks.  Atomic on exhaustion. */
int dlmk_cache_fork_sequence(dlmk_kv_cache *cache, uint64_t src_seq, uint64_t dst_seq,
                             int32_t *pairs, uint32_t pairs_capacity, uint32_t *n_pairs,
                             dlmk_kv_exhausted *err);

/* Extension, prefix sharing without copies (the paged form of dlm's prefix
 * cache, which clones a KvSnapshot: src/batching.rs:32-72,
 * src/forward/orchestrator.rs:73-105).  dst lists exactly src's blocks; each
 * block's reference count grows by one and nothing is allocated or copied.
 * Full blocks are never written again, so they stay shared for good; before
 * either sequence appends into a shared partially-filled last block it must
 * go through dlmk_cache_append_tokens_cow. */
int dlmk_cache_fork_sequence_shared(dlmk_kv_cache *cache, uint64_t src_seq, uint64_t dst_seq);
/* Extension: append_tokens that first replaces a shared partially-filled last
 * block by a private block.  *n_pairs is 0 or 1; when 1, cow_pair (host
 * int32[2]) = {shared block, private block}, to be copied with
 * dlmk_copy_blocks before the sequence's new tokens are written.  Capacity for
 * the copy and the new blocks is checked first (atomic, as append_tokens). */
int dlmk_cache_append_tokens_cow(dlmk_kv_cache *cache, uint64_t seq_id, uint64_t n,
                                 int32_t *cow_pair, uint32_t *n_pairs, dlmk_kv_exhausted *err);
/* Number of block tables listing `block` (0: free or out of range). */
uint32_t dlmk_cache_block_refcount(const dlmk_kv_cache *cache, uint32_t block);
/* sequence_len, paged.rs:200-202 (0 if unknown). */
uint64_t dlmk_cache_sequence_len(const dlmk_kv_cache *cache, uint64_t seq_id);
/* block_table, paged.rs:205-207: copies up to cap ids into out (may be NULL)
 * and returns the table length, or -1 for an unknown sequence. */
int64_t dlmk_cache_block_table(const dlmk_kv_cache *cache, uint64_t seq_id, uint32_t *out,
                               uint64_t cap);
/* num_sequences / stats, paged.rs:210-227 and the pool counters :137-160. */
uint64_t dlmk_cache_num_sequences(const dlmk_kv_cache *cache);
void dlmk_cache_stats(const dlmk_kv_cache *cache, dlmk_kv_cache_stats *out);
/* The free stack bottom-to-top (top is handed out next); returns its length. */
uint32_t dlmk_cache_free_list(const dlmk_kv_cache *cache, uint32_t *out, uint32_t cap);

/* Device-side views of the books (host arrays, to be uploaded by the caller).
 * slot_mapping: slots of tokens [start_pos, start_pos+n) of seq_id
 * (slot = block * block_size + offset); those tokens must already be appended.
 * block_tables: row s = table of seq_ids[s] padded with 0 to max_blocks;
 * ctx_lens[s] = its length (DLMK_ERR_INVALID_ARG if a table is longer). */
int dlmk_cache_slot_mapping(const dlmk_kv_cache *cache, uint64_t seq_id, uint64_t start_pos,
                            uint64_t n, int64_t *slot_mapping);
int dlmk_cache_fill_block_tables(const dlmk_kv_cache *cache, const uint64_t *seq_ids,
                                 uint32_t n_seqs, uint32_t max_blocks, int32_t *block_tables,
                                 int32_t *ctx_lens);

/* ======================================================================== */
/* Device entry points (hand-written HIP for gfx950).                       */
/* ======================================================================== */

/* Paged KV append: replaces copy_kernel x2 at kernels.cu:361-363 (and
 * KvLayerCache::append, src/forward/cpu.rs:765-795).  k_src/v_src are
 * [n_tok][num_kv_heads][head_dim]; token i goes to slot_mapping[i].  A negative
 * slot, or one >= num_blocks * block_size, is skipped.  A bit copy (f32, f16,
 * bf16).  Per-token decode and per-chunk prefill alike.  Pools and sources
 * must be 16-byte aligned, else DLMK_ERR_INVALID_ARG. */
int dlmk_kv_append(void *stream, void *k_pool, void *v_pool, const void *k_src,
                   const void *v_src, const int64_t *slot_mapping, int64_t n_tok,
                   int num_kv_heads, int head_dim, int block_size, int64_t num_blocks,
                   int dtype);

/* Workspace bytes dlmk_paged_decode_attention needs for these bounds. */
size_t dlmk_paged_attention_workspace_size(int num_seqs, int num_q_per_seq, int num_q_heads,
                                           int head_dim, int block_size, int max_blocks_per_seq);

/* Paged GQA decode attention: replaces attention_kernel at kernels.cu:210-242
 * (launched at :365-366) and attention() at src/forward/cpu.rs:1126-1151.
 *   q   [num_seqs][num_q_per_seq][num_q_heads][head_dim], same dtype as the pools
 *   out [num_seqs][num_q_per_seq][num_q_heads][head_dim], out_dtype
 *   block_tables int32 [num_seqs][max_blocks_per_seq], ctx_lens int32 [num_seqs]
 * Query j of sequence s attends causally to the first
 * ctx_lens[s] - num_q_per_seq + j + 1 tokens (num_q_per_seq > 1 is the
 * speculative-verify case; 1 is plain decode); a query with no visible token
 * gets zeros.  score = dot(q, k) * scale; softmax; out = sum p * v.
 * Block ids outside [0, num_blocks) are treated as masked tokens; a context
 * length above max_blocks_per_seq * block_size is clamped to it.
 * Contexts are split into fixed partitions processed in parallel and merged by
 * log-sum-exp in a second pass; workspace holds the partials
 * (>= dlmk_paged_attention_workspace_size bytes, 256-byte aligned).
 * Geometry: block_size 16; any num_q_heads / num_kv_heads group and
 * num_q_per_seq; head_dim a multiple of 4 (f32) or 8 (f16, bf16) up to 256;
 * otherwise DLMK_ERR_UNSUPPORTED.  q and the pools (and, for the step and
 * quantized variants, the new tokens and the scales) must be 16-byte
 * aligned, else DLMK_ERR_INVALID_ARG. */
int dlmk_paged_decode_attention(void *stream, void *out, int out_dtype, const void *q,
                                const void *k_pool, const void *v_pool, int dtype,
                                const int32_t *block_tables, const int32_t *ctx_lens,
                                int num_seqs, int num_q_per_seq, int num_q_heads,
                                int num_kv_heads, int head_dim, int block_size,
                                int max_blocks_per_seq, int64_t num_blocks, float scale,
                                void *workspace, size_t workspace_bytes);

/* Fused decode step: appends each sequence's num_q_per_seq newest tokens and
 * runs dlmk_paged_decode_attention over them in the same launches, with no
 * separate append kernel (the reference does the two back to back inside
 * dlm_decode_block, kernels.cu:361-366): the attention reads the new tokens
 * from k_new / v_new, and the pools are written by the split-K combine
 * launch, or by the partition launch when there is no combine.
 * k_new / v_new are [num_seqs][num_q_per_seq][num_kv_heads][head_dim] in the
 * pool dtype; token j of sequence s goes to position ctx_lens[s] -
 * num_q_per_seq + j through block_tables (so ctx_lens already counts them and
 * the table already holds their blocks, as PagedKvCache::append_tokens
 * leaves it).  The pools receive exactly the bits dlmk_kv_append would write;
 * out equals dlmk_kv_append followed by dlmk_paged_decode_attention. */
int dlmk_paged_decode_step(void *stream, void *out, int out_dtype, const void *q, void *k_pool,
                           void *v_pool, int dtype, const void *k_new, const void *v_new,
                           const int32_t *block_tables, const int32_t *ctx_lens, int num_seqs,
                           int num_q_per_seq, int num_q_heads, int num_kv_heads, int head_dim,
                           int block_size, int max_blocks_per_seq, int64_t num_blocks, float scale,
                           void *workspace, size_t workspace_bytes);

/* Allocation-free paged decode attention.  No counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as dlmk_paged_decode_attention without the workspace:
 * the split-K partials live in a library-owned device array of
 * DLMK_NOALLOC_SCRATCH_BYTES per GPU (allocated with the code object, kept
 * until the process ends).  Calls whose partials would exceed it return
 * DLMK_ERR_WORKSPACE before launching anything.  Nothing in the array needs
 * to start at zero; every call on one GPU shares it, so calls that overlap on
 * one GPU (concurrent streams) race.  Never calls hipMalloc or hipFree. */
#define DLMK_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int dlmk_paged_decode_attention_noalloc(void *stream, void *out, int out_dtype, const void *q,
                                        const void *k_pool, const void *v_pool, int dtype,
                                        const int32_t *block_tables, const int32_t *ctx_lens,
                                        int num_seqs, int num_q_per_seq, int num_q_heads,
                                        int num_kv_heads, int head_dim, int block_size,
                                        int max_blocks_per_seq, int64_t num_blocks, float scale);

/* Quantized KV pools (dlm's --kv-quant int8 / int4, KvLayerCache at
 * src/forward/cpu.rs:622-711).  Each token carries one f32 scale per pool over
 * its whole kv_dim (num_kv_heads * head_dim values): scale = max|x| / qmax
 * (qmax 127 / 7), code = round-half-away(x / scale) clamped to +-qmax, and an
 * all-zero token has scale 0 and zero codes.  head_dim is a multiple of 64.
 * Codes are stored offset binary: int8 code c as the byte c + 128, int4 code
 * c as the nibble c + 8, two to a byte (low nibble the even element).
 * Layouts per layer (block_size 16), each (block, kv head) tile:
 *   K [d/KG][16 tokens][KG dims]: KG = 16 (int8); int4 KG = 32 if
 *     d % 128 == 0, else 16.
 *   V [d/(16 VG)][4 token quads][16][VG dims][4 tokens]: VG = 4 (int8);
 *     int4 VG = 8 if d % 128 == 0, else 4 (an int4 byte holds one token's
 *     dims 2p and 2p+1).  Dim j of token t sits at quarter j / (16 VG), quad
 *     t / 4, group (j / VG) % 16, element j % VG, token t % 4.
 *   scales: k_scales / v_scales f32 [num_blocks][16] (slot order).
 * Each lane of the attention kernel loads 16 bytes of a tile at a time (8 at
 * int4 d = 64, where a whole tile is 512 bytes).
 * Append: replaces KvLayerCache::append's quantizing branch (cpu.rs:765-795,
 * quantize_i8 / quantize_i4 at :672-711).  k_src / v_src are
 * [n_tok][num_kv_heads][head_dim] in src_dtype (f32, f16, bf16); token i goes
 * to slot_mapping[i]; negative or out-of-pool slots are skipped.  quant is
 * DLMK_I8 or DLMK_I4. */
int dlmk_kv_append_quant(void *stream, void *k_pool, void *v_pool, float *k_scales,
                         float *v_scales, const void *k_src, const void *v_src, int src_dtype,
                         const int64_t *slot_mapping, int64_t n_tok, int num_kv_heads,
                         int head_dim, int block_size, int64_t num_blocks, int quant);

/* Paged decode attention over quantized pools: replaces attention() with
 * key_head_dot / value_head_accumulate's dequantizing branches
 * (cpu.rs:798-846, :1126-1151).  q is f16; every other argument, the
 * causal rule, masking and the workspace are as in dlmk_paged_decode_attention
 * (the same workspace size function applies).  Scores are
 * dot(q, k_code) * k_scale * scale; values are v_code * v_scale. */
int dlmk_paged_decode_attention_quant(void *stream, void *out, int out_dtype, const void *q,
                                      const void *k_pool, const void *v_pool,
                                      const float *k_scales, const float *v_scales, int quant,
                                      const int32_t *block_tables, const int32_t *ctx_lens,
                                      int num_seqs, int num_q_per_seq, int num_q_heads,
                                      int num_kv_heads, int head_dim, int block_size,
                                      int max_blocks_per_seq, int64_t num_blocks, float scale,
                                      void *workspace, size_t workspace_bytes);

/* Block copy for fork / copy-on-write: for each pairs[i] = (src, dst) (device
 * int32[n][2]) copy block src to block dst in both pools.  block_bytes is the
 * size of one block of one pool (num_kv_heads * block_size * head_dim * elem
 * bytes), a multiple of 16.  Pairs must not chain (no dst is another's src).
 * Ids outside [0, num_blocks) are skipped.  The pools (and below, the
 * staging buffer) must be 16-byte aligned, else DLMK_ERR_INVALID_ARG. */
int dlmk_copy_blocks(void *stream, void *k_pool, void *v_pool, const int32_t *pairs, int64_t n,
                     size_t block_bytes, int64_t num_blocks);

/* Swap gather: staging (device) [n][2][block_bytes] <- (K block, V block) of
 * block_ids[i].  Swap scatter is the inverse.  Ids outside the pool are skipped. */
int dlmk_gather_blocks(void *stream, void *staging, const void *k_pool, const void *v_pool,
                       const int32_t *block_ids, int64_t n, size_t block_bytes,
                       int64_t num_blocks);
int dlmk_scatter_blocks(void *stream, void *k_pool, void *v_pool, const void *staging,
                        const int32_t *block_ids, int64_t n, size_t block_bytes,
                        int64_t num_blocks);

/* Swap out to / in from pinned host memory: gather into dev_staging, then one
 * hipMemcpyAsync D2H (swap_out); or one H2D then scatter (swap_in).  host_buf is
 * [n][2][block_bytes]; dev_staging must hold 2 * n * block_bytes.  The async
 * copy is the PCIe analogue of dlm's pinned streaming upload
 * (src/forward/streaming_gpu.rs:139-164; src/gpu/ffi_hip.rs:44-50). */
int dlmk_swap_out(void *stream, void *host_buf, const void *k_pool, const void *v_pool,
                  const int32_t *block_ids, int64_t n, size_t block_bytes, int64_t num_blocks,
                  void *dev_staging, size_t staging_bytes);
int dlmk_swap_in(void *stream, void *k_pool, void *v_pool, const void *host_buf,
                 const int32_t *block_ids, int64_t n, size_t block_bytes, int64_t num_blocks,
                 void *dev_staging, size_t staging_bytes);

/* One decode block over the paged cache: replaces dlm_decode_block
 * (src/gpu/kernels.cu:313-392, declared at src/forward/gpu.rs:34-64; the CPU
 * oracle is decode_block, src/forward/cpu.rs:1156-1219).  Same arguments in
 * the same order, with three changes:
 *   - kv_keys / kv_values (one contiguous f32 history per kernel) become this
 *     layer's f32 pools k_pool [num_blocks][num_kv_heads][head_dim/4][16][4]
 *     and v_pool [num_blocks][num_kv_heads][head_dim][16], addressed through
 *     the sequence's device block table (int32 [max_blocks_per_seq]);
 *   - an explicit stream, first, instead of the default stream;
 *   - a caller-owned workspace (dlmk_decode_block_workspace_size bytes,
 *     256-byte aligned) instead of thread_local scratch (kernels.cu:283-306).
 * The new token's K (after RoPE) and V go to position num_positions
 * (block block_table[num_positions / 16], offset num_positions % 16; those
 * blocks must already be the sequence's, as PagedKvCache::append_tokens
 * leaves them); attention covers positions 0..num_positions.  x [hidden] is
 * updated in place.  q/k/v_bias may be NULL; inv_freq [head_dim/2] is the
 * host-computed rope_inv_freqs (src/forward/cpu.rs:1057-1092).  Weight rows
 * are read 16 bytes at a time: hidden_size, q_dim, inter and (int4/int8) the
 * group size must be multiples of 4 (f32), 8 (bf16, f16), 32 (int4) or 16
 * (int8) elements, else DLMK_ERR_UNSUPPORTED; head_dim is even, a multiple of
 * 4 and at most 256, with any GQA group (the f32 paged attention kernel).
 * Returns 0 or an error code; never synchronises. */
size_t dlmk_decode_block_workspace_size(int hidden_size, int q_dim, int kv_dim, int num_heads,
                                        int head_dim, int inter, int max_blocks_per_seq);
int dlmk_decode_block_paged(
    void *stream, int hidden_size, int q_dim, int kv_dim, int num_heads, int num_kv_heads,
    int head_dim, int inter, float rms_eps, int w_dtype, int w_group_size, const void *q_proj,
    const void *k_proj, const void *v_proj, const void *o_proj, const void *gate_proj,
    const void *up_proj, const void *down_proj, const float *in_norm, const float *post_norm,
    const float *q_bias, const float *k_bias, const float *v_bias, const float *inv_freq,
    float *x, void *k_pool, void *v_pool, int64_t num_blocks, const int32_t *block_table,
    int max_blocks_per_seq, int num_positions, int position, void *workspace,
    size_t workspace_bytes);

/* The decode block over num_tokens consecutive tokens in one pass: the
 * batched target verify of a speculative round.  dlm verifies a draft one
 * token at a time, re-running the target per position
 * (SpeculativeSession::step, src/speculative.rs:145-185); this runs the
 * gamma + 1 tokens [last, d1 .. d_gamma] through a layer together.  Same
 * arguments as dlmk_decode_block_paged plus num_tokens (>= 1): x is
 * [num_tokens][hidden] (updated in place); token j's K/V go to position
 * num_positions + j and its RoPE angle uses position + j; token j attends
 * causally to positions 0 .. num_positions + j (dlmk_paged_decode_attention
 * with num_q_per_seq = num_tokens).  Each GEMV stage reads its weights once
 * per group of up to 8 tokens whose inputs fit 64 KiB of LDS together (one
 * token at a time for inputs wider than 8192 floats).  The result per token
 * is the sequential decode block's up to float rounding.  Workspace:
 * dlmk_verify_block_workspace_size(..., num_tokens) bytes, 256-byte aligned.
 * No counterpart in the reference's FFI; rejected tokens are rolled back by
 * the caller (dlmk_cache_truncate_sequence) -- their pool slots are simply
 * overwritten by the next append. */
size_t dlmk_verify_block_workspace_size(int hidden_size, int q_dim, int kv_dim, int num_heads,
                                        int head_dim, int inter, int max_blocks_per_seq,
                                        int num_tokens);
int dlmk_verify_block_paged(
    void *stream, int hidden_size, int q_dim, int kv_dim, int num_heads, int num_kv_heads,
    int head_dim, int inter, float rms_eps, int w_dtype, int w_group_size, const void *q_proj,
    const void *k_proj, const void *v_proj, const void *o_proj, const void *gate_proj,
    const void *up_proj, const void *down_proj, const float *in_norm, const float *post_norm,
    const float *q_bias, const float *k_bias, const float *v_bias, const float *inv_freq,
    float *x, void *k_pool, void *v_pool, int64_t num_blocks, const int32_t *block_table,
    int max_blocks_per_seq, int num_positions, int position, int num_tokens, void *workspace,
    size_t workspace_bytes);

/* Pinned host memory, PinnedBuffer (src/memory/pinned.rs:38-112) analogue.
 * dlmk_alloc_pinned: page-locked, zero-initialised, rounded up to whole 4 KiB
 * pages (PinnedBuffer::with_len, pinned.rs:59-67); bytes == 0 returns
 * DLMK_ERR_INVALID_ARG (DlmError::HostAlloc there) and sets *ptr to NULL, as
 * does any failure.  dlmk_free_pinned(NULL) is a no-op returning 0. */
int dlmk_alloc_pinned(void **ptr, size_t bytes);
int dlmk_free_pinned(void *ptr);

#ifdef __cplusplus
}
#endif

#endif /* DLMK_H */
