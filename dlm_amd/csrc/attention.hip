// Paged GQA decode attention entry points (dlmk_paged_decode_attention,
// dlmk_paged_decode_step, dlmk_paged_decode_attention_quant): argument checks,
// workspace layout and dispatch to the per-format kernels (attention_*.hip).
//
// Replaces attention_kernel (src/gpu/kernels.cu:210-242) and the CPU
// attention() (src/forward/cpu.rs:1126-1151); the kernels and their design are
// described in attention_kernels.h.
#include "attention_kernels.h"

#include <mutex>

extern "C" {

size_t dlmk_paged_attention_workspace_size(int num_seqs, int num_q_per_seq, int num_q_heads,
                                           int head_dim, int block_size, int max_blocks_per_seq) {
    (void)block_size;
    if (num_seqs <= 0 || num_q_per_seq <= 0 || num_q_heads <= 0 || head_dim <= 0 ||
        max_blocks_per_seq <= 0)
        return 0;
    const int64_t parts = parts_for(max_blocks_per_seq, kMinPartition);
    if (parts <= 1) return 0;
    const int64_t rows = (int64_t)num_seqs * num_q_per_seq * num_q_heads;
    const int64_t o_bytes = rows * parts * head_dim * 4;
    const int64_t o_aligned = (o_bytes + 255) / 256 * 256;
    return (size_t)(o_aligned + rows * parts * 2 * 4);
}

}  // extern "C"

namespace {

int paged_attention_impl(const char *who, void *stream, void *out, int out_dtype, const void *q,
                         void *k_pool, void *v_pool, int dtype, const float *k_scales,
                         const float *v_scales, const void *k_new,
                         const void *v_new, const int32_t *block_tables, const int32_t *ctx_lens,
                         int num_seqs, int num_q_per_seq, int num_q_heads, int num_kv_heads,
                         int head_dim, int block_size, int max_blocks_per_seq, int64_t num_blocks,
                         float scale, void *workspace, size_t workspace_bytes,
                         bool exact_workspace = false) {
    if (num_seqs < 0 || num_q_per_seq <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
        head_dim <= 0 || max_blocks_per_seq <= 0 || num_blocks < 0)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: bad sizes", who);
    if (num_q_heads % num_kv_heads != 0)
        return dlmk::fail(DLMK_ERR_INVALID_ARG,
                          "%s: %d query heads not a multiple of %d kv heads", who,
                          num_q_heads, num_kv_heads);
    if (num_seqs == 0) return DLMK_OK;
    if (!out || !q || !k_pool || !v_pool || !block_tables || !ctx_lens)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: null pointer", who);
    const bool quant = dtype == DLMK_I8 || dtype == DLMK_I4;
    if (quant && (!k_scales || !v_scales))
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: null scale pointer", who);
    if (quant && k_new)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED, "%s: no fused append into quantized pools", who);
    // Q, the pools and the new tokens are read (and the new tokens stored) 16
    // bytes a lane, and the scales 16 bytes a lane group.
    const auto misaligned = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 != 0; };
    if (misaligned(q) || misaligned(k_pool) || misaligned(v_pool) || misaligned(k_new) ||
        misaligned(v_new) || misaligned(k_scales) || misaligned(v_scales))
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: q, pools, new tokens and scales must be "
                          "16-byte aligned", who);
    if (block_size != kBlock)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED,
                          "%s: block_size %d unsupported (16)", who, block_size);
    if (out_dtype != DLMK_F32 && out_dtype != DLMK_F16 && out_dtype != DLMK_BF16)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: bad out dtype %d", who,
                          out_dtype);
    if ((int64_t)num_seqs * num_kv_heads > 0x7fffffff ||
        parts_for(max_blocks_per_seq, kMinPartition) > 65534 || num_seqs > 65535)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED, "%s: grid too large", who);

    Args a;
    a.out = out;
    a.out_dtype = out_dtype;
    a.q = q;
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.k_scales = k_scales;
    a.v_scales = v_scales;
    a.k_new = k_new;
    a.v_new = v_new;
    a.tables = block_tables;
    a.ctx_lens = ctx_lens;
    a.B = num_seqs;
    a.NQ = num_q_per_seq;
    a.Hq = num_q_heads;
    a.Hkv = num_kv_heads;
    a.max_blocks = max_blocks_per_seq;
    a.D = head_dim;
    a.num_blocks = num_blocks;
    a.scale = scale;
    a.stream = (hipStream_t)stream;
    a.workspace = nullptr;
    a.ws_bytes = 0;
    const int64_t parts = parts_for(max_blocks_per_seq, kMinPartition);
    if (parts > 1) {
        // The documented bound (dlmk_paged_attention_workspace_size) holds for
        // every kernel; the launch checks the exact need of the partition size
        // it picks (exact_workspace: only that check, for a fixed-size buffer).
        const size_t need = dlmk_paged_attention_workspace_size(
            num_seqs, num_q_per_seq, num_q_heads, head_dim, block_size, max_blocks_per_seq);
        if (!workspace || (!exact_workspace && workspace_bytes < need))
            return dlmk::fail(DLMK_ERR_WORKSPACE,
                              "%s: workspace %zu bytes, need %zu", who,
                              workspace_bytes, need);
        if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
            return dlmk::fail(DLMK_ERR_INVALID_ARG,
                              "%s: workspace not 256-byte aligned", who);
        a.workspace = workspace;
        a.ws_bytes = workspace_bytes;
    }
    switch (dtype) {
        case DLMK_F32: return dlmk_attn::dispatch_f32(a, head_dim);
        case DLMK_F16: return dlmk_attn::dispatch_f16(a, head_dim);
        case DLMK_BF16: return dlmk_attn::dispatch_bf16(a, head_dim);
        case DLMK_I8: return dlmk_attn::dispatch_i8(a, head_dim);
        case DLMK_I4: return dlmk_attn::dispatch_i4(a, head_dim);
        default:
            return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: bad KV dtype %d", who,
                              dtype);
    }
}

}  // namespace

extern "C" {

int dlmk_paged_decode_attention(void *stream, void *out, int out_dtype, const void *q,
                                const void *k_pool, const void *v_pool, int dtype,
                                const int32_t *block_tables, const int32_t *ctx_lens,
                                int num_seqs, int num_q_per_seq, int num_q_heads,
                                int num_kv_heads, int head_dim, int block_size,
                                int max_blocks_per_seq, int64_t num_blocks, float scale,
                                void *workspace, size_t workspace_bytes) {
    // Without new tokens the kernels never write the pools.
    return paged_attention_impl("dlmk_paged_decode_attention", stream, out, out_dtype, q,
                                const_cast<void *>(k_pool), const_cast<void *>(v_pool), dtype,
                                nullptr, nullptr, nullptr, nullptr, block_tables, ctx_lens, num_seqs,
                                num_q_per_seq, num_q_heads, num_kv_heads, head_dim, block_size,
                                max_blocks_per_seq, num_blocks, scale, workspace, workspace_bytes);
}

int dlmk_paged_decode_step(void *stream, void *out, int out_dtype, const void *q, void *k_pool,
                           void *v_pool, int dtype, const void *k_new, const void *v_new,
                           const int32_t *block_tables, const int32_t *ctx_lens, int num_seqs,
                           int num_q_per_seq, int num_q_heads, int num_kv_heads, int head_dim,
                           int block_size, int max_blocks_per_seq, int64_t num_blocks, float scale,
                           void *workspace, size_t workspace_bytes) {
    if (num_seqs > 0 && (!k_new || !v_new))
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_paged_decode_step: null new-token pointer");
    return paged_attention_impl("dlmk_paged_decode_step", stream, out, out_dtype, q, k_pool,
                                v_pool, dtype, nullptr, nullptr, k_new, v_new, block_tables, ctx_lens, num_seqs,
                                num_q_per_seq, num_q_heads, num_kv_heads, head_dim, block_size,
                                max_blocks_per_seq, num_blocks, scale, workspace, workspace_bytes);
}

}  // extern "C"

extern "C" {

int dlmk_paged_decode_attention_quant(void *stream, void *out, int out_dtype, const void *q,
                                      const void *k_pool, const void *v_pool,
                                      const float *k_scales, const float *v_scales, int quant,
                                      const int32_t *block_tables, const int32_t *ctx_lens,
                                      int num_seqs, int num_q_per_seq, int num_q_heads,
                                      int num_kv_heads, int head_dim, int block_size,
                                      int max_blocks_per_seq, int64_t num_blocks, float scale,
                                      void *workspace, size_t workspace_bytes) {
    if (quant != DLMK_I8 && quant != DLMK_I4)
        return dlmk::fail(DLMK_ERR_INVALID_ARG,
                          "dlmk_paged_decode_attention_quant: bad quant %d", quant);
    return paged_attention_impl("dlmk_paged_decode_attention_quant", stream, out, out_dtype, q,
                                const_cast<void *>(k_pool), const_cast<void *>(v_pool), quant,
                                k_scales, v_scales, nullptr, nullptr, block_tables, ctx_lens,
                                num_seqs, num_q_per_seq, num_q_heads, num_kv_heads, head_dim,
                                block_size, max_blocks_per_seq, num_blocks, scale, workspace,
                                workspace_bytes);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free attention (dlmk_paged_decode_attention_noalloc): the split-K
// partials live in a file-scope device array instead of a caller workspace.
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kScratchBytes = DLMK_NOALLOC_SCRATCH_BYTES;

}  // namespace

// One copy per GPU the library runs on, held until the process ends.  In host
// code `scratch` names a host-side stand-in: kernels only ever receive the
// device address hipGetSymbolAddress returns (scratch_for_stream below).
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// The device address of `scratch` on the device that runs `stream` (the
// current device for the null stream), looked up once per device with that
// device current.
int scratch_for_stream(hipStream_t stream, void **out) {
    int cur = 0, dev = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return dlmk::fail((int)e, "hipGetDevice: %s", hipGetErrorString(e));
    dev = cur;
    if (stream != nullptr) {
        e = hipStreamGetDevice(stream, &dev);
        if (e != hipSuccess)
            return dlmk::fail((int)e, "hipStreamGetDevice: %s", hipGetErrorString(e));
    }
    if (dev < 0 || dev >= kMaxDevices)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED, "device %d beyond the scratch table", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess)
            return dlmk::fail((int)e, "hipSetDevice(%d): %s", dev, hipGetErrorString(e));
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (dev != cur) hipSetDevice(cur);
        if (e != hipSuccess)
            return dlmk::fail((int)e, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return DLMK_OK;
}

}  // namespace

extern "C" {

int dlmk_paged_decode_attention_noalloc(void *stream, void *out, int out_dtype, const void *q,
                                        const void *k_pool, const void *v_pool, int dtype,
                                        const int32_t *block_tables, const int32_t *ctx_lens,
                                        int num_seqs, int num_q_per_seq, int num_q_heads,
                                        int num_kv_heads, int head_dim, int block_size,
                                        int max_blocks_per_seq, int64_t num_blocks, float scale) {
    void *ws = nullptr;
    const int rc = scratch_for_stream((hipStream_t)stream, &ws);
    if (rc != DLMK_OK) return rc;
    return paged_attention_impl("dlmk_paged_decode_attention_noalloc", stream, out, out_dtype, q,
                                const_cast<void *>(k_pool), const_cast<void *>(v_pool), dtype,
                                nullptr, nullptr, nullptr, nullptr, block_tables, ctx_lens, num_seqs,
                                num_q_per_seq, num_q_heads, num_kv_heads, head_dim, block_size,
                                max_blocks_per_seq, num_blocks, scale, ws, kScratchBytes,
                                /*exact_workspace=*/true);
}

}  // extern "C"
