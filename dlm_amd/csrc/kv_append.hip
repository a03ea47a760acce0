// Paged KV append (dlmk_kv_append).
//
// Replaces the reference's contiguous append -- two copy_kernel launches into
// slot `num_positions` of a flat f32 buffer (src/gpu/kernels.cu:267-270 used at
// :361-363) -- with one launch that scatters every token of a decode step or a
// prefill chunk into its physical block through a slot mapping.  It is a pure
// bit copy, so f32, f16 and bf16 share one kernel keyed on element size.
//
// Thread mapping: one thread moves one 16-byte chunk (X = 16 / elem_bytes
// consecutive dims) of one (token, kv head).  Tokens are the fastest-varying
// index inside a wavefront, so lanes holding consecutive tokens of the same
// block write one contiguous run of K chunks ([d/X][bs][X] rows) and, per dim,
// one contiguous run of V elements ([d][bs] rows).

#include <hip/hip_runtime.h>

#include "dlmk.h"
#include "dlmk_internal.h"

namespace {

constexpr int kThreads = 256;

template <int EB>
struct Bits;
template <>
struct Bits<2> {
    using type = uint16_t;
};
template <>
struct Bits<4> {
    using type = uint32_t;
};

template <int EB>
__global__ __launch_bounds__(kThreads) void kv_append_kernel(
    char *__restrict__ k_pool, char *__restrict__ v_pool, const char *__restrict__ k_src,
    const char *__restrict__ v_src, const int64_t *__restrict__ slots, int64_t n_tok,
    int num_kv_heads, int head_dim, int block_size, int64_t num_slots) {
    using E = typename Bits<EB>::type;
    constexpr int X = 16 / EB;
    const int64_t tok = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (tok >= n_tok) return;
    const int cpl = head_dim / X;            // 16-byte chunks per head row
    const int head = blockIdx.y / cpl;       // blockIdx.y = head * cpl + chunk
    const int chunk = blockIdx.y - head * cpl;
    const int64_t slot = slots[tok];
    if (slot < 0 || slot >= num_slots) return;
    const int64_t blk = slot / block_size;
    const int t = (int)(slot - blk * block_size);

    const int64_t src_off = ((tok * num_kv_heads + head) * head_dim + (int64_t)chunk * X) * EB;
    const uint4 kc = *reinterpret_cast<const uint4 *>(k_src + src_off);
    const uint4 vc = *reinterpret_cast<const uint4 *>(v_src + src_off);

    const int64_t tile = ((blk * num_kv_heads + head) * (int64_t)head_dim * block_size) * EB;
    // K tile [d/X][bs][X]: chunk row `chunk`, token t.
    *reinterpret_cast<uint4 *>(k_pool + tile + ((int64_t)chunk * block_size + t) * 16) = kc;
    // V tile [d][bs]: element (dim, t).
    E ve[X];
    __builtin_memcpy(ve, &vc, 16);
    E *vrow = reinterpret_cast<E *>(v_pool + tile) + (int64_t)chunk * X * block_size + t;
#pragma unroll
    for (int e = 0; e < X; ++e) vrow[(int64_t)e * block_size] = ve[e];
}

}  // namespace

extern "C" int dlmk_kv_append(void *stream, void *k_pool, void *v_pool, const void *k_src,
                              const void *v_src, const int64_t *slot_mapping, int64_t n_tok,
                              int num_kv_heads, int head_dim, int block_size,
                              int64_t num_blocks, int dtype) {
    if (n_tok < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks < 0)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_kv_append: bad sizes (n_tok %lld, heads %d, dim %d, bs %d)",
                          (long long)n_tok, num_kv_heads, head_dim, block_size);
    if (n_tok == 0) return DLMK_OK;
    if (!k_pool || !v_pool || !k_src || !v_src || !slot_mapping)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_kv_append: null pointer");
    int eb;
    switch (dtype) {
        case DLMK_F32: eb = 4; break;
        case DLMK_F16:
        case DLMK_BF16: eb = 2; break;
        default: return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_kv_append: unknown dtype %d", dtype);
    }
    if ((head_dim * eb) % 16 != 0)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED, "dlmk_kv_append: head_dim*elem_bytes (%d) not a multiple of 16",
                          head_dim * eb);
    const int cpl = head_dim * eb / 16;
    const int64_t gy = (int64_t)num_kv_heads * cpl;
    const int64_t gx = dlmk::ceil_div(n_tok, kThreads);
    if (gy > 65535 || gx > 0x7fffffff)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED, "dlmk_kv_append: grid too large");
    dim3 grid((unsigned)gx, (unsigned)gy);
    auto s = (hipStream_t)stream;
    const int64_t num_slots = num_blocks * block_size;
    if (eb == 2)
        hipLaunchKernelGGL(kv_append_kernel<2>, grid, dim3(kThreads), 0, s, (char *)k_pool,
                           (char *)v_pool, (const char *)k_src, (const char *)v_src, slot_mapping,
                           n_tok, num_kv_heads, head_dim, block_size, num_slots);
    else
        hipLaunchKernelGGL(kv_append_kernel<4>, grid, dim3(kThreads), 0, s, (char *)k_pool,
                           (char *)v_pool, (const char *)k_src, (const char *)v_src, slot_mapping,
                           n_tok, num_kv_heads, head_dim, block_size, num_slots);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return dlmk::fail((int)e, "dlmk_kv_append launch: %s", hipGetErrorString(e));
    return DLMK_OK;
}
