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

// ---------------------------------------------------------------------------
// Quantizing append for int8 / int4 pools (dlmk_kv_append_quant).
//
// KvLayerCache::append for the Int8 / Int4 stores (src/forward/cpu.rs:780-793,
// quantize_i8 / quantize_i4 at :667-700): each token's K (and V) vector over
// the whole kv_dim gets one scale max|x| / 127 (or / 7) and codes
// round(x / scale) clamped to +-127 (+-7), an all-zero vector scale 0.  One
// wavefront per token: a wave max-reduction, then the codes go to the paged
// layout -- int8 K [d/8][16][8], V [d][16]; int4 K [d/8][16][4] and
// V [d/2][16] bytes holding two consecutive dims of one token (low nibble for
// the even dim), so a byte never mixes tokens and appends never share one.
// ---------------------------------------------------------------------------
template <typename S>
__device__ __forceinline__ float to_f32(S x) {
    return (float)x;
}

template <int QBITS, typename S>
__global__ __launch_bounds__(256) void kv_append_quant_kernel(
    uint8_t *__restrict__ k_pool, uint8_t *__restrict__ v_pool, float *__restrict__ k_scales,
    float *__restrict__ v_scales, const S *__restrict__ k_src, const S *__restrict__ v_src,
    const int64_t *__restrict__ slots, int64_t n_tok, int num_kv_heads, int head_dim,
    int block_size, int64_t num_slots) {
    const int64_t tok = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (tok >= n_tok) return;
    const int64_t slot = slots[tok];
    if (slot < 0 || slot >= num_slots) return;
    const int64_t blk = slot / block_size;
    const int t = (int)(slot - blk * block_size);
    const int d = head_dim, kv_dim = num_kv_heads * head_dim;
    const float qmax = QBITS == 8 ? 127.f : 7.f;
    const int64_t tile_bytes = (int64_t)d * block_size * QBITS / 8;
#pragma unroll
    for (int which = 0; which < 2; ++which) {
        const S *src = (which ? v_src : k_src) + tok * kv_dim;
        uint8_t *pool = which ? v_pool : k_pool;
        float mx = 0.f;
        for (int e = lane; e < kv_dim; e += 64) mx = fmaxf(mx, fabsf(to_f32(src[e])));
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const float scale = mx / qmax;
        const bool zero = !(scale > 0.f);
        if (lane == 0) (which ? v_scales : k_scales)[slot] = zero ? 0.f : scale;
        auto code = [&](float x) -> int {
            return zero ? 0 : (int)fminf(fmaxf(roundf(x / scale), -qmax), qmax);
        };
        if (QBITS == 8) {
            for (int e = lane; e < kv_dim; e += 64) {
                const int h = e / d, j = e - h * d;
                uint8_t *tile = pool + (blk * num_kv_heads + h) * tile_bytes;
                const int64_t off = which ? (int64_t)j * block_size + t
                                          : ((int64_t)(j / 8) * block_size + t) * 8 + j % 8;
                tile[off] = (uint8_t)(int8_t)code(to_f32(src[e]));
            }
        } else {
            for (int pe = lane; pe < kv_dim / 2; pe += 64) {
                const int e = 2 * pe, h = e / d, j = e - h * d;
                uint8_t *tile = pool + (blk * num_kv_heads + h) * tile_bytes;
                const uint8_t byte = (uint8_t)((code(to_f32(src[e])) & 0x0f) |
                                               ((code(to_f32(src[e + 1])) & 0x0f) << 4));
                const int64_t off = which ? (int64_t)(j / 2) * block_size + t
                                          : ((int64_t)(j / 8) * block_size + t) * 4 + (j % 8) / 2;
                tile[off] = byte;
            }
        }
    }
}

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

extern "C" int dlmk_kv_append_quant(void *stream, void *k_pool, void *v_pool, float *k_scales,
                                    float *v_scales, const void *k_src, const void *v_src,
                                    int src_dtype, const int64_t *slot_mapping, int64_t n_tok,
                                    int num_kv_heads, int head_dim, int block_size,
                                    int64_t num_blocks, int quant) {
    if (n_tok < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks < 0)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_kv_append_quant: bad sizes");
    if (n_tok == 0) return DLMK_OK;
    if (!k_pool || !v_pool || !k_scales || !v_scales || !k_src || !v_src || !slot_mapping)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_kv_append_quant: null pointer");
    if (quant != DLMK_I8 && quant != DLMK_I4)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_kv_append_quant: quant %d is not int8/int4", quant);
    if (head_dim % 8 != 0 || block_size != 16)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED,
                          "dlmk_kv_append_quant: head_dim %d (multiple of 8) / block_size %d (16)",
                          head_dim, block_size);
    const int64_t gx = dlmk::ceil_div(n_tok, 4);
    if (gx > 0x7fffffff) return dlmk::fail(DLMK_ERR_UNSUPPORTED, "dlmk_kv_append_quant: grid too large");
    auto s = (hipStream_t)stream;
    const int64_t num_slots = num_blocks * block_size;
    auto kp = (uint8_t *)k_pool, vp = (uint8_t *)v_pool;
#define DLMK_LAUNCH(Q, S)                                                                       \
    hipLaunchKernelGGL((kv_append_quant_kernel<Q, S>), dim3((unsigned)gx), dim3(256), 0, s, kp, vp, \
                       k_scales, v_scales, (const S *)k_src, (const S *)v_src, slot_mapping,     \
                       n_tok, num_kv_heads, head_dim, block_size, num_slots)
    const int q = quant == DLMK_I8 ? 8 : 4;
    switch (src_dtype * 16 + q) {
        case DLMK_F32 * 16 + 8: DLMK_LAUNCH(8, float); break;
        case DLMK_F32 * 16 + 4: DLMK_LAUNCH(4, float); break;
        case DLMK_F16 * 16 + 8: DLMK_LAUNCH(8, _Float16); break;
        case DLMK_F16 * 16 + 4: DLMK_LAUNCH(4, _Float16); break;
        case DLMK_BF16 * 16 + 8: DLMK_LAUNCH(8, __bf16); break;
        case DLMK_BF16 * 16 + 4: DLMK_LAUNCH(4, __bf16); break;
        default:
            return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_kv_append_quant: bad source dtype %d",
                              src_dtype);
    }
#undef DLMK_LAUNCH
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return dlmk::fail((int)e, "dlmk_kv_append_quant launch: %s", hipGetErrorString(e));
    return DLMK_OK;
}
