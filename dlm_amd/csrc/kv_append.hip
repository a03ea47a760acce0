// Paged KV append (dlmk_kv_append).
//
// Replaces the reference's contiguous append -- two copy_kernel launches into
// slot `num_positions` of a flat f32 buffer (src/gpu/kernels.cu:267-270 used at
// :361-363) -- with one launch that scatters every token of a decode step or a
// prefill chunk into its physical block through a slot mapping.  It is a pure
// bit copy, so f32, f16 and bf16 share the kernels, keyed on element size.
// Appends of 512 tokens or more in 16-token blocks use kv_append_run_kernel
// (below); the rest use kv_append_kernel.
//
// kv_append_kernel thread mapping: one thread moves CPT 16-byte chunks (X = 16 / elem_bytes
// consecutive dims each) of one (token, kv head).  Tokens are the fastest-varying
// index inside a wavefront, so lanes holding consecutive tokens of the same
// block write one contiguous run of K chunks ([d/X][bs][X] rows) and, per dim,
// one contiguous run of V elements ([d][bs] rows).

#include <hip/hip_runtime.h>

#include "dlmk.h"
#include "dlmk_internal.h"

namespace {

constexpr int kThreads = 256;

#ifndef DLMK_STORE_NT
#define DLMK_STORE_NT 1
#endif
// Pool stores: non-temporal (write around the caches).  The attention kernels
// stream the pools with non-temporal loads, and those measured ~5 us slower
// per launch at the 8B shape when the lines they read were written through
// the caches by the step before.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <typename V>
__device__ __forceinline__ void pool_store(V *p, V v) {
#if DLMK_STORE_NT
    __builtin_nontemporal_store(v, p);
#else
    *p = v;
#endif
}
__device__ __forceinline__ void pool_store(uint4 *p, uint4 v) {
    pool_store(reinterpret_cast<u32x4 *>(p), __builtin_bit_cast(u32x4, v));
}

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

template <int EB, int CPT>
__global__ __launch_bounds__(kThreads) void kv_append_kernel(
    char *__restrict__ k_pool, char *__restrict__ v_pool, const char *__restrict__ k_src,
    const char *__restrict__ v_src, const int64_t *__restrict__ slots, int64_t n_tok,
    int num_kv_heads, int head_dim, int block_size, int64_t num_slots) {
    using E = typename Bits<EB>::type;
    constexpr int X = 16 / EB;
    const int64_t tok = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (tok >= n_tok) return;
    const int gpl = head_dim / X / CPT;      // groups of CPT 16-byte chunks per head row
    const int head = blockIdx.y / gpl;       // blockIdx.y = head * gpl + group
    const int chunk0 = (blockIdx.y - head * gpl) * CPT;
    const int64_t slot = slots[tok];
    if (slot < 0 || slot >= num_slots) return;
    const int64_t blk = slot / block_size;
    const int t = (int)(slot - blk * block_size);

    const int64_t src_off = ((tok * num_kv_heads + head) * head_dim + (int64_t)chunk0 * X) * EB;
    uint4 kc[CPT], vc[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        kc[c] = reinterpret_cast<const uint4 *>(k_src + src_off)[c];
        vc[c] = reinterpret_cast<const uint4 *>(v_src + src_off)[c];
    }

    const int64_t tile = ((blk * num_kv_heads + head) * (int64_t)head_dim * block_size) * EB;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int chunk = chunk0 + c;
        // K tile [d/X][bs][X]: chunk row `chunk`, token t.
        pool_store(reinterpret_cast<uint4 *>(k_pool + tile + ((int64_t)chunk * block_size + t) * 16), kc[c]);
        // V tile [d][bs]: element (dim, t).
        E ve[X];
        __builtin_memcpy(ve, &vc[c], 16);
        E *vrow = reinterpret_cast<E *>(v_pool + tile) + (int64_t)chunk * X * block_size + t;
#pragma unroll
        for (int e = 0; e < X; ++e) pool_store(&vrow[(int64_t)e * block_size], ve[e]);
    }
}

// Prefill-sized appends (block size 16): one work-group per run of 16
// consecutive source tokens and one kv head, 16 * cpl threads (cpl = 16-byte
// chunks per head row; thread i holds chunk i % cpl of token i / cpl), so each
// token's head row is read by cpl consecutive lanes.  When the run's slots
// fill one block in order -- every full block of a prefill chunk -- the K and
// V tiles are transposed in LDS and written as one contiguous run of 16-byte
// stores; otherwise each thread stores its own chunk as kv_append_kernel does.
// LDS rows are padded by one 16-byte unit per chunk to spread the banks.
constexpr int kRunTokens = 16;
constexpr int kRunMaxThreads = 1024;
constexpr int64_t kRunMinTokens = 512;

template <int EB>
__global__ __launch_bounds__(kRunMaxThreads) void kv_append_run_kernel(
    char *__restrict__ k_pool, char *__restrict__ v_pool, const char *__restrict__ k_src,
    const char *__restrict__ v_src, const int64_t *__restrict__ slots, int64_t n_tok,
    int num_kv_heads, int head_dim, int64_t num_slots) {
    using E = typename Bits<EB>::type;
    constexpr int X = 16 / EB, BS = kRunTokens, PAD = BS + 1;
    __shared__ uint4 k_lds[kRunMaxThreads / BS * PAD];
    __shared__ uint4 v_lds[kRunMaxThreads / BS * PAD];
    const int cpl = head_dim / X;
    const int i = threadIdx.x, t = i / cpl, chunk = i - t * cpl;
    const int head = blockIdx.y;
    const int64_t tok0 = (int64_t)blockIdx.x * BS, tok = tok0 + t;
    const bool have = tok < n_tok;
    int64_t slot = -1;
    uint4 kc = {0, 0, 0, 0}, vc = {0, 0, 0, 0};
    if (have) {
        slot = slots[tok];
        const int64_t off = ((tok * num_kv_heads + head) * head_dim) * EB + (int64_t)chunk * 16;
        kc = *reinterpret_cast<const uint4 *>(k_src + off);
        vc = *reinterpret_cast<const uint4 *>(v_src + off);
    }
    const int64_t slot0 = slots[tok0];  // tok0 < n_tok: the grid is ceil(n_tok / 16) runs
    const bool in_run = have && slot0 >= 0 && slot0 % BS == 0 && slot0 + BS <= num_slots && slot == slot0 + t;
    if (__syncthreads_and(in_run)) {
        // K tile [cpl][16][X]: this chunk is unit chunk * 16 + t.  V tile
        // [d][16]: element (chunk * X + e, t); 16-byte unit u of the tile is
        // chunk u / 16 of it.
        k_lds[chunk * PAD + t] = kc;
        E ve[X];
        __builtin_memcpy(ve, &vc, 16);
        E *vrow = reinterpret_cast<E *>(v_lds + chunk * PAD);
#pragma unroll
        for (int e = 0; e < X; ++e) vrow[e * BS + t] = ve[e];
        __syncthreads();
        const int64_t tile = ((slot0 / BS) * num_kv_heads + head) * (int64_t)head_dim * BS * EB;
        const int u = (i / BS) * PAD + i % BS;
        reinterpret_cast<uint4 *>(k_pool + tile)[i] = k_lds[u];
        reinterpret_cast<uint4 *>(v_pool + tile)[i] = v_lds[u];
    } else if (have && slot >= 0 && slot < num_slots) {
        const int64_t blk = slot / BS;
        const int tt = (int)(slot - blk * BS);
        const int64_t tile = ((blk * num_kv_heads + head) * (int64_t)head_dim * BS) * EB;
        *reinterpret_cast<uint4 *>(k_pool + tile + ((int64_t)chunk * BS + tt) * 16) = kc;
        E ve[X];
        __builtin_memcpy(ve, &vc, 16);
        E *vrow = reinterpret_cast<E *>(v_pool + tile) + (int64_t)chunk * X * BS + tt;
#pragma unroll
        for (int e = 0; e < X; ++e) vrow[(int64_t)e * BS] = ve[e];
    }
}

}  // namespace

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Quantizing append for int8 / int4 pools (dlmk_kv_append_quant).
//
// KvLayerCache::append for the Int8 / Int4 stores (src/forward/cpu.rs:780-793,
// quantize_i8 / quantize_i4 at :672-701): each token's K (and V) vector over
// the whole kv_dim gets one scale max|x| / 127 (or / 7) and codes
// round(x / scale) clamped to +-127 (+-7) -- NaN quotients give code 0, as
// Rust's saturating `as i8` does -- and an all-zero vector scale 0.
//
// One work-group per token: threads 0..127 own K's 8-dim chunks t, t + 128,
// ... (kept in registers), threads 128..255 V's: one 16-byte source load per
// chunk (two for f32), a max-reduction over the pool's two waves, then the
// stores into the tiles the attention kernel reads 16 bytes a lane at a time
// (head_dim a multiple of 64; KG, VG as below):
//   K [d/KG][16 tokens][KG dims], KG = 16 (int8) or 32 / 16 (int4, d % 128
//     == 0 or not): a chunk is one 8-byte (int8) or 4-byte (int4) store;
//   V [d/(16 VG)][4 token quads][16][VG dims][4 tokens], VG = 4 (int8) or
//     8 / 4 (int4): one byte per dim (int8) or per dim pair (int4, low nibble
//     the even dim, so a byte never mixes tokens and appends never share one).
// Codes are stored offset binary (int8 c as the byte c + 128, int4 c as the
// nibble c + 8), so the attention kernel widens them without a sign flip.
template <typename S>
__device__ __forceinline__ void load8(const S *p, float (&x)[8]) {
    if constexpr (sizeof(S) == 4) {
        const u32x4 a = reinterpret_cast<const u32x4 *>(p)[0];
        const u32x4 b = reinterpret_cast<const u32x4 *>(p)[1];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            x[k] = __uint_as_float(a[k]);
            x[4 + k] = __uint_as_float(b[k]);
        }
    } else {
        const u32x4 raw = *reinterpret_cast<const u32x4 *>(p);
        S e[8];
        __builtin_memcpy(e, &raw, 16);
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = (float)e[k];
    }
}

__device__ __forceinline__ int quant_code(float x, float inv_ok, float scale, float qmax) {
    const float r = roundf(x / scale);
    return (inv_ok == 0.f || r != r) ? 0 : (int)fminf(fmaxf(r, -qmax), qmax);
}

// Stores the 8 offset-binary codes q of dims j .. j + 7 of token t into the
// (block, kv head) tile at `tile` (K if which == 0, else V), in the layouts
// described above.
template <int QBITS>
__device__ __forceinline__ void place_chunk(uint8_t *tile, int which, int j, int t, int d,
                                            const int (&q)[8]) {
    constexpr int BS = 16;
    const int KG = QBITS == 8 ? 16 : (d % 128 == 0 ? 32 : 16);
    const int VG = QBITS == 8 ? 4 : (d % 128 == 0 ? 8 : 4);
    const int VLANE = VG * QBITS / 2;
    // V: dim jj of this token sits at lane group (jj / VG) % 16 of
    // quarter jj / (16 VG), word (jj % VG) / (dims per byte), byte t % 4.
    const int vq = j / (16 * VG), vn = (j % (16 * VG)) / VG, vk = j % VG;
    uint8_t *vbase = tile + ((int64_t)(vq * 4 + t / 4) * 16 + vn) * VLANE + t % 4;
    if constexpr (QBITS == 8) {
        if (which == 0) {
            u32x2 w;
            w[0] = (q[0] & 0xff) | (q[1] & 0xff) << 8 | (q[2] & 0xff) << 16 | (uint32_t)(q[3] & 0xff) << 24;
            w[1] = (q[4] & 0xff) | (q[5] & 0xff) << 8 | (q[6] & 0xff) << 16 | (uint32_t)(q[7] & 0xff) << 24;
            *reinterpret_cast<u32x2 *>(tile + ((j / KG) * BS + t) * KG + j % KG) = w;
        } else {
            // 8 dims = two lane groups of VG = 4 (vk == 0).
#pragma unroll
            for (int k = 0; k < 8; ++k) vbase[(k / 4) * VLANE + (k % 4) * 4] = (uint8_t)q[k];
        }
    } else {
        uint8_t by[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) by[m] = (uint8_t)((q[2 * m] & 0x0f) | (q[2 * m + 1] & 0x0f) << 4);
        if (which == 0) {
            uint32_t w = by[0] | by[1] << 8 | by[2] << 16 | (uint32_t)by[3] << 24;
            *reinterpret_cast<uint32_t *>(tile + ((j / KG) * BS + t) * (KG / 2) + (j % KG) / 2) = w;
        } else {
            // Dim pair m of the chunk: VG = 8 keeps the chunk in one lane
            // group (words vk/2 .. +3); VG = 4 spans two (vk == 0).
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int jj = vk + 2 * m;
                vbase[(jj / VG) * VLANE + ((jj % VG) / 2) * 4] = by[m];
            }
        }
    }
}

template <int QBITS, typename S, int NC>
__global__ __launch_bounds__(256) void kv_append_quant_kernel(
    uint8_t *__restrict__ k_pool, uint8_t *__restrict__ v_pool, float *__restrict__ k_scales,
    float *__restrict__ v_scales, const S *__restrict__ k_src, const S *__restrict__ v_src,
    const int64_t *__restrict__ slots, int64_t n_tok, int num_kv_heads, int head_dim,
    int64_t num_slots) {
    constexpr int BS = 16;
    // One work-group per token: threads 0..127 quantize K, 128..255 V, each
    // over chunks lt, lt + 128, ... (NC of them); a pool's max meets across
    // its two waves in LDS.
    __shared__ float red[4];
    const int64_t tok = blockIdx.x;
    const int lane = threadIdx.x & 63, which = threadIdx.x >> 7, lt = threadIdx.x & 127;
    if (tok >= n_tok) return;  // the grid is n_tok work-groups; uniform per work-group
    const int64_t slot = slots[tok];
    if (slot < 0 || slot >= num_slots) return;
    const int64_t blk = slot / BS;
    const int t = (int)(slot - blk * BS);
    const int d = head_dim, kv_dim = num_kv_heads * head_dim, nchunks = kv_dim / 8;
    const float qmax = QBITS == 8 ? 127.f : 7.f;
    const int64_t tile_bytes = (int64_t)d * BS * QBITS / 8;
    {
        const S *src = (which ? v_src : k_src) + tok * kv_dim;
        uint8_t *pool = which ? v_pool : k_pool;
        float x[NC][8];
        float mx = 0.f;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = lt + 128 * i;
            if (c < nchunks) {
                load8(src + 8 * c, x[i]);
            } else {
#pragma unroll
                for (int k = 0; k < 8; ++k) x[i][k] = 0.f;
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) mx = fmaxf(mx, fabsf(x[i][k]));
        }
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        if (lane == 0) red[threadIdx.x >> 6] = mx;
        __syncthreads();
        mx = fmaxf(red[2 * which], red[2 * which + 1]);
        const float scale = mx / qmax;
        const float ok = scale > 0.f ? 1.f : 0.f;
        if (lt == 0) (which ? v_scales : k_scales)[slot] = ok != 0.f ? scale : 0.f;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = lt + 128 * i;
            if (c >= nchunks) continue;
            const int h = (8 * c) / d, j = 8 * c - h * d;
            uint8_t *tile = pool + (blk * num_kv_heads + h) * tile_bytes;
            int q[8];
#pragma unroll
            // Offset binary in the pools: code c is stored as c + 128 (c + 8).
            for (int k = 0; k < 8; ++k) q[k] = quant_code(x[i][k], ok, scale, qmax) + (QBITS == 8 ? 128 : 8);
            place_chunk<QBITS>(tile, which, j, t, d, q);
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
    auto s = (hipStream_t)stream;
    const int64_t num_slots = num_blocks * block_size;
    // Prefill-sized appends in 16-token blocks: runs of 16 tokens per
    // work-group (coalesced source rows, whole-tile stores for full blocks;
    // 2096 tokens 9.6 -> 5.7 us, a 16384-token prefill 5.55 -> 6.38 TB/s).
    if (n_tok >= kRunMinTokens && block_size == kRunTokens && cpl * kRunTokens <= kRunMaxThreads) {
        const int64_t rx = dlmk::ceil_div(n_tok, (int64_t)kRunTokens);
        if (rx > 0x7fffffff || num_kv_heads > 65535)
            return dlmk::fail(DLMK_ERR_UNSUPPORTED, "dlmk_kv_append: grid too large");
        dim3 rgrid((unsigned)rx, (unsigned)num_kv_heads);
        if (eb == 2)
            hipLaunchKernelGGL(kv_append_run_kernel<2>, rgrid, dim3(cpl * kRunTokens), 0, s, (char *)k_pool,
                               (char *)v_pool, (const char *)k_src, (const char *)v_src, slot_mapping, n_tok,
                               num_kv_heads, head_dim, num_slots);
        else
            hipLaunchKernelGGL(kv_append_run_kernel<4>, rgrid, dim3(cpl * kRunTokens), 0, s, (char *)k_pool,
                               (char *)v_pool, (const char *)k_src, (const char *)v_src, slot_mapping, n_tok,
                               num_kv_heads, head_dim, num_slots);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return dlmk::fail((int)e, "dlmk_kv_append launch: %s", hipGetErrorString(e));
        return DLMK_OK;
    }
    // Outside the run kernel's range: two chunks per thread for appends of
    // 512 tokens or more where the head row allows (a 2096-token append 13.4
    // -> 9.5 us in 16-token blocks), one for decode-sized ones (64 tokens:
    // 2.70 us against 3.11 with two).
    const int cpt = cpl % 2 == 0 && n_tok >= 512 ? 2 : 1;
    const int64_t gy = (int64_t)num_kv_heads * cpl / cpt;
    const int64_t gx = dlmk::ceil_div(n_tok, kThreads);
    if (gy > 65535 || gx > 0x7fffffff)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED, "dlmk_kv_append: grid too large");
    dim3 grid((unsigned)gx, (unsigned)gy);
#define DLMK_APPEND_LAUNCH(EB, CPT)                                                               \
    hipLaunchKernelGGL((kv_append_kernel<EB, CPT>), grid, dim3(kThreads), 0, s, (char *)k_pool,    \
                       (char *)v_pool, (const char *)k_src, (const char *)v_src, slot_mapping, n_tok, \
                       num_kv_heads, head_dim, block_size, num_slots)
    if (eb == 2) {
        if (cpt == 2)
            DLMK_APPEND_LAUNCH(2, 2);
        else
            DLMK_APPEND_LAUNCH(2, 1);
    } else {
        if (cpt == 2)
            DLMK_APPEND_LAUNCH(4, 2);
        else
            DLMK_APPEND_LAUNCH(4, 1);
    }
#undef DLMK_APPEND_LAUNCH
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return dlmk::fail((int)e, "dlmk_kv_append launch: %s", hipGetErrorString(e));
    return DLMK_OK;
}

// Prefill-sized int8 appends: one work-group per run of 16 consecutive
// source tokens, 512 threads (256 per pool; 16 lanes per token, RC chunks
// each, so a token's max is a 16-lane shuffle reduction).  When the run's
// slots fill one block in order, the codes are placed into an LDS image of
// the block's tiles (every kv head) and the image is copied out with 16-byte
// stores; otherwise each thread places its codes straight into the pool.
constexpr int kQuantRunMaxKvDim = 1024;
constexpr int64_t kQuantRunMinTokens = 512;

template <int QBITS, typename S, int RC>
__global__ __launch_bounds__(512) void kv_append_quant_run_kernel(
    uint8_t *__restrict__ k_pool, uint8_t *__restrict__ v_pool, float *__restrict__ k_scales,
    float *__restrict__ v_scales, const S *__restrict__ k_src, const S *__restrict__ v_src,
    const int64_t *__restrict__ slots, int64_t n_tok, int num_kv_heads, int head_dim,
    int64_t num_slots) {
    constexpr int BS = 16;
    __shared__ __attribute__((aligned(16))) uint8_t img[2][kQuantRunMaxKvDim * BS * QBITS / 8];
    const int which = threadIdx.x >> 8, lt = threadIdx.x & 255, tt = lt >> 4, sub = lt & 15;
    const int64_t tok0 = (int64_t)blockIdx.x * BS, tok = tok0 + tt;
    const bool have = tok < n_tok;
    const int d = head_dim, kv_dim = num_kv_heads * head_dim;
    const float qmax = QBITS == 8 ? 127.f : 7.f;
    const S *src = (which ? v_src : k_src) + (have ? tok : tok0) * kv_dim;
    float x[RC][8];
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < RC; ++i) {
        load8(src + 8 * (sub + 16 * i), x[i]);
#pragma unroll
        for (int k = 0; k < 8; ++k) mx = fmaxf(mx, fabsf(x[i][k]));
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    const int64_t slot = have ? slots[tok] : -1;
    const int64_t slot0 = slots[tok0];  // tok0 < n_tok: the grid is ceil(n_tok / 16) runs
    const bool in_run = have && slot0 >= 0 && slot0 % BS == 0 && slot0 + BS <= num_slots && slot == slot0 + tt;
    const bool full = __syncthreads_and(in_run);
    const bool valid = have && slot >= 0 && slot < num_slots;
    const float scale = mx / qmax;
    const float ok = scale > 0.f ? 1.f : 0.f;
    if (valid && sub == 0) (which ? v_scales : k_scales)[slot] = ok != 0.f ? scale : 0.f;
    uint8_t *pool = which ? v_pool : k_pool;
    const int64_t tile_bytes = (int64_t)d * BS * QBITS / 8;
    if (valid) {
        const int64_t blk = slot / BS;
        const int t = (int)(slot - blk * BS);
#pragma unroll
        for (int i = 0; i < RC; ++i) {
            const int c = sub + 16 * i;
            const int h = (8 * c) / d, j = 8 * c - h * d;
            uint8_t *tile = full ? img[which] + h * tile_bytes : pool + (blk * num_kv_heads + h) * tile_bytes;
            int q[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) q[k] = quant_code(x[i][k], ok, scale, qmax) + (QBITS == 8 ? 128 : 8);
            place_chunk<QBITS>(tile, which, j, t, d, q);
        }
    }
    if (full) {  // uniform over the work-group
        __syncthreads();
        const int64_t units = num_kv_heads * tile_bytes / 16;
        uint4 *dst = reinterpret_cast<uint4 *>(pool + (slot0 / BS) * num_kv_heads * tile_bytes);
        const uint4 *from = reinterpret_cast<const uint4 *>(img[which]);
        for (int64_t u = lt; u < units; u += 256) dst[u] = from[u];
    }
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
    if (head_dim % 64 != 0 || block_size != 16)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED,
                          "dlmk_kv_append_quant: head_dim %d (multiple of 64) / block_size %d (16)",
                          head_dim, block_size);
    const int64_t kv_dim = (int64_t)num_kv_heads * head_dim;
    const int64_t chunks_per_lane = dlmk::ceil_div(kv_dim / 8, 128);
    if (chunks_per_lane > 8)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED,
                          "dlmk_kv_append_quant: kv_dim %lld above 8192", (long long)kv_dim);
    if (reinterpret_cast<uintptr_t>(k_src) % 16 || reinterpret_cast<uintptr_t>(v_src) % 16)
        return dlmk::fail(DLMK_ERR_INVALID_ARG,
                          "dlmk_kv_append_quant: k_src / v_src not 16-byte aligned");
    const int nc = chunks_per_lane <= 1 ? 1 : chunks_per_lane <= 2 ? 2 : chunks_per_lane <= 4 ? 4 : 8;
    // Runs of 16 tokens per work-group for prefill-sized int8 appends with
    // kv_dim 512 or 1024 (4 or 8 chunks per lane): config 3's 2096 tokens
    // 12.36 -> 11.56 us.  int4 measured slower that way (8.55 -> 11.59 us)
    // and keeps one work-group per token.
    const int rc = quant == DLMK_I8 && n_tok >= kQuantRunMinTokens &&
                           (kv_dim == 512 || kv_dim == kQuantRunMaxKvDim)
                       ? (int)(kv_dim / 8 / 16) : 0;
    const int64_t gx = n_tok;
    if (gx > 0x7fffffff) return dlmk::fail(DLMK_ERR_UNSUPPORTED, "dlmk_kv_append_quant: grid too large");
    auto s = (hipStream_t)stream;
    const int64_t num_slots = num_blocks * block_size;
    auto kp = (uint8_t *)k_pool, vp = (uint8_t *)v_pool;
#define DLMK_LAUNCH_NC(Q, S, NC)                                                                \
    hipLaunchKernelGGL((kv_append_quant_kernel<Q, S, NC>), dim3((unsigned)gx), dim3(256), 0, s, kp, \
                       vp, k_scales, v_scales, (const S *)k_src, (const S *)v_src, slot_mapping,  \
                       n_tok, num_kv_heads, head_dim, num_slots)
#define DLMK_LAUNCH_RUN(Q, S, RC)                                                                    \
    hipLaunchKernelGGL((kv_append_quant_run_kernel<Q, S, RC>), dim3((unsigned)dlmk::ceil_div(n_tok, (int64_t)16)), \
                       dim3(512), 0, s, kp, vp, k_scales, v_scales, (const S *)k_src, (const S *)v_src,         \
                       slot_mapping, n_tok, num_kv_heads, head_dim, num_slots)
#define DLMK_LAUNCH(Q, S)                                             \
    if (rc == 4) {                                                    \
        DLMK_LAUNCH_RUN(Q, S, 4);                                     \
        break;                                                        \
    }                                                                 \
    if (rc == 8) {                                                    \
        DLMK_LAUNCH_RUN(Q, S, 8);                                     \
        break;                                                        \
    }                                                                 \
    switch (nc) {                                                     \
        case 1: DLMK_LAUNCH_NC(Q, S, 1); break;                       \
        case 2: DLMK_LAUNCH_NC(Q, S, 2); break;                       \
        case 4: DLMK_LAUNCH_NC(Q, S, 4); break;                       \
        default: DLMK_LAUNCH_NC(Q, S, 8); break;                      \
    }
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
#undef DLMK_LAUNCH_NC
#undef DLMK_LAUNCH_RUN
#undef DLMK_LAUNCH
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return dlmk::fail((int)e, "dlmk_kv_append_quant launch: %s", hipGetErrorString(e));
    return DLMK_OK;
}
