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

// The 8 codes of a chunk, packed as stored (offset binary): int8 w0 = bytes
// c0..c3 + 128, w1 = c4..c7 + 128; int4 w0 byte m = (c_2m + 8) | (c_2m+1 + 8)
// << 4, where c = clamp(round(x / scale), -qmax, qmax) (round half away
// from zero; NaN quotients and scale 0 give 0).  No division per element:
// Ziv's rounding test (A. Ziv, "Fast evaluation of elementary
// mathematical functions with correctly rounded last bit", ACM TOMS 17(3),
// 1991) -- evaluate cheaply with a known error bound, and take the exact path
// only when the bound cannot decide the rounding.  inv = 1 / scale is
// correctly rounded and |x| <= max, so y = x * inv differs from x / scale by
// at most |x / scale| 2^-23 <= 128 2^-23 = 2^-16, and the rounded quotient
// fl(x / scale) from x / scale by at most half an ulp, 2^-17.  roundf and
// rintf agree except at the half-integers, and change value only there; so
// when y is more than 2^-14 away from every half-integer (|y - rint(y)| <
// 1/2 - 2^-14), rint(y) == roundf(fl(x / scale)).  Otherwise -- about 2^-13
// of the elements, and every non-finite y (NaN input, scale 0 or a scale
// whose reciprocal overflows: then y is NaN or infinite) -- the chunk takes
// the division.  Codes are packed with v_cvt_pk_u8_f32.
template <int QBITS>
__device__ __forceinline__ void quant_chunk(const float (&x)[8], float inv_ok, float scale,
                                            float inv, uint32_t &w0, uint32_t &w1) {
    constexpr float qmax = QBITS == 8 ? 127.f : 7.f, bias = QBITS == 8 ? 128.f : 8.f;
    float r[8];
    bool exact = true;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float y = x[k] * inv;
        r[k] = __builtin_rintf(y);
        exact = exact && fabsf(y - r[k]) < 0.5f - 0x1p-14f;
    }
    if (!exact) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float q = roundf(x[k] / scale);
            r[k] = (inv_ok == 0.f || q != q) ? 0.f : q;
        }
    }
    float c[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) c[k] = __builtin_amdgcn_fmed3f(r[k], -qmax, qmax) + bias;
    if constexpr (QBITS == 8) {
        w0 = w1 = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            w0 = __builtin_amdgcn_cvt_pk_u8_f32(c[k], k, w0);
            w1 = __builtin_amdgcn_cvt_pk_u8_f32(c[4 + k], k, w1);
        }
    } else {
        w0 = w1 = 0;
#pragma unroll
        for (int m = 0; m < 4; ++m) w0 = __builtin_amdgcn_cvt_pk_u8_f32(fmaf(c[2 * m + 1], 16.f, c[2 * m]), m, w0);
    }
}

// Stores a chunk's packed codes (quant_chunk) of dims j .. j + 7 of token t
// into the (block, kv head) tile at `tile` (K if which == 0, else V), in the
// layouts described above.
template <int QBITS>
__device__ __forceinline__ void place_chunk(uint8_t *tile, int which, int j, int t, int d,
                                            uint32_t w0, uint32_t w1) {
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
            *reinterpret_cast<u32x2 *>(tile + ((j / KG) * BS + t) * KG + j % KG) = u32x2{w0, w1};
        } else {
            // 8 dims = two lane groups of VG = 4 (vk == 0).
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                vbase[k * 4] = (uint8_t)(w0 >> (8 * k));
                vbase[VLANE + k * 4] = (uint8_t)(w1 >> (8 * k));
            }
        }
    } else {
        if (which == 0) {
            *reinterpret_cast<uint32_t *>(tile + ((j / KG) * BS + t) * (KG / 2) + (j % KG) / 2) = w0;
        } else {
            // Dim pair m of the chunk: VG = 8 keeps the chunk in one lane
            // group (words vk/2 .. +3); VG = 4 spans two (vk == 0).
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int jj = vk + 2 * m;
                vbase[(jj / VG) * VLANE + ((jj % VG) / 2) * 4] = (uint8_t)(w0 >> (8 * m));
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
        const float inv = 1.0f / scale;
        if (lt == 0) (which ? v_scales : k_scales)[slot] = ok != 0.f ? scale : 0.f;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = lt + 128 * i;
            if (c >= nchunks) continue;
            const int h = (8 * c) / d, j = 8 * c - h * d;
            uint8_t *tile = pool + (blk * num_kv_heads + h) * tile_bytes;
            uint32_t w0, w1;
            quant_chunk<QBITS>(x[i], ok, scale, inv, w0, w1);
            place_chunk<QBITS>(tile, which, j, t, d, w0, w1);
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
    if (!dlmk::aligned16(k_pool) || !dlmk::aligned16(v_pool) || !dlmk::aligned16(k_src) ||
        !dlmk::aligned16(v_src))
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_kv_append: pools and sources must be 16-byte aligned");
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

// Quantizing appends of kQuadMinTokens or more (kv_dim <= 4096): one
// work-group per quad of 4 consecutive source tokens and one pool (grid.y: K
// or V), kQuadWaves waves.  Lane (e, sub) of wave w holds token e's 8-dim
// chunks sub + 16 (w + kQuadWaves i), i < RC.  A token's max is a 16-lane
// shuffle reduction, then a max over the waves in LDS.  Codes come from
// quant_chunk.  K chunks are one 8-byte (int8) or 4-byte (int4) store per
// lane, as place_chunk does.  A V word holds one dim (int8) or dim pair
// (int4) of a token quad (V layout above), so when the 4 tokens fill one quad
// of one block (slots s .. s + 3, s % 4 == 0), the 4 lanes sharing a chunk
// transpose their packed codes (4 x 4 bytes, lane shuffles) and each stores
// whole words; otherwise V bytes are stored as place_chunk does.
// Measured at configs[2] (2096 tokens, kv_dim 1024, f16 source), bench.py
// graph replays, int8 / int4:
//   LDS image of whole blocks (byte stores, 72% of its LDS cycles bank
//   conflicts by SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE) / one work-group
//   per token: 11.6 / 8.5 us;
//   1 wave per quad (16 lanes per token, 64 elements a lane, ~4500
//   instructions in one dependent chain): 11.4 / 12.1 us;
//   8 waves: 9.3 / 8.4 us; 4 waves (2 chunks a lane): 7.0 / 6.9 us;
//   2 waves: 7.5 / 7.8 us.
// Decode-sized appends (64 tokens) are faster one work-group per token
// (3.4 / 3.2 us against 4.6 / 3.6 us).
#ifndef DLMK_QUAD_WAVES
#define DLMK_QUAD_WAVES 4
#endif
constexpr int kQuadWaves = DLMK_QUAD_WAVES;
#ifndef DLMK_QUAD_MIN_TOKENS
#define DLMK_QUAD_MIN_TOKENS 256
#endif
constexpr int64_t kQuadMinTokens = DLMK_QUAD_MIN_TOKENS;

// Lanes sub + 16 t (t = 0..3) hold token t's packed word a; lane sub + 16 e
// gets word e of the transpose: byte t = byte e of token t's word.
__device__ __forceinline__ uint32_t quad_transpose(uint32_t a, int e, int sub) {
    uint32_t r = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t at = (uint32_t)__shfl((int)a, sub + 16 * t, 64);
        r |= ((at >> (8 * e)) & 0xffu) << (8 * t);
    }
    return r;
}

template <int QBITS, typename S, int RC>
__global__ __launch_bounds__(64 * kQuadWaves) void kv_append_quant_quad_kernel(
    uint8_t *__restrict__ k_pool, uint8_t *__restrict__ v_pool, float *__restrict__ k_scales,
    float *__restrict__ v_scales, const S *__restrict__ k_src, const S *__restrict__ v_src,
    const int64_t *__restrict__ slots, int64_t n_tok, int num_kv_heads, int head_dim,
    int64_t num_slots) {
    constexpr int BS = 16;
    __shared__ float red[kQuadWaves][4];
    const int which = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, e = lane >> 4, sub = lane & 15;
    const int64_t tok = (int64_t)blockIdx.x * 4 + e;
    const bool have = tok < n_tok;
    const int64_t slot = have ? slots[tok] : -1;
    const int d = head_dim, kv_dim = num_kv_heads * head_dim, nchunks = kv_dim / 8;
    constexpr float qmax = QBITS == 8 ? 127.f : 7.f;
    const S *src = (which ? v_src : k_src) + (have ? tok : 0) * (int64_t)kv_dim;
    float x[RC][8];
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < RC; ++i) {
        const int c = sub + 16 * (wave + kQuadWaves * i);
        if (have && c < nchunks) {
            load8(src + 8 * c, x[i]);
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) x[i][k] = 0.f;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) mx = fmaxf(mx, fabsf(x[i][k]));
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (sub == 0) red[wave][e] = mx;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kQuadWaves; ++w) mx = fmaxf(mx, red[w][e]);
    const bool valid = have && slot >= 0 && slot < num_slots;
    const float scale = mx / qmax;
    const float ok = scale > 0.f ? 1.f : 0.f;
    const float inv = 1.0f / scale;
    if (valid && wave == 0 && sub == 0) (which ? v_scales : k_scales)[slot] = ok != 0.f ? scale : 0.f;
    // Do the 4 tokens fill one quad of one block?  (The same 4 slots in every
    // wave: uniform over the work-group.)
    const int lo = (int)(slot & 0xffffffff), hi = (int)(slot >> 32);
    const int64_t s0 = ((int64_t)__shfl(hi, sub, 64) << 32) | (uint32_t)__shfl(lo, sub, 64);
    const bool quad = __all(valid && s0 % 4 == 0 && slot == s0 + e);
    uint8_t *pool = which ? v_pool : k_pool;
    const int64_t tile_bytes = (int64_t)d * BS * QBITS / 8;
    const int64_t blk = valid ? slot / BS : 0;
    const int t = valid ? (int)(slot - blk * BS) : 0;
#pragma unroll
    for (int i = 0; i < RC; ++i) {
        const int c = sub + 16 * (wave + kQuadWaves * i);
        const bool live = valid && c < nchunks;
        const int h = (8 * c) / d, j = 8 * c - h * d;
        uint8_t *tile = pool + (blk * num_kv_heads + h) * tile_bytes;
        uint32_t w0, w1;
        quant_chunk<QBITS>(x[i], ok, scale, inv, w0, w1);
        if (which == 0 || !quad) {  // uniform per wave
            if (live) place_chunk<QBITS>(tile, which, j, t, d, w0, w1);
            continue;
        }
        const int VG = QBITS == 8 ? 4 : (d % 128 == 0 ? 8 : 4);
        const int VLANE = VG * QBITS / 2;
        const int vq = j / (16 * VG), vn = (j % (16 * VG)) / VG, vk = j % VG;
        uint8_t *vbase = tile + ((int64_t)(vq * 4 + t / 4) * 16 + vn) * VLANE;  // the quad's word 0
        if constexpr (QBITS == 8) {
            // Words: dims 0..3 and 4..7 of the chunk; lane e stores dims e and 4 + e.
            const uint32_t r0 = quad_transpose(w0, e, sub), r1 = quad_transpose(w1, e, sub);
            if (live) {
                *reinterpret_cast<uint32_t *>(vbase + e * 4) = r0;
                *reinterpret_cast<uint32_t *>(vbase + VLANE + e * 4) = r1;
            }
        } else {
            // Word: byte m = dims 2m, 2m + 1 of the token; lane e stores dim pair e.
            const uint32_t r = quad_transpose(w0, e, sub);
            const int jj = vk + 2 * e;
            if (live) *reinterpret_cast<uint32_t *>(vbase + (jj / VG) * VLANE + ((jj % VG) / 2) * 4) = r;
        }
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
    if (!dlmk::aligned16(k_src) || !dlmk::aligned16(v_src) || !dlmk::aligned16(k_pool) ||
        !dlmk::aligned16(v_pool))
        return dlmk::fail(DLMK_ERR_INVALID_ARG,
                          "dlmk_kv_append_quant: sources and pools must be 16-byte aligned");
    const int nc = chunks_per_lane <= 1 ? 1 : chunks_per_lane <= 2 ? 2 : chunks_per_lane <= 4 ? 4 : 8;
    // Token quads (quad kernel) for appends of kQuadMinTokens or more; else
    // one work-group of 256 threads per token.
    const int64_t lane_chunks = dlmk::ceil_div(kv_dim / 8, (int64_t)(16 * kQuadWaves));
    const int rc = n_tok >= kQuadMinTokens && lane_chunks <= 8
                       ? (lane_chunks <= 1 ? 1 : lane_chunks <= 2 ? 2 : lane_chunks <= 4 ? 4 : 8)
                       : 0;
    const int64_t gx = n_tok;
    if (gx > 0x7fffffff) return dlmk::fail(DLMK_ERR_UNSUPPORTED, "dlmk_kv_append_quant: grid too large");
    auto s = (hipStream_t)stream;
    const int64_t num_slots = num_blocks * block_size;
    auto kp = (uint8_t *)k_pool, vp = (uint8_t *)v_pool;
#define DLMK_LAUNCH_NC(Q, S, NC)                                                                \
    hipLaunchKernelGGL((kv_append_quant_kernel<Q, S, NC>), dim3((unsigned)gx), dim3(256), 0, s, kp, \
                       vp, k_scales, v_scales, (const S *)k_src, (const S *)v_src, slot_mapping,  \
                       n_tok, num_kv_heads, head_dim, num_slots)
#define DLMK_LAUNCH_QUAD(Q, S, RC)                                                                   \
    hipLaunchKernelGGL((kv_append_quant_quad_kernel<Q, S, RC>),                                      \
                       dim3((unsigned)dlmk::ceil_div(n_tok, (int64_t)4), 2), dim3(64 * kQuadWaves), 0, s, \
                       kp, vp,                                                                       \
                       k_scales, v_scales, (const S *)k_src, (const S *)v_src, slot_mapping, n_tok,  \
                       num_kv_heads, head_dim, num_slots)
#define DLMK_LAUNCH(Q, S)                                             \
    switch (rc) {                                                     \
        case 1: DLMK_LAUNCH_QUAD(Q, S, 1); break;                     \
        case 2: DLMK_LAUNCH_QUAD(Q, S, 2); break;                     \
        case 4: DLMK_LAUNCH_QUAD(Q, S, 4); break;                     \
        case 8: DLMK_LAUNCH_QUAD(Q, S, 8); break;                     \
        default:                                                      \
            switch (nc) {                                             \
                case 1: DLMK_LAUNCH_NC(Q, S, 1); break;               \
                case 2: DLMK_LAUNCH_NC(Q, S, 2); break;               \
                case 4: DLMK_LAUNCH_NC(Q, S, 4); break;               \
                default: DLMK_LAUNCH_NC(Q, S, 8); break;              \
            }                                                         \
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
#undef DLMK_LAUNCH_QUAD
#undef DLMK_LAUNCH
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return dlmk::fail((int)e, "dlmk_kv_append_quant launch: %s", hipGetErrorString(e));
    return DLMK_OK;
}
