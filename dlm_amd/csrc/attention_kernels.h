#pragma once
// Paged GQA decode attention kernels (dlmk_paged_decode_attention) for gfx950.
// Included by attention.hip (entry points) and by one translation unit per
// pool format (attention_<format>.hip), which instantiate the kernels.
//
// Replaces attention_kernel (src/gpu/kernels.cu:210-242: one thread per query
// head, serial over a contiguous f32 history) and the CPU attention()
// (src/forward/cpu.rs:1126-1151).  Same maths -- score = dot(q, k) * scale,
// softmax over the visible positions, out = sum p * v -- evaluated as a
// streaming, HBM-bound pass over the paged pools.
//
// Work decomposition (both kernels).  One work-group owns one (sequence, kv
// head, partition of P tokens) and serves every query row that reads that kv
// head: the GQA group times the num_q_per_seq verify queries (ROWS rows).  K/V
// bytes of a partition are therefore read from HBM exactly once.  Partition
// blocks are dealt to the NW wavefronts round-robin.  Each wave computes an
// exact softmax over its own tokens (max over all its scores first, so no
// rescaling), the waves are merged in LDS, and partitions of one sequence are
// merged by log-sum-exp in a second kernel (a sequence whose context fits one
// partition is finished by the first).  Everything runs in the log2 domain
// with log2(e) folded into the scale.
//
// f16 / bf16 pools: matrix-core kernel.  Per 16-token block and wave:
//   S^T (16 tokens x 16 rows) = K (16 x d) . Q^T (d x 16)
//     v_mfma_f32_16x16x32_{f16,bf16}, d/32 steps.  A K-tile load of lane l
//     (chunk row l/16 + 4i of token l%16, 16 bytes) is exactly the A operand,
//     the query rows (zero-padded to 16) are the B operand.  The accumulator
//     lands as lane l = (row l%16, tokens 4(l/16)..+3).
//   O (16 rows x d) += P (16 x 16 tokens) . V (16 tokens x d)
//     v_mfma_f32_16x16x16_{f16,bf16}, d/16 steps.  S^T's accumulator layout
//     IS the A-operand layout of this product, so P never leaves registers;
//     the B operand is 4 tokens x 1 dim = 8 contiguous bytes of the V tile
//     [d][16].
// int8 / int4 pools: the same kernel over f16 operands widened in registers
//   from tiles laid out for 16-byte loads per lane (storage codecs below);
//   query groups of up to 4 rows (int4: 8) run paged_attn_packed_kernel,
//   which puts 4 (2) blocks into one score tile instead of padding it with
//   zero query rows.
// f32 pools, and geometries the tuned kernels are not instantiated for:
//   paged_attn_generic_kernel, the same tiling with the head dim, GQA group
//   and query count at run time (f32 on v_mfma_f32_16x16x4_f32).

#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>

#include "dlmk.h"
#include "dlmk_internal.h"

// Launch arguments shared by the entry points and the per-format dispatchers.
namespace dlmk_attn {
struct Args {
    void *out;
    int out_dtype;
    const void *q;
    void *k_pool, *v_pool;
    const float *k_scales, *v_scales;  // quantized pools: one f32 per (block, token slot)
    const void *k_new, *v_new;         // fused decode step: tokens appended in the same launch
    const int32_t *tables, *ctx_lens;
    int B, NQ, Hq, Hkv, max_blocks;
    int64_t num_blocks;
    float scale;
    int D;               // head dim
    void *workspace;     // split-K partials, 256-byte aligned (may be NULL if never needed)
    size_t ws_bytes;     // bytes available at workspace
    hipStream_t stream;
};

// Per-format dispatchers (one translation unit each): launch the partition
// kernel (and the combine kernel) for head_dim and GQA group a.Hq / a.Hkv.
int dispatch_f32(const Args &a, int head_dim);
int dispatch_f16(const Args &a, int head_dim);
int dispatch_bf16(const Args &a, int head_dim);
int dispatch_i8(const Args &a, int head_dim);
int dispatch_i4(const Args &a, int head_dim);
}  // namespace dlmk_attn

namespace {

using dlmk_attn::Args;

constexpr int kBlock = 16;          // tokens per KV block (dlm: src/main.rs:455)
constexpr int kMinPartition = 64;  // smallest partition of any kernel (sizes the workspace)
constexpr float kLog2e = 1.4426950408889634f;

// Matrix-core kernel shape: waves per work-group, blocks per wave, prefetch
// depth in tile loads (overridable at build time for tuning sweeps).
#ifndef DLMK_MFMA_NW
#define DLMK_MFMA_NW 4
#endif
#ifndef DLMK_MFMA_NB
#define DLMK_MFMA_NB 16
#endif
#ifndef DLMK_MFMA_PD
#define DLMK_MFMA_PD 2
#endif
// Minimum waves per SIMD for the quantized-pool kernels: half the bytes per
// tile leave the per-tile latency chain exposed, so they trade registers for
// occupancy.
#ifndef DLMK_MFMA_QWAVES
#define DLMK_MFMA_QWAVES 3
#endif
// Prefetch depth for int8 / int4 pools, whose tiles are 2x / 4x smaller.
#ifndef DLMK_MFMA_PDQ
#define DLMK_MFMA_PDQ 2
#endif
// Prefetch depth of paged_attn_packed_kernel, in 16-byte loads per lane, for
// 4 blocks per score tile (groups of up to 4 rows) and for 2 (5-8 rows).
// Measured (attention only, two runs): 4 blocks, configs[1]: int4 50.4 /
// 52.2 / 52.0% of HBM peak at depth 2 / 4 / 8, int8 65.3 / 67.0 / 67.5%;
// 2 blocks, configs[3] int4: 56.9 / 54.0 / 54.4% at depth 2 / 4 / 8.
#ifndef DLMK_MFMA_PDP4
#define DLMK_MFMA_PDP4 8
#endif
#ifndef DLMK_MFMA_PDP2
#define DLMK_MFMA_PDP2 2
#endif
// Minimum waves per SIMD the register allocation must allow for every pool
// format (0: per-format defaults above; a tuning override).
#ifndef DLMK_MFMA_WPE
#define DLMK_MFMA_WPE 0
#endif
// Quantized pools that run paged_attn_packed_kernel (bit 0: int4 with at
// most 8 query rows, bit 1: int8 with at most 4, bit 2: int8 with 5-8).
// Measured at configs[1] (4 rows) and configs[3] (8 rows), attention only:
// int4 47.4 -> 49.6% and 55.0 -> 57.3% of HBM peak; int8 63.9 -> 65.5% with
// 4 rows but 67.9 -> 64.2% with 8.
#ifndef DLMK_MFMA_PACKED
#define DLMK_MFMA_PACKED 3
#endif
// int8 rows of more than this many partitions take the unpacked kernel:
// configs[2] (rows up to 8704 tokens, 9 partitions) 66.1 -> 67.2% of HBM peak
// that way; configs[1] (4 partitions) keeps the packed kernel's 67.7%.
#ifndef DLMK_PACKED_I8_MAXPARTS
#define DLMK_PACKED_I8_MAXPARTS 4
#endif
// Blocks per wave for int8 pools.
#ifndef DLMK_MFMA_Q8NB
#define DLMK_MFMA_Q8NB 16
#endif
// 1: stream K/V tiles with non-temporal loads (no reuse, keep them out of L2/MALL).
#ifndef DLMK_MFMA_NT
#define DLMK_MFMA_NT 1
#endif

// Pool stores of new tokens: non-temporal (written around the caches).  The
// kernels stream the pools with non-temporal loads; read back that way, lines
// written through the caches by an earlier launch measured several us slower
// per launch at the 8B shape.
template <typename V>
__device__ __forceinline__ void pool_store(V *p, V v) {
    __builtin_nontemporal_store(v, p);
}

template <typename V>
__device__ __forceinline__ V stream_load(const V *p) {
#if DLMK_MFMA_NT
    return __builtin_nontemporal_load(p);
#else
    return *p;
#endif
}

// Tile loads through a buffer resource covering one tile: a masked tile gets
// num_records 0, and its loads return zeros without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void *tile, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(tile), 0, bytes, 0x00020000);
}
template <typename T>
__device__ __forceinline__ T buf_load(__amdgpu_buffer_rsrc_t r, int byte_off) {
    constexpr int aux = DLMK_MFMA_NT ? 2 : 0;  // nt
    if constexpr (sizeof(T) == 16)
        return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, aux));
    else
        return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, aux));
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void store_out(void *out, int out_dtype, int64_t idx, float v) {
    if (out_dtype == DLMK_F32) {
        static_cast<float *>(out)[idx] = v;
    } else if (out_dtype == DLMK_F16) {
        static_cast<_Float16 *>(out)[idx] = (_Float16)v;
    } else {
        static_cast<__bf16 *>(out)[idx] = (__bf16)v;  // round to nearest even
    }
}

template <int W>
__device__ __forceinline__ float xor_sum(float v) {
#pragma unroll
    for (int o = 1; o < W; o <<= 1) v += __shfl_xor(v, o);
    return v;
}

template <int W>
__device__ __forceinline__ float xor_max(float v) {
#pragma unroll
    for (int o = 1; o < W; o <<= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ int parts_of(int ctx, int P) { return ctx > P ? (ctx + P - 1) / P : 1; }

// Shared epilogue: merge the NW waves' (m, l, O) of one work-group and either
// finish the rows (single-partition sequence) or store the partition partial.
// The ROWS x NW merge weights 2^(m_w - M) are computed once into LDS, so the
// per-element pass is a plain weighted sum of the waves' O.
// o_lds rows may be padded (DS > D) to keep the waves' stores conflict-free.
template <int ROWS, int D, int NW, int GQA, int NQ, int DS>
__device__ __forceinline__ void merge_waves(const float (&o_lds)[NW][ROWS][DS],
                                            const float (&ml_lds)[NW][ROWS][2], void *out,
                                            int out_dtype, int seq, int kvh, int part,
                                            int nparts, int num_q_heads, int max_parts,
                                            float *ws_o, float *ws_ml) {
    __shared__ float fac[ROWS][NW];
    __shared__ float rowML[ROWS][2];
    if (threadIdx.x < ROWS) {
        const int r = threadIdx.x;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, ml_lds[w][r][0]);
        float L = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float mw = ml_lds[w][r][0];
            const float f = (M == -INFINITY || mw == -INFINITY) ? 0.f : exp2f(mw - M);
            fac[r][w] = f;
            L = fmaf(f, ml_lds[w][r][1], L);
        }
        rowML[r][0] = M;
        rowML[r][1] = L;
    }
    __syncthreads();
    // Four consecutive dims per thread: 16-byte LDS reads and partial stores.
    static_assert(D % 4 == 0, "float4 merge");
    for (int idx = threadIdx.x; idx < ROWS * D / 4; idx += NW * 64) {
        const int r = idx / (D / 4), d = 4 * (idx - r * (D / 4));
        float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float4 v = *reinterpret_cast<const float4 *>(&o_lds[w][r][d]);
            const float f = fac[r][w];
            O.x = fmaf(f, v.x, O.x);
            O.y = fmaf(f, v.y, O.y);
            O.z = fmaf(f, v.z, O.z);
            O.w = fmaf(f, v.w, O.w);
        }
        const float L = rowML[r][1];
        const int j = r / GQA, h = kvh * GQA + r % GQA;
        const int64_t row = (int64_t)(seq * NQ + j) * num_q_heads + h;
        if (nparts == 1) {
            store_out(out, out_dtype, row * D + d, L > 0.f ? O.x / L : 0.f);
            store_out(out, out_dtype, row * D + d + 1, L > 0.f ? O.y / L : 0.f);
            store_out(out, out_dtype, row * D + d + 2, L > 0.f ? O.z / L : 0.f);
            store_out(out, out_dtype, row * D + d + 3, L > 0.f ? O.w / L : 0.f);
        } else {
            const int64_t slot = row * max_parts + part;
            *reinterpret_cast<float4 *>(&ws_o[slot * D + d]) = O;
            if (d == 0) {
                ws_ml[2 * slot] = rowML[r][0];
                ws_ml[2 * slot + 1] = L;
            }
        }
    }
}

// 1: a wave processes its NB blocks last first (measured 100.4 against
// 101.4 us a launch at the 8B shape, configs[1]).
#ifndef DLMK_MFMA_REV
#define DLMK_MFMA_REV 1
#endif
// Position of a wave's b-th processed block among its NB blocks.
__device__ __forceinline__ int wave_block(int b, int nb) { return DLMK_MFMA_REV ? nb - 1 - b : b; }

// Fused decode step, append work-group: threads tid, tid + nthreads, ...
// store the K and V of sequence seq's newest nq positions for every kv head,
// (kv head, position, dim) flattened over the threads (the bits
// dlmk_kv_append writes; masked or out-of-pool blocks skipped).
template <typename T, int D>
__device__ __forceinline__ void append_new_tokens(T *k_pool, T *v_pool, const T *k_new,
                                                  const T *v_new, const int32_t *block_tables,
                                                  const int32_t *ctx_lens, int seq,
                                                  int num_kv_heads, int nq, int max_blocks,
                                                  int64_t num_blocks, int tid, int nthreads) {
    constexpr int X = 16 / sizeof(T);
    constexpr int TILE = D * kBlock;
    const int ctx = min(ctx_lens[seq], max_blocks * kBlock);
    // K: a token's 8-dim chunk is 16 contiguous bytes of the tile (one store;
    // 103.6 -> 103.3 us a step at the 8B shape against one element a thread).
    typedef uint32_t w4t __attribute__((ext_vector_type(4)));
    for (int e = tid; e < num_kv_heads * nq * (D / X); e += nthreads) {
        const int c = e % (D / X), j = (e / (D / X)) % nq, kvh = e / ((D / X) * nq), p = ctx - nq + j;
        if (p < 0) continue;
        const int64_t blk = block_tables[(int64_t)seq * max_blocks + p / kBlock];
        if (blk < 0 || blk >= num_blocks) continue;
        const int t = p % kBlock;
        const int64_t base = (blk * num_kv_heads + kvh) * TILE;
        const int64_t src = ((int64_t)(seq * nq + j) * num_kv_heads + kvh) * D + c * X;
        pool_store(reinterpret_cast<w4t *>(&k_pool[base + (c * kBlock + t) * X]),
                   *reinterpret_cast<const w4t *>(&k_new[src]));
    }
    // V: one element per (dim, token) in the [D][16] tile.
    for (int e = tid; e < num_kv_heads * nq * D; e += nthreads) {
        const int dim = e % D, j = (e / D) % nq, kvh = e / (D * nq), p = ctx - nq + j;
        if (p < 0) continue;
        const int64_t blk = block_tables[(int64_t)seq * max_blocks + p / kBlock];
        if (blk < 0 || blk >= num_blocks) continue;
        const int t = p % kBlock;
        const int64_t base = (blk * num_kv_heads + kvh) * TILE;
        const int64_t src = ((int64_t)(seq * nq + j) * num_kv_heads + kvh) * D + dim;
        pool_store(&v_pool[base + dim * kBlock + t], v_new[src]);
    }
}

__device__ __forceinline__ bool holds_new(int lb, int ctx, int nq) {
    return lb * kBlock < ctx && lb * kBlock + kBlock > ctx - nq;
}

// ---------------------------------------------------------------------------
// Matrix-core partition kernel (f16 / bf16 pools).
// ---------------------------------------------------------------------------
template <typename T>
struct Mfma;

template <>
struct Mfma<_Float16> {
    using elem = _Float16;
    using x8 = f16x8;
    using x4 = f16x4;
    static __device__ __forceinline__ f32x4 qk(x8 a, x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 pv(x4 a, x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mfma<__bf16> {
    using elem = __bf16;
    using x8 = bf16x8;
    using x4 = bf16x4;
    static __device__ __forceinline__ f32x4 qk(x8 a, x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 pv(x4 a, x4 b, f32x4 c) {
        typedef short s16x4 __attribute__((ext_vector_type(4)));
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                         __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
    }
};

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Exact widening of small integer codes to f16 without conversions: the f16
// with bit pattern 0x64uu is 1024 + uu for any byte uu, so a code c stored
// offset binary as the unsigned byte (or nibble) c + b and placed under a
// 0x64 high byte is the f16 value B + c with B = 1024 + b.  v_perm_b32 builds two such halves from bytes lo,
// lo + 1 of w in one op.  The bias is not subtracted per element: the kernel
// removes B * sum(q) from each score and B * sum(p) from each output row
// (dot products are linear in the codes), which takes one VALU op per code
// pair off the inner loops.  B + c is exact in f16 (|B + c| < 2048) and the
// products are exact in the f32 accumulators, so the only extra rounding is
// f32 accumulation of the larger partial sums (about 2^-24 * B relative to
// the q or p magnitudes).
template <int LO>
__device__ __forceinline__ f16x2 biased_pair(uint32_t w) {
    constexpr uint32_t sel = 0x04000400u | (uint32_t)LO | (uint32_t)(LO + 1) << 16;
    return __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, w, sel));
}

// Four biased byte codes (bytes 0..3 of w) -> f16x4 of B + c.
__device__ __forceinline__ f16x4 biased4(uint32_t w) {
    const f16x2 a = biased_pair<0>(w), b = biased_pair<2>(w);
    return f16x4{a[0], a[1], b[0], b[1]};
}

// Four bytes of w whose low nibbles are zero -> f16x4 of 1 + byte / 1024: the
// byte goes under a 0x3C high byte (exponent 0), so a nibble n held in the
// byte's high half becomes 1 + n / 64.  With the nibble in mantissa bits 4-7
// instead of 0-3, the bias is 72 code units (1 + 8/64 against a unit of 1/64)
// rather than 1032: small enough for the kernel to remove it from the score
// after the dot product, as for int8 codes (1152 units against codes 16x
// larger).
__device__ __forceinline__ f16x4 unit4(uint32_t w) {
    const f16x2 a = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x3c3c3c3cu, w, 0x04010400u));
    const f16x2 b = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x3c3c3c3cu, w, 0x04030402u));
    return f16x4{a[0], a[1], b[0], b[1]};
}

// Storage codecs of the matrix-core kernel, one per pool format and head
// dim D.  A codec says where a lane's K and V bytes sit in a (block, kv head)
// tile and how they become MFMA operands:
//   QK (S^T = K.Q^T, 16x16x32): step i takes 8 dims of token n (lane n + 16g)
//     from K load i / SK, sub-step i % SK; q_chunk(i, g) is the 8-dim Q chunk
//     those 8 K dims pair with, and q_op permutes a Q chunk into the order
//     k_op emits K in (the dot product does not care which dims pair up, only
//     that both sides agree).
//   PV (O = P.V, 16x16x16): step k takes 4 tokens (4g .. 4g + 3) of one dim,
//     from V load k / SV, sub-step k % SV; its output column n is dim
//     v_dim(k, n).
// Each lane loads 16 bytes per instruction wherever a tile holds that many
// per lane: the int8 kernel with 8-byte K and 4-byte V loads reached 62% of
// the read bandwidth a pure 16-byte read of the same tiles reaches 77%.
//   Quantized codecs keep one f32 scale per token: K scales multiply the
//     score, V scales multiply the probabilities (p * v_scale, 4 values per
//     lane, instead of 32 widened values).  Codes widen to f16 exactly, as
//     kBias + code (the kernel removes the bias).
template <typename E, int D>
struct CodecFloat {  // f16 / bf16 pools: K [d/8][16][8], V [d][16] elements
    static constexpr int kCodeBits = 16;
    using QT = E;
    using Op = Mfma<E>;
    using KRaw = typename Op::x8;
    using VRaw = typename Op::x4;
    static constexpr bool kScaled = false;
    static constexpr bool kBufLoads = true;
    static constexpr int kMinWaves = 1;  // memory-bound at the compiler's allocation
    static constexpr float kBias = 0.f, kBiasK = 0.f, kKScale = 1.f;
    static constexpr int64_t kTileBytes = (int64_t)D * kBlock * sizeof(E);
    static constexpr int SK = 1, KL = D / 32, SV = 1, VL = D / 16;
    static __device__ __forceinline__ KRaw load_k(const uint8_t *tile, int i, int lane) {
        return stream_load(reinterpret_cast<const KRaw *>(tile) + 64 * i + lane);
    }
    static __device__ __forceinline__ VRaw load_v(const uint8_t *tile, int k, int lane) {
        const int g = lane >> 4, n = lane & 15;
        return stream_load(reinterpret_cast<const VRaw *>(tile) + ((16 * k + n) * kBlock + 4 * g) / 4);
    }
    static __device__ __forceinline__ int k_off(int i, int lane) { return (64 * i + lane) * (int)sizeof(KRaw); }
    static __device__ __forceinline__ int v_off(int k, int lane) {
        const int g = lane >> 4, n = lane & 15;
        return ((16 * k + n) * kBlock + 4 * g) / 4 * (int)sizeof(VRaw);
    }
    static __device__ __forceinline__ int q_chunk(int i, int g) { return 4 * i + g; }
    static __device__ __forceinline__ KRaw q_op(KRaw q) { return q; }
    static __device__ __forceinline__ typename Op::x8 k_op(KRaw r, int) { return r; }
    static __device__ __forceinline__ typename Op::x4 v_op(VRaw r, int) { return r; }
    static __device__ __forceinline__ int v_dim(int k, int n) { return 16 * k + n; }
};

template <int D>
using CodecF16 = CodecFloat<_Float16, D>;
template <int D>
using CodecBF16 = CodecFloat<__bf16, D>;

// Quantized tiles (head dim a multiple of 64), int4 codes two to a byte with
// the even element in the low nibble:
//   K [D/KG][16 tokens][KG dims]: one lane load = KG dims of token n = SK
//     QK steps (8 dims each);
//   V [D/(16 VG)][4 token quads][16][VG dims][4 tokens]: one lane load = 4
//     tokens x VG dims = VG PV steps, lane n holding dims VG n .. VG n + VG - 1
//     of its quarter.
template <int D>
struct CodecI8 {  // KG = 16, VG = 4: 16-byte K and V loads
    static constexpr int kCodeBits = 8;
    using QT = _Float16;
    using Op = Mfma<_Float16>;
    using KRaw = u32x4;
    using VRaw = u32x4;
    static constexpr bool kScaled = true;
    static constexpr bool kBufLoads = true;
    static constexpr float kBias = 1024.f + 128.f, kBiasK = kBias, kKScale = 1.f;  // bytes c + 128
    static constexpr int kMinWaves = D <= 128 ? DLMK_MFMA_QWAVES : 1;
    static constexpr int64_t kTileBytes = (int64_t)D * kBlock;
    static constexpr int KG = 16, VG = 4;  // dims per K / V load of a lane
    static constexpr int SK = 2, KL = D / 64, SV = 4, VL = D / 64;
    static __device__ __forceinline__ KRaw load_k(const uint8_t *tile, int p, int lane) {
        return stream_load(reinterpret_cast<const KRaw *>(tile) + 64 * p + lane);
    }
    static __device__ __forceinline__ VRaw load_v(const uint8_t *tile, int l, int lane) {
        return stream_load(reinterpret_cast<const VRaw *>(tile) + 64 * l + lane);
    }
    static __device__ __forceinline__ int k_off(int p, int lane) { return (64 * p + lane) * (int)sizeof(KRaw); }
    static __device__ __forceinline__ int v_off(int l, int lane) { return (64 * l + lane) * (int)sizeof(VRaw); }
    static __device__ __forceinline__ int q_chunk(int i, int g) { return 8 * (i >> 1) + 2 * g + (i & 1); }
    static __device__ __forceinline__ f16x8 q_op(f16x8 q) { return q; }
    static __device__ __forceinline__ f16x8 k_op(KRaw r, int s) {
        const f16x4 a = biased4(r[2 * s]), b = biased4(r[2 * s + 1]);
        return f16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    }
    static __device__ __forceinline__ f16x4 v_op(VRaw r, int kk) { return biased4(r[kk]); }
    static __device__ __forceinline__ int v_dim(int k, int n) { return 64 * (k >> 2) + 4 * n + (k & 3); }
};

template <int D>
struct CodecI4 {  // KG, VG = 32, 8 (D % 128 == 0: 16-byte loads) or 16, 4 (D = 64: 8-byte loads, a whole tile)
    static constexpr int kCodeBits = 4;
    static constexpr bool kWide = D % 128 == 0;
    static constexpr int KG = kWide ? 32 : 16, VG = kWide ? 8 : 4;
    using QT = _Float16;
    using Op = Mfma<_Float16>;
    using KRaw = typename std::conditional<kWide, u32x4, u32x2>::type;
    using VRaw = KRaw;
    static constexpr bool kScaled = true;
    static constexpr bool kBufLoads = false;  // measured slower with them (configs[3] -1.3 points)
    // K nibbles widen to 1 + (c + 8) / 64 (unit4): the score is
    // (dot - 1.125 * sum(q)) * k_scale * 64, the 64 folded into the softmax
    // scale.  The 0x64 widening of the V codes
    // (B + c, B = 1032) would put a 1032-unit bias on K as well, whose f32
    // cancellation in the scores, scaled by a large token's K scale, reached
    // the output tolerance; the V bias is relative to p * v_scale, which the
    // output is divided by.
    static constexpr float kBias = 1024.f + 8.f;  // V nibbles c + 8
    static constexpr float kBiasK = 1.125f, kKScale = 64.f;
    static constexpr int kMinWaves = D <= 128 ? DLMK_MFMA_QWAVES : 1;
    static constexpr int64_t kTileBytes = (int64_t)D * kBlock / 2;
    static constexpr int SK = KG / 8, KL = D / (4 * KG), SV = VG, VL = D / (16 * VG);
    static __device__ __forceinline__ KRaw load_k(const uint8_t *tile, int p, int lane) {
        return stream_load(reinterpret_cast<const KRaw *>(tile) + 64 * p + lane);
    }
    static __device__ __forceinline__ VRaw load_v(const uint8_t *tile, int l, int lane) {
        return stream_load(reinterpret_cast<const VRaw *>(tile) + 64 * l + lane);
    }
    static __device__ __forceinline__ int k_off(int p, int lane) { return (64 * p + lane) * (int)sizeof(KRaw); }
    static __device__ __forceinline__ int v_off(int l, int lane) { return (64 * l + lane) * (int)sizeof(VRaw); }
    static __device__ __forceinline__ int q_chunk(int i, int g) { return SK * (4 * (i / SK) + g) + i % SK; }
    // k_op emits a word's elements in the order 0 2 4 6 1 3 5 7 (even nibbles, then odd).
    static __device__ __forceinline__ f16x8 q_op(f16x8 q) {
        return f16x8{q[0], q[2], q[4], q[6], q[1], q[3], q[5], q[7]};
    }
    static __device__ __forceinline__ f16x8 k_op(KRaw r, int s) {
        const uint32_t x = r[s];  // nibbles c + 8
        const f16x4 a = unit4((x << 4) & 0xf0f0f0f0u), b = unit4(x & 0xf0f0f0f0u);
        return f16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    }
    // Word kk / 2 holds dims kk & ~1 (low nibbles) and kk | 1 of 4 tokens.
    static __device__ __forceinline__ f16x4 v_op(VRaw r, int kk) {
        return biased4((r[kk >> 1] >> (4 * (kk & 1))) & 0x0f0f0f0fu);
    }
    static __device__ __forceinline__ int v_dim(int k, int n) { return 16 * VG * (k / VG) + VG * n + k % VG; }
};

#if DLMK_MFMA_WPE
#define DLMK_MFMA_ATTRS __attribute__((amdgpu_waves_per_eu(DLMK_MFMA_WPE)))
#else
#define DLMK_MFMA_ATTRS __attribute__((amdgpu_waves_per_eu(C::kMinWaves)))
#endif

template <typename C, int D, int GQA, int NQ, int NW, int NB, int PD>
__global__ __launch_bounds__(NW * 64) DLMK_MFMA_ATTRS void paged_attn_mfma_kernel(
    void *__restrict__ out, int out_dtype, const typename C::QT *__restrict__ q,
    uint8_t *__restrict__ k_pool, uint8_t *__restrict__ v_pool,
    const float *__restrict__ k_scales, const float *__restrict__ v_scales,
    const typename C::QT *__restrict__ k_new, const typename C::QT *__restrict__ v_new,
    const int32_t *__restrict__ block_tables, const int32_t *__restrict__ ctx_lens,
    int num_q_heads, int num_kv_heads, int max_blocks, int64_t num_blocks, float scale_log2,
    int max_parts, float *__restrict__ ws_o, float *__restrict__ ws_ml, int append_row) {
    using M = typename C::Op;
    using x8 = typename M::x8;
    using x4 = typename M::x4;
    using PT = typename M::elem;
    using QT = typename C::QT;
    constexpr int ROWS = GQA * NQ;
    constexpr int KI = D / 32;           // QK steps per block
    constexpr int VN = D / 16;           // PV steps per block
    constexpr int P = NW * NB * kBlock;  // tokens per work-group
    constexpr int64_t TILE = C::kTileBytes;  // bytes per (block, kv head)
    static_assert(ROWS <= 16 && D % 32 == 0, "unsupported geometry");

    // Rows padded by 16 bytes: rows D * 4 bytes apart sit in the same LDS banks,
    // and the epilogue's stores write several rows per instruction.
    __shared__ __attribute__((aligned(16))) float o_lds[NW][ROWS][D + 4];
    __shared__ float ml_lds[NW][ROWS][2];

    // blockIdx.x = seq * num_kv_heads + kv head, blockIdx.y = partition: the
    // dispatcher deals consecutive work-groups to the 8 XCDs round-robin, so
    // with the (sequence, head) pair fastest every XCD gets the same mix of
    // full and ragged partitions (partition-fastest would pin each XCD to one
    // partition index, and late partitions exist only for long contexts).
    // Partitions are dealt last index first: the high indices (long contexts
    // only, mostly full) start early and the grid ends on partition 0, where
    // the short sequences' small work-groups fill the drain (+1 point of HBM
    // peak over first-index-first at the 8B shape).
    if constexpr (!C::kScaled) {
        // Fused decode step: the partition work-groups take the new tokens
        // from k_new / v_new in registers instead of the pools.  When a
        // combine launch follows, it stores them into the pools (configs[1]
        // step 100.4 -> 99.9 us against 97.7 for the attention pair);
        // otherwise the first row of the grid (dealt first) does, one
        // work-group per sequence (the row's work-groups of kv head 0)
        // covering all its kv heads.
        // Measured at the 8B shape (configs[1], step / attention alone):
        //   stores issued by the partition waves themselves, behind a fence:
        //     109.8 / 100.4 us; from the owning wave's substitution
        //     registers, no fence: 108.6 / 100.5 us;
        //   append row, one work-group per (sequence, kv head): 105.2 / 100.7;
        //   the same row as the grid's last (dealt last): 105.6 / 100.7 (per
        //   sequence and dealt last: 103.9 against 103.6 dealt first);
        //   one work-group per sequence: 103.9-104.4 / 100.7-101.0;
        //   per 4 or 16 sequences: 107.6 / 111.1 us;
        //   whole 32-byte sectors rewritten (read, substitute, store by lane
        //   pairs), not the tokens' 2-byte elements: 112.0 against 103.5 us.
        // With the row's stores skipped (wrong results, timing only) the step
        // takes 100.6 us and without the substitution 103.1: the 2.7 us left
        // over the attention is the stores themselves.  Issued by the combine
        // launch instead they still cost 2.2 us: each V element is a 2-byte
        // write into a different 32-byte row of the [d][16] tile (as plain
        // stores through the caches instead of non-temporal: 104.4 us).
        if (append_row && blockIdx.y == 0) {
            if (blockIdx.x % num_kv_heads == 0)
                append_new_tokens<QT, D>(reinterpret_cast<QT *>(k_pool), reinterpret_cast<QT *>(v_pool),
                                         k_new, v_new, block_tables, ctx_lens, blockIdx.x / num_kv_heads,
                                         num_kv_heads, NQ, max_blocks, num_blocks, threadIdx.x, NW * 64);
            return;
        }
    }
    const int part = gridDim.y - 1 - blockIdx.y;
    const int kvh = blockIdx.x % num_kv_heads, seq = blockIdx.x / num_kv_heads;
    // A length beyond the table width is clamped: no read past a table row and
    // no partition index past max_parts.
    const int ctx = min(ctx_lens[seq], max_blocks * kBlock);
    const int nparts = parts_of(ctx, P);
    if (part >= nparts) return;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, n = lane & 15;  // lane group, row (QK) / dim (PV) index
    const int nblk_seq = (ctx + kBlock - 1) / kBlock;
    const int32_t *table = block_tables + (int64_t)seq * max_blocks;

    // Q^T operand: row n of the group, chunk q_chunk(i, g) (zeroed beyond
    // ROWS below).  Lanes past ROWS load row n % ROWS, so the loads carry no
    // branches (a masked load would make its first use wait for it).
    x8 qb[KI];
    {
        const int r = n % ROWS;
        const int j = r / GQA, h = kvh * GQA + r % GQA;
        const x8 *qp = reinterpret_cast<const x8 *>(q + ((int64_t)(seq * NQ + j) * num_q_heads + h) * D);
#pragma unroll
        for (int i = 0; i < KI; ++i) qb[i] = qp[C::q_chunk(i, g)];
    }
    // Causal limit of this lane's row (verify query n / GQA).
    const int limit = n < ROWS ? ctx - NQ + n / GQA + 1 : ctx;

    // This wave's blocks: partition block b*NW + wave.  Blocks past the
    // context (or with an id outside the pool) are masked: their loads are
    // pointed at the wave's first block, so that every load is issued
    // unconditionally, and with buffer loads (f16 / bf16 and int8 pools) the
    // tile's resource has no records, so they return zeros without touching
    // memory.  Re-reads of the first block had partly come from HBM:
    // configs[1] 71.0 -> 72.9% of HBM peak and traffic 1.047 -> 1.017x the
    // algorithmic bytes, configs[4] 65.9 -> 67.5%, int8 60.5 -> 61.6%; int4
    // measured a point slower and keeps global loads of the first block.
    int lbs[NB];
    int64_t blk[NB];
    bool ok[NB];
    int nvalid = 0;
    // The table reads are unconditional (index clamped into the row), so the
    // NB scalar loads go out back to back and share one wait; a guarded read
    // per block would serialise NB memory round trips before the first tile.
    int32_t raw[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int lb = part * (NW * NB) + wave_block(b, NB) * NW + wave;
        raw[b] = table[max(min(lb, nblk_seq - 1), 0)];
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int lb = part * (NW * NB) + wave_block(b, NB) * NW + wave;
        const int64_t id = lb < nblk_seq ? (int64_t)raw[b] : -1;
        lbs[b] = lb;
        ok[b] = id >= 0 && id < num_blocks;
        blk[b] = id;
        nvalid += ok[b];
    }

    float m = -INFINITY, lsum = 0.f;
    f32x4 accp = {0.f, 0.f, 0.f, 0.f};  // quantized pools: P row sums (rows 4g + j)
    f32x4 acc[VN];
#pragma unroll
    for (int k = 0; k < VN; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Fused decode step: the newest NQ positions ctx - NQ .. ctx - 1 may not
    // be in the pools yet (the append work-groups store them concurrently).
    // They span at most two consecutive logical blocks, which belong to
    // different waves (blocks are dealt round-robin), so a wave owns at most
    // one of them (bnew).  The wave loads that block's tiles as usual, reads
    // the new tokens' K/V from k_new / v_new alongside, and substitutes them
    // lane by lane: the same bits the append writes, whichever bytes the tile
    // load saw.
    static_assert(NW >= 2, "new-token blocks must land on different waves");
    int bnew = -1;
    if constexpr (!C::kScaled) {
        if (k_new != nullptr) {
#pragma unroll
            for (int b = 0; b < NB; ++b)
                if (ok[b] && holds_new(lbs[b], ctx, NQ)) bnew = b;
        }
    }
    bnew = __builtin_amdgcn_readfirstlane(bnew);
    const int lb_new = part * (NW * NB) + wave_block(bnew, NB) * NW + wave;
    const int first_new = ctx - NQ;
    // K: lane (token n, group g) covers chunk rows 4i + g of token n.
    const int jk = lb_new * kBlock + n - first_new;
    const bool k_is_new = jk >= 0 && jk < NQ;
    x8 knew[KI];
    x4 vnew[VN];
    if constexpr (!C::kScaled) {
        if (bnew >= 0) {
            const QT *kr = k_new + ((int64_t)(seq * NQ + min(max(jk, 0), NQ - 1)) * num_kv_heads + kvh) * D;
#pragma unroll
            for (int i = 0; i < KI; ++i) knew[i] = reinterpret_cast<const x8 *>(kr)[4 * i + g];
            // V: lane (dim n of step k, group g) covers tokens 4g .. 4g + 3.
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int jv = min(max(lb_new * kBlock + 4 * g + e - first_new, 0), NQ - 1);
                const QT *vr = v_new + ((int64_t)(seq * NQ + jv) * num_kv_heads + kvh) * D;
#pragma unroll
                for (int k = 0; k < VN; ++k) vnew[k][e] = vr[16 * k + n];
            }
        }
    }

    if (nvalid > 0) {
        int64_t first = 0;
#pragma unroll
        for (int b = NB - 1; b >= 0; --b)
            if (ok[b]) first = blk[b];
#pragma unroll
        for (int b = 0; b < NB; ++b)
            if (!ok[b]) blk[b] = first;

        // Software pipeline over the wave's 2*NB tile loads (K tiles of
        // blocks 0..NB-1, then V tiles): load stage t + PD is issued before
        // stage t is consumed, and scheduling barriers keep the compiler from
        // sinking the loads next to their uses.
        typename C::KRaw kb[NB][C::KL];
        typename C::VRaw vb[NB][C::VL];
        f32x4 ksc[NB], vsc[NB];
        // A stage's scale load goes out before its code loads, fenced by a
        // scheduling barrier: loads complete in issue order, so waiting for
        // a scale never waits for a later stage's codes.
        auto issue = [&](int t) {
            if (t < NB) {
                if constexpr (C::kScaled) {
                    ksc[t] = *reinterpret_cast<const f32x4 *>(k_scales + blk[t] * kBlock + 4 * g);
                    __builtin_amdgcn_sched_barrier(0);
                }
                const uint8_t *kt = k_pool + (blk[t] * num_kv_heads + kvh) * TILE;
                if constexpr (C::kBufLoads) {
                    const auto rk = tile_rsrc(kt, ok[t] ? (int)TILE : 0);
#pragma unroll
                    for (int i = 0; i < C::KL; ++i) kb[t][i] = buf_load<typename C::KRaw>(rk, C::k_off(i, lane));
                } else {
#pragma unroll
                    for (int i = 0; i < C::KL; ++i) kb[t][i] = C::load_k(kt, i, lane);
                }
            } else if (t < 2 * NB) {
                if constexpr (C::kScaled) {
                    vsc[t - NB] = *reinterpret_cast<const f32x4 *>(v_scales + blk[t - NB] * kBlock + 4 * g);
                    __builtin_amdgcn_sched_barrier(0);
                }
                const uint8_t *vt = v_pool + (blk[t - NB] * num_kv_heads + kvh) * TILE;
                if constexpr (C::kBufLoads) {
                    const auto rv = tile_rsrc(vt, ok[t - NB] ? (int)TILE : 0);
#pragma unroll
                    for (int l = 0; l < C::VL; ++l) vb[t - NB][l] = buf_load<typename C::VRaw>(rv, C::v_off(l, lane));
                } else {
#pragma unroll
                    for (int l = 0; l < C::VL; ++l) vb[t - NB][l] = C::load_v(vt, l, lane);
                }
            }
        };
#pragma unroll
        for (int t = 0; t < PD; ++t) issue(t);
        __builtin_amdgcn_sched_barrier(0);
        // Q operand in the order k_op emits K (zero rows past ROWS), after the
        // first tile loads are out.
#pragma unroll
        for (int i = 0; i < KI; ++i) qb[i] = n < ROWS ? C::q_op(qb[i]) : x8{};
        // Sum of row n's Q operand (as the MFMA sees it): the score bias is
        // kBiasK * qsum.
        float qsum = 0.f;
        // Softmax scale with the codec's score unit folded in (exact: a power of two).
        const float sl2 = scale_log2 * C::kKScale;
        if constexpr (C::kBiasK != 0.f) {
#pragma unroll
            for (int i = 0; i < KI; ++i)
#pragma unroll
                for (int e = 0; e < 8; ++e) qsum += (float)qb[i][e];
            qsum += __shfl_xor(qsum, 16);
            qsum += __shfl_xor(qsum, 32);
        }

        // Scores S^T: s[b][j] = row n, token 4g + j of block b.
        float s[NB][4];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            issue(b + PD);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (!C::kScaled) {
                if (b == bnew) {
#pragma unroll
                    for (int i = 0; i < KI; ++i) kb[b][i] = k_is_new ? knew[i] : kb[b][i];
                }
            }
            // Two accumulators (even / odd steps) halve the dependent MFMA chain.
            f32x4 c = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < KI; i += 2) {
                c = M::qk(C::k_op(kb[b][i / C::SK], i % C::SK), qb[i], c);
                c1 = M::qk(C::k_op(kb[b][(i + 1) / C::SK], (i + 1) % C::SK), qb[i + 1], c1);
            }
            c += c1;
            if constexpr (C::kScaled) {
#pragma unroll
                for (int j = 0; j < 4; ++j) c[j] = fmaf(-C::kBiasK, qsum, c[j]) * ksc[b][j];
            }
            // Every row sees all 16 tokens of this block (all blocks but a
            // sequence's last, for one query): no masking (wave-uniform).
            // Quantized pools only: the f16 kernel is memory-bound and
            // measured 0.3 points slower with the branch.
            const bool full = C::kScaled && __builtin_amdgcn_readfirstlane(
                ok[b] && (lbs[b] + 1) * kBlock <= ctx - NQ + 1);
            if (full) {
#pragma unroll
                for (int j = 0; j < 4; ++j) s[b][j] = c[j] * sl2;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int pos = lbs[b] * kBlock + 4 * g + j;
                    s[b][j] = (ok[b] && pos < limit) ? c[j] * sl2 : -INFINITY;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }

        // Exact per-wave row max: own scores, then the 4 lane groups.
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int j = 0; j < 4; ++j) m = fmaxf(m, s[b][j]);
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        // A row with no valid score (m = -inf) subtracts 0 instead: its
        // scores are all -inf and exponentiate to 0 without a select per score.
        const float msub = m == -INFINITY ? 0.f : m;

        // O += P . V.  Float pools: P rounded to the operand type, and l sums
        // the rounded P.  Quantized pools: the operand is p * v_scale (l sums
        // p), so the widened codes need no per-element scaling.
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            issue(NB + b + PD);
            __builtin_amdgcn_sched_barrier(0);
            // Tokens at or past `valid` are outside the context (stale bytes,
            // maybe NaN) or belong to a masked block (another block's bytes).
            const int valid = __builtin_amdgcn_readfirstlane(ok[b] ? ctx - lbs[b] * kBlock : 0);
            x4 pa;
            // v_exp_f32 directly: s - m <= 0 (or -inf, giving 0), and
            // results below 2^-126 (flushed) do not matter next to the row max's 1.
            float p4[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) p4[j] = __builtin_amdgcn_exp2f(s[b][j] - msub);
            if constexpr (C::kScaled) {
                // Past `valid` p is 0 already; the select keeps a NaN scale
                // out.  int4: blocks wholly inside the context skip it
                // (wave-uniform; the int8 kernel spills with the branch).
                if (C::kCodeBits == 4 && valid >= kBlock) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) pa[j] = (PT)(p4[j] * vsc[b][j]);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) pa[j] = (PT)(4 * g + j < valid ? p4[j] * vsc[b][j] : 0.f);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float p = p4[j];
                if constexpr (C::kScaled) {
                    lsum += p;
                } else {
                    const PT ph = (PT)p;
                    pa[j] = ph;
                    lsum += (float)ph;
                }
            }
            if constexpr (C::kScaled) {
                // Row sums of the operand the MFMA sees, subnormals included,
                // on the matrix pipe: P . ones leaves row 4g + j's sum in
                // column n of accp[j] (v_dot2_f32_f16 flushes subnormal f16
                // and the bias turns any difference into kBias times that
                // much output error).
                const x4 ones = {(PT)1.f, (PT)1.f, (PT)1.f, (PT)1.f};
                accp = M::pv(pa, ones, accp);
            }
            typename M::x4 vo[VN];
#pragma unroll
            for (int k = 0; k < VN; ++k) vo[k] = C::v_op(vb[b][k / C::SV], k % C::SV);
            if constexpr (!C::kScaled) {
                if (b == bnew) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int jv = lb_new * kBlock + 4 * g + e - first_new;
                        if (jv >= 0 && jv < NQ) {
#pragma unroll
                            for (int k = 0; k < VN; ++k) vo[k][e] = vnew[k][e];
                        }
                    }
                }
                // Float V can hold NaN past the context, and 0 * NaN is NaN:
                // zero it.  A wave-uniform branch, taken only by partial blocks.
                if (valid < kBlock) {
#pragma unroll
                    for (int k = 0; k < VN; ++k)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            vo[k][e] = 4 * g + e < valid ? vo[k][e] : (PT)0.f;
                }
            }
#pragma unroll
            for (int k = 0; k < VN; ++k) acc[k] = M::pv(pa, vo[k], acc[k]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    if constexpr (C::kScaled) {
        // Output bias of row 4g + j: kBias * (row's P sum).
        float ob[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) ob[j] = C::kBias * accp[j];
#pragma unroll
        for (int k = 0; k < VN; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[k][j] -= ob[j];
    }

    // acc[k][j] = O[row 4g + j][dim v_dim(k, n)].
#pragma unroll
    for (int k = 0; k < VN; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (4 * g + j < ROWS) o_lds[wave][4 * g + j][C::v_dim(k, n)] = acc[k][j];
    if (g == 0 && n < ROWS) {
        ml_lds[wave][n][0] = m;
        ml_lds[wave][n][1] = lsum;
    }
    __syncthreads();
    merge_waves<ROWS, D, NW, GQA, NQ>(o_lds, ml_lds, out, out_dtype, seq, kvh, part, nparts,
                                      num_q_heads, max_parts, ws_o, ws_ml);
}


// ---------------------------------------------------------------------------
// Packed matrix-core kernel for quantized pools and query groups of at most 8
// rows (GQA group x verify queries).  paged_attn_mfma_kernel gives every
// 16-token block its own 16-column score tile, so with 4 rows 12 of the 16
// columns are padding: their scores, softmax arithmetic and registers are
// spent for nothing.  Here one MFMA tile holds T = 16 / RP blocks (RP = 4 or
// 8 columns a block), block tau of a group of T in columns RP*tau .. +RP-1:
//
//   S^T (16 tokens x (T blocks x RP rows)) = sum over 16-lane groups g of
//       K_{block of g} (16 x 8 dims) . Qdiag (8 dims x 16 columns)
//   Lane group g always feeds the same block tau(g) = g / (4 / T) of the
//   group (all of its token's K row for T = 4, half of it for T = 2); the B
//   operand is Q in the columns of block tau(g) and zero elsewhere (block
//   diagonal).  It is read from LDS: each lane's address is fixed for the
//   launch (its row of Q, or a zero line when its column belongs to another
//   block), so the operand costs one ds_read and no VALU per step.
//   The accumulator leaves lane (column n, group g) with tokens 4g..4g+3 of
//   block n / RP, row n % RP: every lane holds real scores.
//
//   O^T (16 dims x (T x RP)) += V^T (16 dims x 16 tokens) . Pdiag (16 tokens x 16)
//   At step sigma lane group g feeds token quad g ^ (sigma * 4 / T) of its
//   block's V; the matching P values sit in lane group g ^ (sigma * 4 / T) of
//   the same column, fetched by one xor shuffle and zeroed where the column
//   belongs to another block.  The T blocks' partial outputs of a row are
//   summed across columns (DPP row rotations) once per wave.
//
// Same MFMA count per block as the unpacked kernel, 4x (T = 4) fewer scores
// per lane, and no zero query rows in the score arithmetic.
// ---------------------------------------------------------------------------
// v + v rotated by R lanes within each row of 16 (DPP row_ror).
template <int R>
__device__ __forceinline__ float row_ror_add(float v) {
    const int r = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x120 + R, 0xf, 0xf, false);
    return v + __builtin_bit_cast(float, r);
}

template <typename C, int D, int GQA, int NQ, int NW, int NB, int PD>
__global__ __launch_bounds__(NW * 64) DLMK_MFMA_ATTRS void paged_attn_packed_kernel(
    void *__restrict__ out, int out_dtype, const typename C::QT *__restrict__ q,
    const uint8_t *__restrict__ k_pool, const uint8_t *__restrict__ v_pool,
    const float *__restrict__ k_scales, const float *__restrict__ v_scales,
    const int32_t *__restrict__ block_tables, const int32_t *__restrict__ ctx_lens,
    int num_q_heads, int num_kv_heads, int max_blocks, int64_t num_blocks, float scale_log2,
    int max_parts, float *__restrict__ ws_o, float *__restrict__ ws_ml) {
    using M = typename C::Op;
    using x8 = typename M::x8;
    using x4 = typename M::x4;
    using PT = typename M::elem;
    using QT = typename C::QT;
    using KRaw = typename C::KRaw;
    using VRaw = typename C::VRaw;
    constexpr int ROWS = GQA * NQ;
    static_assert(C::kScaled && ROWS <= 8 && D % 64 == 0, "packed kernel: quantized pools, <= 8 rows");
    constexpr int RP = ROWS <= 4 ? 4 : 8;  // columns per block
    constexpr int T = 16 / RP;             // blocks per MFMA tile
    constexpr int G = 4 / T;               // lane groups per block
    constexpr int NG = NB / T;             // block groups per wave
    static_assert(NB % T == 0, "blocks per wave must fill the block groups");
    static_assert(NB <= 32, "block validity is a 32-bit mask");
    constexpr int CH = D / 8 / G;          // 8-dim chunks a lane group feeds per block = QK steps per group
    constexpr int SK = C::KG / 8;          // chunks per K load
    constexpr int NLK = CH / SK;           // K loads per lane per group
    constexpr int NLV = T * C::VL;         // V loads per lane per group
    constexpr int NK = NG * NLK, NV = NG * NLV;
    constexpr int QS = CH;                 // QK steps per group
    constexpr int QP = 3;                  // Q operand reads in flight ahead of the MFMAs
    constexpr int VN = D / 16;
    constexpr int P = NW * NB * kBlock;
    constexpr int64_t TILE = C::kTileBytes;

    // Rows padded by 16 bytes: rows D * 4 bytes apart sit in the same LDS banks,
    // and the epilogue's stores write several rows per instruction.
    __shared__ __attribute__((aligned(16))) float o_lds[NW][ROWS][D + 4];
    __shared__ float ml_lds[NW][ROWS][2];
    // Q rows in operand order, then one zero line.  Rows are padded by 16
    // bytes: at D * 2 bytes apart (a multiple of the 256-byte bank cycle) the
    // rows one read instruction touches would sit in the same banks.
    constexpr int QSTR = D + 8;
    __shared__ __attribute__((aligned(16))) QT q_lds[RP * QSTR + CH * 8];
    __shared__ float qsum_lds[RP];

    const int part = gridDim.y - 1 - blockIdx.y;
    const int kvh = blockIdx.x % num_kv_heads, seq = blockIdx.x / num_kv_heads;
    const int ctx = min(ctx_lens[seq], max_blocks * kBlock);
    const int nparts = parts_of(ctx, P);
    if (part >= nparts) return;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, n = lane & 15;
    const int tcol = n / RP, r = n % RP;   // this lane's score column: block tcol of a group, row r
    const int tg = g / G, gs = g % G;      // block this lane group feeds, and its part of the K row
    const int nblk_seq = (ctx + kBlock - 1) / kBlock;
    const int32_t *table = block_tables + (int64_t)seq * max_blocks;

    // Stage Q (operand order, rows past ROWS zero) and each row's operand sum.
    {
        constexpr int CPR = D / 8;  // chunks per row
        static_assert(RP * CPR <= NW * 64, "one chunk per thread");
        const int idx = threadIdx.x;
        if (idx < RP * CPR) {
            const int rr = idx / CPR, c = idx % CPR;
            x8 v = {};
            if (rr < ROWS) {
                const int j = rr / GQA, h = kvh * GQA + rr % GQA;
                v = C::q_op(reinterpret_cast<const x8 *>(q + ((int64_t)(seq * NQ + j) * num_q_heads + h) * D)[c]);
            }
            *reinterpret_cast<x8 *>(&q_lds[rr * QSTR + 8 * c]) = v;
            float sum = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) sum += (float)v[e];
#pragma unroll
            for (int o = 1; o < CPR; o <<= 1) sum += __shfl_xor(sum, o);
            if (c == 0) qsum_lds[rr] = sum;
        }
        for (int e = threadIdx.x; e < CH; e += NW * 64) *reinterpret_cast<x8 *>(&q_lds[RP * QSTR + 8 * e]) = x8{};
    }

    // Logical block of this wave's b-th block and its validity (wave-uniform
    // bit mask).  Each lane also reads, per block group, the pool ids of the
    // block its lane group loads (tg) and of its score column's block (tcol):
    // a clamped table index, and block 0 for ids outside the pool, so every
    // load is issued unconditionally and stays inside the pool.
    const auto lbof = [&](int b) { return part * (NW * NB) + wave_block(b, NB) * NW + wave; };
    uint32_t okm = 0;
    {
        int32_t bid[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) bid[b] = table[max(min(lbof(b), nblk_seq - 1), 0)];
#pragma unroll
        for (int b = 0; b < NB; ++b)
            okm |= (uint32_t)(lbof(b) < nblk_seq && bid[b] >= 0 && bid[b] < num_blocks) << b;
    }
    const int nvalid = __builtin_popcount(okm);
    int32_t idt[NG], ids[NG];
#pragma unroll
    for (int u = 0; u < NG; ++u) {
        idt[u] = table[max(min(lbof(u * T + tg), nblk_seq - 1), 0)];
        ids[u] = table[max(min(lbof(u * T + tcol), nblk_seq - 1), 0)];
    }
    __syncthreads();

    float m = -INFINITY, lsum = 0.f;
    f32x4 accp = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc[VN];
#pragma unroll
    for (int k = 0; k < VN; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int limit = r < ROWS ? ctx - NQ + r / GQA + 1 : ctx;

    if (nvalid > 0) {
        // This lane's Q operand line: its row's chunks for its part of the K
        // row, or zeros when its column belongs to another block.
        const int qline = (tcol == tg && r < ROWS) ? r * QSTR + gs * CH * 8 : RP * QSTR;
        const float qsum = qsum_lds[r];
        const float sl2 = scale_log2 * C::kKScale;

        const auto inpool = [&](int32_t id) { return id >= 0 && id < num_blocks ? id : 0; };
        KRaw kr[NK];
        VRaw vr[NV];
        f32x4 ksc[NG], vsc[NG];
        int64_t kto[NG], vto[NG];  // this lane group's tile offset in group u
        // Flat load sequence: the groups' K loads, then their V loads; the
        // scales of a group go out before its first code load.
        auto issue = [&](int t) {
            if (t < NK) {
                const int u = t / NLK, x = t % NLK;
                if (x == 0) {
                    ksc[u] = *reinterpret_cast<const f32x4 *>(k_scales + (int64_t)inpool(ids[u]) * kBlock + 4 * g);
                    __builtin_amdgcn_sched_barrier(0);
                    kto[u] = ((int64_t)inpool(idt[u]) * num_kv_heads + kvh) * TILE;
                }
                const KRaw *kt = reinterpret_cast<const KRaw *>(k_pool + kto[u]);
                kr[t] = stream_load(kt + (gs * NLK + x) * kBlock + n);
            } else if (t < NK + NV) {
                const int tv = t - NK;
                const int u = tv / NLV, y = tv % NLV, sg = y / C::VL, l = y % C::VL;
                if (y == 0) {
                    vsc[u] = *reinterpret_cast<const f32x4 *>(v_scales + (int64_t)inpool(ids[u]) * kBlock + 4 * g);
                    __builtin_amdgcn_sched_barrier(0);
                    vto[u] = ((int64_t)inpool(idt[u]) * num_kv_heads + kvh) * TILE;
                }
                const VRaw *vt = reinterpret_cast<const VRaw *>(v_pool + vto[u]);
                vr[tv] = stream_load(vt + 64 * l + 16 * (g ^ (sg * G)) + n);
            }
        };
#pragma unroll
        for (int t = 0; t < PD; ++t) issue(t);
        __builtin_amdgcn_sched_barrier(0);

        // Scores: s[u][j] = row r, token 4g + j of block u*T + tcol.
        float s[NG][4];
#pragma unroll
        for (int u = 0; u < NG; ++u) {
            f32x4 c = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
            // The Q operand is re-read from LDS for every group: an opaque
            // copy of the line offset keeps the compiler from holding all
            // QS operands in registers across groups.
            int ql = qline;
            asm volatile("" : "+v"(ql));
            // Operand reads run QP steps ahead of their MFMA (LDS latency).
            x8 bq[QS];
#pragma unroll
            for (int i = 0; i < QP && i < QS; ++i) bq[i] = *reinterpret_cast<const x8 *>(&q_lds[ql + 8 * i]);
#pragma unroll
            for (int x = 0; x < NLK; ++x) {
                issue(u * NLK + x + PD);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int e = 0; e < SK; ++e) {
                    const int i = x * SK + e;
                    if (i + QP < QS) bq[i + QP] = *reinterpret_cast<const x8 *>(&q_lds[ql + 8 * (i + QP)]);
                    if (i & 1)
                        c1 = M::qk(C::k_op(kr[u * NLK + x], e), bq[i], c1);
                    else
                        c = M::qk(C::k_op(kr[u * NLK + x], e), bq[i], c);
                }
            }
            c += c1;
#pragma unroll
            for (int j = 0; j < 4; ++j) c[j] = fmaf(-C::kBiasK, qsum, c[j]) * ksc[u][j];
            bool full = true;
#pragma unroll
            for (int tau = 0; tau < T; ++tau)
                full = full && ((okm >> (u * T + tau)) & 1) && (lbof(u * T + tau) + 1) * kBlock <= ctx - NQ + 1;
            if (full) {
#pragma unroll
                for (int j = 0; j < 4; ++j) s[u][j] = c[j] * sl2;
            } else {
                const int lb = part * (NW * NB) + wave_block(u * T + tcol, NB) * NW + wave;
                const bool okc = (okm >> (u * T + tcol)) & 1;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int pos = lb * kBlock + 4 * g + j;
                    s[u][j] = (okc && pos < limit) ? c[j] * sl2 : -INFINITY;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }

        // Row max over every block group and lane of the row (columns
        // RP*t + r for all t, all lane groups).
#pragma unroll
        for (int u = 0; u < NG; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) m = fmaxf(m, s[u][j]);
#pragma unroll
        for (int o = RP; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
        const float msub = m == -INFINITY ? 0.f : m;

        const x4 ones = {(PT)1.f, (PT)1.f, (PT)1.f, (PT)1.f};
#pragma unroll
        for (int u = 0; u < NG; ++u) {
            float p4[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) p4[j] = __builtin_amdgcn_exp2f(s[u][j] - msub);
            bool full = true;
#pragma unroll
            for (int tau = 0; tau < T; ++tau)
                full = full && ((okm >> (u * T + tau)) & 1) && (lbof(u * T + tau) + 1) * kBlock <= ctx;
            x4 pa;
            if (full) {
#pragma unroll
                for (int j = 0; j < 4; ++j) pa[j] = (PT)(p4[j] * vsc[u][j]);
            } else {
                // Past `valid` p is 0 already; the select keeps a NaN scale out.
                const int lb = part * (NW * NB) + wave_block(u * T + tcol, NB) * NW + wave;
                const int valid = ((okm >> (u * T + tcol)) & 1) ? ctx - lb * kBlock : 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) pa[j] = (PT)(4 * g + j < valid ? p4[j] * vsc[u][j] : 0.f);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) lsum += p4[j];
            const u32x2 pw = __builtin_bit_cast(u32x2, pa);
#pragma unroll
            for (int sg = 0; sg < T; ++sg) {
#pragma unroll
                for (int l = 0; l < C::VL; ++l) {
                    issue(NK + u * NLV + sg * C::VL + l + PD);
                    __builtin_amdgcn_sched_barrier(0);
                }
                // P of this step: token quad g ^ (sg * G) of column block tcol,
                // held by lane group g ^ (sg * G); zero outside block tg's columns.
                u32x2 w = pw;
                if (sg != 0) {
                    w[0] = __shfl_xor(pw[0], 16 * sg * G);
                    w[1] = __shfl_xor(pw[1], 16 * sg * G);
                }
                const x4 bp = tcol == tg ? __builtin_bit_cast(x4, w) : x4{};
                accp = M::pv(ones, bp, accp);
#pragma unroll
                for (int k = 0; k < VN; ++k) {
                    const x4 vo = C::v_op(vr[u * NLV + sg * C::VL + k / C::SV], k % C::SV);
                    acc[k] = M::pv(vo, bp, acc[k]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
#pragma unroll
    for (int o = RP; o < 64; o <<= 1) lsum += __shfl_xor(lsum, o);
    // Output bias of column n: kBias * (its P operand sum); then the T blocks'
    // partials of row r (columns r, RP + r, ...) are summed.
#pragma unroll
    for (int k = 0; k < VN; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float v = acc[k][j] - C::kBias * accp[j];
            if constexpr (T == 4) v = row_ror_add<8>(row_ror_add<4>(v));
            else v = row_ror_add<8>(v);
            acc[k][j] = v;
        }

    // acc[k][j] (columns n < RP) = O[row n][dim v_dim(k, 4g + j)].
    if (n < ROWS) {
#pragma unroll
        for (int k = 0; k < VN; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j) o_lds[wave][n][C::v_dim(k, 4 * g + j)] = acc[k][j];
        if (g == 0) {
            ml_lds[wave][n][0] = m;
            ml_lds[wave][n][1] = lsum;
        }
    }
    __syncthreads();
    merge_waves<ROWS, D, NW, GQA, NQ>(o_lds, ml_lds, out, out_dtype, seq, kvh, part, nparts,
                                      num_q_heads, max_parts, ws_o, ws_ml);
}

// ---------------------------------------------------------------------------
// Generic matrix-core partition kernel: any head dim hd <= DP (a multiple of
// the pool's 16-byte chunk), any GQA group and query count (row groups of 16
// query rows), f32 / f16 / bf16 pools.  The same tiling as
// paged_attn_mfma_kernel with the geometry at run time: lanes of chunk rows
// or dims past hd load an in-tile address (chunk row / dim 0) and meet zero Q
// (scores) or are never stored (outputs), so any hd works without padding the
// pools.  f32 pools use v_mfma_f32_16x16x4_f32: one 16-byte K chunk of a lane
// is 4 steps of 4 dims, one 16-byte V load 4 tokens of one dim (4 steps).
// ---------------------------------------------------------------------------
template <typename T>
struct GenOp;

template <>
struct GenOp<float> {
    using KRaw = f32x4;  // 4 dims of one token (K) / 4 tokens of one dim (V)
    using VRaw = f32x4;
    using P4 = f32x4;    // P operand: 4 tokens of one row, kept in f32
    static constexpr int X = 4;  // elements per 16-byte chunk
    static __device__ __forceinline__ void qk(KRaw k, KRaw q, f32x4 &c0, f32x4 &c1) {
        c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(k[0], q[0], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(k[1], q[1], c1, 0, 0, 0);
        c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(k[2], q[2], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(k[3], q[3], c1, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 pv(P4 p, VRaw v, f32x4 c) {
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(p[0], v[0], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(p[1], v[1], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(p[2], v[2], c, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_16x16x4f32(p[3], v[3], c, 0, 0, 0);
    }
    static __device__ __forceinline__ float round_p(float p) { return p; }
};

template <typename E>
struct GenOpHalf {  // f16 / bf16: one 16-byte chunk is one 16x16x32 step
    using M = Mfma<E>;
    using KRaw = typename M::x8;
    using VRaw = typename M::x4;
    using P4 = typename M::x4;
    static constexpr int X = 8;
    static __device__ __forceinline__ void qk(KRaw k, KRaw q, f32x4 &c0, f32x4 &) {
        c0 = M::qk(k, q, c0);
    }
    static __device__ __forceinline__ f32x4 pv(P4 p, VRaw v, f32x4 c) { return M::pv(p, v, c); }
    static __device__ __forceinline__ E round_p(float p) { return (E)p; }
};
template <>
struct GenOp<_Float16> : GenOpHalf<_Float16> {};
template <>
struct GenOp<__bf16> : GenOpHalf<__bf16> {};

// Runtime geometry of the generic kernel.
struct GenGeom {
    int hd;        // head dim (<= DP)
    int gqa, nq;   // query heads per kv head, queries per sequence
    int n_rg;      // row groups of 16 rows per (sequence, kv head)
};

template <typename T, int DP, int NW, int NB, int PD, bool FUSED>
__global__ __launch_bounds__(NW * 64) void paged_attn_generic_kernel(
    void *__restrict__ out, int out_dtype, const T *__restrict__ q, T *__restrict__ k_pool,
    T *__restrict__ v_pool, const T *__restrict__ k_new, const T *__restrict__ v_new,
    const int32_t *__restrict__ block_tables, const int32_t *__restrict__ ctx_lens, GenGeom geo,
    int num_q_heads, int num_kv_heads, int max_blocks, int64_t num_blocks, float scale_log2,
    int max_parts, float *__restrict__ ws_o, float *__restrict__ ws_ml) {
    using G = GenOp<T>;
    using KRaw = typename G::KRaw;
    using VRaw = typename G::VRaw;
    constexpr int X = G::X;
    constexpr int KL = DP / X / 4;   // 16-byte K (and Q) loads per lane per block
    constexpr int VN = DP / 16;      // 16-dim PV steps (one V load each) per block
    constexpr int P = NW * NB * kBlock;
    static_assert(DP % (4 * X) == 0 && DP % 16 == 0, "unsupported padded head dim");
    static_assert(NW >= 2, "new-token blocks must land on different waves");

    // Rows padded by 16 bytes: the epilogue stores 4 rows per instruction.
    __shared__ __attribute__((aligned(16))) float o_lds[NW][16][DP + 4];
    __shared__ float ml_lds[NW][16][2];

    const int hd = geo.hd, gqa = geo.gqa, nq = geo.nq;
    const int64_t tile = (int64_t)hd * kBlock;  // elements per (block, kv head) tile
    const int rg = blockIdx.x % geo.n_rg;
    const int kvh = (blockIdx.x / geo.n_rg) % num_kv_heads;
    const int seq = blockIdx.x / geo.n_rg / num_kv_heads;

    if (FUSED && blockIdx.y == 0) {
        // Fused decode step: the first grid row stores the new tokens, one
        // work-group per sequence (row group 0 of kv head 0) over all kv
        // heads, as paged_attn_mfma_kernel; the partition work-groups
        // substitute them from k_new / v_new.
        if (rg == 0 && kvh == 0) {
            const int ctx = min(ctx_lens[seq], max_blocks * kBlock);
            for (int e = threadIdx.x; e < num_kv_heads * nq * hd; e += NW * 64) {
                const int dim = e % hd, j = (e / hd) % nq, h = e / (hd * nq), p = ctx - nq + j;
                if (p < 0) continue;
                const int64_t blk = block_tables[(int64_t)seq * max_blocks + p / kBlock];
                if (blk < 0 || blk >= num_blocks) continue;
                const int t = p % kBlock;
                const int64_t base = (blk * num_kv_heads + h) * tile;
                const int64_t src = ((int64_t)(seq * nq + j) * num_kv_heads + h) * hd + dim;
                pool_store(&k_pool[base + (dim / X * kBlock + t) * X + dim % X], k_new[src]);
                pool_store(&v_pool[base + dim * kBlock + t], v_new[src]);
            }
        }
        return;
    }
    // Partitions last index first (as paged_attn_mfma_kernel); with the
    // append row at blockIdx.y 0 this still maps rows 1.. onto max_parts - 1 .. 0.
    const int part = gridDim.y - 1 - blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, n = lane & 15;
    const int32_t *table = block_tables + (int64_t)seq * max_blocks;
    const int rows = gqa * nq;
    const int rows_here = min(16, rows - rg * 16);

    // Context length, table entries (clamped to the row, not to the context)
    // and the query go out together: no load waits on another before the
    // first tile (config 1: 6.94 -> 6.70 us; the same change measured no
    // difference in paged_attn_mfma_kernel's large grids, whose start-up
    // overlaps other work-groups' streams).
    int32_t raw[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int lb = part * (NW * NB) + wave_block(b, NB) * NW + wave;
        raw[b] = table[min(lb, max_blocks - 1)];
    }
    // Row n of this group: query j, head h.  Lanes past the group's rows load
    // a valid row and are zeroed below.
    const int r = rg * 16 + min(n, rows_here - 1);
    const int qj = r / gqa, qh = kvh * gqa + r % gqa;
    // This lane's chunk rows 4l + g (clamped into the tile past hd / X).
    const int nchunk = hd / X;
    int crow[KL];
#pragma unroll
    for (int l = 0; l < KL; ++l) crow[l] = 4 * l + g < nchunk ? 4 * l + g : 0;
    KRaw qb[KL];
    {
        const KRaw *qp = reinterpret_cast<const KRaw *>(q + ((int64_t)(seq * nq + qj) * num_q_heads + qh) * hd);
#pragma unroll
        for (int l = 0; l < KL; ++l) qb[l] = qp[crow[l]];
    }
    const int len = ctx_lens[seq];
#pragma unroll
    for (int b = 0; b < NB; ++b) asm volatile("" ::"s"(raw[b]), "s"(len));
    const int ctx = min(len, max_blocks * kBlock);
    const int nparts = parts_of(ctx, P);
    if (part >= nparts) return;
    const int nblk_seq = (ctx + kBlock - 1) / kBlock;
    const int limit = ctx - nq + qj + 1;

    int lbs[NB];
    int64_t blk[NB];
    bool ok[NB];
    int nvalid = 0;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int lb = part * (NW * NB) + wave_block(b, NB) * NW + wave;
        const int64_t id = lb < nblk_seq ? (int64_t)raw[b] : -1;
        lbs[b] = lb;
        ok[b] = id >= 0 && id < num_blocks;
        blk[b] = id;
        nvalid += ok[b];
    }

    float m = -INFINITY, lsum = 0.f;
    f32x4 acc[VN];
#pragma unroll
    for (int k = 0; k < VN; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Fused step: this wave's block holding new tokens, if any (see
    // paged_attn_mfma_kernel), and the new tokens' chunks in registers.
    int bnew = -1;
    if constexpr (FUSED) {
#pragma unroll
        for (int b = 0; b < NB; ++b)
            if (ok[b] && holds_new(lbs[b], ctx, nq)) bnew = b;
    }
    bnew = __builtin_amdgcn_readfirstlane(bnew);
    const int lb_new = part * (NW * NB) + wave_block(max(bnew, 0), NB) * NW + wave;
    const int first_new = ctx - nq;
    const int jk = lb_new * kBlock + n - first_new;
    const bool k_is_new = jk >= 0 && jk < nq;
    KRaw knew[KL];
    VRaw vnew[VN];
    int vdim[VN];
#pragma unroll
    for (int k = 0; k < VN; ++k) vdim[k] = 16 * k + n < hd ? 16 * k + n : 0;
    if (FUSED && bnew >= 0) {
        const KRaw *kr = reinterpret_cast<const KRaw *>(
            k_new + ((int64_t)(seq * nq + min(max(jk, 0), nq - 1)) * num_kv_heads + kvh) * hd);
#pragma unroll
        for (int l = 0; l < KL; ++l) knew[l] = kr[crow[l]];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int jv = min(max(lb_new * kBlock + 4 * g + e - first_new, 0), nq - 1);
            const T *vr = v_new + ((int64_t)(seq * nq + jv) * num_kv_heads + kvh) * hd;
#pragma unroll
            for (int k = 0; k < VN; ++k) vnew[k][e] = vr[vdim[k]];
        }
    }

    if (nvalid > 0) {
        int64_t first = 0;
#pragma unroll
        for (int b = NB - 1; b >= 0; --b)
            if (ok[b]) first = blk[b];
#pragma unroll
        for (int b = 0; b < NB; ++b)
            if (!ok[b]) blk[b] = first;

        KRaw kb[NB][KL];
        VRaw vb[NB][VN];
        auto issue = [&](int t) {
            if (t < NB) {
                const KRaw *kt = reinterpret_cast<const KRaw *>(k_pool + (blk[t] * num_kv_heads + kvh) * tile);
#pragma unroll
                for (int l = 0; l < KL; ++l) kb[t][l] = stream_load(kt + crow[l] * kBlock + n);
            } else if (t < 2 * NB) {
                const VRaw *vt = reinterpret_cast<const VRaw *>(v_pool + (blk[t - NB] * num_kv_heads + kvh) * tile);
#pragma unroll
                for (int k = 0; k < VN; ++k) vb[t - NB][k] = stream_load(vt + vdim[k] * 4 + g);
            }
        };
#pragma unroll
        for (int t = 0; t < PD; ++t) issue(t);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int l = 0; l < KL; ++l) qb[l] = n < rows_here && 4 * l + g < nchunk ? qb[l] : KRaw{};

        float s[NB][4];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            issue(b + PD);
            __builtin_amdgcn_sched_barrier(0);
            if (FUSED && b == bnew) {
#pragma unroll
                for (int l = 0; l < KL; ++l) kb[b][l] = k_is_new ? knew[l] : kb[b][l];
            }
            f32x4 c = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int l = 0; l < KL; ++l) {
                if (l & 1)
                    G::qk(kb[b][l], qb[l], c1, c);
                else
                    G::qk(kb[b][l], qb[l], c, c1);
            }
            c += c1;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int pos = lbs[b] * kBlock + 4 * g + j;
                s[b][j] = (ok[b] && pos < limit) ? c[j] * scale_log2 : -INFINITY;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int j = 0; j < 4; ++j) m = fmaxf(m, s[b][j]);
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));

#pragma unroll
        for (int b = 0; b < NB; ++b) {
            issue(NB + b + PD);
            __builtin_amdgcn_sched_barrier(0);
            const int valid = __builtin_amdgcn_readfirstlane(ok[b] ? ctx - lbs[b] * kBlock : 0);
            typename G::P4 pa;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float p = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s[b][j] - m);
                pa[j] = G::round_p(p);
                lsum += (float)pa[j];
            }
            VRaw vo[VN];
#pragma unroll
            for (int k = 0; k < VN; ++k) vo[k] = vb[b][k];
            if (FUSED && b == bnew) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int jv = lb_new * kBlock + 4 * g + e - first_new;
                    if (jv >= 0 && jv < nq) {
#pragma unroll
                        for (int k = 0; k < VN; ++k) vo[k][e] = vnew[k][e];
                    }
                }
            }
            // V past the context can hold NaN, and 0 * NaN is NaN: zero it.
            if (valid < kBlock) {
#pragma unroll
                for (int k = 0; k < VN; ++k)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        vo[k][e] = 4 * g + e < valid ? vo[k][e] : (T)0.f;
            }
#pragma unroll
            for (int k = 0; k < VN; ++k) acc[k] = G::pv(pa, vo[k], acc[k]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);

    // acc[k][j] = O[row 4g + j][dim 16k + n].
#pragma unroll
    for (int k = 0; k < VN; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) o_lds[wave][4 * g + j][16 * k + n] = acc[k][j];
    if (g == 0) {
        ml_lds[wave][n][0] = m;
        ml_lds[wave][n][1] = lsum;
    }
    __syncthreads();

    // Merge the waves (as merge_waves, with the geometry at run time).
    __shared__ float fac[16][NW];
    __shared__ float rowML[16][2];
    if (threadIdx.x < 16) {
        const int rr = threadIdx.x;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, ml_lds[w][rr][0]);
        float L = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float mw = ml_lds[w][rr][0];
            const float f = (M == -INFINITY || mw == -INFINITY) ? 0.f : exp2f(mw - M);
            fac[rr][w] = f;
            L = fmaf(f, ml_lds[w][rr][1], L);
        }
        rowML[rr][0] = M;
        rowML[rr][1] = L;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < rows_here * hd; idx += NW * 64) {
        const int rr = idx / hd, d = idx - rr * hd;
        float O = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) O = fmaf(fac[rr][w], o_lds[w][rr][d], O);
        const float L = rowML[rr][1];
        const int gr = rg * 16 + rr, j = gr / gqa, h = kvh * gqa + gr % gqa;
        const int64_t row = (int64_t)(seq * nq + j) * num_q_heads + h;
        if (nparts == 1) {
            store_out(out, out_dtype, row * hd + d, L > 0.f ? O / L : 0.f);
        } else {
            const int64_t slot = row * max_parts + part;
            ws_o[slot * hd + d] = O;
            if (d == 0) {
                ws_ml[2 * slot] = rowML[rr][0];
                ws_ml[2 * slot + 1] = L;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Pass 2: log-sum-exp merge of a sequence's partitions.  Rows of up to
// kCombineBatch partitions: one wave per (query row, sequence), kCombineWaves
// rows per work-group.
// ---------------------------------------------------------------------------
constexpr int kCombineWaves = 4;
constexpr int kCombineBatch = 8;

// DPL dims per lane: head dim D <= 64 * DPL (dims past D are read clamped and
// never stored).
// Fused decode step over f16 / bf16 pools: the new tokens' K and V are
// stored into the pools by the combine launch, which runs after every
// partition work-group has read them from k_new / v_new in registers and
// has memory bandwidth to spare.  16-bit elements are copied as bits.
struct NewTokens {
    uint16_t *k_pool, *v_pool;
    const uint16_t *k_new, *v_new;  // null: nothing to store
    const int32_t *tables;
    int max_blocks, num_kv_heads, gqa, nq;
    int64_t num_blocks;
};

// Wave-wide store of query token j's K and V for kv head kvh of sequence seq
// (position ctx - nq + j; K [blk][Hkv][d/8][16][8], V [blk][Hkv][d][16]; a
// block id outside the pool is skipped), the bits dlmk_kv_append writes.
__device__ __forceinline__ void store_new_token(const NewTokens &nt, int seq, int j, int kvh, int ctx,
                                                int D, int lane) {
    const int p = ctx - nt.nq + j;
    if (p < 0) return;
    const int64_t blk = nt.tables[(int64_t)seq * nt.max_blocks + p / kBlock];
    if (blk < 0 || blk >= nt.num_blocks) return;
    const int t = p % kBlock;
    const int64_t base = (blk * nt.num_kv_heads + kvh) * (int64_t)D * kBlock;
    const int64_t src = ((int64_t)(seq * nt.nq + j) * nt.num_kv_heads + kvh) * D;
    typedef uint32_t w4t __attribute__((ext_vector_type(4)));
    for (int c = lane; c < D / 8; c += 64)
        pool_store(reinterpret_cast<w4t *>(&nt.k_pool[base + (c * kBlock + t) * 8]),
                   *reinterpret_cast<const w4t *>(&nt.k_new[src + 8 * c]));
    for (int e = lane; e < D; e += 64) pool_store(&nt.v_pool[base + e * kBlock + t], nt.v_new[src + e]);
}

template <int DPL>
__global__ __launch_bounds__(64 * kCombineWaves) void paged_attn_combine_wave_kernel(
    void *__restrict__ out, int out_dtype, const float *__restrict__ ws_o,
    const float *__restrict__ ws_ml, const int32_t *__restrict__ ctx_lens, int rows_per_seq,
    int max_blocks, int partition, int max_parts, int D, NewTokens nt) {
    constexpr int B = kCombineBatch;  // partitions loaded per batch
    // One wave per (sequence, query row), kCombineWaves rows per work-group:
    // the wave folds all of the row's partitions itself (online rescale), so
    // no cross-wave merge and a quarter of the work-groups of one per row.
    const int seq = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * kCombineWaves + (threadIdx.x >> 6);
    if (r >= rows_per_seq) return;
    const int64_t row = (int64_t)seq * rows_per_seq + r;
    const float *ml = ws_ml + 2 * row * max_parts;
    const float *o = ws_o + row * max_parts * D;

    float mb[B], lb[B], ob[B][DPL];
    auto load = [&](int p0, int last) {
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const int p = min(p0 + i, last);
            mb[i] = ml[2 * p];
            lb[i] = ml[2 * p + 1];
#pragma unroll
            for (int k = 0; k < DPL; ++k) ob[i][k] = o[(int64_t)p * D + min(lane + 64 * k, D - 1)];
        }
    };
    // The first batch is read before the context length is known (every
    // slot below max_parts exists; only those below nparts are used), so
    // rows of up to B partitions cost one memory round trip.
    load(0, max_parts - 1);
    const int ctx = min(ctx_lens[seq], max_blocks * kBlock);
    const int nparts = parts_of(ctx, partition);
    if (nt.k_new != nullptr) {
        // Row r = j * Hq + h: the first row of each kv head's group stores
        // that head's token j.
        const int hq = nt.num_kv_heads * nt.gqa, h = r % hq;
        if (h % nt.gqa == 0) store_new_token(nt, seq, r / hq, h / nt.gqa, ctx, D, lane);
    }
    if (nparts == 1) return;

    float m = -INFINITY, L = 0.f, O[DPL];
#pragma unroll
    for (int k = 0; k < DPL; ++k) O[k] = 0.f;
    for (int p0 = 0;;) {
#pragma unroll
        for (int i = 0; i < B; ++i) {
            if (p0 + i >= nparts) break;
            const float mn = fmaxf(m, mb[i]);
            if (mn == -INFINITY) continue;  // both empty
            const float fa = m == -INFINITY ? 0.f : exp2f(m - mn);
            const float fb = mb[i] == -INFINITY ? 0.f : exp2f(mb[i] - mn);
            L = fa * L + fb * lb[i];
#pragma unroll
            for (int k = 0; k < DPL; ++k) O[k] = fa * O[k] + fb * ob[i][k];
            m = mn;
        }
        p0 += B;
        if (p0 >= nparts) break;
        load(p0, nparts - 1);
    }
#pragma unroll
    for (int k = 0; k < DPL; ++k)
        if (lane + 64 * k < D) store_out(out, out_dtype, row * D + lane + 64 * k, L > 0.f ? O[k] / L : 0.f);
}

// Rows of more than kCombineBatch partitions: one work-group of
// kCombineWaves waves per (query row, sequence).  Wave w folds partitions
// w, w + W, ... in batches of 8 with an online rescale (its first batch loaded
// before the context length arrives), and the waves merge once in LDS.
template <int DPL>
__global__ __launch_bounds__(64 * kCombineWaves) void paged_attn_combine_wg_kernel(
    void *__restrict__ out, int out_dtype, const float *__restrict__ ws_o,
    const float *__restrict__ ws_ml, const int32_t *__restrict__ ctx_lens, int rows_per_seq,
    int max_blocks, int partition, int max_parts, int D, NewTokens nt) {
    constexpr int W = kCombineWaves;
    __shared__ float wml[W][2];
    __shared__ float so[W][64 * DPL + 1];
    const int seq = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row = (int64_t)seq * rows_per_seq + blockIdx.x;
    const float *ml = ws_ml + 2 * row * max_parts;
    const float *o = ws_o + row * max_parts * D;

    // Wave w's first batch -- partitions w, w + W, ..., w + (B - 1) W,
    // clamped into the row -- is loaded before the context length is known
    // (every slot below max_parts exists; only those below nparts are
    // folded), so rows of up to B x W partitions cost one memory round trip.
    // Later partitions fold in further batches with an online rescale; the W
    // waves then merge once.
    constexpr int B = 8;
    float m = -INFINITY, L = 0.f, O[DPL];
#pragma unroll
    for (int k = 0; k < DPL; ++k) O[k] = 0.f;
    float mb[B], lb[B], ob[B][DPL];
    auto load = [&](int p0, int last) {
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const int p = min(p0 + i * W, last);
            mb[i] = ml[2 * p];
            lb[i] = ml[2 * p + 1];
#pragma unroll
            for (int k = 0; k < DPL; ++k) ob[i][k] = o[(int64_t)p * D + min(lane + 64 * k, D - 1)];
        }
    };
    load(wave, max_parts - 1);
    const int ctx = min(ctx_lens[seq], max_blocks * kBlock);
    const int nparts = parts_of(ctx, partition);
    if (nt.k_new != nullptr && wave == 0) {
        const int r = blockIdx.x, hq = nt.num_kv_heads * nt.gqa, h = r % hq;
        if (h % nt.gqa == 0) store_new_token(nt, seq, r / hq, h / nt.gqa, ctx, D, lane);
    }
    if (nparts == 1) return;
    for (int p0 = wave;;) {
#pragma unroll
        for (int i = 0; i < B; ++i) {
            if (p0 + i * W >= nparts) break;
            const float mn = fmaxf(m, mb[i]);
            if (mn == -INFINITY) continue;  // both empty
            const float fa = m == -INFINITY ? 0.f : exp2f(m - mn);
            const float fb = mb[i] == -INFINITY ? 0.f : exp2f(mb[i] - mn);
            L = fa * L + fb * lb[i];
#pragma unroll
            for (int k = 0; k < DPL; ++k) O[k] = fa * O[k] + fb * ob[i][k];
            m = mn;
        }
        p0 += B * W;
        if (p0 >= nparts) break;
        load(p0, nparts - 1);
    }
#pragma unroll
    for (int k = 0; k < DPL; ++k) so[wave][lane + 64 * k] = O[k];
    if (lane == 0) {
        wml[wave][0] = m;
        wml[wave][1] = L;
    }
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) M = fmaxf(M, wml[w][0]);
    float fw[W], Lt = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
        fw[w] = (M == -INFINITY || wml[w][0] == -INFINITY) ? 0.f : exp2f(wml[w][0] - M);
        Lt = fmaf(fw[w], wml[w][1], Lt);
    }
    for (int d = threadIdx.x; d < D; d += 64 * W) {
        float Ot = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) Ot = fmaf(fw[w], so[w][d], Ot);
        store_out(out, out_dtype, row * D + d, Lt > 0.f ? Ot / Lt : 0.f);
    }
}

// ---------------------------------------------------------------------------
// Host dispatch.
// ---------------------------------------------------------------------------

inline int64_t parts_for(int max_blocks, int partition) {
    int64_t tokens = (int64_t)max_blocks * kBlock;
    return tokens > partition ? dlmk::ceil_div(tokens, partition) : 1;
}

// Combine launch for DPL dims per lane (head dim <= 64 * DPL).
template <int DPL>
void launch_combine(const Args &a, int partition, int max_parts, float *ws_o, float *ws_ml,
                    const NewTokens &nt) {
    // Rows of up to kCombineBatch partitions: a wave per row (config 5
    // 64.9 -> 66.2%); longer rows: a work-group per row, whose four waves
    // share the row's partitions (the wave-per-row kernel was 0.8 points
    // slower at config 4's 32 partitions and 2.9 us slower in the decode
    // block's 32).
    if (max_parts > kCombineBatch)
        hipLaunchKernelGGL(paged_attn_combine_wg_kernel<DPL>, dim3((unsigned)(a.NQ * a.Hq), (unsigned)a.B),
                           dim3(64 * kCombineWaves), 0, a.stream, a.out, a.out_dtype, ws_o, ws_ml, a.ctx_lens,
                           a.NQ * a.Hq, a.max_blocks, partition, max_parts, a.D, nt);
    else
        hipLaunchKernelGGL(paged_attn_combine_wave_kernel<DPL>,
                           dim3((unsigned)((a.NQ * a.Hq + kCombineWaves - 1) / kCombineWaves), (unsigned)a.B),
                           dim3(64 * kCombineWaves), 0, a.stream, a.out, a.out_dtype, ws_o, ws_ml, a.ctx_lens,
                           a.NQ * a.Hq, a.max_blocks, partition, max_parts, a.D, nt);
}

// Launches the partition kernel through `launch(grid, max_parts, ws_o, ws_ml)`
// over grid_x x max_parts work-groups, then the combine kernel when a
// sequence can span several partitions.
// combine_appends: a fused decode step whose partition launch has no append
// row when it is followed by a combine launch; the combine stores the new
// tokens instead.
template <typename Launch>
int launch_pair(const Args &a, int partition, int64_t grid_x, Launch launch, bool combine_appends = false) {
    const int max_parts = (int)parts_for(a.max_blocks, partition);
    float *ws_o = nullptr, *ws_ml = nullptr;
    if (grid_x > 0x7fffffff)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED, "paged attention: grid too large");
    if (max_parts > 1) {
        // Workspace layout for this partition size: O partials
        // [rows][max_parts][D] f32, then (m, l) pairs [rows][max_parts][2].
        const int64_t rows = (int64_t)a.B * a.NQ * a.Hq;
        const int64_t o_bytes = (rows * max_parts * a.D * 4 + 255) / 256 * 256;
        const int64_t need = o_bytes + rows * max_parts * 2 * 4;
        if (!a.workspace || (int64_t)a.ws_bytes < need)
            return dlmk::fail(DLMK_ERR_WORKSPACE,
                              "paged attention: split-K partials need %lld bytes, the workspace "
                              "holds %zu", (long long)need, a.ws_bytes);
        ws_o = static_cast<float *>(a.workspace);
        ws_ml = reinterpret_cast<float *>(static_cast<char *>(a.workspace) + o_bytes);
    }
    launch(dim3((unsigned)grid_x, (unsigned)max_parts), max_parts, ws_o, ws_ml);
    if (max_parts > 1) {
        NewTokens nt{};
        if (combine_appends && a.k_new != nullptr)
            nt = NewTokens{static_cast<uint16_t *>(a.k_pool), static_cast<uint16_t *>(a.v_pool),
                           static_cast<const uint16_t *>(a.k_new), static_cast<const uint16_t *>(a.v_new),
                           a.tables, a.max_blocks, a.Hkv, a.Hq / a.Hkv, a.NQ, a.num_blocks};
        switch ((a.D + 63) / 64) {
            case 1: launch_combine<1>(a, partition, max_parts, ws_o, ws_ml, nt); break;
            case 2: launch_combine<2>(a, partition, max_parts, ws_o, ws_ml, nt); break;
            case 3: launch_combine<3>(a, partition, max_parts, ws_o, ws_ml, nt); break;
            default: launch_combine<4>(a, partition, max_parts, ws_o, ws_ml, nt); break;
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return dlmk::fail((int)e, "paged attention launch: %s", hipGetErrorString(e));
    return DLMK_OK;
}

// Matrix-core path: NW waves x NB blocks per partition, pool format C.
template <typename C, int D, int GQA, int NQ, int NB>
int launch_mfma_nb(const Args &a) {
    constexpr int NW = DLMK_MFMA_NW;
    constexpr int PD = C::kScaled ? DLMK_MFMA_PDQ : DLMK_MFMA_PD;
    static_assert(NW * NB * kBlock >= kMinPartition, "partition below the workspace bound");
    using QT = typename C::QT;
    return launch_pair(a, NW * NB * kBlock, (int64_t)a.B * a.Hkv,
                       [&](dim3 grid, int max_parts, float *ws_o, float *ws_ml) {
        constexpr int kPackBit = C::kCodeBits == 4 ? 1 : GQA * NQ <= 4 ? 2 : 4;
        const bool pack_rows = C::kCodeBits == 4 || max_parts <= DLMK_PACKED_I8_MAXPARTS;
        if constexpr (C::kScaled && GQA * NQ <= 8 && (DLMK_MFMA_PACKED & kPackBit)) if (pack_rows) {
            constexpr int PDP = GQA * NQ <= 4 ? DLMK_MFMA_PDP4 : DLMK_MFMA_PDP2;
            hipLaunchKernelGGL((paged_attn_packed_kernel<C, D, GQA, NQ, NW, NB, PDP>), grid, dim3(NW * 64), 0,
                               a.stream, a.out, a.out_dtype, static_cast<const QT *>(a.q),
                               static_cast<const uint8_t *>(a.k_pool), static_cast<const uint8_t *>(a.v_pool),
                               a.k_scales, a.v_scales, a.tables, a.ctx_lens, a.Hq, a.Hkv, a.max_blocks,
                               a.num_blocks, a.scale * kLog2e, max_parts, ws_o, ws_ml);
            return;
        }
        // Fused decode step: the new tokens are stored by the combine launch
        // when there is one, else by one more grid row of append work-groups.
        const int append_row = !C::kScaled && a.k_new != nullptr && max_parts == 1;
        if (append_row) grid.y += 1;
        hipLaunchKernelGGL((paged_attn_mfma_kernel<C, D, GQA, NQ, NW, NB, PD>), grid, dim3(NW * 64), 0,
                           a.stream, a.out, a.out_dtype, static_cast<const QT *>(a.q),
                           static_cast<uint8_t *>(a.k_pool), static_cast<uint8_t *>(a.v_pool),
                           a.k_scales, a.v_scales, static_cast<const QT *>(a.k_new),
                           static_cast<const QT *>(a.v_new), a.tables, a.ctx_lens, a.Hq, a.Hkv,
                           a.max_blocks, a.num_blocks, a.scale * kLog2e, max_parts, ws_o, ws_ml, append_row);
    }, !C::kScaled && a.k_new != nullptr);
}

// Partition shape per launch.  f16 / bf16 and int8 pools: 16 blocks per wave
// (1024-token partitions).  int4 pools: 8 blocks per wave (512-token
// partitions) when every row then fits the one-wave combine (max_blocks * 16
// <= 8 x 512 tokens: configs[1] and shorter), else 16 (long rows: configs[3],
// whose 64 partitions of 512 tokens lost 2 points to 32 of 1024).  Measured
// at configs[1], attention only, two runs each: int4 42.5 / 41.6% of HBM peak
// with 8 blocks against 40.7 / 40.9% with 16; int8 60.9 / 60.9% with 8
// against 61.6 / 61.5% with 16.
#ifndef DLMK_MFMA_QNB_SHORT
#define DLMK_MFMA_QNB_SHORT 8
#endif
template <typename C, int D, int GQA, int NQ>
int launch_mfma(const Args &a) {
    if constexpr (C::kScaled && C::kCodeBits == 4 && DLMK_MFMA_QNB_SHORT != DLMK_MFMA_NB) {
        constexpr int NBS = DLMK_MFMA_QNB_SHORT;
        if (parts_for(a.max_blocks, DLMK_MFMA_NW * NBS * kBlock) <= kCombineBatch)
            return launch_mfma_nb<C, D, GQA, NQ, NBS>(a);
    }
    if constexpr (C::kScaled && C::kCodeBits == 8) return launch_mfma_nb<C, D, GQA, NQ, DLMK_MFMA_Q8NB>(a);
    return launch_mfma_nb<C, D, GQA, NQ, DLMK_MFMA_NB>(a);
}

// Generic kernel, NB blocks per wave (FUSED: with the fused step's append).
template <typename T, int DP, int NB, bool FUSED>
int launch_generic_nb(const Args &a) {
    constexpr int NW = 4, PD = 2;
    static_assert(NW * NB * kBlock >= kMinPartition, "partition below the workspace bound");
    const int gqa = a.Hq / a.Hkv;
    const GenGeom geo{a.D, gqa, a.NQ, (gqa * a.NQ + 15) / 16};
    return launch_pair(a, NW * NB * kBlock, (int64_t)a.B * a.Hkv * geo.n_rg,
                       [&](dim3 grid, int max_parts, float *ws_o, float *ws_ml) {
        if (FUSED) grid.y += 1;  // the fused step's append row
        hipLaunchKernelGGL((paged_attn_generic_kernel<T, DP, NW, NB, PD, FUSED>), grid, dim3(NW * 64), 0,
                           a.stream, a.out, a.out_dtype, static_cast<const T *>(a.q),
                           static_cast<T *>(a.k_pool), static_cast<T *>(a.v_pool),
                           static_cast<const T *>(a.k_new), static_cast<const T *>(a.v_new),
                           a.tables, a.ctx_lens, geo, a.Hq, a.Hkv, a.max_blocks, a.num_blocks,
                           a.scale * kLog2e, max_parts, ws_o, ws_ml);
    });
}

// Partition size by grid: the large partitions when that grid fills the chip
// (kGenFullGrid work-groups); otherwise 128-token partitions while they still
// give kGenMinGrid work-groups (a single decoding sequence, as in
// dlmk_decode_block_paged, has num_kv_heads x ctx / 128 of them: 128 at the
// 8B shape and ctx 2048), else 64-token ones.
constexpr int64_t kGenFullGrid = 1024;
constexpr int64_t kGenMinGrid = 128;

template <typename T, int DP, bool FUSED>
int launch_generic_f(const Args &a) {
    // Large partitions: 256 tokens of f32 (NB 4) or 1024 of f16 / bf16 (NB
    // 16).  The fused step picks the same shape as the plain launch, so its
    // output is the same bits as append + attention.
    constexpr int NB_BIG = sizeof(T) == 4 ? 4 : 16;
    const int64_t rgs = (a.Hq / a.Hkv * a.NQ + 15) / 16;
    const auto grid = [&](int p) { return (int64_t)a.B * a.Hkv * rgs * parts_for(a.max_blocks, p); };
#ifdef DLMK_GEN_FORCE_NB
    if (DLMK_GEN_FORCE_NB == 1) return launch_generic_nb<T, DP, 1, FUSED>(a);
    if (DLMK_GEN_FORCE_NB == 2) return launch_generic_nb<T, DP, 2, FUSED>(a);
#endif
    if (grid(4 * NB_BIG * kBlock) >= kGenFullGrid) return launch_generic_nb<T, DP, NB_BIG, FUSED>(a);
    if (grid(4 * 2 * kBlock) >= kGenMinGrid) return launch_generic_nb<T, DP, 2, FUSED>(a);
    return launch_generic_nb<T, DP, 1, FUSED>(a);
}

template <typename T, int DP>
int launch_generic(const Args &a) {
    return a.k_new != nullptr ? launch_generic_f<T, DP, true>(a) : launch_generic_f<T, DP, false>(a);
}

// Padded head dims of the generic kernel: hd is rounded up to the next one.
// f32 pools: multiples of 4 up to 256; f16 / bf16: multiples of 8 up to 256.
template <typename T>
int dispatch_generic(const Args &a) {
    const int hd = a.D;
    if constexpr (sizeof(T) == 4) {
        if (hd % 4 != 0 || hd > 256) return -1;
        if (hd <= 16) return launch_generic<T, 16>(a);
        if (hd <= 32) return launch_generic<T, 32>(a);
        if (hd <= 48) return launch_generic<T, 48>(a);
        if (hd <= 64) return launch_generic<T, 64>(a);
        if (hd <= 80) return launch_generic<T, 80>(a);
        if (hd <= 96) return launch_generic<T, 96>(a);
        if (hd <= 128) return launch_generic<T, 128>(a);
        if (hd <= 192) return launch_generic<T, 192>(a);
        return launch_generic<T, 256>(a);
    } else {
        if (hd % 8 != 0 || hd > 256) return -1;
        if (hd <= 32) return launch_generic<T, 32>(a);
        if (hd <= 64) return launch_generic<T, 64>(a);
        if (hd <= 96) return launch_generic<T, 96>(a);
        if (hd <= 128) return launch_generic<T, 128>(a);
        if (hd <= 160) return launch_generic<T, 160>(a);
        if (hd <= 192) return launch_generic<T, 192>(a);
        return launch_generic<T, 256>(a);
    }
}

// (GQA group, queries) pairs with an instantiated paged_attn_mfma_kernel.
inline bool mfma_rows(int gqa, int nq) {
    switch (gqa * 16 + nq) {
        case 1 * 16 + 1: case 1 * 16 + 2: case 1 * 16 + 4:
        case 2 * 16 + 1: case 2 * 16 + 2: case 2 * 16 + 4:
        case 4 * 16 + 1: case 4 * 16 + 2: case 4 * 16 + 4:
        case 8 * 16 + 1: case 8 * 16 + 2:
        case 16 * 16 + 1: return true;
        default: return false;
    }
}

inline int unsupported_rows(int gqa, int nq) {
    return dlmk::fail(DLMK_ERR_UNSUPPORTED,
                      "paged attention: no kernel for GQA group %d x %d queries", gqa, nq);
}

template <template <int> class CD, int D>
int dispatch_mfma(const Args &a, int gqa) {
    using C = CD<D>;
    switch (gqa * 16 + a.NQ) {
        case 1 * 16 + 1: return launch_mfma<C, D, 1, 1>(a);
        case 1 * 16 + 2: return launch_mfma<C, D, 1, 2>(a);
        case 1 * 16 + 4: return launch_mfma<C, D, 1, 4>(a);
        case 2 * 16 + 1: return launch_mfma<C, D, 2, 1>(a);
        case 2 * 16 + 2: return launch_mfma<C, D, 2, 2>(a);
        case 2 * 16 + 4: return launch_mfma<C, D, 2, 4>(a);
        case 4 * 16 + 1: return launch_mfma<C, D, 4, 1>(a);
        case 4 * 16 + 2: return launch_mfma<C, D, 4, 2>(a);
        case 4 * 16 + 4: return launch_mfma<C, D, 4, 4>(a);
        case 8 * 16 + 1: return launch_mfma<C, D, 8, 1>(a);
        case 8 * 16 + 2: return launch_mfma<C, D, 8, 2>(a);
        case 16 * 16 + 1: return launch_mfma<C, D, 16, 1>(a);
        default: return unsupported_rows(gqa, a.NQ);
    }
}

inline int bad_dim(int head_dim, const char *dims) {
    return dlmk::fail(DLMK_ERR_UNSUPPORTED,
                      "paged attention: head_dim %d unsupported for this dtype (%s)",
                      head_dim, dims);
}

}  // namespace
