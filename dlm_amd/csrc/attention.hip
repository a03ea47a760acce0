// Paged GQA decode attention (dlmk_paged_decode_attention) for gfx950.
//
// Replaces attention_kernel (src/gpu/kernels.cu:210-242: one thread per query
// head, serial over a contiguous f32 history) and the CPU attention()
// (src/forward/cpu.rs:1126-1151).  Same maths -- score = dot(q, k) * scale,
// softmax over the visible positions, out = sum p * v -- evaluated as a
// streaming, HBM-bound pass over the paged pools.
//
// Work decomposition.  One work-group owns one (sequence, kv head, partition of
// kPartition = 256 tokens) and serves every query row that reads that kv head:
// the GQA group times the num_q_per_seq verify queries (ROWS rows).  K/V bytes
// of a partition are therefore read from HBM exactly once.  Each wavefront owns
// BPW consecutive 16-token blocks and issues all their K and V loads (16 bytes
// per lane, each instruction one contiguous KiB of a tile) before doing any
// maths, so a wave keeps BPW * 8 KiB (f16, d=128) in flight.
//
//   K tile [d/X][16][X]: load i of lane l is chunk row l/16 + 4i of token l%16,
//     so one lane accumulates a 4-chunk partial dot for one token and the
//     score needs only a 4-way cross-lane sum (xor 16, xor 32).
//   V tile [d][16]: load i of lane l is X consecutive tokens of one dim, so a
//     lane's accumulator is ROWS x (loads) floats and the final sum is across
//     the 16/X lanes sharing a dim.
//
// Softmax is computed per wave over its own tokens (max, exp2, sum, all in
// the log2 domain with log2(e) folded into the scale), the waves are merged in
// LDS, and partitions of one sequence are merged by log-sum-exp in a second
// kernel.  A sequence whose context fits one partition is finished by the
// first kernel.

#include <hip/hip_runtime.h>

#include <cmath>

#include "dlmk.h"
#include "dlmk_internal.h"

namespace {

constexpr int kBlock = 16;        // tokens per KV block (dlm: src/main.rs:455)
constexpr int kPartition = 256;   // tokens per work-group
constexpr float kLog2e = 1.4426950408889634f;

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <typename T>
struct Elem;
template <>
struct Elem<float> {
    static constexpr int X = 4;
};
template <>
struct Elem<_Float16> {
    static constexpr int X = 8;
};

// acc + dot of two 16-byte chunks.
template <typename T>
__device__ __forceinline__ float dot_chunk(const uint4 &a, const uint4 &b, float acc);

template <>
__device__ __forceinline__ float dot_chunk<float>(const uint4 &a, const uint4 &b, float acc) {
    acc = fmaf(__uint_as_float(a.x), __uint_as_float(b.x), acc);
    acc = fmaf(__uint_as_float(a.y), __uint_as_float(b.y), acc);
    acc = fmaf(__uint_as_float(a.z), __uint_as_float(b.z), acc);
    acc = fmaf(__uint_as_float(a.w), __uint_as_float(b.w), acc);
    return acc;
}

template <>
__device__ __forceinline__ float dot_chunk<_Float16>(const uint4 &a, const uint4 &b, float acc) {
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a.x), __builtin_bit_cast(f16x2, b.x), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a.y), __builtin_bit_cast(f16x2, b.y), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a.z), __builtin_bit_cast(f16x2, b.z), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a.w), __builtin_bit_cast(f16x2, b.w), acc, false);
    return acc;
}

// Widen one 16-byte chunk to X floats (exact).
template <typename T>
__device__ __forceinline__ void widen(const uint4 &c, float *out);

template <>
__device__ __forceinline__ void widen<float>(const uint4 &c, float *out) {
    out[0] = __uint_as_float(c.x);
    out[1] = __uint_as_float(c.y);
    out[2] = __uint_as_float(c.z);
    out[3] = __uint_as_float(c.w);
}

template <>
__device__ __forceinline__ void widen<_Float16>(const uint4 &c, float *out) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f16x2 h = __builtin_bit_cast(f16x2, w[i]);
        out[2 * i] = (float)h[0];
        out[2 * i + 1] = (float)h[1];
    }
}

__device__ __forceinline__ void store_out(void *out, int out_dtype, int64_t idx, float v) {
    if (out_dtype == DLMK_F32) {
        static_cast<float *>(out)[idx] = v;
    } else if (out_dtype == DLMK_F16) {
        static_cast<_Float16 *>(out)[idx] = (_Float16)v;
    } else {
        // bf16, round to nearest even (NaN kept quiet).
        uint32_t u = __float_as_uint(v);
        uint16_t r = (u & 0x7fffffffu) > 0x7f800000u
                         ? (uint16_t)((u >> 16) | 0x40)
                         : (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
        static_cast<uint16_t *>(out)[idx] = r;
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

// ---------------------------------------------------------------------------
// Pass 1: one work-group per (partition, kv head, sequence).
// ---------------------------------------------------------------------------
template <typename T, int D, int GQA, int NQ, int NWAVES>
__global__ __launch_bounds__(NWAVES * 64) void paged_attn_partition_kernel(
    void *__restrict__ out, int out_dtype, const T *__restrict__ q,
    const T *__restrict__ k_pool, const T *__restrict__ v_pool,
    const int32_t *__restrict__ block_tables, const int32_t *__restrict__ ctx_lens,
    int num_q_heads, int num_kv_heads, int max_blocks, int64_t num_blocks, float scale_log2,
    int max_parts, float *__restrict__ ws_o, float *__restrict__ ws_ml) {
    constexpr int X = Elem<T>::X;          // elements per 16-byte chunk
    constexpr int CPL = D / X;             // chunks per token row
    constexpr int KI = CPL / 4;            // 16-byte loads per lane per block (K and V alike)
    constexpr int CPD = kBlock / X;        // V chunks per dim row of a tile
    constexpr int ROWS = GQA * NQ;
    constexpr int BPW = kPartition / kBlock / NWAVES;  // blocks per wave
    constexpr int TILE = D * kBlock;       // elements per (block, kv head) tile
    static_assert(CPL % 4 == 0 && BPW >= 1, "unsupported geometry");

    __shared__ float p_lds[NWAVES][BPW][ROWS][kBlock];
    __shared__ float o_lds[NWAVES][ROWS][D];
    __shared__ float ml_lds[NWAVES][ROWS][2];

    const int part = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    // A length beyond the table width is clamped: no read past a table row and
    // no partition index past max_parts.
    const int ctx = min(ctx_lens[seq], max_blocks * kBlock);
    const int nparts = ctx > kPartition ? (ctx + kPartition - 1) / kPartition : 1;
    if (part >= nparts) return;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nblk_seq = (ctx + kBlock - 1) / kBlock;
    const int first_lb = part * (kPartition / kBlock) + wave * BPW;
    const int32_t *table = block_tables + (int64_t)seq * max_blocks;

    // Physical ids of this wave's blocks (wave-uniform).
    int64_t blk[BPW];
#pragma unroll
    for (int b = 0; b < BPW; ++b) {
        const int lb = first_lb + b;
        int64_t id = lb < nblk_seq ? (int64_t)table[lb] : -1;
        blk[b] = (id >= 0 && id < num_blocks) ? id : -1;
    }

    // Issue every K and V load of the wave up front.
    uint4 kb[BPW][KI], vb[BPW][KI];
#pragma unroll
    for (int b = 0; b < BPW; ++b) {
        if (blk[b] >= 0) {
            const int64_t base = (blk[b] * num_kv_heads + kvh) * TILE;
            const uint4 *kp = reinterpret_cast<const uint4 *>(k_pool + base);
            const uint4 *vp = reinterpret_cast<const uint4 *>(v_pool + base);
#pragma unroll
            for (int i = 0; i < KI; ++i) kb[b][i] = kp[64 * i + lane];
#pragma unroll
            for (int i = 0; i < KI; ++i) vb[b][i] = vp[64 * i + lane];
        } else {
#pragma unroll
            for (int i = 0; i < KI; ++i) kb[b][i] = vb[b][i] = make_uint4(0, 0, 0, 0);
        }
    }

    // Query chunks matching this lane's K chunks.
    uint4 qr[ROWS][KI];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        const int j = r / GQA, h = kvh * GQA + r % GQA;
        const uint4 *qp = reinterpret_cast<const uint4 *>(
            q + ((int64_t)(seq * NQ + j) * num_q_heads + h) * D);
#pragma unroll
        for (int i = 0; i < KI; ++i) qr[r][i] = qp[(lane >> 4) + 4 * i];
    }

    // Scores for token lane%16 of each block; log2 domain.
    const int tok = lane & 15;
    float s[BPW][ROWS];
#pragma unroll
    for (int b = 0; b < BPW; ++b)
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < KI; ++i) acc = dot_chunk<T>(qr[r][i], kb[b][i], acc);
            acc += __shfl_xor(acc, 16);
            acc += __shfl_xor(acc, 32);
            s[b][r] = acc;
        }

    float m[ROWS], l[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        const int limit = ctx - NQ + r / GQA + 1;  // causal limit of verify query r/GQA
        float mx = -INFINITY;
#pragma unroll
        for (int b = 0; b < BPW; ++b) {
            const int pos = (first_lb + b) * kBlock + tok;
            const bool vis = blk[b] >= 0 && pos < limit;
            s[b][r] = vis ? s[b][r] * scale_log2 : -INFINITY;
            mx = fmaxf(mx, s[b][r]);
        }
        mx = xor_max<16>(mx);
        float sum = 0.f;
#pragma unroll
        for (int b = 0; b < BPW; ++b) {
            const float p = mx == -INFINITY ? 0.f : exp2f(s[b][r] - mx);
            s[b][r] = p;
            sum += p;
        }
        m[r] = mx;
        l[r] = xor_sum<16>(sum);
    }

    // Probabilities to LDS: lane group g (= lane/16) writes rows r with r%4 == g.
#pragma unroll
    for (int b = 0; b < BPW; ++b)
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
            if ((r & 3) == (lane >> 4)) p_lds[wave][b][r][tok] = s[b][r];
    __syncthreads();

    // acc[r][i] covers dim (64 i + lane) / CPD over tokens tg*X .. tg*X+X-1.
    const int tg = lane % CPD;
    float acc[ROWS][KI];
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int i = 0; i < KI; ++i) acc[r][i] = 0.f;

#pragma unroll
    for (int b = 0; b < BPW; ++b) {
        if (blk[b] < 0) continue;
        float pr[ROWS][X];
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
#pragma unroll
            for (int e = 0; e < X; ++e) pr[r][e] = p_lds[wave][b][r][tg * X + e];
        // Tokens past the context in the last block hold stale bytes (maybe
        // NaN); zero them so p = 0 contributes exactly nothing.
        const int valid = ctx - (first_lb + b) * kBlock;
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            float v[X];
            widen<T>(vb[b][i], v);
            if (valid < kBlock) {
#pragma unroll
                for (int e = 0; e < X; ++e)
                    if (tg * X + e >= valid) v[e] = 0.f;
            }
#pragma unroll
            for (int r = 0; r < ROWS; ++r)
#pragma unroll
                for (int e = 0; e < X; ++e) acc[r][i] = fmaf(pr[r][e], v[e], acc[r][i]);
        }
    }

#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int i = 0; i < KI; ++i) acc[r][i] = xor_sum<CPD>(acc[r][i]);

    if (tg == 0) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
#pragma unroll
            for (int i = 0; i < KI; ++i) o_lds[wave][r][(64 * i + lane) / CPD] = acc[r][i];
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            ml_lds[wave][r][0] = m[r];
            ml_lds[wave][r][1] = l[r];
        }
    }
    __syncthreads();

    // Merge the waves; finish or write the partition's partial.
    for (int idx = threadIdx.x; idx < ROWS * D; idx += NWAVES * 64) {
        const int r = idx / D, d = idx - r * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NWAVES; ++w) M = fmaxf(M, ml_lds[w][r][0]);
        float O = 0.f, L = 0.f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < NWAVES; ++w) {
                const float mw = ml_lds[w][r][0];
                const float f = mw == -INFINITY ? 0.f : exp2f(mw - M);
                L = fmaf(f, ml_lds[w][r][1], L);
                O = fmaf(f, o_lds[w][r][d], O);
            }
        }
        const int j = r / GQA, h = kvh * GQA + r % GQA;
        const int64_t row = (int64_t)(seq * NQ + j) * num_q_heads + h;
        if (nparts == 1) {
            store_out(out, out_dtype, row * D + d, L > 0.f ? O / L : 0.f);
        } else {
            const int64_t slot = row * max_parts + part;
            ws_o[slot * D + d] = O;
            if (d == 0) {
                ws_ml[2 * slot] = M;
                ws_ml[2 * slot + 1] = L;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Pass 2: log-sum-exp merge of a sequence's partitions, one wave per query row.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(64) void paged_attn_combine_kernel(
    void *__restrict__ out, int out_dtype, const float *__restrict__ ws_o,
    const float *__restrict__ ws_ml, const int32_t *__restrict__ ctx_lens, int rows_per_seq,
    int max_parts) {
    constexpr int DPL = D / 64;  // dims per lane
    const int seq = blockIdx.y;
    const int ctx = min(ctx_lens[seq], max_parts * kPartition);
    const int nparts = ctx > kPartition ? (ctx + kPartition - 1) / kPartition : 1;
    if (nparts == 1) return;
    const int lane = threadIdx.x;
    const int64_t row = (int64_t)seq * rows_per_seq + blockIdx.x;
    const float *ml = ws_ml + 2 * row * max_parts;
    const float *o = ws_o + row * max_parts * D;

    float M = -INFINITY;
    for (int p = lane; p < nparts; p += 64) M = fmaxf(M, ml[2 * p]);
    M = xor_max<64>(M);

    float O[DPL], L = 0.f;
#pragma unroll
    for (int k = 0; k < DPL; ++k) O[k] = 0.f;
    if (M != -INFINITY) {
        for (int p = 0; p < nparts; ++p) {
            const float mp = ml[2 * p];
            const float f = mp == -INFINITY ? 0.f : exp2f(mp - M);
            L = fmaf(f, ml[2 * p + 1], L);
#pragma unroll
            for (int k = 0; k < DPL; ++k) O[k] = fmaf(f, o[(int64_t)p * D + lane + 64 * k], O[k]);
        }
    }
#pragma unroll
    for (int k = 0; k < DPL; ++k)
        store_out(out, out_dtype, row * D + lane + 64 * k, L > 0.f ? O[k] / L : 0.f);
}

// ---------------------------------------------------------------------------
// Host dispatch.
// ---------------------------------------------------------------------------
struct Args {
    void *out;
    int out_dtype;
    const void *q, *k_pool, *v_pool;
    const int32_t *tables, *ctx_lens;
    int B, NQ, Hq, Hkv, max_blocks;
    int64_t num_blocks;
    float scale;
    float *ws_o, *ws_ml;
    int max_parts;
    hipStream_t stream;
};

template <typename T, int D, int GQA, int NQ>
int launch(const Args &a) {
    constexpr int ROWS = GQA * NQ;
    constexpr int NWAVES = ROWS <= 4 ? 4 : 8;
    dim3 grid((unsigned)a.max_parts, (unsigned)a.Hkv, (unsigned)a.B);
    hipLaunchKernelGGL((paged_attn_partition_kernel<T, D, GQA, NQ, NWAVES>), grid,
                       dim3(NWAVES * 64), 0, a.stream, a.out, a.out_dtype,
                       static_cast<const T *>(a.q), static_cast<const T *>(a.k_pool),
                       static_cast<const T *>(a.v_pool), a.tables, a.ctx_lens, a.Hq, a.Hkv,
                       a.max_blocks, a.num_blocks, a.scale * kLog2e, a.max_parts, a.ws_o,
                       a.ws_ml);
    if (a.max_parts > 1)
        hipLaunchKernelGGL(paged_attn_combine_kernel<D>, dim3((unsigned)(a.NQ * a.Hq), (unsigned)a.B),
                           dim3(64), 0, a.stream, a.out, a.out_dtype, a.ws_o, a.ws_ml,
                           a.ctx_lens, a.NQ * a.Hq, a.max_parts);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return dlmk::fail((int)e, "dlmk_paged_decode_attention launch: %s", hipGetErrorString(e));
    return DLMK_OK;
}

template <typename T, int D>
int dispatch_rows(const Args &a, int gqa) {
    switch (gqa * 16 + a.NQ) {
        case 1 * 16 + 1: return launch<T, D, 1, 1>(a);
        case 1 * 16 + 2: return launch<T, D, 1, 2>(a);
        case 1 * 16 + 4: return launch<T, D, 1, 4>(a);
        case 2 * 16 + 1: return launch<T, D, 2, 1>(a);
        case 2 * 16 + 2: return launch<T, D, 2, 2>(a);
        case 2 * 16 + 4: return launch<T, D, 2, 4>(a);
        case 4 * 16 + 1: return launch<T, D, 4, 1>(a);
        case 4 * 16 + 2: return launch<T, D, 4, 2>(a);
        case 8 * 16 + 1: return launch<T, D, 8, 1>(a);
        default:
            return dlmk::fail(DLMK_ERR_UNSUPPORTED,
                              "dlmk_paged_decode_attention: no kernel for GQA group %d x %d queries",
                              gqa, a.NQ);
    }
}

template <typename T>
int dispatch_dim(const Args &a, int head_dim, int gqa) {
    switch (head_dim) {
        case 64: return dispatch_rows<T, 64>(a, gqa);
        case 128: return dispatch_rows<T, 128>(a, gqa);
        default:
            return dlmk::fail(DLMK_ERR_UNSUPPORTED,
                              "dlmk_paged_decode_attention: head_dim %d unsupported (64, 128)",
                              head_dim);
    }
}

int64_t parts_for(int max_blocks) {
    int64_t tokens = (int64_t)max_blocks * kBlock;
    return tokens > kPartition ? dlmk::ceil_div(tokens, kPartition) : 1;
}

}  // namespace

extern "C" {

size_t dlmk_paged_attention_workspace_size(int num_seqs, int num_q_per_seq, int num_q_heads,
                                           int head_dim, int block_size, int max_blocks_per_seq) {
    (void)block_size;
    if (num_seqs <= 0 || num_q_per_seq <= 0 || num_q_heads <= 0 || head_dim <= 0 ||
        max_blocks_per_seq <= 0)
        return 0;
    const int64_t parts = parts_for(max_blocks_per_seq);
    if (parts <= 1) return 0;
    const int64_t rows = (int64_t)num_seqs * num_q_per_seq * num_q_heads;
    const int64_t o_bytes = rows * parts * head_dim * 4;
    const int64_t o_aligned = (o_bytes + 255) / 256 * 256;
    return (size_t)(o_aligned + rows * parts * 2 * 4);
}

int dlmk_paged_decode_attention(void *stream, void *out, int out_dtype, const void *q,
                                const void *k_pool, const void *v_pool, int dtype,
                                const int32_t *block_tables, const int32_t *ctx_lens,
                                int num_seqs, int num_q_per_seq, int num_q_heads,
                                int num_kv_heads, int head_dim, int block_size,
                                int max_blocks_per_seq, int64_t num_blocks, float scale,
                                void *workspace, size_t workspace_bytes) {
    if (num_seqs < 0 || num_q_per_seq <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
        head_dim <= 0 || max_blocks_per_seq <= 0 || num_blocks < 0)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_paged_decode_attention: bad sizes");
    if (num_q_heads % num_kv_heads != 0)
        return dlmk::fail(DLMK_ERR_INVALID_ARG,
                          "dlmk_paged_decode_attention: %d query heads not a multiple of %d kv heads",
                          num_q_heads, num_kv_heads);
    if (num_seqs == 0) return DLMK_OK;
    if (!out || !q || !k_pool || !v_pool || !block_tables || !ctx_lens)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_paged_decode_attention: null pointer");
    if (block_size != kBlock)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED,
                          "dlmk_paged_decode_attention: block_size %d unsupported (16)", block_size);
    if (out_dtype != DLMK_F32 && out_dtype != DLMK_F16 && out_dtype != DLMK_BF16)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_paged_decode_attention: bad out dtype %d",
                          out_dtype);
    if (num_seqs > 65535 || num_kv_heads > 65535)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED, "dlmk_paged_decode_attention: grid too large");

    Args a;
    a.out = out;
    a.out_dtype = out_dtype;
    a.q = q;
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.tables = block_tables;
    a.ctx_lens = ctx_lens;
    a.B = num_seqs;
    a.NQ = num_q_per_seq;
    a.Hq = num_q_heads;
    a.Hkv = num_kv_heads;
    a.max_blocks = max_blocks_per_seq;
    a.num_blocks = num_blocks;
    a.scale = scale;
    a.stream = (hipStream_t)stream;
    a.max_parts = (int)parts_for(max_blocks_per_seq);
    a.ws_o = nullptr;
    a.ws_ml = nullptr;
    if (a.max_parts > 1) {
        const size_t need = dlmk_paged_attention_workspace_size(
            num_seqs, num_q_per_seq, num_q_heads, head_dim, block_size, max_blocks_per_seq);
        if (!workspace || workspace_bytes < need)
            return dlmk::fail(DLMK_ERR_WORKSPACE,
                              "dlmk_paged_decode_attention: workspace %zu bytes, need %zu",
                              workspace_bytes, need);
        if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
            return dlmk::fail(DLMK_ERR_INVALID_ARG,
                              "dlmk_paged_decode_attention: workspace not 256-byte aligned");
        const int64_t rows = (int64_t)num_seqs * num_q_per_seq * num_q_heads;
        const int64_t o_bytes = rows * a.max_parts * head_dim * 4;
        a.ws_o = static_cast<float *>(workspace);
        a.ws_ml = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                            (o_bytes + 255) / 256 * 256);
    }
    const int gqa = num_q_heads / num_kv_heads;
    switch (dtype) {
        case DLMK_F32: return dispatch_dim<float>(a, head_dim, gqa);
        case DLMK_F16: return dispatch_dim<_Float16>(a, head_dim, gqa);
        default:
            return dlmk::fail(DLMK_ERR_UNSUPPORTED,
                              "dlmk_paged_decode_attention: KV dtype %d unsupported (f32, f16)", dtype);
    }
}

}  // extern "C"
