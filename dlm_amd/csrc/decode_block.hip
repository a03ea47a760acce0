// One transformer decode block over the paged KV cache (dlmk_decode_block_paged).
//
// The drop-in for dlm_decode_block (src/gpu/kernels.cu:313-392) with its
// contiguous, per-kernel f32 KV history (kv_keys / kv_values written at slot
// num_positions, :361-363, then attention over it, :365-366) replaced by the
// layer's paged pools and the sequence's block table.  The maths follows
// decode_block (src/forward/cpu.rs:1156-1219): rmsnorm -> q/k/v projections
// (+ biases) -> RoPE -> append -> GQA attention -> o_proj + residual ->
// rmsnorm -> SwiGLU MLP + residual.  Weights stay in their checkpoint dtype
// (f32, bf16, f16, or dlm's int4/int8 group-affine blobs) and are decoded in
// registers, as the reference's load_w<> does.
//
// Kernels (all HBM-bound on the weights at decode batch 1):
//   gemv_kernel          x staged once per work-group in LDS as f32 planes
//                        (both rmsnorms are folded into that staging); a grid
//                        of resident work-groups; RW output rows per wave,
//                        16-byte weight loads, 16 in flight per lane (8 per
//                        matrix for SwiGLU) plus the next step's prefetched,
//                        wave reduction; epilogue = residual add, (two
//                        matrices) SwiGLU, or, for q, k and v as one launch,
//                        biases and RoPE (NeoX split-half, host-computed
//                        inv_freq) over row pairs of one head,
//                        with the new token's K and V written straight into
//                        the pools at the slot the block table gives; it also
//                        writes the context length the attention reads.
// Attention is dlmk_paged_decode_attention (f32 pools).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "dlmk.h"
#include "dlmk_internal.h"

namespace {

constexpr int kBlock = 16;  // tokens per KV block
#ifndef DLMK_GEMV_WAVES
#define DLMK_GEMV_WAVES 4
#endif
constexpr int kGemvWaves = DLMK_GEMV_WAVES;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Non-temporal load with its result type pinned to the pointee: called on a
// vector pointer directly, the builtin's result can come back as one element
// (then splatted), and only a dword is loaded.
template <typename V>
__device__ __forceinline__ V stream_load(const V *p) {
    return __builtin_nontemporal_load(p);
}

template <int W>
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 1; o < W; o <<= 1) v += __shfl_xor(v, o);
    return v;
}

// ---------------------------------------------------------------------------
// Weight chunks: 16 bytes of one row hold E elements.  dot_chunk returns
// sum_e w_e * x_e for the chunk starting at element j0 of row `row`.
// Quantized blobs (QuantLayout, src/forward/cpu.rs:132-159): codes, then f32
// scales and zero-points per group of `gs` elements; a chunk never straddles
// a group (gs is a multiple of E, checked by the host), so it is
// scale * (sum c_e x_e - zero * sum x_e).
// ---------------------------------------------------------------------------
template <int DT>
struct WChunk;

template <>
struct WChunk<DLMK_W_F32> {
    static constexpr int E = 4;
    static __device__ __forceinline__ float dot(u32x4 r, const float *xs, const uint8_t *, int64_t,
                                                int64_t, int64_t, int64_t) {
        // Whole-vector bit casts only: a bit cast of one element of a vector
        // (r[e], r.y) reads the vector's first element with this compiler.
        typedef float f4 __attribute__((ext_vector_type(4)));
        const f4 f = __builtin_bit_cast(f4, r);
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) s += f[e] * xs[e];
        return s;
    }
};

template <>
struct WChunk<DLMK_W_BF16> {
    static constexpr int E = 8;
    static __device__ __forceinline__ float dot(u32x4 r, const float *xs, const uint8_t *, int64_t,
                                                int64_t, int64_t, int64_t) {
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            s += __builtin_bit_cast(float, r[e] << 16) * xs[2 * e];
            s += __builtin_bit_cast(float, r[e] & 0xffff0000u) * xs[2 * e + 1];
        }
        return s;
    }
};

template <>
struct WChunk<DLMK_W_F16> {
    static constexpr int E = 8;
    static __device__ __forceinline__ float dot(u32x4 r, const float *xs, const uint8_t *, int64_t,
                                                int64_t, int64_t, int64_t) {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        const h8 h = __builtin_bit_cast(h8, r);
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) s += (float)h[e] * xs[e];
        return s;
    }
};

template <>
struct WChunk<DLMK_W_INT4> {
    static constexpr int E = 32;  // two codes a byte, low nibble = even element
    static __device__ __forceinline__ float dot(u32x4 r, const float *xs, const uint8_t *blob,
                                                int64_t scales_off, int64_t zeros_off, int64_t gs,
                                                int64_t i0) {
        float cx = 0.f, sx = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const float x = xs[8 * e + b];
                cx += (float)((r[e] >> (4 * b)) & 15u) * x;
                sx += x;
            }
        const int64_t g = i0 / gs;
        const float scale = *reinterpret_cast<const float *>(blob + scales_off + 4 * g);
        const float zero = *reinterpret_cast<const float *>(blob + zeros_off + 4 * g);
        return scale * (cx - zero * sx);
    }
};

template <>
struct WChunk<DLMK_W_INT8> {
    static constexpr int E = 16;  // one code a byte
    static __device__ __forceinline__ float dot(u32x4 r, const float *xs, const uint8_t *blob,
                                                int64_t scales_off, int64_t zeros_off, int64_t gs,
                                                int64_t i0) {
        float cx = 0.f, sx = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const float x = xs[4 * e + b];
                cx += (float)((r[e] >> (8 * b)) & 255u) * x;
                sx += x;
            }
        const int64_t g = i0 / gs;
        const float scale = *reinterpret_cast<const float *>(blob + scales_off + 4 * g);
        const float zero = *reinterpret_cast<const float *>(blob + zeros_off + 4 * g);
        return scale * (cx - zero * sx);
    }
};

// Byte offsets of a quantized blob of n elements (QuantLayout).
struct QOffsets {
    int64_t scales, zeros;
};

__host__ __device__ inline QOffsets qoffsets(int dt, int64_t n, int64_t gs) {
    const int64_t code_bytes = dt == DLMK_W_INT4 ? (n + 1) / 2 : n;
    const int64_t s = (code_bytes + 3) / 4 * 4;
    const int64_t groups = gs > 0 ? (n + gs - 1) / gs : 0;
    return QOffsets{s, s + groups * 4};
}

enum Epilogue { kAddInto = 1, kSwiGLU = 2, kRopeAppend = 3 };

// Up to three matrices over the same input, as one launch (q, k and v share
// the normalised hidden state).  A segment's rows follow the previous
// segment's in the launch's row numbering.
struct GemvSeg {
    const uint8_t *W, *W2;  // W2: the up projection of the SwiGLU epilogue
    const float *bias;      // kRopeAppend: may be null
    float *out;             // token t's outputs start at out + t * ostride
    int rows, ostride;
};

// kRopeAppend: segments q, k, v (+ biases); q is rotated in place into its
// output, the rotated k and v go straight into the pools.
struct RopeArgs {
    const float *inv_freq;
    float *k_pool, *v_pool;
    const int32_t *table;
    int64_t num_blocks;
    int num_kv_heads, head_dim, num_positions, position;
    int32_t *ctx_len;
};

struct GemvArgs {
    GemvSeg seg[3];
    int nseg, total_rows, in_dim, gs;
    int nt;               // tokens (x rows [nt][x_stride]); the kernel's NT >= nt
    // Column slice: this launch covers weight columns col0 .. col0 + in_dim of
    // rows row_elems long (kAddInto only; otherwise col0 0, in_dim ==
    // row_elems), reading x[t][col0 ..] with rows x_stride floats apart.
    int col0, row_elems, x_stride;
    const float *x;
    const float *norm_w;  // non-null: x is staged as rmsnorm(x) * norm_w
    float eps;
    RopeArgs rope;
};

// Row-major [rows][in_dim] matrices times x.  Work-group: kGemvWaves waves
// and x staged once in LDS as f32 -- normalised on the way when norm_w is set
// (rmsnorm, src/forward/cpu.rs:934-943: every work-group sums the squares in
// the same order, so all see the same factor).  Wave w of work-group b takes
// launch rows (b * kGemvWaves + w) * RW + k * gridDim.x * kGemvWaves * RW,
// RW rows at a time, so a grid of resident work-groups amortises the staging
// over several rows and each x read over RW rows: 16-byte weight loads, U in
// flight per lane per row, a wave reduction per row.  Epilogues: kAddInto
// out[o] += dot (the residual); kSwiGLU out[o] = silu(dot(W)) * dot(W2);
// kRopeAppend (q, k, v + biases, then RoPE and the paged append).
//
// Measured on the 8B layer (bf16): the x reads from LDS, not the weight
// stream, bounded these kernels -- down_proj took 34.9 us with the dot
// products and 20.9 us with them replaced by a register-only reduction, against
// 18.1 us for a pure read of its weights with the same grid.  Conflict-free
// planes of x and one x read per RW rows took it to 23.3 us.
template <int RW>
struct RowGroup {  // RW launch rows resolved to their segments
    GemvSeg g[RW];
    int o[RW], si[RW];
    QOffsets qo[RW];
};

// RoPE pair (rope_inplace, src/forward/cpu.rs:1094-1114: NeoX split-half,
// host-computed inv_freq) of rows `row` (dim i of its head) and row + d/2 of
// segment si: q rotated into out; k rotated and v as they are into the pools
// at position num_positions of the sequence (table[p / 16], offset p % 16, f32
// layouts K [blk][Hkv][d/4][16][4], V [blk][Hkv][d][16]); a block id outside
// the pool is skipped (the attention masks it).
__device__ __forceinline__ void rope_store(const RopeArgs &r, int si, float *out, int row, float a,
                                           float b, int tok) {
    const int d = r.head_dim, half = d / 2, h = row / d, i = row % d;
    if (si < 2) {
        const float ang = (float)(r.position + tok) * r.inv_freq[i];
        const float sn = sinf(ang), cs = cosf(ang);
        const float ra = a * cs - b * sn, rb = a * sn + b * cs;
        a = ra;
        b = rb;
    }
    if (si == 0) {
        out[row] = a;
        out[row + half] = b;
        return;
    }
    const int pos = r.num_positions + tok;
    const int64_t blk = r.table[pos / kBlock];
    if (blk < 0 || blk >= r.num_blocks) return;
    const int t = pos % kBlock;
    const int64_t tile = (blk * r.num_kv_heads + h) * (int64_t)d * kBlock;
    if (si == 1) {
        float *kt = r.k_pool + tile;
        kt[((i / 4) * kBlock + t) * 4 + i % 4] = a;
        kt[(((i + half) / 4) * kBlock + t) * 4 + (i + half) % 4] = b;
    } else {
        float *vt = r.v_pool + tile;
        vt[(int64_t)i * kBlock + t] = a;
        vt[(int64_t)(i + half) * kBlock + t] = b;
    }
}

template <int DT, int EPI, int RW, int U, int NT>
__global__ __launch_bounds__(64 * kGemvWaves) void gemv_kernel(GemvArgs a) {
    using C = WChunk<DT>;
    constexpr int E = C::E;
    constexpr bool kTwo = EPI == kSwiGLU;
    extern __shared__ float xs[];
    __shared__ float red[NT][kGemvWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int in_dim = a.in_dim;
    const int chunks = in_dim / E;
    const int64_t row_bytes = (int64_t)a.row_elems * 16 / E;
    const int cc0 = a.col0 / E;  // first chunk of the slice
    const int rstride = gridDim.x * kGemvWaves * RW;

    // A wave's work is a sequence of steps (RW rows, chunk block c0 of U * 64
    // chunks): rows r0, r0 + rstride, ..., each over c0 = 0, 64U, ... .  The
    // loads of step s + 1 are issued before step s is computed (two register
    // buffers, A and B), and the first step's loads go out before x is
    // staged, so the weight stream never waits on the x round trip or on a
    // step's arithmetic.
    auto resolve = [&](int r0, RowGroup<RW> &R) {
#pragma unroll
        for (int j = 0; j < RW; ++j) {
            // Segment of launch row r0 + j (explicit selects: a dynamically
            // indexed kernel-argument array would be copied to scratch).  Rows
            // past the end repeat the last row, and are not stored.
            int rr = min(r0 + j, a.total_rows - 1);
            R.g[j] = a.seg[0];
            R.si[j] = 0;
            if (a.nseg > 1 && rr >= a.seg[0].rows) {
                rr -= a.seg[0].rows;
                R.g[j] = a.seg[1];
                R.si[j] = 1;
                if (a.nseg > 2 && rr >= a.seg[1].rows) {
                    rr -= a.seg[1].rows;
                    R.g[j] = a.seg[2];
                    R.si[j] = 2;
                }
            }
            if constexpr (EPI == kRopeAppend) {
                // Launch rows 2p, 2p + 1 are rows i and i + d/2 of one head
                // (p = head * d/2 + i): the RoPE pair lands in one wave.
                const int half = a.rope.head_dim / 2, pr = rr >> 1;
                rr = (pr / half) * a.rope.head_dim + pr % half + (rr & 1) * half;
            }
            R.o[j] = rr;
            R.qo[j] = qoffsets(DT, (int64_t)R.g[j].rows * a.row_elems, a.gs);
        }
    };
    auto issue = [&](const RowGroup<RW> &R, int c0, u32x4 (&w1)[RW][U], u32x4 (&w2)[RW][U]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = min(c0 + u * 64 + lane, chunks - 1);
#pragma unroll
            for (int j = 0; j < RW; ++j) {
                w1[j][u] = stream_load(reinterpret_cast<const u32x4 *>(R.g[j].W + R.o[j] * row_bytes) + cc0 + c);
                if constexpr (kTwo)
                    w2[j][u] = stream_load(reinterpret_cast<const u32x4 *>(R.g[j].W2 + R.o[j] * row_bytes) + cc0 + c);
            }
        }
    };

    if constexpr (EPI == kRopeAppend)
        if (blockIdx.x == 0 && threadIdx.x == 0) *a.rope.ctx_len = a.rope.num_positions + a.nt;
    int r0 = (blockIdx.x * kGemvWaves + wave) * RW, c0 = 0;
    RowGroup<RW> RA, RB;
    u32x4 wa1[RW][U], wa2[RW][U], wb1[RW][U], wb2[RW][U];
    if (r0 < a.total_rows) {
        resolve(r0, RA);
        issue(RA, 0, wa1, wa2);
    }
    __builtin_amdgcn_sched_barrier(0);

    // Stage x with 16-byte loads, kStageUnroll in flight per thread (in_dim is
    // a multiple of 4: every weight dtype reads at least 4 elements a chunk),
    // summing the squares on the way; then normalise in place.  LDS holds x
    // as E/4 planes of float4, plane q holding elements 4q .. 4q + 3 of every
    // chunk: lanes reading consecutive chunks read consecutive 16-byte slots
    // (no bank conflicts; chunk-major storage conflicts 2-way for bf16 and
    // more for the quantized dtypes).  Token t's planes follow token t - 1's
    // (t * in_dim floats in); tokens past nt are staged as zeros.
    constexpr int kStageUnroll = 8;
    const int n4 = in_dim / 4;
    float4 *xs4 = reinterpret_cast<float4 *>(xs);
    // The norm weights of this thread's first kNormPre normalise-pass slots,
    // loaded with x (not after the reduction's barrier).
    constexpr int kNormPre = 4;
    float4 nwv[kNormPre];
    if (a.norm_w != nullptr) {
#pragma unroll
        for (int j = 0; j < kNormPre; ++j) {
            const int k = threadIdx.x + j * 64 * kGemvWaves;
            if (k < n4) {
                const float *nw = a.norm_w + (k % chunks) * E + 4 * (k / chunks);
                nwv[j] = make_float4(nw[0], nw[1], nw[2], nw[3]);
            }
        }
    }
    float ss[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        ss[t] = 0.f;
        const float4 *x4 = reinterpret_cast<const float4 *>(a.x + (int64_t)t * a.x_stride + a.col0);
        float4 *xt4 = xs4 + t * n4;
        const bool live = t < a.nt;
        for (int i0 = 0; i0 < n4; i0 += 64 * kGemvWaves * kStageUnroll) {
            float4 v[kStageUnroll];
#pragma unroll
            for (int u = 0; u < kStageUnroll; ++u) {
                const int i = i0 + u * 64 * kGemvWaves + threadIdx.x;
                v[u] = live && i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < kStageUnroll; ++u) {
                const int i = i0 + u * 64 * kGemvWaves + threadIdx.x;
                if (i < n4) {
                    xt4[(i % (E / 4)) * chunks + i / (E / 4)] = v[u];
                    ss[t] += v[u].x * v[u].x + v[u].y * v[u].y + v[u].z * v[u].z + v[u].w * v[u].w;
                }
            }
        }
    }
    if (a.norm_w != nullptr) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            ss[t] = wave_sum<64>(ss[t]);
            if (lane == 0) red[t][wave] = ss[t];
        }
        __syncthreads();
        float inv[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float tot = 0.f;
#pragma unroll
            for (int w = 0; w < kGemvWaves; ++w) tot += red[t][w];
            inv[t] = 1.0f / sqrtf(tot / (float)in_dim + a.eps);
        }
        auto norm4 = [&](int k, float4 w) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float4 v = xs4[t * n4 + k];
                v.x = v.x * inv[t] * w.x;
                v.y = v.y * inv[t] * w.y;
                v.z = v.z * inv[t] * w.z;
                v.w = v.w * inv[t] * w.w;
                xs4[t * n4 + k] = v;
            }
        };
#pragma unroll
        for (int j = 0; j < kNormPre; ++j) {
            const int k = threadIdx.x + j * 64 * kGemvWaves;
            if (k < n4) norm4(k, nwv[j]);
        }
        for (int k = threadIdx.x + kNormPre * 64 * kGemvWaves; k < n4; k += 64 * kGemvWaves) {
            const float *nw = a.norm_w + (k % chunks) * E + 4 * (k / chunks);
            norm4(k, make_float4(nw[0], nw[1], nw[2], nw[3]));
        }
    }
    __syncthreads();

    float acc[RW][NT], acc2[RW][NT];
#pragma unroll
    for (int j = 0; j < RW; ++j)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[j][t] = acc2[j][t] = 0.f;

    // One step: issue the next step's loads into (Rn, wn), then consume
    // (Rc, wc) at (r0, c0); finish the rows after their last chunk block.
    // Returns false when the wave has no further step.
    auto step = [&](RowGroup<RW> &Rc, u32x4 (&wc1)[RW][U], u32x4 (&wc2)[RW][U], RowGroup<RW> &Rn,
                    u32x4 (&wn1)[RW][U], u32x4 (&wn2)[RW][U]) -> bool {
        int r1 = r0, c1 = c0 + 64 * U;
        const bool last = c1 >= chunks;
        if (last) {
            c1 = 0;
            r1 += rstride;
        }
        if (r1 < a.total_rows) {
            resolve(r1, Rn);  // scalar work; a struct copy here defeats SROA
            issue(Rn, c1, wn1, wn2);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + u * 64 + lane;
            if (c < chunks) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    if (NT > 1 && t >= a.nt) break;
                    float xv[E];  // token t's x of this chunk, read once for the RW rows
#pragma unroll
                    for (int q = 0; q < E / 4; ++q) {
                        const float4 v = xs4[t * n4 + q * chunks + c];
                        xv[4 * q] = v.x;
                        xv[4 * q + 1] = v.y;
                        xv[4 * q + 2] = v.z;
                        xv[4 * q + 3] = v.w;
                    }
#pragma unroll
                    for (int j = 0; j < RW; ++j) {
                        const int64_t i0 = (int64_t)Rc.o[j] * a.row_elems + a.col0 + (int64_t)c * E;
                        acc[j][t] += C::dot(wc1[j][u], xv, Rc.g[j].W, Rc.qo[j].scales, Rc.qo[j].zeros, a.gs, i0);
                        if constexpr (kTwo)
                            acc2[j][t] += C::dot(wc2[j][u], xv, Rc.g[j].W2, Rc.qo[j].scales, Rc.qo[j].zeros, a.gs, i0);
                    }
                }
            }
        }
        if constexpr (EPI == kRopeAppend) {
            static_assert(RW == 2, "RoPE pairs need two rows per wave");
            if (last) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    float s[2];
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        s[j] = wave_sum<64>(acc[j][t]);
                        if (Rc.g[j].bias) s[j] += Rc.g[j].bias[Rc.o[j]];
                        acc[j][t] = acc2[j][t] = 0.f;
                    }
                    if (lane == 0 && r0 < a.total_rows && t < a.nt)
                        rope_store(a.rope, Rc.si[0], Rc.g[0].out + (int64_t)t * Rc.g[0].ostride, Rc.o[0],
                                   s[0], s[1], t);
                }
            }
        } else if (last) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int j = 0; j < RW; ++j) {
                    const float s1 = wave_sum<64>(acc[j][t]);
                    const float s2 = kTwo ? wave_sum<64>(acc2[j][t]) : 0.f;
                    if (lane == 0 && r0 + j < a.total_rows && t < a.nt) {
                        float *o = Rc.g[j].out + (int64_t)t * Rc.g[j].ostride + Rc.o[j];
                        if constexpr (EPI == kAddInto) {
                            *o = *o + s1;
                        } else {
                            // silu(gate) * up, cpu.rs:960-975
                            *o = s1 / (1.0f + expf(-s1)) * s2;
                        }
                    }
                    acc[j][t] = acc2[j][t] = 0.f;
                }
        }
        r0 = r1;
        c0 = c1;
        return r0 < a.total_rows;
    };
    if (r0 < a.total_rows) {
        while (step(RA, wa1, wa2, RB, wb1, wb2) && step(RB, wb1, wb2, RA, wa1, wa2)) {
        }
    }
}


int w_elems_per_chunk(int dt) {
    switch (dt) {
        case DLMK_W_F32: return 4;
        case DLMK_W_BF16:
        case DLMK_W_F16: return 8;
        case DLMK_W_INT4: return 32;
        case DLMK_W_INT8: return 16;
        default: return 0;
    }
}

int device_cus() {
    static int cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (cus[dev] == 0) {
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c < 1)
            c = 1;
        cus[dev] = c;
    }
    return cus[dev];
}

// Resident work-groups only (the occupancy of this instantiation with its
// LDS), so every work-group runs from the start and stages x once for all
// its rows.
template <int DT, int EPI, int RW, int U, int NT>
void launch_gemv_rw(hipStream_t st, const GemvArgs &a) {
    const auto kernel = gemv_kernel<DT, EPI, RW, U, NT>;
    const size_t lds = (size_t)NT * a.in_dim * sizeof(float);
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 64 * kGemvWaves, lds) !=
            hipSuccess || per_cu < 1)
        per_cu = 1;
    const int want = (a.total_rows + kGemvWaves * RW - 1) / (kGemvWaves * RW);
    const int grid = std::max(1, std::min(want, device_cus() * per_cu));
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * kGemvWaves), lds, st, a);
}

// T weight loads in flight per lane -- 16, or 8 per matrix for SwiGLU and 8 for
// one-token residual launches: rows of at least T loads per lane run one at a
// time, shorter rows 2 or 4 at once.
// Several tokens (NT > 1) do NT times the arithmetic per load and hold NT
// accumulators per row: one row per wave (two for the RoPE pairs) and 8 (4
// per matrix) loads in flight.  Measured on two Llama-3-8B layers, verify of
// 2 / 5 / 8 tokens: 114.8 / 291.3 / 338.4 us a layer, against 114.0 / 301.1
// / 360.2 with 16 / NT loads (at least 2) and 117.6 / 305.8 / 362.6 with 16.
template <int DT, int EPI, int NT>
void launch_gemv_epi(hipStream_t st, const GemvArgs &a) {
    constexpr int T0 = EPI == kSwiGLU ? 8 : 16;
    // One-token residual launches (o_proj, down_proj): 8 loads in flight per
    // lane, whose registers allow more resident waves (8B layer 95.2 -> 94.1
    // us; the verify's several-token launches keep T0 / 2).
    constexpr int T = NT == 1 ? (EPI == kAddInto ? 8 : T0) : T0 / 2;
    if constexpr (EPI == kRopeAppend) {
        // RoPE pairs: two rows per wave.  One token: 4 loads per row, whose
        // registers allow 3 waves per SIMD, so the 8B layer's 6144 q/k/v rows
        // fit one pass of resident work-groups (14.2 -> 13.1 us; 8 loads per
        // row held 2 waves per SIMD and took 1.5 passes).
        constexpr int UR = NT == 1 ? T / 4 : T / 2;
        launch_gemv_rw<DT, EPI, 2, (UR > 1 ? UR : 1), NT>(st, a);
    } else if constexpr (NT > 1) {
        launch_gemv_rw<DT, EPI, 1, T, NT>(st, a);
    } else {
        const int per_lane = (a.in_dim / WChunk<DT>::E + 63) / 64;  // chunk loads per lane per row
        if (per_lane >= T)
            launch_gemv_rw<DT, EPI, 1, T, NT>(st, a);
        else if (per_lane >= T / 2)
            launch_gemv_rw<DT, EPI, 2, T / 2, NT>(st, a);
        else
            launch_gemv_rw<DT, EPI, 4, T / 4, NT>(st, a);
    }
}

template <int DT, int NT>
void launch_gemv_nt(int epi, hipStream_t st, const GemvArgs &a) {
    if (epi == kAddInto)
        launch_gemv_epi<DT, kAddInto, NT>(st, a);
    else if (epi == kSwiGLU)
        launch_gemv_epi<DT, kSwiGLU, NT>(st, a);
    else
        launch_gemv_epi<DT, kRopeAppend, NT>(st, a);
}

// Token counts the kernel is instantiated for; a launch of nt tokens runs
// the smallest NT >= nt (tokens past nt are zeros and never stored).
template <int DT>
void launch_gemv(int epi, hipStream_t st, const GemvArgs &a) {
    if (a.nt <= 1)
        launch_gemv_nt<DT, 1>(epi, st, a);
    else if (a.nt <= 2)
        launch_gemv_nt<DT, 2>(epi, st, a);
    else if (a.nt <= 4)
        launch_gemv_nt<DT, 4>(epi, st, a);
    else
        launch_gemv_nt<DT, 8>(epi, st, a);
}

constexpr int kMaxTokensPerLaunch = 8;
constexpr int64_t kGemvLdsMax = 64 * 1024;  // bytes of staged x per work-group

void gemv_launch(int dt, int epi, hipStream_t st, const GemvArgs &a) {
    switch (dt) {
        case DLMK_W_F32: launch_gemv<DLMK_W_F32>(epi, st, a); break;
        case DLMK_W_BF16: launch_gemv<DLMK_W_BF16>(epi, st, a); break;
        case DLMK_W_F16: launch_gemv<DLMK_W_F16>(epi, st, a); break;
        case DLMK_W_INT4: launch_gemv<DLMK_W_INT4>(epi, st, a); break;
        default: launch_gemv<DLMK_W_INT8>(epi, st, a); break;
    }
}

// n tokens through one GEMV stage, in groups of at most kMaxTokensPerLaunch
// tokens whose inputs are staged in LDS together, so each weight row is read
// once per group -- the point of verifying a draft in one pass.  Launches
// that normalise their input (norm_w) stage whole rows: as many tokens as
// kGemvLdsMax holds.  Residual launches (kAddInto, no norm) take a group of up
// to 8 tokens over column slices sized to kGemvLdsMax instead, each launch
// adding its slice's partial dot products into the output (for one token,
// and whenever a whole row fits, one slice).
void gemv(int dt, int epi, hipStream_t st, const GemvArgs &a, int n) {
    const int64_t row_bytes = (int64_t)a.in_dim * sizeof(float);
    const bool sliced = epi == kAddInto && a.norm_w == nullptr && n > 1;
    int fit = sliced ? kMaxTokensPerLaunch
                     : (int)std::min<int64_t>(kMaxTokensPerLaunch, kGemvLdsMax / row_bytes);
    // Whole instantiated NT sizes: 8, 4, 2, 1 (a padded NT also takes LDS).
    fit = fit >= 8 ? 8 : fit >= 4 ? 4 : fit >= 2 ? 2 : 1;
    for (int t0 = 0; t0 < n; t0 += fit) {
        GemvArgs b = a;
        b.nt = std::min(fit, n - t0);
        b.x = a.x + (int64_t)t0 * a.x_stride;
        for (int i = 0; i < b.nseg; ++i) b.seg[i].out += (int64_t)t0 * b.seg[i].ostride;
        b.rope.num_positions += t0;
        b.rope.position += t0;
        const int nt_pad = b.nt <= 1 ? 1 : b.nt <= 2 ? 2 : b.nt <= 4 ? 4 : 8;
        // Slice width: a multiple of the chunk (and of the quantization group,
        // so no group straddles two launches).
        const int unit = std::max(w_elems_per_chunk(dt), a.gs > 0 ? a.gs : 1);
        int width = a.in_dim;
        if (sliced && (int64_t)nt_pad * a.in_dim * (int64_t)sizeof(float) > kGemvLdsMax)
            width = std::max(unit, (int)(kGemvLdsMax / ((int64_t)nt_pad * sizeof(float))) / unit * unit);
        for (int c0 = 0; c0 < a.in_dim; c0 += width) {
            GemvArgs c = b;
            c.col0 = c0;
            c.in_dim = std::min(width, a.in_dim - c0);
            gemv_launch(dt, epi, st, c);
        }
    }
}

GemvArgs gemv_args(const float *x, int in_dim, int gs, const float *norm_w, float eps) {
    GemvArgs a{};
    a.x = x;
    a.in_dim = in_dim;
    a.row_elems = in_dim;
    a.x_stride = in_dim;
    a.col0 = 0;
    a.gs = gs;
    a.norm_w = norm_w;
    a.eps = eps;
    return a;
}

// ostride: floats between consecutive tokens' outputs.
void add_seg(GemvArgs &a, const void *W, const void *W2, const float *bias, float *out, int rows,
             int ostride) {
    a.seg[a.nseg++] = GemvSeg{static_cast<const uint8_t *>(W), static_cast<const uint8_t *>(W2),
                              bias, out, rows, ostride};
    a.total_rows += rows;
}

// Workspace regions, each on a 256-byte boundary, for n tokens: q[n][qd],
// k[kvd], v[kvd] (the k / v segments' outputs go to the pools; these are
// never written), ctx[n][qd], act[n][inter], ctx_len (int32), then the
// attention workspace.
struct BlockWs {
    int64_t q, k, v, ctx, act, ctx_len, attn, total;
};

BlockWs block_ws(int qd, int kvd, int inter, int n, int64_t attn_bytes) {
    const auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
    BlockWs w;
    w.q = 0;
    w.k = up(w.q + 4LL * qd * n);
    w.v = up(w.k + 4LL * kvd);
    w.ctx = up(w.v + 4LL * kvd);
    w.act = up(w.ctx + 4LL * qd * n);
    w.ctx_len = up(w.act + 4LL * inter * n);
    w.attn = up(w.ctx_len + 4);
    w.total = w.attn + attn_bytes;
    return w;
}

size_t block_workspace_size(int hidden_size, int q_dim, int kv_dim, int num_heads, int head_dim,
                            int inter, int max_blocks_per_seq, int n) {
    if (hidden_size <= 0 || q_dim <= 0 || kv_dim <= 0 || num_heads <= 0 || head_dim <= 0 ||
        inter <= 0 || max_blocks_per_seq <= 0 || n <= 0)
        return 0;
    const size_t attn = dlmk_paged_attention_workspace_size(1, n, num_heads, head_dim, kBlock,
                                                            max_blocks_per_seq);
    return (size_t)block_ws(q_dim, kv_dim, inter, n, (int64_t)attn).total;
}

// dlmk_decode_block_paged (n = 1) and dlmk_verify_block_paged: n consecutive
// tokens at positions num_positions .. num_positions + n - 1 (RoPE angles
// from position .. position + n - 1), x [n][hidden] in place.
int block_impl(const char *who, void *stream, int hidden_size, int q_dim, int kv_dim,
               int num_heads, int num_kv_heads, int head_dim, int inter, float rms_eps,
               int w_dtype, int w_group_size, const void *q_proj, const void *k_proj,
               const void *v_proj, const void *o_proj, const void *gate_proj, const void *up_proj,
               const void *down_proj, const float *in_norm, const float *post_norm,
               const float *q_bias, const float *k_bias, const float *v_bias,
               const float *inv_freq, float *x, void *k_pool, void *v_pool, int64_t num_blocks,
               const int32_t *block_table, int max_blocks_per_seq, int num_positions,
               int position, int n, void *workspace, size_t workspace_bytes) {
    if (hidden_size <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || inter <= 0 ||
        max_blocks_per_seq <= 0 || num_positions < 0 || num_blocks < 1 || n < 1 ||
        q_dim != num_heads * head_dim || kv_dim != num_kv_heads * head_dim ||
        num_heads % num_kv_heads != 0 || head_dim % 2 != 0)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: inconsistent sizes", who);
    if ((int64_t)num_positions + n > (int64_t)max_blocks_per_seq * kBlock)
        return dlmk::fail(DLMK_ERR_INVALID_ARG,
                          "%s: positions %d..%d beyond the block table (%d blocks)", who,
                          num_positions, num_positions + n - 1, max_blocks_per_seq);
    if (!q_proj || !k_proj || !v_proj || !o_proj || !gate_proj || !up_proj || !down_proj ||
        !in_norm || !post_norm || !inv_freq || !x || !k_pool || !v_pool || !block_table)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: null pointer", who);
    const int E = w_elems_per_chunk(w_dtype);
    if (E == 0) return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: bad weight dtype %d", who, w_dtype);
    const bool quant = w_dtype == DLMK_W_INT4 || w_dtype == DLMK_W_INT8;
    if (hidden_size % E || q_dim % E || inter % E || (quant && (w_group_size <= 0 || w_group_size % E)))
        return dlmk::fail(DLMK_ERR_UNSUPPORTED,
                          "%s: hidden %d, q_dim %d, inter %d%s must be multiples of %d", who,
                          hidden_size, q_dim, inter, quant ? " and the group size" : "", E);
    const int64_t lds_max = (int64_t)std::max(hidden_size, std::max(q_dim, inter)) * 4;
    if (lds_max > kGemvLdsMax)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED, "%s: input width %lld floats exceeds LDS", who,
                          (long long)(lds_max / 4));
    const size_t attn_need = dlmk_paged_attention_workspace_size(1, n, num_heads, head_dim, kBlock,
                                                                 max_blocks_per_seq);
    const BlockWs ws = block_ws(q_dim, kv_dim, inter, n, (int64_t)attn_need);
    if (!workspace || (int64_t)workspace_bytes < ws.total)
        return dlmk::fail(DLMK_ERR_WORKSPACE, "%s: workspace %zu bytes, need %lld", who,
                          workspace_bytes, (long long)ws.total);
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: workspace not 256-byte aligned", who);

    hipStream_t st = static_cast<hipStream_t>(stream);
    char *base = static_cast<char *>(workspace);
    float *q = reinterpret_cast<float *>(base + ws.q);
    float *k = reinterpret_cast<float *>(base + ws.k);
    float *v = reinterpret_cast<float *>(base + ws.v);
    float *ctx = reinterpret_cast<float *>(base + ws.ctx);
    float *act = reinterpret_cast<float *>(base + ws.act);
    int32_t *ctx_len = reinterpret_cast<int32_t *>(base + ws.ctx_len);
    const int gs = quant ? w_group_size : 0;

    // Attention sublayer: rmsnorm folded into the q/k/v launch's staging.
    GemvArgs qkv = gemv_args(x, hidden_size, gs, in_norm, rms_eps);
    add_seg(qkv, q_proj, nullptr, q_bias, q, q_dim, q_dim);
    add_seg(qkv, k_proj, nullptr, k_bias, k, kv_dim, 0);
    add_seg(qkv, v_proj, nullptr, v_bias, v, kv_dim, 0);
    // RoPE and the append are the launch's epilogue (rows paired per head).
    qkv.rope = RopeArgs{inv_freq, static_cast<float *>(k_pool), static_cast<float *>(v_pool),
                        block_table, num_blocks, num_kv_heads, head_dim, num_positions, position,
                        ctx_len};
    gemv(w_dtype, kRopeAppend, st, qkv, n);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return dlmk::fail((int)e, "%s launch: %s", who, hipGetErrorString(e));
    // n causal queries: token j sees positions 0 .. num_positions + j.
    const int rc = dlmk_paged_decode_attention(
        stream, ctx, DLMK_F32, q, k_pool, v_pool, DLMK_F32, block_table, ctx_len, 1, n, num_heads,
        num_kv_heads, head_dim, kBlock, max_blocks_per_seq, num_blocks,
        1.0f / sqrtf((float)head_dim), attn_need ? base + ws.attn : nullptr, attn_need);
    if (rc != DLMK_OK) return rc;
    GemvArgs oproj = gemv_args(ctx, q_dim, gs, nullptr, 0.f);
    add_seg(oproj, o_proj, nullptr, nullptr, x, hidden_size, hidden_size);
    gemv(w_dtype, kAddInto, st, oproj, n);

    // MLP sublayer (SwiGLU): the post-attention rmsnorm folded into the
    // gate/up launch's staging.
    GemvArgs gu = gemv_args(x, hidden_size, gs, post_norm, rms_eps);
    add_seg(gu, gate_proj, up_proj, nullptr, act, inter, inter);
    gemv(w_dtype, kSwiGLU, st, gu, n);
    GemvArgs down = gemv_args(act, inter, gs, nullptr, 0.f);
    add_seg(down, down_proj, nullptr, nullptr, x, hidden_size, hidden_size);
    gemv(w_dtype, kAddInto, st, down, n);
    e = hipGetLastError();
    if (e != hipSuccess) return dlmk::fail((int)e, "%s launch: %s", who, hipGetErrorString(e));
    return DLMK_OK;
}

}  // namespace

extern "C" {

size_t dlmk_decode_block_workspace_size(int hidden_size, int q_dim, int kv_dim, int num_heads,
                                        int head_dim, int inter, int max_blocks_per_seq) {
    return block_workspace_size(hidden_size, q_dim, kv_dim, num_heads, head_dim, inter,
                                max_blocks_per_seq, 1);
}

int dlmk_decode_block_paged(
    void *stream, int hidden_size, int q_dim, int kv_dim, int num_heads, int num_kv_heads,
    int head_dim, int inter, float rms_eps, int w_dtype, int w_group_size, const void *q_proj,
    const void *k_proj, const void *v_proj, const void *o_proj, const void *gate_proj,
    const void *up_proj, const void *down_proj, const float *in_norm, const float *post_norm,
    const float *q_bias, const float *k_bias, const float *v_bias, const float *inv_freq,
    float *x, void *k_pool, void *v_pool, int64_t num_blocks, const int32_t *block_table,
    int max_blocks_per_seq, int num_positions, int position, void *workspace,
    size_t workspace_bytes) {
    return block_impl("dlmk_decode_block_paged", stream, hidden_size, q_dim, kv_dim, num_heads,
                      num_kv_heads, head_dim, inter, rms_eps, w_dtype, w_group_size, q_proj,
                      k_proj, v_proj, o_proj, gate_proj, up_proj, down_proj, in_norm, post_norm,
                      q_bias, k_bias, v_bias, inv_freq, x, k_pool, v_pool, num_blocks,
                      block_table, max_blocks_per_seq, num_positions, position, 1, workspace,
                      workspace_bytes);
}

size_t dlmk_verify_block_workspace_size(int hidden_size, int q_dim, int kv_dim, int num_heads,
                                        int head_dim, int inter, int max_blocks_per_seq,
                                        int num_tokens) {
    return block_workspace_size(hidden_size, q_dim, kv_dim, num_heads, head_dim, inter,
                                max_blocks_per_seq, num_tokens);
}

int dlmk_verify_block_paged(
    void *stream, int hidden_size, int q_dim, int kv_dim, int num_heads, int num_kv_heads,
    int head_dim, int inter, float rms_eps, int w_dtype, int w_group_size, const void *q_proj,
    const void *k_proj, const void *v_proj, const void *o_proj, const void *gate_proj,
    const void *up_proj, const void *down_proj, const float *in_norm, const float *post_norm,
    const float *q_bias, const float *k_bias, const float *v_bias, const float *inv_freq,
    float *x, void *k_pool, void *v_pool, int64_t num_blocks, const int32_t *block_table,
    int max_blocks_per_seq, int num_positions, int position, int num_tokens, void *workspace,
    size_t workspace_bytes) {
    return block_impl("dlmk_verify_block_paged", stream, hidden_size, q_dim, kv_dim, num_heads,
                      num_kv_heads, head_dim, inter, rms_eps, w_dtype, w_group_size, q_proj,
                      k_proj, v_proj, o_proj, gate_proj, up_proj, down_proj, in_norm, post_norm,
                      q_bias, k_bias, v_bias, inv_freq, x, k_pool, v_pool, num_blocks,
                      block_table, max_blocks_per_seq, num_positions, position, num_tokens,
                      workspace, workspace_bytes);
}

}  // extern "C"
