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
//   rmsnorm_kernel       one 1024-thread work-group.
//   gemv_kernel          x staged once per work-group in LDS as f32; one wave
//                        per output row, 16-byte weight loads, 8 in flight per
//                        lane, wave reduction; epilogue = bias store, residual
//                        add, or (two matrices) SwiGLU.
//   rope_append_kernel   RoPE on q and k (NeoX split-half, host-computed
//                        inv_freq), then the new token's K and V straight into
//                        the pools at the slot the block table gives; also
//                        writes the context length the attention reads.
// Attention is dlmk_paged_decode_attention (f32 pools).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "dlmk.h"
#include "dlmk_internal.h"

namespace {

constexpr int kBlock = 16;  // tokens per KV block
constexpr int kGemvWaves = 4;
constexpr int kGemvUnroll = 8;  // 16-byte weight loads in flight per lane

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
// rmsnorm (src/forward/cpu.rs:934-943): out = x * (1 / sqrt(mean(x^2) + eps)) * w.
// ---------------------------------------------------------------------------
constexpr int kNormThreads = 1024;

__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float *__restrict__ x,
                                                               const float *__restrict__ w,
                                                               float *__restrict__ out, int n,
                                                               float eps) {
    __shared__ float part[kNormThreads / 64];
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += kNormThreads) ss += x[i] * x[i];
    ss = wave_sum<64>(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < kNormThreads / 64; ++i) tot += part[i];
    const float inv = 1.0f / sqrtf(tot / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += kNormThreads) out[i] = x[i] * inv * w[i];
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

enum Epilogue { kStoreBias = 0, kAddInto = 1, kSwiGLU = 2 };

// out_dim rows of a row-major [out_dim][in_dim] matrix W (and, for SwiGLU, of
// a second matrix W2) times x.  Work-group: kGemvWaves waves; x is staged in
// LDS once; wave w of work-group b takes rows (b * kGemvWaves + w) +
// k * gridDim.x * kGemvWaves.  Epilogues: kStoreBias out[o] = dot (+ bias[o]);
// kAddInto out[o] += dot (the residual); kSwiGLU out[o] = silu(dot) * dot2.
template <int DT, int EPI>
__global__ __launch_bounds__(64 * kGemvWaves) void gemv_kernel(
    const uint8_t *__restrict__ W, const uint8_t *__restrict__ W2, const float *__restrict__ x,
    const float *__restrict__ bias, float *__restrict__ out, int out_dim, int in_dim, int gs) {
    using C = WChunk<DT>;
    constexpr int E = C::E;
    extern __shared__ float xs[];
    for (int i = threadIdx.x; i < in_dim; i += 64 * kGemvWaves) xs[i] = x[i];
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t n = (int64_t)out_dim * in_dim;
    const QOffsets qo = qoffsets(DT, n, gs);
    const int chunks = in_dim / E;
    const int64_t row_bytes = (int64_t)in_dim * 16 / E;
    for (int o = blockIdx.x * kGemvWaves + wave; o < out_dim; o += gridDim.x * kGemvWaves) {
        const u32x4 *wr = reinterpret_cast<const u32x4 *>(W + o * row_bytes);
        const u32x4 *wr2 = EPI == kSwiGLU ? reinterpret_cast<const u32x4 *>(W2 + o * row_bytes)
                                          : nullptr;
        float s = 0.f, s2 = 0.f;
        for (int c0 = 0; c0 < chunks; c0 += 64 * kGemvUnroll) {
            u32x4 r[kGemvUnroll], r2[kGemvUnroll];
#pragma unroll
            for (int u = 0; u < kGemvUnroll; ++u) {
                const int c = min(c0 + u * 64 + lane, chunks - 1);
                r[u] = stream_load(wr + c);
                if constexpr (EPI == kSwiGLU) r2[u] = stream_load(wr2 + c);
            }
#pragma unroll
            for (int u = 0; u < kGemvUnroll; ++u) {
                const int c = c0 + u * 64 + lane;
                if (c < chunks) {
                    const int64_t i0 = (int64_t)o * in_dim + (int64_t)c * E;
                    s += C::dot(r[u], xs + c * E, W, qo.scales, qo.zeros, gs, i0);
                    if constexpr (EPI == kSwiGLU)
                        s2 += C::dot(r2[u], xs + c * E, W2, qo.scales, qo.zeros, gs, i0);
                }
            }
        }
        s = wave_sum<64>(s);
        if constexpr (EPI == kSwiGLU) s2 = wave_sum<64>(s2);
        if (lane == 0) {
            if constexpr (EPI == kStoreBias) {
                out[o] = s + (bias ? bias[o] : 0.f);
            } else if constexpr (EPI == kAddInto) {
                out[o] = out[o] + s;
            } else {
                out[o] = s / (1.0f + expf(-s)) * s2;  // silu(gate) * up, src/forward/cpu.rs:960-975
            }
        }
    }
}

// ---------------------------------------------------------------------------
// RoPE (rope_inplace, src/forward/cpu.rs:1094-1114) on q in place and on k,
// then the token's K (rotated) and V go to position num_positions of the
// sequence: block table[p / 16], offset p % 16, in the f32 pool layouts
// K [blk][Hkv][d/4][16][4], V [blk][Hkv][d][16].  A block id outside the pool
// is skipped (the attention masks it).  Thread 0 writes the context length.
// ---------------------------------------------------------------------------
__global__ void rope_append_kernel(float *__restrict__ q, const float *__restrict__ k,
                                   const float *__restrict__ v, const float *__restrict__ inv_freq,
                                   float *__restrict__ k_pool, float *__restrict__ v_pool,
                                   const int32_t *__restrict__ table, int64_t num_blocks,
                                   int num_heads, int num_kv_heads, int head_dim, int num_positions,
                                   int position, int32_t *__restrict__ ctx_len) {
    const int half = head_dim / 2;
    const int nq = num_heads * half, nk = num_kv_heads * half, nv = num_kv_heads * head_dim;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx == 0) *ctx_len = num_positions + 1;
    const int64_t blk = table[num_positions / kBlock];
    const int t = num_positions % kBlock;
    const bool in_pool = blk >= 0 && blk < num_blocks;
    const int64_t tile = (int64_t)head_dim * kBlock;
    if (idx < nq + nk) {
        const bool is_q = idx < nq;
        const int r = is_q ? idx : idx - nq;
        const int h = r / half, i = r % half;
        const float ang = (float)position * inv_freq[i];
        const float sn = sinf(ang), cs = cosf(ang);
        const float *src = is_q ? q : k;
        const float a = src[h * head_dim + i], b = src[h * head_dim + i + half];
        const float ra = a * cs - b * sn, rb = a * sn + b * cs;
        if (is_q) {
            q[h * head_dim + i] = ra;
            q[h * head_dim + i + half] = rb;
        } else if (in_pool) {
            float *kt = k_pool + (blk * num_kv_heads + h) * tile;
            kt[((i / 4) * kBlock + t) * 4 + i % 4] = ra;
            kt[(((i + half) / 4) * kBlock + t) * 4 + (i + half) % 4] = rb;
        }
    } else if (idx < nq + nk + nv && in_pool) {
        const int r = idx - nq - nk;
        const int h = r / head_dim, j = r % head_dim;
        v_pool[(blk * num_kv_heads + h) * tile + (int64_t)j * kBlock + t] = v[r];
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

int gemv_grid(int out_dim) {
    return std::max(1, std::min((out_dim + kGemvWaves - 1) / kGemvWaves, 1024));
}

template <int DT>
void launch_gemv(int epi, hipStream_t st, const void *W, const void *W2, const float *x,
                 const float *bias, float *out, int out_dim, int in_dim, int gs) {
    const size_t lds = (size_t)in_dim * sizeof(float);
    const auto *w = static_cast<const uint8_t *>(W);
    const auto *w2 = static_cast<const uint8_t *>(W2);
    const dim3 grid(gemv_grid(out_dim)), block(64 * kGemvWaves);
    if (epi == kStoreBias)
        hipLaunchKernelGGL((gemv_kernel<DT, kStoreBias>), grid, block, lds, st, w, w2, x, bias, out,
                           out_dim, in_dim, gs);
    else if (epi == kAddInto)
        hipLaunchKernelGGL((gemv_kernel<DT, kAddInto>), grid, block, lds, st, w, w2, x, bias, out,
                           out_dim, in_dim, gs);
    else
        hipLaunchKernelGGL((gemv_kernel<DT, kSwiGLU>), grid, block, lds, st, w, w2, x, bias, out,
                           out_dim, in_dim, gs);
}

void gemv(int dt, int epi, hipStream_t st, const void *W, const void *W2, const float *x,
          const float *bias, float *out, int out_dim, int in_dim, int gs) {
    switch (dt) {
        case DLMK_W_F32: launch_gemv<DLMK_W_F32>(epi, st, W, W2, x, bias, out, out_dim, in_dim, gs); break;
        case DLMK_W_BF16: launch_gemv<DLMK_W_BF16>(epi, st, W, W2, x, bias, out, out_dim, in_dim, gs); break;
        case DLMK_W_F16: launch_gemv<DLMK_W_F16>(epi, st, W, W2, x, bias, out, out_dim, in_dim, gs); break;
        case DLMK_W_INT4: launch_gemv<DLMK_W_INT4>(epi, st, W, W2, x, bias, out, out_dim, in_dim, gs); break;
        default: launch_gemv<DLMK_W_INT8>(epi, st, W, W2, x, bias, out, out_dim, in_dim, gs); break;
    }
}

// Workspace regions, each on a 256-byte boundary: normed[H], q[qd], k[kvd],
// v[kvd], ctx[qd], act[inter], ctx_len (int32), then the attention workspace.
struct BlockWs {
    int64_t normed, q, k, v, ctx, act, ctx_len, attn, total;
};

BlockWs block_ws(int H, int qd, int kvd, int inter, int64_t attn_bytes) {
    const auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
    BlockWs w;
    w.normed = 0;
    w.q = up(w.normed + 4LL * H);
    w.k = up(w.q + 4LL * qd);
    w.v = up(w.k + 4LL * kvd);
    w.ctx = up(w.v + 4LL * kvd);
    w.act = up(w.ctx + 4LL * qd);
    w.ctx_len = up(w.act + 4LL * inter);
    w.attn = up(w.ctx_len + 4);
    w.total = w.attn + attn_bytes;
    return w;
}

}  // namespace

extern "C" {

size_t dlmk_decode_block_workspace_size(int hidden_size, int q_dim, int kv_dim, int num_heads,
                                        int head_dim, int inter, int max_blocks_per_seq) {
    if (hidden_size <= 0 || q_dim <= 0 || kv_dim <= 0 || num_heads <= 0 || head_dim <= 0 ||
        inter <= 0 || max_blocks_per_seq <= 0)
        return 0;
    const size_t attn = dlmk_paged_attention_workspace_size(1, 1, num_heads, head_dim, kBlock,
                                                            max_blocks_per_seq);
    return (size_t)block_ws(hidden_size, q_dim, kv_dim, inter, (int64_t)attn).total;
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
    static const char *who = "dlmk_decode_block_paged";
    if (hidden_size <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || inter <= 0 ||
        max_blocks_per_seq <= 0 || num_positions < 0 || num_blocks < 1 ||
        q_dim != num_heads * head_dim || kv_dim != num_kv_heads * head_dim ||
        num_heads % num_kv_heads != 0 || head_dim % 2 != 0)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: inconsistent sizes", who);
    if ((int64_t)num_positions + 1 > (int64_t)max_blocks_per_seq * kBlock)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: position %d beyond the block table (%d blocks)",
                          who, num_positions, max_blocks_per_seq);
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
    if (lds_max > 64 * 1024)
        return dlmk::fail(DLMK_ERR_UNSUPPORTED, "%s: input width %lld floats exceeds LDS", who,
                          (long long)(lds_max / 4));
    const size_t attn_need = dlmk_paged_attention_workspace_size(1, 1, num_heads, head_dim, kBlock,
                                                                 max_blocks_per_seq);
    const BlockWs ws = block_ws(hidden_size, q_dim, kv_dim, inter, (int64_t)attn_need);
    if (!workspace || (int64_t)workspace_bytes < ws.total)
        return dlmk::fail(DLMK_ERR_WORKSPACE, "%s: workspace %zu bytes, need %lld", who,
                          workspace_bytes, (long long)ws.total);
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: workspace not 256-byte aligned", who);

    hipStream_t st = static_cast<hipStream_t>(stream);
    char *base = static_cast<char *>(workspace);
    float *normed = reinterpret_cast<float *>(base + ws.normed);
    float *q = reinterpret_cast<float *>(base + ws.q);
    float *k = reinterpret_cast<float *>(base + ws.k);
    float *v = reinterpret_cast<float *>(base + ws.v);
    float *ctx = reinterpret_cast<float *>(base + ws.ctx);
    float *act = reinterpret_cast<float *>(base + ws.act);
    int32_t *ctx_len = reinterpret_cast<int32_t *>(base + ws.ctx_len);
    const int gs = quant ? w_group_size : 0;

    // Attention sublayer.
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(kNormThreads), 0, st, x, in_norm, normed,
                       hidden_size, rms_eps);
    gemv(w_dtype, kStoreBias, st, q_proj, nullptr, normed, q_bias, q, q_dim, hidden_size, gs);
    gemv(w_dtype, kStoreBias, st, k_proj, nullptr, normed, k_bias, k, kv_dim, hidden_size, gs);
    gemv(w_dtype, kStoreBias, st, v_proj, nullptr, normed, v_bias, v, kv_dim, hidden_size, gs);
    const int rope_threads = (num_heads + num_kv_heads) * (head_dim / 2) + kv_dim;
    hipLaunchKernelGGL(rope_append_kernel, dim3((rope_threads + 255) / 256), dim3(256), 0, st, q,
                       k, v, inv_freq, static_cast<float *>(k_pool), static_cast<float *>(v_pool),
                       block_table, num_blocks, num_heads, num_kv_heads, head_dim, num_positions,
                       position, ctx_len);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return dlmk::fail((int)e, "%s launch: %s", who, hipGetErrorString(e));
    const int rc = dlmk_paged_decode_attention(
        stream, ctx, DLMK_F32, q, k_pool, v_pool, DLMK_F32, block_table, ctx_len, 1, 1, num_heads,
        num_kv_heads, head_dim, kBlock, max_blocks_per_seq, num_blocks,
        1.0f / sqrtf((float)head_dim), attn_need ? base + ws.attn : nullptr, attn_need);
    if (rc != DLMK_OK) return rc;
    gemv(w_dtype, kAddInto, st, o_proj, nullptr, ctx, nullptr, x, hidden_size, q_dim, gs);

    // MLP sublayer (SwiGLU).
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(kNormThreads), 0, st, x, post_norm, normed,
                       hidden_size, rms_eps);
    gemv(w_dtype, kSwiGLU, st, gate_proj, up_proj, normed, nullptr, act, inter, hidden_size, gs);
    gemv(w_dtype, kAddInto, st, down_proj, nullptr, act, nullptr, x, hidden_size, inter, gs);
    e = hipGetLastError();
    if (e != hipSuccess) return dlmk::fail((int)e, "%s launch: %s", who, hipGetErrorString(e));
    return DLMK_OK;
}

}  // extern "C"
