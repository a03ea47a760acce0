// Block copy (fork / copy-on-write) and swap gather/scatter.
//
// No counterpart exists in the reference: dlm forks a sequence by deep-cloning
// its contiguous KvLayerCache (KvSnapshot, src/forward/orchestrator.rs:73-105)
// and has no KV swap (src/swap plans weight windows).  Here a fork copies whole
// physical blocks, and swap moves blocks through a contiguous device staging
// buffer so the PCIe transfer is one large hipMemcpyAsync.
//
// All three kernels are byte moves of `block_bytes` per (item, pool): one
// work-group per (item, pool) streams the block in 16-byte chunks, each thread
// keeping kUnroll loads in flight before it stores.

#include <hip/hip_runtime.h>

#include "dlmk.h"
#include "dlmk_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void move_block(char *__restrict__ dst, const char *__restrict__ src,
                                           int64_t chunks) {
    const u32x4 *s = reinterpret_cast<const u32x4 *>(src);
    u32x4 *d = reinterpret_cast<u32x4 *>(dst);
    int64_t c = threadIdx.x;
    for (; c + (kUnroll - 1) * kThreads < chunks; c += kUnroll * kThreads) {
        u32x4 r[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) r[u] = __builtin_nontemporal_load(s + c + u * kThreads);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) __builtin_nontemporal_store(r[u], d + c + u * kThreads);
    }
    for (; c < chunks; c += kThreads) __builtin_nontemporal_store(__builtin_nontemporal_load(s + c), d + c);
}

// blockIdx.x = pair index, blockIdx.y = pool (0 = K, 1 = V).
__global__ __launch_bounds__(kThreads) void copy_blocks_kernel(char *k_pool, char *v_pool,
                                                               const int32_t *__restrict__ pairs,
                                                               int64_t block_bytes,
                                                               int64_t num_blocks) {
    const int64_t i = blockIdx.x;
    const int64_t src = pairs[2 * i], dst = pairs[2 * i + 1];
    if (src < 0 || src >= num_blocks || dst < 0 || dst >= num_blocks || src == dst) return;
    char *pool = blockIdx.y ? v_pool : k_pool;
    move_block(pool + dst * block_bytes, pool + src * block_bytes, block_bytes / 16);
}

// staging[i][pool] <- pool[ids[i]]
__global__ __launch_bounds__(kThreads) void gather_blocks_kernel(char *__restrict__ staging,
                                                                 const char *k_pool,
                                                                 const char *v_pool,
                                                                 const int32_t *__restrict__ ids,
                                                                 int64_t block_bytes,
                                                                 int64_t num_blocks) {
    const int64_t i = blockIdx.x;
    const int64_t id = ids[i];
    if (id < 0 || id >= num_blocks) return;
    const char *pool = blockIdx.y ? v_pool : k_pool;
    move_block(staging + (2 * i + blockIdx.y) * block_bytes, pool + id * block_bytes,
               block_bytes / 16);
}

// pool[ids[i]] <- staging[i][pool]
__global__ __launch_bounds__(kThreads) void scatter_blocks_kernel(char *k_pool, char *v_pool,
                                                                  const char *__restrict__ staging,
                                                                  const int32_t *__restrict__ ids,
                                                                  int64_t block_bytes,
                                                                  int64_t num_blocks) {
    const int64_t i = blockIdx.x;
    const int64_t id = ids[i];
    if (id < 0 || id >= num_blocks) return;
    char *pool = blockIdx.y ? v_pool : k_pool;
    move_block(pool + id * block_bytes, staging + (2 * i + blockIdx.y) * block_bytes,
               block_bytes / 16);
}

int check(const char *who, int64_t n, size_t block_bytes, int64_t num_blocks) {
    if (n < 0 || num_blocks < 0)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: negative count", who);
    if (block_bytes == 0 || block_bytes % 16 != 0)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "%s: block_bytes %zu is not a positive multiple of 16",
                          who, block_bytes);
    if (n > 0x7fffffff) return dlmk::fail(DLMK_ERR_UNSUPPORTED, "%s: too many blocks", who);
    return DLMK_OK;
}

int launched(const char *who) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return dlmk::fail((int)e, "%s launch: %s", who, hipGetErrorString(e));
    return DLMK_OK;
}

}  // namespace

extern "C" {

int dlmk_copy_blocks(void *stream, void *k_pool, void *v_pool, const int32_t *pairs, int64_t n,
                     size_t block_bytes, int64_t num_blocks) {
    if (int rc = check("dlmk_copy_blocks", n, block_bytes, num_blocks)) return rc;
    if (n == 0) return DLMK_OK;
    if (!k_pool || !v_pool || !pairs)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_copy_blocks: null pointer");
    if (!dlmk::aligned16(k_pool) || !dlmk::aligned16(v_pool))
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_copy_blocks: pools and staging must be 16-byte aligned");
    hipLaunchKernelGGL(copy_blocks_kernel, dim3((unsigned)n, 2), dim3(kThreads), 0,
                       (hipStream_t)stream, (char *)k_pool, (char *)v_pool, pairs,
                       (int64_t)block_bytes, num_blocks);
    return launched("dlmk_copy_blocks");
}

int dlmk_gather_blocks(void *stream, void *staging, const void *k_pool, const void *v_pool,
                       const int32_t *block_ids, int64_t n, size_t block_bytes,
                       int64_t num_blocks) {
    if (int rc = check("dlmk_gather_blocks", n, block_bytes, num_blocks)) return rc;
    if (n == 0) return DLMK_OK;
    if (!staging || !k_pool || !v_pool || !block_ids)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_gather_blocks: null pointer");
    if (!dlmk::aligned16(staging) || !dlmk::aligned16(k_pool) || !dlmk::aligned16(v_pool))
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_gather_blocks: pools and staging must be 16-byte aligned");
    hipLaunchKernelGGL(gather_blocks_kernel, dim3((unsigned)n, 2), dim3(kThreads), 0,
                       (hipStream_t)stream, (char *)staging, (const char *)k_pool,
                       (const char *)v_pool, block_ids, (int64_t)block_bytes, num_blocks);
    return launched("dlmk_gather_blocks");
}

int dlmk_scatter_blocks(void *stream, void *k_pool, void *v_pool, const void *staging,
                        const int32_t *block_ids, int64_t n, size_t block_bytes,
                        int64_t num_blocks) {
    if (int rc = check("dlmk_scatter_blocks", n, block_bytes, num_blocks)) return rc;
    if (n == 0) return DLMK_OK;
    if (!staging || !k_pool || !v_pool || !block_ids)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_scatter_blocks: null pointer");
    if (!dlmk::aligned16(staging) || !dlmk::aligned16(k_pool) || !dlmk::aligned16(v_pool))
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_scatter_blocks: pools and staging must be 16-byte aligned");
    hipLaunchKernelGGL(scatter_blocks_kernel, dim3((unsigned)n, 2), dim3(kThreads), 0,
                       (hipStream_t)stream, (char *)k_pool, (char *)v_pool,
                       (const char *)staging, block_ids, (int64_t)block_bytes, num_blocks);
    return launched("dlmk_scatter_blocks");
}

int dlmk_swap_out(void *stream, void *host_buf, const void *k_pool, const void *v_pool,
                  const int32_t *block_ids, int64_t n, size_t block_bytes, int64_t num_blocks,
                  void *dev_staging, size_t staging_bytes) {
    if (int rc = check("dlmk_swap_out", n, block_bytes, num_blocks)) return rc;
    if (n == 0) return DLMK_OK;
    const size_t bytes = 2 * (size_t)n * block_bytes;
    if (!host_buf || !dev_staging)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_swap_out: null buffer");
    if (staging_bytes < bytes)
        return dlmk::fail(DLMK_ERR_WORKSPACE, "dlmk_swap_out: staging holds %zu bytes, need %zu",
                          staging_bytes, bytes);
    if (int rc = dlmk_gather_blocks(stream, dev_staging, k_pool, v_pool, block_ids, n,
                                    block_bytes, num_blocks))
        return rc;
    hipError_t e = hipMemcpyAsync(host_buf, dev_staging, bytes, hipMemcpyDeviceToHost,
                                  (hipStream_t)stream);
    if (e != hipSuccess) return dlmk::fail((int)e, "dlmk_swap_out copy: %s", hipGetErrorString(e));
    return DLMK_OK;
}

int dlmk_swap_in(void *stream, void *k_pool, void *v_pool, const void *host_buf,
                 const int32_t *block_ids, int64_t n, size_t block_bytes, int64_t num_blocks,
                 void *dev_staging, size_t staging_bytes) {
    if (int rc = check("dlmk_swap_in", n, block_bytes, num_blocks)) return rc;
    if (n == 0) return DLMK_OK;
    const size_t bytes = 2 * (size_t)n * block_bytes;
    if (!host_buf || !dev_staging)
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_swap_in: null buffer");
    if (staging_bytes < bytes)
        return dlmk::fail(DLMK_ERR_WORKSPACE, "dlmk_swap_in: staging holds %zu bytes, need %zu",
                          staging_bytes, bytes);
    hipError_t e = hipMemcpyAsync(dev_staging, host_buf, bytes, hipMemcpyHostToDevice,
                                  (hipStream_t)stream);
    if (e != hipSuccess) return dlmk::fail((int)e, "dlmk_swap_in copy: %s", hipGetErrorString(e));
    return dlmk_scatter_blocks(stream, k_pool, v_pool, dev_staging, block_ids, n, block_bytes,
                               num_blocks);
}

}  // extern "C"
