// Error reporting and pinned host memory for libdlmk.so.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>

#include "dlmk.h"
#include "dlmk_internal.h"

namespace dlmk {

static thread_local char g_last_error[512] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

}  // namespace dlmk

extern "C" {

int dlmk_abi_version(void) { return DLMK_ABI_VERSION; }

const char *dlmk_get_last_error_string(void) { return dlmk::g_last_error; }

// Page-locked host memory (PinnedBuffer::with_len, src/memory/pinned.rs:59-67):
// a zero-byte request is an error (DlmError::HostAlloc{bytes: 0}), the
// allocation is rounded up to whole 4 KiB pages, and the bytes start at zero.
int dlmk_alloc_pinned(void **ptr, size_t bytes) {
    if (!ptr) return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_alloc_pinned: null out pointer");
    *ptr = nullptr;
    if (bytes == 0) return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_alloc_pinned: zero bytes");
    constexpr size_t kPage = 4096;
    if (bytes > SIZE_MAX - (kPage - 1))
        return dlmk::fail(DLMK_ERR_INVALID_ARG, "dlmk_alloc_pinned: %zu bytes overflows", bytes);
    const size_t capacity = (bytes + kPage - 1) / kPage * kPage;
    hipError_t e = hipHostMalloc(ptr, capacity, hipHostMallocDefault);
    if (e != hipSuccess) {
        *ptr = nullptr;
        return dlmk::fail((int)e, "hipHostMalloc(%zu): %s", capacity, hipGetErrorString(e));
    }
    memset(*ptr, 0, capacity);
    return DLMK_OK;
}

int dlmk_free_pinned(void *ptr) {
    if (!ptr) return DLMK_OK;
    hipError_t e = hipHostFree(ptr);
    if (e != hipSuccess) return dlmk::fail((int)e, "hipHostFree: %s", hipGetErrorString(e));
    return DLMK_OK;
}

}  // extern "C"
