// Shared helpers of libdlmk.so (not part of the public ABI).
#pragma once

#include <cstdarg>
#include <cstdint>

namespace dlmk {

// Records a printf-style message as this thread's last error.
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

// set_error + return `code` (a DLMK_ERR_* or hipError_t value).
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// The kernels move 16 bytes a lane: operands must start on a 16-byte boundary.
inline bool aligned16(const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace dlmk
