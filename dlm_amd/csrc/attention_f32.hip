// Paged decode attention over f32 pools (dlm's KV dtype, KvStore::Full,
// src/forward/cpu.rs:641-650): the generic matrix-core kernel of
// attention_kernels.h (v_mfma_f32_16x16x4_f32), any head dim that is a
// multiple of 4 up to 256 and any GQA group / query count.
#include "attention_kernels.h"

namespace dlmk_attn {

int dispatch_f32(const Args &a, int head_dim) {
    const int rc = dispatch_generic<float>(a);
    return rc == -1 ? bad_dim(head_dim, "multiples of 4 up to 256") : rc;
}

}  // namespace dlmk_attn
