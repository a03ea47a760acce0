// Paged decode attention over bf16 pools: the tuned matrix-core kernel for
// head dims 64, 128 and 256 with an instantiated (GQA group, queries) pair,
// the generic kernel for every other head dim that is a multiple of 8 up to
// 256 and for larger query groups.
#include "attention_kernels.h"

namespace dlmk_attn {

int dispatch_bf16(const Args &a, int head_dim) {
    const int gqa = a.Hq / a.Hkv;
    if (mfma_rows(gqa, a.NQ)) {
        switch (head_dim) {
            case 64: return dispatch_mfma<CodecBF16, 64>(a, gqa);
            case 128: return dispatch_mfma<CodecBF16, 128>(a, gqa);
            case 256: return dispatch_mfma<CodecBF16, 256>(a, gqa);
            default: break;
        }
    }
    const int rc = dispatch_generic<__bf16>(a);
    return rc == -1 ? bad_dim(head_dim, "multiples of 8 up to 256") : rc;
}

}  // namespace dlmk_attn
