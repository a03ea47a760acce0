// Paged decode attention over bf16 pools (matrix-core kernel): instantiates and launches
// the kernels of attention_kernels.h for the supported head dims.
#include "attention_kernels.h"

namespace dlmk_attn {

int dispatch_bf16(const Args &a, int head_dim) {
    const int gqa = a.Hq / a.Hkv;
    switch (head_dim) {
        case 64: return dispatch_mfma<CodecBF16, 64>(a, gqa);
        case 128: return dispatch_mfma<CodecBF16, 128>(a, gqa);
        case 256: return dispatch_mfma<CodecBF16, 256>(a, gqa);
        default: return bad_dim(head_dim, "64, 128, 256");
    }
}

}  // namespace dlmk_attn
