// Paged decode attention over f32 pools (VALU kernel): instantiates and launches
// the kernels of attention_kernels.h for the supported head dims.
#include "attention_kernels.h"

namespace dlmk_attn {

int dispatch_f32(const Args &a, int head_dim) {
    const int gqa = a.Hq / a.Hkv;
    switch (head_dim) {
        case 64: return dispatch_valu<64>(a, gqa);
        case 128: return dispatch_valu<128>(a, gqa);
        default: return bad_dim(head_dim, "64, 128");
    }
}

}  // namespace dlmk_attn
