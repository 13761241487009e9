// Instantiations of the attention kernel for float16 K/V caches (icl_attention_kernel.h).
#include "icl_attention_kernel.h"

namespace nori {
namespace attn {

int launch_f16(int dp, int mode, int nw, const Args& a, hipStream_t stream) {
    return launch_dtype<NORI_F16>(dp, mode, nw, a, stream);
}

}  // namespace attn
}  // namespace nori
