// Instantiations of the attention kernel for int8 (codes + fp32 row scales) K/V caches (icl_attention_kernel.h).
#include "icl_attention_kernel.h"

namespace nori {
namespace attn {

int launch_i8(int dp, bool ones, int nw, const Args& a, hipStream_t stream) {
    return launch_dtype<NORI_I8>(dp, ones, nw, a, stream);
}

namespace {

template <int DP, bool ONES>
int occupancy(int nw) {
    int n = 0;
    hipError_t e;
    if constexpr (DP <= 48) {
        if (nw == 16) {
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, icl_attention_kernel<DP, NORI_I8, ONES, 16>, 16 * 64, 0);
            return e == hipSuccess ? n : 1;
        }
    }
    if (nw == 8) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, icl_attention_kernel<DP, NORI_I8, ONES, 8>, 8 * 64, 0);
    else e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, icl_attention_kernel<DP, NORI_I8, ONES, 2>, 2 * 64, 0);
    return e == hipSuccess ? n : 1;
}

}  // namespace

int resident_workgroups(int dp, bool ones, int nw) {
    // cached per shape: the answer depends only on the compiled kernel and the device
    static int cache[8][2][3] = {};
    const int di = dp / 16 - 1, oi = ones ? 1 : 0, ni = nw == 16 ? 2 : (nw == 8 ? 1 : 0);
    if (di < 0 || di > 7) return 1;
    int& slot = cache[di][oi][ni];
    if (slot == 0) {
        switch (dp) {
            case 16: slot = occupancy<16, true>(nw); break;
            case 32: slot = ones ? occupancy<32, true>(nw) : occupancy<32, false>(nw); break;
            case 48: slot = occupancy<48, true>(nw); break;
            case 64: slot = ones ? occupancy<64, true>(nw) : occupancy<64, false>(nw); break;
            case 80: slot = occupancy<80, true>(nw); break;
            case 96: slot = ones ? occupancy<96, true>(nw) : occupancy<96, false>(nw); break;
            case 112: slot = occupancy<112, true>(nw); break;
            default: slot = ones ? occupancy<128, true>(nw) : occupancy<128, false>(nw); break;
        }
        if (slot <= 0) slot = 1;
    }
    return slot;
}

}  // namespace attn
}  // namespace nori
