// Instantiations of the attention kernel for int8 (codes + fp32 row scales) K/V caches (icl_attention_kernel.h).
#include "icl_attention_kernel.h"

namespace nori {
namespace attn {

int launch_i8(int dp, int mode, int nw, const Args& a, hipStream_t stream) {
    return launch_dtype<NORI_I8>(dp, mode, nw, a, stream);
}

namespace {

template <int DP, int MODE>
int occupancy(int nw) {
    int n = 0;
    hipError_t e;
    if constexpr (has_16_waves(DP, MODE)) {
        if (nw == 16) {
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, icl_attention_kernel<DP, NORI_I8, MODE, 16>, 16 * 64, 0);
            return e == hipSuccess ? n : 1;
        }
    }
    if constexpr (has_5_waves(DP)) {
        if (nw == 5) {
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, icl_attention_kernel<DP, NORI_I8, MODE, 5>, 5 * 64, 0);
            return e == hipSuccess ? n : 1;
        }
    }
    if (nw == 8) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, icl_attention_kernel<DP, NORI_I8, MODE, 8>, 8 * 64, 0);
    else e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, icl_attention_kernel<DP, NORI_I8, MODE, 2>, 2 * 64, 0);
    return e == hipSuccess ? n : 1;
}

template <int DP, int OTHER>
int occupancy_of(int mode, int nw) {
    return mode == kFold ? occupancy<DP, kFold>(nw) : occupancy<DP, OTHER>(nw);
}

}  // namespace

int resident_workgroups(int dp, int mode, int nw) {
    // cached per shape: the answer depends only on the compiled kernel and the device
    static int cache[8][2][4] = {};
    const int di = dp / 16 - 1, ni = nw == 16 ? 2 : (nw == 8 ? 1 : (nw == 5 ? 3 : 0));
    if (di < 0 || di > 7 || mode < 0 || mode > 1) return 1;
    int& slot = cache[di][mode][ni];
    if (slot == 0) {
        switch (dp) {
            case 16: slot = occupancy_of<16, kValu>(mode, nw); break;
            case 32: slot = occupancy_of<32, kValu>(mode, nw); break;
            case 48: slot = occupancy_of<48, kValu>(mode, nw); break;
            case 64: slot = occupancy_of<64, kValu>(mode, nw); break;
            case 80: slot = occupancy_of<80, kValu>(mode, nw); break;
            case 96: slot = occupancy_of<96, kValu>(mode, nw); break;
            case 112: slot = occupancy_of<112, kValu>(mode, nw); break;
            default: slot = occupancy_of<128, kValu>(mode, nw); break;
        }
        if (slot <= 0) slot = 1;
    }
    return slot;
}

}  // namespace attn
}  // namespace nori
