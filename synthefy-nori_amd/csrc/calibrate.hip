// Measurement only: the dense f16 MFMA rate this GPU sustains on given operand data.
//
// MI355X's 2.5 PFLOP/s dense f16 figure assumes the 2.4 GHz peak engine clock. Under a dense
// MFMA load the clock is set by the power limit, and the power an MFMA draws depends on its
// operand bits, so the rate a kernel can reach depends on its data. This kernel runs nothing
// but v_mfma_f32_32x32x16_f16, cycling through eight operand register sets per wavefront
// (read once from `operands`), so the caller can time the ceiling for random operands
// against, for example, all-zero ones. It has no counterpart in the reference.
#include "nori_common.h"

namespace {

using namespace nori;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kProbeThreads = 256;  // four wavefronts
constexpr int kProbeBlocksPerCu = 4;  // four wavefronts per SIMD

__global__ void __launch_bounds__(kProbeThreads) mfma_f16_probe_kernel(const u32x4* ops, int64_t n_vec, int iters,
                                                                     float* sink, int64_t sink_len) {
    const int lane = threadIdx.x & 63;
    u32x4 a[8], b[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        a[s] = ops[(((int64_t)blockIdx.x * 16 + s) * 64 + lane) % n_vec];
        b[s] = ops[(((int64_t)blockIdx.x * 16 + 8 + s) * 64 + lane) % n_vec];
    }
    f32x16 c[4] = {};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int s = 0; s < 8; ++s)
            c[s & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a[s]), __builtin_bit_cast(f16x8, b[s]),
                                                             c[s & 3], 0, 0, 0);
    }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc += c[0][i] + c[1][i] + c[2][i] + c[3][i];
    sink[((int64_t)blockIdx.x * kProbeThreads + threadIdx.x) % sink_len] = acc;
}

}  // namespace

extern "C" int64_t nori_mfma_f16_probe_flop(int64_t iters) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return -1;
    // workgroups x wavefronts x iterations x 8 MFMAs x 2*32*32*16 FLOP
    return (int64_t)cus * kProbeBlocksPerCu * 4 * iters * 8 * 32768;
}

extern "C" int nori_mfma_f16_probe(const void* operands, int64_t n_vec, int32_t iters, float* sink, int64_t sink_len,
                                   void* stream) {
    clear_error();
    if (!operands || !sink || n_vec <= 0 || sink_len <= 0 || iters <= 0)
        return fail(NORI_ERR_INVALID, "mfma_f16_probe: needs operands (n_vec > 0), a sink (sink_len > 0) and iters > 0");
    if ((uintptr_t)operands % 16) return fail(NORI_ERR_INVALID, "mfma_f16_probe: operands must be 16-byte aligned");
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return fail(NORI_ERR_RUNTIME, "mfma_f16_probe: cannot query the device");
    hipLaunchKernelGGL(mfma_f16_probe_kernel, dim3((unsigned)(cus * kProbeBlocksPerCu)), dim3(kProbeThreads), 0,
                       (hipStream_t)stream, reinterpret_cast<const u32x4*>(operands), n_vec, (int)iters, sink, sink_len);
    return launch_status("mfma_f16_probe");
}
