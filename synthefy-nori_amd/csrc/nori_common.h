// Shared device helpers and host-side status plumbing for libnori_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nori_hip.h"

namespace nori {

// ---------------------------------------------------------------- host status
// Records a formatted message for nori_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the thread-local message.
void clear_error();
// Maps the last launch error of this thread to a status (NORI_OK when none).
int launch_status(const char* what);

inline int dtype_size(int dt) {
    switch (dt) {
        case NORI_F32: return 4;
        case NORI_F16: return 2;
        case NORI_BF16: return 2;
        case NORI_I8: return 1;
        default: return 0;
    }
}

// Compute units of the current device (256 on MI355X; that when the query fails).
inline int device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
    return cus;
}

inline const char* dtype_name(int dt) {
    switch (dt) {
        case NORI_F32: return "float32";
        case NORI_F16: return "float16";
        case NORI_BF16: return "bfloat16";
        case NORI_I8: return "int8";
        default: return "unknown";
    }
}

// ---------------------------------------------------------------- device types
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- conversions
// All float -> 16-bit conversions round to nearest even (the hardware default mode),
// which is what torch's .to(dtype) and its per-op result rounding do.
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Hides an fp32 value from instruction selection. The backend otherwise folds a multiply
// (or fma) followed by a narrowing to fp16 into one v_fma_mixlo_f16, which rounds the exact
// product straight to fp16; torch rounds it to fp32 first and then to fp16.
__device__ __forceinline__ float pin_f32(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    __bf16 h = (__bf16)pin_f32(f);
    return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    _Float16 h = (_Float16)pin_f32(f);
    return __builtin_bit_cast(uint16_t, h);
}

template <int DT>
__device__ __forceinline__ float load_elem(const void* p, int64_t i) {
    if constexpr (DT == NORI_F32) return reinterpret_cast<const float*>(p)[i];
    else if constexpr (DT == NORI_F16) return f16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    else return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void store_elem(void* p, int64_t i, float v) {
    if constexpr (DT == NORI_F32) reinterpret_cast<float*>(p)[i] = v;
    else if constexpr (DT == NORI_F16) reinterpret_cast<uint16_t*>(p)[i] = f32_to_f16(v);
    else reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
}

// Round an fp32 value to dtype DT and widen it back: the per-op result rounding of torch.
template <int DT>
__device__ __forceinline__ float round_to(float v) {
    if constexpr (DT == NORI_F32) return v;
    else if constexpr (DT == NORI_F16) return f16_to_f32(f32_to_f16(v));
    else return bf16_to_f32(f32_to_bf16(v));
}

}  // namespace nori

// Dispatch a runtime float dtype onto a template parameter named DT_ (F32/F16/BF16).
#define NORI_DISPATCH_FLOAT(dt, DT_, ...)                                     \
    switch (dt) {                                                            \
        case NORI_F32: { constexpr int DT_ = NORI_F32; __VA_ARGS__; } break;  \
        case NORI_F16: { constexpr int DT_ = NORI_F16; __VA_ARGS__; } break;  \
        case NORI_BF16: { constexpr int DT_ = NORI_BF16; __VA_ARGS__; } break; \
        default: break;                                                      \
    }
