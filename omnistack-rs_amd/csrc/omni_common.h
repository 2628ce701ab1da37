// Shared device/host helpers for the gfx950 codec + attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "omnistack_amd.h"

namespace omni {

// Thread-local error message (host side).
void set_error(const char *fmt, ...);

#define OMNI_CHECK_ARG(cond, ...)                   \
    do {                                            \
        if (!(cond)) {                              \
            ::omni::set_error(__VA_ARGS__);         \
            return OMNI_EINVAL;                     \
        }                                           \
    } while (0)

#define OMNI_CHECK_LAUNCH(what)                                              \
    do {                                                                     \
        hipError_t e_ = hipGetLastError();                                   \
        if (e_ != hipSuccess) {                                              \
            ::omni::set_error("%s: %s", what, hipGetErrorString(e_));        \
            return OMNI_ERUNTIME;                                            \
        }                                                                    \
    } while (0)

static inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// Compute units of the current device, queried once per device (a full
// property query costs far more than a launch; 256 if it fails).
static inline int device_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        cached[dev] = (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
                          ? n : 256;
    }
    return cached[dev];
}

// fp32 1/sqrt(D) exactly as torch forms `x * (1.0 / math.sqrt(D))` on an fp32
// tensor: the Python double is rounded to fp32 before the multiply.
static inline float inv_sqrt_dim_f32(int D) { return (float)(1.0 / __builtin_sqrt((double)D)); }

// ── element conversions (round-to-nearest-even, like torch) ─────────────

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(((uint32_t)h) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);  // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
    _Float16 h = (_Float16)f;  // IEEE conversion, round-to-nearest-even
    return __builtin_bit_cast(uint16_t, h);
}

// Load element i of a tensor of the given dtype as fp32.
__device__ __forceinline__ float load_as_f32(const void *p, int dtype, int64_t i) {
    if (dtype == OMNI_F32) return reinterpret_cast<const float *>(p)[i];
    uint16_t h = reinterpret_cast<const uint16_t *>(p)[i];
    return dtype == OMNI_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

// Round an fp32 value to `dtype` and back (identity for f32).
__device__ __forceinline__ float round_to_dtype(float v, int dtype) {
    if (dtype == OMNI_BF16) return bf16_to_f32(f32_to_bf16_rne(v));
    if (dtype == OMNI_F16) return f16_to_f32(f32_to_f16_rne(v));
    return v;
}

__device__ __forceinline__ void store_from_f32(void *p, int dtype, int64_t i, float v) {
    if (dtype == OMNI_F32) {
        reinterpret_cast<float *>(p)[i] = v;
    } else if (dtype == OMNI_BF16) {
        reinterpret_cast<uint16_t *>(p)[i] = f32_to_bf16_rne(v);
    } else {
        reinterpret_cast<uint16_t *>(p)[i] = f32_to_f16_rne(v);
    }
}

static inline int dtype_size(int dtype) { return dtype == OMNI_F32 ? 4 : 2; }
static inline bool dtype_ok(int dtype) { return dtype == OMNI_F32 || dtype == OMNI_F16 || dtype == OMNI_BF16; }
static inline bool head_dim_ok(int D) { return D == 128 || D == 32; }

}  // namespace omni
