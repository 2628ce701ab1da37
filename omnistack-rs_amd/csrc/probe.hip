// Streaming-read bandwidth probe: the HBM read rate a plain kernel reaches
// on this device, measured beside the decode kernel (which reads its packed
// cache once and writes almost nothing).  Each block XOR-folds its
// grid-stride share of 16-byte words and writes one partial, so the loads
// cannot be dropped and the result can be checked on the host: the XOR of
// all partials is the XOR of every 32-bit word of the buffer.
#include "omni_common.h"

namespace omni {

typedef uint32_t probe_u4 __attribute__((ext_vector_type(4)));
constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 8;       // independent 16-byte loads in flight per thread

__global__ __launch_bounds__(kProbeThreads) void hbm_read_kernel(const probe_u4 *__restrict__ p, int64_t n16,
                                                                  uint32_t *partials) {
    const int64_t stride = (int64_t)gridDim.x * kProbeThreads;
    int64_t i = (int64_t)blockIdx.x * kProbeThreads + threadIdx.x;
    uint32_t acc = 0u;
    for (; i + (kProbeUnroll - 1) * stride < n16; i += kProbeUnroll * stride) {
        probe_u4 v[kProbeUnroll];
#pragma unroll
        for (int k = 0; k < kProbeUnroll; ++k) v[k] = __builtin_nontemporal_load(p + i + k * stride);
#pragma unroll
        for (int k = 0; k < kProbeUnroll; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    for (; i < n16; i += stride) {
        const probe_u4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, m);
    __shared__ uint32_t wx[kProbeThreads / 64];
    if ((threadIdx.x & 63) == 0) wx[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t r = 0u;
#pragma unroll
        for (int w = 0; w < kProbeThreads / 64; ++w) r ^= wx[w];
        partials[blockIdx.x] = r;
    }
}

}  // namespace omni

using namespace omni;

extern "C" int omni_hbm_read_probe(const void *buf, size_t bytes, uint32_t *partials, int n_partials,
                                   void *stream) {
    OMNI_CHECK_ARG(n_partials >= 1 && n_partials <= (1 << 20),
                   "omni_hbm_read_probe: n_partials must be in [1, 2^20], got %d", n_partials);
    OMNI_CHECK_ARG(bytes % 16 == 0, "omni_hbm_read_probe: bytes must be a multiple of 16, got %zu", bytes);
    OMNI_CHECK_ARG(partials && (buf || bytes == 0), "omni_hbm_read_probe: NULL pointer");
    OMNI_CHECK_ARG(((uintptr_t)buf & 15u) == 0, "omni_hbm_read_probe: buffer must be 16-byte aligned");
    hipLaunchKernelGGL(hbm_read_kernel, dim3((unsigned)n_partials), dim3(kProbeThreads), 0, as_stream(stream),
                       reinterpret_cast<const probe_u4 *>(buf), (int64_t)(bytes / 16), partials);
    OMNI_CHECK_LAUNCH("omni_hbm_read_probe");
    return OMNI_OK;
}
