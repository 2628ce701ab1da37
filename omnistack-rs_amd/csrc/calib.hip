// Lloyd-Max INT4 codebook calibration on the GPU (gfx950).
//
// Reference: LloydMaxCalibrator.fit (omnistack_rs/quantization/codebook.py:
// 64-108), driven per kv head by calibrate_per_group (:148-172) in the bake
// (scripts/run_criteo_benchmark.py:357-362).  Same recipe:
//   init   16 equal-count bins of the sorted samples (bin size
//          bs = n / 16; the n % 16 largest samples are in no bin), centroid
//          = mean of its bin;
//   iterate  code = first-index argmin_k fp32 |x - c_k|; c_k = mean of the
//          samples coded k (an empty cell keeps its centroid); stop after
//          max_iters or when the largest fp32 move |c_new - c_old| < tol
//          (the moved centroids are kept);
//   result sorted ascending.
// The sort is replaced by four radix-select passes (8 bits each, all 16
// order statistics x_(r*bs - 1) at once) and one pass that sums the samples
// below each of them: bin r's sum is F(r bs) - F((r-1) bs) with
// F(m) = sum(x < v) + v (m - #(x < v)) for v the m-th smallest sample.
// Sums are accumulated in fp64 per thread, then over threads and blocks in a
// fixed order, so results are deterministic; means are rounded to fp32 once.
// (The reference's fp32 `mean()` rounds along the way: its last bits can
// differ, and so can a convergence decision taken at the tolerance.)
// Samples must be finite.
//
// Layout: group g's samples are rows of `inner` contiguous elements:
// element e of group g is x[(e / inner) * outer_stride + g * group_stride +
// e % inner], e < outer * inner.  A flat vector is outer = 1; head h of a
// (B, H, T, D) cache is outer = B, inner = T*D, outer_stride = H*T*D,
// group_stride = T*D.
#include <math.h>

#include "omni_common.h"

namespace omni {

constexpr int kLmK = 16;            // centroids
constexpr int kLmThreads = 256;
constexpr int kLmMaxBlocks = 240;   // blocks per group (grid-stride)
constexpr int kLmIntervals = kLmK + 1;

struct LmArgs {
    const void *x;
    int64_t outer, inner, outer_stride, group_stride, n, bs;
    int blocks;
    int max_iters;
    float tol;
    // workspace (per group g)
    uint32_t *hist;      // [g][16][256] radix histograms of the unique prefixes
    uint32_t *prefix;    // [g][16] key prefix of each order statistic
    int64_t *krank;      // [g][16] its rank among samples with that prefix
    uint32_t *uprefix;   // [g][17]: [0] = number of unique prefixes, then the prefixes
    double *psum;        // [g][blocks][17] block partial sums
    uint64_t *pcnt;      // [g][blocks][17] block partial counts
    float *cent;         // [g][16] current centroids
    int *state;          // [g][2]: converged, iterations run
    float *out;          // [g][16]
};

__device__ __forceinline__ uint32_t lm_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float lm_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

template <int DT>
__device__ __forceinline__ float lm_load(const LmArgs &a, int64_t o, int64_t i, int g) {
    const int64_t idx = o * a.outer_stride + (int64_t)g * a.group_stride + i;
    if constexpr (DT == OMNI_F32) return reinterpret_cast<const float *>(a.x)[idx];
    const uint16_t h = reinterpret_cast<const uint16_t *>(a.x)[idx];
    if constexpr (DT == OMNI_BF16) return bf16_to_f32(h);
    return f16_to_f32(h);
}

// Visit this thread's elements of group g in a fixed order:
// e = start, start + stride, ... (grid-stride over the flattened index,
// the (row, column) pair advanced without division).
// Eight loads are issued before the eight samples are used (the loop is
// otherwise bound by one memory latency per sample).
template <int DT, typename F>
__device__ __forceinline__ void lm_for_each(const LmArgs &a, int g, F &&f) {
    constexpr int U = 8;
    const int64_t stride = (int64_t)a.blocks * kLmThreads;
    const int64_t start = (int64_t)blockIdx.x * kLmThreads + threadIdx.x;
    if (start >= a.n) return;
    const int64_t so = stride / a.inner, si = stride % a.inner;
    int64_t o = start / a.inner, i = start % a.inner;
    for (int64_t e = start; e < a.n; e += U * stride) {
        float xv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            xv[u] = e + u * stride < a.n ? lm_load<DT>(a, o, i, g) : 0.0f;
            o += so;
            i += si;
            if (i >= a.inner) {
                i -= a.inner;
                ++o;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (e + u * stride < a.n) f(xv[u]);
    }
}

__global__ void lm_clear_kernel(LmArgs a) {
    const int g = blockIdx.y;
    uint32_t *h = a.hist + (size_t)g * kLmK * 256;
    for (int s = threadIdx.x; s < kLmK * 256; s += blockDim.x) h[s] = 0u;
    if (threadIdx.x < kLmK) {
        a.prefix[g * kLmK + threadIdx.x] = 0u;
        a.krank[g * kLmK + threadIdx.x] = (int64_t)(threadIdx.x + 1) * a.bs - 1;
    }
    if (threadIdx.x == 0) {
        a.uprefix[g * (kLmK + 1)] = 1u;       // one unique (empty) prefix
        a.uprefix[g * (kLmK + 1) + 1] = 0u;
        a.state[2 * g] = 0;
        a.state[2 * g + 1] = 0;
    }
}

// Radix pass: histogram of key digit `pass` (bits 31-24 first) over the
// samples whose higher digits equal one of the unique prefixes.
template <int DT>
__global__ __launch_bounds__(kLmThreads) void lm_radix_kernel(LmArgs a, int pass) {
    const int g = blockIdx.y;
    __shared__ uint32_t lh[kLmK * 256];
    __shared__ uint32_t up[kLmK];
    const uint32_t nu = a.uprefix[g * (kLmK + 1)];
    for (int s = threadIdx.x; s < kLmK * 256; s += kLmThreads) lh[s] = 0u;
    if (threadIdx.x < kLmK) up[threadIdx.x] = a.uprefix[g * (kLmK + 1) + 1 + threadIdx.x];
    __syncthreads();
    const int shift = 24 - 8 * pass;
    lm_for_each<DT>(a, g, [&](float x) {
        const uint32_t key = lm_key(x);
        const uint32_t hi = pass == 0 ? 0u : key >> (shift + 8);
        const uint32_t dig = (key >> shift) & 0xffu;
        for (uint32_t u = 0; u < nu; ++u)
            if (up[u] == hi) {
                atomicAdd(&lh[u * 256 + dig], 1u);
                break;
            }
    });
    __syncthreads();
    uint32_t *h = a.hist + (size_t)g * kLmK * 256;
    for (int s = threadIdx.x; s < (int)nu * 256; s += kLmThreads)
        if (lh[s]) atomicAdd(&h[s], lh[s]);
}

// After a radix pass: each order statistic picks its digit (one wave per
// statistic: a prefix sum of the 256 bin counts over the lanes, four bins
// per lane), the unique prefixes for the next pass are listed, and the
// histograms are cleared.
__global__ __launch_bounds__(256) void lm_select_kernel(LmArgs a) {
    const int g = blockIdx.y;
    uint32_t *h = a.hist + (size_t)g * kLmK * 256;
    uint32_t *upg = a.uprefix + g * (kLmK + 1);
    __shared__ uint32_t newp[kLmK];
    const uint32_t nu = upg[0];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int j = w; j < kLmK; j += 4) {
        const uint32_t p = a.prefix[g * kLmK + j];
        uint32_t u = 0;
        while (u + 1 < nu && upg[1 + u] != p) ++u;
        const int64_t k = a.krank[g * kLmK + j];
        const uint4 c4 = reinterpret_cast<const uint4 *>(h + u * 256)[lane];
        const uint64_t mine = (uint64_t)c4.x + c4.y + c4.z + c4.w;
        uint64_t incl = mine;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint64_t y = __shfl_up(incl, off);
            if (lane >= off) incl += y;
        }
        // the bin holding rank k lies in the first lane whose inclusive count exceeds k
        const uint64_t over = __ballot(incl > (uint64_t)k);
        const int L = over ? __ffsll((unsigned long long)over) - 1 : 63;
        int64_t kk = k - (int64_t)__shfl(incl - mine, L);
        const uint32_t b0 = __shfl(c4.x, L), b1 = __shfl(c4.y, L), b2 = __shfl(c4.z, L);
        int d = 4 * L;
        if (kk >= (int64_t)b0) {
            kk -= b0;
            ++d;
            if (kk >= (int64_t)b1) {
                kk -= b1;
                ++d;
                if (kk >= (int64_t)b2) {
                    kk -= b2;
                    ++d;
                }
            }
        }
        if (lane == 0) {
            a.krank[g * kLmK + j] = kk;
            newp[j] = (p << 8) | (uint32_t)d;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t n = 0;
        for (int j = 0; j < kLmK; ++j) {
            a.prefix[g * kLmK + j] = newp[j];
            if (n == 0 || upg[n] != newp[j]) upg[1 + n++] = newp[j];   // prefixes ascend with j
        }
        upg[0] = n;
    }
    for (int t = threadIdx.x; t < kLmK * 256; t += blockDim.x) h[t] = 0u;
}

// Adds x to this thread's own LDS slot (fp64 sum, count).  Slots are
// private to a thread, so the additions happen in its program order (the
// same sums as register accumulators, without a 17-way select per sample).
__device__ __forceinline__ void lm_slot_add(double *sum, uint32_t *cnt, float x) {
    __hip_atomic_fetch_add(sum, (double)x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Block-wide fixed-order sum of nq (sum, count) pairs into the partials:
// an xor tree inside each wave, then the four waves in order.
__device__ __forceinline__ void lm_block_store(const LmArgs &a, int g, double (&s)[kLmIntervals],
                                               uint64_t (&c)[kLmIntervals], int nq) {
    constexpr int nwv = kLmThreads / 64;
    __shared__ double ws[nwv][kLmIntervals];
    __shared__ uint64_t wc[nwv][kLmIntervals];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1)
#pragma unroll
        for (int q = 0; q < kLmIntervals; ++q) {
            s[q] += __shfl_xor(s[q], m);
            c[q] += (uint64_t)__shfl_xor((unsigned long long)c[q], m);
        }
    if (lane == 0)
#pragma unroll
        for (int q = 0; q < kLmIntervals; ++q) {
            ws[w][q] = s[q];
            wc[w][q] = c[q];
        }
    __syncthreads();
    if (t < nq) {
        double ts = ws[0][t];
        uint64_t tc = wc[0][t];
#pragma unroll
        for (int v = 1; v < nwv; ++v) {
            ts += ws[v][t];
            tc += wc[v][t];
        }
        const size_t o = ((size_t)g * a.blocks + blockIdx.x) * kLmIntervals + t;
        a.psum[o] = ts;
        a.pcnt[o] = tc;
    }
}

// Sums and counts of the samples in each interval between the 16 order
// statistics v_0 <= ... <= v_15: interval t holds #{j : v_j <= x} = t.
template <int DT>
__global__ __launch_bounds__(kLmThreads) void lm_interval_kernel(LmArgs a) {
    const int g = blockIdx.y;
    __shared__ double ls[kLmIntervals][kLmThreads];
    __shared__ uint32_t lc[kLmIntervals][kLmThreads];
    const int th = threadIdx.x;
    float v[kLmK];
#pragma unroll
    for (int j = 0; j < kLmK; ++j) v[j] = lm_value(a.prefix[g * kLmK + j]);
#pragma unroll
    for (int q = 0; q < kLmIntervals; ++q) {
        ls[q][th] = 0.0;
        lc[q][th] = 0u;
    }
    lm_for_each<DT>(a, g, [&](float x) {
        int t = 0;
#pragma unroll
        for (int j = 0; j < kLmK; ++j) t += v[j] <= x ? 1 : 0;
        lm_slot_add(&ls[t][th], &lc[t][th], x);
    });
    double s[kLmIntervals];
    uint64_t c[kLmIntervals];
#pragma unroll
    for (int q = 0; q < kLmIntervals; ++q) {
        s[q] = ls[q][th];
        c[q] = lc[q][th];
    }
    lm_block_store(a, g, s, c, kLmIntervals);
}

// Initial centroids from the order statistics and the interval sums
// (thread t < 255 sums interval t / 15 over blocks t % 15, t % 15 + 15, ...;
// the 15 partial sums of an interval are then added in order).
__global__ __launch_bounds__(256) void lm_init_kernel(LmArgs a) {
    const int g = blockIdx.y;
    constexpr int kParts = 15;
    __shared__ double ps[kLmIntervals][kParts];
    __shared__ uint64_t pc[kLmIntervals][kParts];
    const int t = threadIdx.x;
    if (t < kLmIntervals * kParts) {
        const int q = t / kParts, part = t % kParts;
        double s = 0.0;
        uint64_t n = 0;
        for (int bl = part; bl < a.blocks; bl += kParts) {
            const size_t o = ((size_t)g * a.blocks + bl) * kLmIntervals + q;
            s += a.psum[o];
            n += a.pcnt[o];
        }
        ps[q][part] = s;
        pc[q][part] = n;
    }
    __syncthreads();
    if (t != 0) return;
    double isum[kLmIntervals];
    uint64_t icnt[kLmIntervals];
    for (int q = 0; q < kLmIntervals; ++q) {
        isum[q] = 0.0;
        icnt[q] = 0;
        for (int part = 0; part < kParts; ++part) {
            isum[q] += ps[q][part];
            icnt[q] += pc[q][part];
        }
    }
    double prev_f = 0.0, s_lt = 0.0;
    uint64_t c_lt = 0;
    for (int j = 0; j < kLmK; ++j) {
        // samples below v_j: intervals 0..j
        s_lt += isum[j];
        c_lt += icnt[j];
        const double vj = (double)lm_value(a.prefix[g * kLmK + j]);
        const double m = (double)((j + 1) * a.bs);
        const double f = s_lt + vj * (m - (double)c_lt);
        a.cent[g * kLmK + j] = (float)((f - prev_f) / (double)a.bs);
        prev_f = f;
    }
}

// One Lloyd step, part 1: per-cell sums and counts under the current centroids.
template <int DT>
__global__ __launch_bounds__(kLmThreads) void lm_assign_kernel(LmArgs a) {
    const int g = blockIdx.y;
    if (a.state[2 * g]) return;                      // converged: uniform for the block
    __shared__ double ls[kLmK][kLmThreads];
    __shared__ uint32_t lc[kLmK][kLmThreads];
    const int th = threadIdx.x;
    float c[kLmK];
#pragma unroll
    for (int k = 0; k < kLmK; ++k) {
        c[k] = a.cent[g * kLmK + k];
        ls[k][th] = 0.0;
        lc[k][th] = 0u;
    }
    lm_for_each<DT>(a, g, [&](float x) {
        int best = 0;
        float bd = fabsf(x - c[0]);
#pragma unroll
        for (int k = 1; k < kLmK; ++k) {
            const float d = fabsf(x - c[k]);
            if (d < bd) {
                bd = d;
                best = k;
            }
        }
        lm_slot_add(&ls[best][th], &lc[best][th], x);
    });
    double s[kLmIntervals];
    uint64_t n[kLmIntervals];
#pragma unroll
    for (int k = 0; k < kLmK; ++k) {
        s[k] = ls[k][th];
        n[k] = lc[k][th];
    }
    s[kLmK] = 0.0;
    n[kLmK] = 0;
    lm_block_store(a, g, s, n, kLmK);
}

// One Lloyd step, part 2: new centroids, the largest move, convergence.
// 256 threads: thread t sums cell t % 16 over blocks t / 16, t / 16 + 16,
// ...; the 16 partial sums of a cell are then added in order.
__global__ __launch_bounds__(256) void lm_update_kernel(LmArgs a) {
    const int g = blockIdx.y;
    __shared__ float moved[kLmK];
    __shared__ double ps[16][kLmK];
    __shared__ uint64_t pc[16][kLmK];
    const int t = threadIdx.x, k = t & (kLmK - 1), part = t >> 4;
    if (a.state[2 * g]) return;
    {
        double s = 0.0;
        uint64_t n = 0;
        for (int bl = part; bl < a.blocks; bl += 16) {
            const size_t o = ((size_t)g * a.blocks + bl) * kLmIntervals + k;
            s += a.psum[o];
            n += a.pcnt[o];
        }
        ps[part][k] = s;
        pc[part][k] = n;
    }
    __syncthreads();
    if (t < kLmK) {
        double s = 0.0;
        uint64_t n = 0;
        for (int p = 0; p < 16; ++p) {
            s += ps[p][k];
            n += pc[p][k];
        }
        const float old = a.cent[g * kLmK + k];
        const float nc = n > 0 ? (float)(s / (double)n) : old;
        moved[k] = fabsf(nc - old);
        a.cent[g * kLmK + k] = nc;
    }
    __syncthreads();
    if (t == 0) {
        float shift = 0.0f;
        for (int j = 0; j < kLmK; ++j) shift = fmaxf(shift, moved[j]);
        a.state[2 * g + 1] += 1;
        if (shift < a.tol) a.state[2 * g] = 1;
    }
}

// Sorted ascending (insertion sort of 16 values) into the output.
__global__ void lm_final_kernel(LmArgs a) {
    const int g = blockIdx.y;
    if (threadIdx.x != 0) return;
    float c[kLmK];
    for (int k = 0; k < kLmK; ++k) c[k] = a.cent[g * kLmK + k];
    for (int i = 1; i < kLmK; ++i) {
        const float v = c[i];
        int j = i - 1;
        while (j >= 0 && c[j] > v) {
            c[j + 1] = c[j];
            --j;
        }
        c[j + 1] = v;
    }
    for (int k = 0; k < kLmK; ++k) a.out[g * kLmK + k] = c[k];
}

static int lm_blocks(int64_t n) {
    const int64_t b = (n + (int64_t)kLmThreads * 8 - 1) / ((int64_t)kLmThreads * 8);
    return (int)(b < 1 ? 1 : (b > kLmMaxBlocks ? kLmMaxBlocks : b));
}

static size_t align256c(size_t x) { return (x + 255) & ~(size_t)255; }

// Workspace carve-up; returns the total bytes (base may be null to size).
static size_t lm_layout(int groups, int blocks, char *base, LmArgs *a) {
    size_t off = 0;
    auto take = [&](size_t bytes) {
        char *p = base ? base + off : nullptr;
        off = align256c(off + bytes);
        return p;
    };
    char *hist = take((size_t)groups * kLmK * 256 * 4);
    char *prefix = take((size_t)groups * kLmK * 4);
    char *krank = take((size_t)groups * kLmK * 8);
    char *up = take((size_t)groups * (kLmK + 1) * 4);
    char *psum = take((size_t)groups * blocks * kLmIntervals * 8);
    char *pcnt = take((size_t)groups * blocks * kLmIntervals * 8);
    char *cent = take((size_t)groups * kLmK * 4);
    char *state = take((size_t)groups * 2 * 4);
    if (a) {
        a->hist = reinterpret_cast<uint32_t *>(hist);
        a->prefix = reinterpret_cast<uint32_t *>(prefix);
        a->krank = reinterpret_cast<int64_t *>(krank);
        a->uprefix = reinterpret_cast<uint32_t *>(up);
        a->psum = reinterpret_cast<double *>(psum);
        a->pcnt = reinterpret_cast<uint64_t *>(pcnt);
        a->cent = reinterpret_cast<float *>(cent);
        a->state = reinterpret_cast<int *>(state);
    }
    return off;
}

template <int DT>
static void lm_launch(const LmArgs &a, int groups, hipStream_t st) {
    const dim3 grid(a.blocks, groups), one(1, groups);
    hipLaunchKernelGGL(lm_clear_kernel, one, dim3(256), 0, st, a);
    for (int pass = 0; pass < 4; ++pass) {
        hipLaunchKernelGGL((lm_radix_kernel<DT>), grid, dim3(kLmThreads), 0, st, a, pass);
        hipLaunchKernelGGL(lm_select_kernel, one, dim3(256), 0, st, a);
    }
    hipLaunchKernelGGL((lm_interval_kernel<DT>), grid, dim3(kLmThreads), 0, st, a);
    hipLaunchKernelGGL(lm_init_kernel, one, dim3(256), 0, st, a);
    for (int it = 0; it < a.max_iters; ++it) {
        hipLaunchKernelGGL((lm_assign_kernel<DT>), grid, dim3(kLmThreads), 0, st, a);
        hipLaunchKernelGGL(lm_update_kernel, one, dim3(256), 0, st, a);
    }
    hipLaunchKernelGGL(lm_final_kernel, one, dim3(64), 0, st, a);
}

__global__ void lm_iters_kernel(const int *state, int groups, int32_t *iters) {
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g < groups) iters[g] = state[2 * g + 1];
}

}  // namespace omni

using namespace omni;

extern "C" size_t omni_lloyd_max_workspace_size(int n_groups, int64_t outer, int64_t inner) {
    if (n_groups <= 0 || outer <= 0 || inner <= 0) return 0;
    return lm_layout(n_groups, lm_blocks(outer * inner), nullptr, nullptr);
}

extern "C" int omni_lloyd_max(const void *x, int x_dtype, int n_groups, int64_t outer, int64_t inner,
                              int64_t outer_stride, int64_t group_stride, int max_iters, float tol,
                              float *codebooks, int32_t *iters_out, void *workspace, size_t workspace_bytes,
                              void *stream) {
    OMNI_CHECK_ARG(dtype_ok(x_dtype), "omni_lloyd_max: bad dtype %d", x_dtype);
    OMNI_CHECK_ARG(n_groups >= 1 && n_groups <= 65535, "omni_lloyd_max: need 1 <= n_groups <= 65535");
    OMNI_CHECK_ARG(outer >= 1 && inner >= 1 && outer_stride >= 0 && group_stride >= 0,
                   "omni_lloyd_max: bad sample layout");
    OMNI_CHECK_ARG(outer <= INT64_MAX / inner, "omni_lloyd_max: too many samples");
    const int64_t n = outer * inner;
    OMNI_CHECK_ARG(n >= kLmK, "omni_lloyd_max: need at least 16 samples per group, got %lld", (long long)n);
    OMNI_CHECK_ARG(max_iters >= 0 && max_iters <= 100000, "omni_lloyd_max: max_iters must be in [0, 100000]");
    OMNI_CHECK_ARG(x && codebooks, "omni_lloyd_max: NULL pointer");
    LmArgs a;
    a.x = x;
    a.outer = outer; a.inner = inner; a.outer_stride = outer_stride; a.group_stride = group_stride;
    a.n = n;
    a.bs = n / kLmK;
    a.blocks = lm_blocks(n);
    a.max_iters = max_iters;
    a.tol = tol;
    a.out = codebooks;
    const size_t need = lm_layout(n_groups, a.blocks, nullptr, nullptr);
    if (workspace == nullptr || workspace_bytes < need) {
        set_error("omni_lloyd_max: workspace of %zu bytes required, %zu given", need, workspace_bytes);
        return OMNI_EWORKSPACE;
    }
    lm_layout(n_groups, a.blocks, reinterpret_cast<char *>(workspace), &a);
    hipStream_t st = as_stream(stream);
    if (x_dtype == OMNI_F32) lm_launch<OMNI_F32>(a, n_groups, st);
    else if (x_dtype == OMNI_BF16) lm_launch<OMNI_BF16>(a, n_groups, st);
    else lm_launch<OMNI_F16>(a, n_groups, st);
    if (iters_out) hipLaunchKernelGGL(lm_iters_kernel, dim3((n_groups + 63) / 64), dim3(64), 0, st, a.state, n_groups,
                                      iters_out);
    OMNI_CHECK_LAUNCH("omni_lloyd_max");
    return OMNI_OK;
}
