// Branchless per-user LoRA gather-apply on queries (gfx950).
//
// Reference semantics: _apply_lora_to_q
// (omnistack_rs/kernels/fused_attention.py:401-430): for each batch row b,
//   delta_r = x[b] @ A[id].T          (T, rank)       fp32
//   delta_q = delta_r @ B[id].T       (T, Hq*D)       fp32
//   q_eff[b] = q[b].float() + delta_q.reshape(T,Hq,D).permute(1,0,2) * alpha
// then cast back to q's dtype; id < 0 leaves q[b] untouched.  Here the
// sentinel is a select on id >= 0, never a multiply-by-zero gate, so NaN or
// Inf in an adapter cannot leak into a sentinel user's query.  An id past the
// bank (only reachable when the host skips validation) yields NaN rows.
//
// One block per (b, t, 1024 outputs): the rank projection delta_r is reduced
// across the lanes of each wave (hidden split over lanes), the block's q and
// B rows are requested before that reduction so their latency overlaps it,
// and each thread then applies four outputs.  Element types are template
// parameters (no per-element dtype branches).
#include <math.h>

#include "omni_common.h"

namespace omni {

constexpr int kLoraThreads = 256;
constexpr int kLoraOutPerThread = 4;
constexpr int kLoraOutPerBlock = kLoraThreads * kLoraOutPerThread;
constexpr int kLoraMaxRank = 64;
constexpr int kLoraJPerWave = kLoraMaxRank / (kLoraThreads / 64);

template <int DT>
struct Elt;
template <>
struct Elt<OMNI_F32> {
    typedef float T;
    __device__ static float f(T v) { return v; }
    __device__ static T from(float v) { return v; }
};
template <>
struct Elt<OMNI_F16> {
    typedef uint16_t T;
    __device__ static float f(T v) { return f16_to_f32(v); }
    __device__ static T from(float v) { return f32_to_f16_rne(v); }
};
template <>
struct Elt<OMNI_BF16> {
    typedef uint16_t T;
    __device__ static float f(T v) { return bf16_to_f32(v); }
    __device__ static T from(float v) { return f32_to_bf16_rne(v); }
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

template <int QT, int WT>
__global__ __launch_bounds__(kLoraThreads) void lora_kernel(
    const void *q_, const void *x_, const void *A_, const void *B_, const int32_t *idx, int Hq, int64_t T,
    int D, int hidden, int rank, int n_loras, float alpha, void *q_out_) {
    typedef typename Elt<QT>::T QE;
    typedef typename Elt<WT>::T WE;
    const QE *q = reinterpret_cast<const QE *>(q_);
    QE *q_out = reinterpret_cast<QE *>(q_out_);
    const WE *x = reinterpret_cast<const WE *>(x_);
    const WE *A = reinterpret_cast<const WE *>(A_);
    const WE *Bw = reinterpret_cast<const WE *>(B_);
    __shared__ float dr[kLoraMaxRank];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t b = blockIdx.z, t = blockIdx.y;
    const int out_dim = Hq * D;
    const int32_t id = idx[b];
    const bool active = id >= 0 && id < n_loras;
    const bool bad = id >= n_loras;
    const int64_t sid = active ? id : 0;

    // this thread's outputs o = base + 4 tid + c; their q values first
    const int obase = blockIdx.x * kLoraOutPerBlock + kLoraOutPerThread * tid;
    float qv[kLoraOutPerThread];
    int64_t qi[kLoraOutPerThread];
#pragma unroll
    for (int c = 0; c < kLoraOutPerThread; ++c) {
        const int o = obase + c < out_dim ? obase + c : out_dim - 1;
        const int hq = o / D, d = o - hq * D;
        qi[c] = ((b * Hq + hq) * T + t) * D + d;
        qv[c] = Elt<QT>::f(q[qi[c]]);
    }

    // delta_r[j] = sum_h x[b][t][h] * A[id][j][h]; wave w takes j = w, w + 4, ...
    {
        float acc[kLoraJPerWave];
#pragma unroll
        for (int jj = 0; jj < kLoraJPerWave; ++jj) acc[jj] = 0.0f;
        const WE *xr = x + (b * T + t) * hidden;
        const WE *Ar = A + sid * rank * (int64_t)hidden;
        for (int h = lane; h < hidden; h += 64) {
            const float xv = Elt<WT>::f(xr[h]);
#pragma unroll
            for (int jj = 0; jj < kLoraJPerWave; ++jj) {
                const int j = wave + 4 * jj;
                if (j < rank) acc[jj] = __builtin_fmaf(xv, Elt<WT>::f(Ar[(int64_t)j * hidden + h]), acc[jj]);
            }
        }
#pragma unroll
        for (int jj = 0; jj < kLoraJPerWave; ++jj) {
            const int j = wave + 4 * jj;
            if (j < rank) {
                const float v = wave_sum(acc[jj]);
                if (lane == 0) dr[j] = v;
            }
        }
    }
    __syncthreads();

    // delta_q[o] = sum_j delta_r[j] * B[id][o][j]
#pragma unroll
    for (int c = 0; c < kLoraOutPerThread; ++c) {
        const int o = obase + c;
        if (o >= out_dim) break;
        const WE *br = Bw + (sid * out_dim + o) * (int64_t)rank;
        float acc = 0.0f;
        for (int j = 0; j < rank; ++j) acc = __builtin_fmaf(dr[j], Elt<WT>::f(br[j]), acc);
        const float upd = Elt<QT>::f(Elt<QT>::from(__fadd_rn(qv[c], __fmul_rn(acc, alpha))));
        const float res = active ? upd : (bad ? __builtin_nanf("") : qv[c]);
        q_out[qi[c]] = Elt<QT>::from(res);
    }
}

template <int QT, int WT>
static void launch_lora(dim3 grid, hipStream_t s, const void *q, const void *x, const void *A, const void *Bw,
                        const int32_t *idx, int Hq, int64_t T, int D, int hidden, int rank, int n_loras,
                        float alpha, void *q_out) {
    hipLaunchKernelGGL((lora_kernel<QT, WT>), grid, dim3(kLoraThreads), 0, s, q, x, A, Bw, idx, Hq, T, D, hidden,
                       rank, n_loras, alpha, q_out);
}

template <int QT>
static void launch_lora_w(int w_dtype, dim3 grid, hipStream_t s, const void *q, const void *x, const void *A,
                          const void *Bw, const int32_t *idx, int Hq, int64_t T, int D, int hidden, int rank,
                          int n_loras, float alpha, void *q_out) {
    if (w_dtype == OMNI_F32)
        launch_lora<QT, OMNI_F32>(grid, s, q, x, A, Bw, idx, Hq, T, D, hidden, rank, n_loras, alpha, q_out);
    else if (w_dtype == OMNI_F16)
        launch_lora<QT, OMNI_F16>(grid, s, q, x, A, Bw, idx, Hq, T, D, hidden, rank, n_loras, alpha, q_out);
    else
        launch_lora<QT, OMNI_BF16>(grid, s, q, x, A, Bw, idx, Hq, T, D, hidden, rank, n_loras, alpha, q_out);
}

}  // namespace omni

using namespace omni;

extern "C" int omni_lora_apply(const void *q, int q_dtype, const void *x, const void *A, const void *Bw,
                               int w_dtype, const int32_t *idx, int64_t B, int Hq, int64_t T,
                               int head_dim, int hidden, int rank, int n_loras, float alpha,
                               void *q_out, void *stream) {
    OMNI_CHECK_ARG(dtype_ok(q_dtype) && dtype_ok(w_dtype), "omni_lora_apply: bad dtype");
    OMNI_CHECK_ARG(B >= 0 && Hq >= 0 && T >= 0 && head_dim > 0 && hidden > 0, "omni_lora_apply: bad shape");
    OMNI_CHECK_ARG(rank >= 1 && rank <= kLoraMaxRank, "omni_lora_apply: rank must be in [1, %d], got %d",
                   kLoraMaxRank, rank);
    OMNI_CHECK_ARG(n_loras >= 1, "omni_lora_apply: n_loras must be >= 1");
    if (B == 0 || Hq == 0 || T == 0) return OMNI_OK;
    OMNI_CHECK_ARG(q && x && A && Bw && idx && q_out, "omni_lora_apply: NULL pointer");
    OMNI_CHECK_ARG(B <= 65535 && T <= 65535, "omni_lora_apply: grid too large (B and T must be <= 65535)");
    OMNI_CHECK_ARG((int64_t)Hq * head_dim <= (int64_t)1 << 30, "omni_lora_apply: n_heads * head_dim too large");
    const int out_dim = Hq * head_dim;
    dim3 grid((unsigned)((out_dim + kLoraOutPerBlock - 1) / kLoraOutPerBlock), (unsigned)T, (unsigned)B);
    hipStream_t s = as_stream(stream);
    if (q_dtype == OMNI_F32)
        launch_lora_w<OMNI_F32>(w_dtype, grid, s, q, x, A, Bw, idx, Hq, T, head_dim, hidden, rank, n_loras, alpha, q_out);
    else if (q_dtype == OMNI_F16)
        launch_lora_w<OMNI_F16>(w_dtype, grid, s, q, x, A, Bw, idx, Hq, T, head_dim, hidden, rank, n_loras, alpha, q_out);
    else
        launch_lora_w<OMNI_BF16>(w_dtype, grid, s, q, x, A, Bw, idx, Hq, T, head_dim, hidden, rank, n_loras, alpha, q_out);
    OMNI_CHECK_LAUNCH("omni_lora_apply");
    return OMNI_OK;
}
