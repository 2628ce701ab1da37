// Branchless per-user LoRA gather-apply on queries (gfx950).
//
// Reference semantics: _apply_lora_to_q
// (omnistack_rs/kernels/fused_attention.py:401-430): for each batch row b,
//   delta_r = x[b] @ A[id].T          (T, rank)       fp32
//   delta_q = delta_r @ B[id].T       (T, Hq*D)       fp32
//   q_eff[b] = q[b].float() + delta_q.reshape(T,Hq,D).permute(1,0,2) * alpha
// then cast back to q's dtype; id < 0 leaves q[b] untouched.  Here the
// sentinel is a select on id >= 0, never a multiply-by-zero gate, so NaN or
// Inf in an adapter cannot leak into a sentinel user's query.
#include <math.h>

#include "omni_common.h"

namespace omni {

constexpr int kLoraThreads = 256;
constexpr int kLoraTok = 8;       // query tokens per block
constexpr int kLoraMaxRank = 64;

__global__ __launch_bounds__(kLoraThreads) void lora_kernel(
    const void *q, int q_dtype, const void *x, const void *A, const void *Bw, int w_dtype,
    const int32_t *idx, int Hq, int64_t T, int D, int hidden, int rank, int n_loras, float alpha,
    void *q_out) {
    __shared__ float dr[kLoraTok][kLoraMaxRank];
    const int64_t b = blockIdx.z;
    const int64_t t0 = (int64_t)blockIdx.y * kLoraTok;
    const int nt = (int)((T - t0) < kLoraTok ? (T - t0) : kLoraTok);
    const int32_t id = idx[b];
    const bool active = id >= 0 && id < n_loras;
    const bool bad = id >= n_loras;
    const int64_t sid = active ? id : 0;

    // delta_r[t][j] = sum_h x[b][t][h] * A[id][j][h]; one thread per (t, j).
    for (int tj = threadIdx.x; tj < nt * rank; tj += blockDim.x) {
        const int tt = tj / rank, j = tj % rank;
        const int64_t xo = (b * T + t0 + tt) * hidden;
        const int64_t ao = (sid * rank + j) * hidden;
        float acc = 0.0f;
        for (int h = 0; h < hidden; ++h)
            acc = __builtin_fmaf(load_as_f32(x, w_dtype, xo + h), load_as_f32(A, w_dtype, ao + h), acc);
        dr[tt][j] = acc;
    }
    __syncthreads();

    const int out_dim = Hq * D;
    const int o = blockIdx.x * blockDim.x + threadIdx.x;
    if (o >= out_dim) return;
    const int hq = o / D, d = o % D;
    const int64_t bo = (sid * out_dim + o) * rank;
    for (int tt = 0; tt < nt; ++tt) {
        float acc = 0.0f;
        for (int j = 0; j < rank; ++j) acc = __builtin_fmaf(dr[tt][j], load_as_f32(Bw, w_dtype, bo + j), acc);
        const int64_t qi = ((b * Hq + hq) * T + t0 + tt) * D + d;
        const float qv = load_as_f32(q, q_dtype, qi);
        const float upd = round_to_dtype(__fadd_rn(qv, __fmul_rn(acc, alpha)), q_dtype);
        const float res = active ? upd : (bad ? __builtin_nanf("") : qv);
        store_from_f32(q_out, q_dtype, qi, res);
    }
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
    OMNI_CHECK_ARG(B <= 65535 && (T + kLoraTok - 1) / kLoraTok <= 65535, "omni_lora_apply: grid too large");
    const int out_dim = Hq * head_dim;
    dim3 grid((unsigned)((out_dim + kLoraThreads - 1) / kLoraThreads), (unsigned)((T + kLoraTok - 1) / kLoraTok),
              (unsigned)B);
    hipLaunchKernelGGL(lora_kernel, grid, dim3(kLoraThreads), 0, as_stream(stream), q, q_dtype, x, A, Bw, w_dtype,
                       idx, Hq, T, head_dim, hidden, rank, n_loras, alpha, q_out);
    OMNI_CHECK_LAUNCH("omni_lora_apply");
    return OMNI_OK;
}
