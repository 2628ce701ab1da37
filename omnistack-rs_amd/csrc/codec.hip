// gfx950 codec kernels: WHT rotation, fused INT4 + QJL encoder, dequantizer.
//
// Bit-level contract (reference deepsheth3/Omnistack-RS, Python/torch):
//   rotation   omnistack_rs/kernels/hadamard.py:51-85   (_wht_torch)
//   encoder    omnistack_rs/kernels/quantize.py:542-590 (quantize_heads)
//              + :361-377 (argmin, nibble pack) + :398-423 (QJL signs)
//   decoder    omnistack_rs/kernels/quantize.py:593-640 (dequantize_heads)
//              + :380-395 (unpack) + :426-451 (QJL reconstruct)
// The library is built with -ffp-contract=off: every fp32 operation below
// rounds exactly where the reference's torch ops round.
#include <math.h>

#include "omni_common.h"

namespace omni {

constexpr int kRowsPerBlock = 256;
constexpr int kProjGroup = 4;   // QJL projections accumulated together per pass

// In-register normalized WHT of one row, reference butterfly order:
// h = 1, 2, ..., D/2; (upper, lower) -> (upper + lower, upper - lower).
template <int D>
__device__ __forceinline__ void wht_row(float (&v)[D], float scale) {
#pragma unroll
    for (int h = 1; h < D; h <<= 1) {
#pragma unroll
        for (int base = 0; base < D; base += 2 * h) {
#pragma unroll
            for (int i = 0; i < h; ++i) {
                float u = v[base + i], l = v[base + h + i];
                v[base + i] = u + l;
                v[base + h + i] = u - l;
            }
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) v[d] = v[d] * scale;
}

template <int D>
__device__ __forceinline__ void load_row(const void *x, int dtype, int64_t row, float (&v)[D]) {
    if (dtype == OMNI_F32) {
        const float4 *p = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(x) + row * D);
#pragma unroll
        for (int k = 0; k < D / 4; ++k) {
            float4 t = p[k];
            v[4 * k] = t.x; v[4 * k + 1] = t.y; v[4 * k + 2] = t.z; v[4 * k + 3] = t.w;
        }
    } else {
        const uint4 *p = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(x) + row * D);
#pragma unroll
        for (int k = 0; k < D / 8; ++k) {
            uint4 t = p[k];
            uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint16_t lo = (uint16_t)(w[j] & 0xffffu), hi = (uint16_t)(w[j] >> 16);
                v[8 * k + 2 * j] = dtype == OMNI_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
                v[8 * k + 2 * j + 1] = dtype == OMNI_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
            }
        }
    }
}

template <int D>
__device__ __forceinline__ void rotate_row(float (&v)[D], int dtype, const int8_t *sign_flip, float scale) {
    if (sign_flip) {
#pragma unroll
        for (int d = 0; d < D; ++d) v[d] = sign_flip[d] < 0 ? -v[d] : v[d];
    }
    wht_row<D>(v, scale);
#pragma unroll
    for (int d = 0; d < D; ++d) v[d] = round_to_dtype(v[d], dtype);
}

// ── omni_wht_rotate ─────────────────────────────────────────────────────

template <int D>
__global__ __launch_bounds__(kRowsPerBlock) void wht_kernel(const void *x, int dtype, int64_t rows,
                                                            const int8_t *sign_flip, void *out, float scale) {
    int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x;
    if (row >= rows) return;
    float v[D];
    load_row<D>(x, dtype, row, v);
    rotate_row<D>(v, dtype, sign_flip, scale);
#pragma unroll
    for (int d = 0; d < D; ++d) store_from_f32(out, dtype, row * D + d, v[d]);
}

// ── omni_encode ─────────────────────────────────────────────────────────
//
// One lane per row; a block covers up to 256 rows of one (b, h), so the
// head's codebook and G are uniform across the block (scalar loads).

// Exact sign of sum_j s_j e_j (s_j = +-1 from the G row bits) by fp64
// Neumaier summation, for the rare projections whose fp32 sum is within its
// rounding bound of zero.  Inlined and fully unrolled so the residual row
// stays in registers (a call would force the whole row to scratch).
template <int D>
__device__ __forceinline__ bool exact_sign_nonneg(const float (&e)[D], const uint32_t *grow) {
    double s = 0.0, c = 0.0;
#pragma unroll
    for (int w = 0; w < D / 32; ++w) {
        const uint32_t gw = grow[w];
#pragma unroll
        for (int jj = 0; jj < 32; ++jj) {
            double y = (double)e[32 * w + jj];
            y = ((gw >> jj) & 1u) ? y : -y;
            const double t = s + y;
            c += (fabs(s) >= fabs(y)) ? ((s - t) + y) : ((y - t) + s);
            s = t;
        }
    }
    return (s + c) >= 0.0;
}

template <int D>
__global__ __launch_bounds__(kRowsPerBlock) void encode_kernel(
    const void *x, int dtype, int64_t T, int H, int rotate, const int8_t *sign_flip,
    const float *codebooks, int per_head, const uint32_t *g_bits,
    uint8_t *nibbles, uint8_t *qjl, float *norms, float scale) {
    constexpr int QD = D / 2;       // QJL projections per row
    constexpr int W = D / 32;       // G words per projection row
    const int h = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int64_t t = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x;
    if (t >= T) return;
    const int64_t row = (b * H + h) * T + t;

    float v[D];
    load_row<D>(x, dtype, row, v);
    if (rotate) rotate_row<D>(v, dtype, sign_flip, scale);

    const float *cbp = codebooks + (per_head ? h * 16 : 0);
    float cb[16];
    bool cb_nan = false;
#pragma unroll
    for (int k = 0; k < 16; ++k) { cb[k] = cbp[k]; cb_nan |= (cb[k] != cb[k]); }

    // Nearest centroid: fp32 |x - c_k|, strictly smaller wins (first index
    // on ties).  A NaN distance is the minimum (torch.argmin); that only
    // matters when the codebook itself holds a NaN: a NaN x gives NaN for
    // every k and keeps code 0 either way.
    uint32_t packed[D / 8];
#pragma unroll
    for (int w = 0; w < D / 8; ++w) packed[w] = 0u;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        float best = fabsf(v[d] - cb[0]);
        int code = 0;
        float cval = cb[0];
#pragma unroll
        for (int k = 1; k < 16; ++k) {
            float dk = fabsf(v[d] - cb[k]);
            bool take = dk < best;
            if (cb_nan) take = take || ((dk != dk) && (best == best));
            best = take ? dk : best;
            code = take ? k : code;
            cval = take ? cb[k] : cval;
        }
        packed[d >> 3] |= (uint32_t)code << (4 * (d & 7));
        v[d] = v[d] - cval;  // residual e_d (fp32), quantize.py:580
    }

    // ||e||_2: fp32 squares (as the reference's fp32 norm forms them) summed
    // in fp64 and rounded once; a sum beyond the fp32 range is +inf, where the
    // reference's fp32 accumulation overflows.
    double ss = 0.0;
    float abs_sum = 0.0f;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        ss += (double)__fmul_rn(v[d], v[d]);
        abs_sum += fabsf(v[d]);
    }
    const float nrm = ss > 3.4028234663852886e38 ? INFINITY : (float)sqrt(ss);

    // QJL signs.  fp32 sequential sums carry |err| <= (D-1) u sum|e_j|; a
    // result farther than D * 2^-24 * abs_sum from zero has a certain sign,
    // anything closer is recomputed exactly.  Non-finite rows take the fp32
    // result's (deterministic) sign like the reference's BLAS does.
    const float bound = abs_sum * ((float)D * 5.9604644775390625e-8f);
    const bool finite_row = isfinite(abs_sum);
    const uint32_t *gh = g_bits + (int64_t)h * QD * W;
    uint32_t sbits[QD / 32 > 0 ? QD / 32 : 1];
#pragma unroll
    for (int k = 0; k < (QD / 32 > 0 ? QD / 32 : 1); ++k) sbits[k] = 0u;
#pragma unroll 1
    for (int i0 = 0; i0 < QD; i0 += kProjGroup) {
        float acc[kProjGroup];
#pragma unroll
        for (int ii = 0; ii < kProjGroup; ++ii) acc[ii] = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            uint32_t gw[kProjGroup];
#pragma unroll
            for (int ii = 0; ii < kProjGroup; ++ii) gw[ii] = gh[(i0 + ii) * W + w];
#pragma unroll
            for (int jj = 0; jj < 32; ++jj) {
#pragma unroll
                for (int ii = 0; ii < kProjGroup; ++ii) {
                    float s = ((gw[ii] >> jj) & 1u) ? 1.0f : -1.0f;
                    acc[ii] = __builtin_fmaf(s, v[32 * w + jj], acc[ii]);
                }
            }
        }
        uint32_t unc = 0u;
#pragma unroll
        for (int ii = 0; ii < kProjGroup; ++ii) {
            const int i = i0 + ii;
            if (finite_row && !(fabsf(acc[ii]) > bound)) unc |= 1u << ii;
            sbits[i >> 5] |= (uint32_t)(acc[ii] >= 0.0f) << (i & 31);
        }
        while (unc) {
            const int ii = __builtin_ctz(unc);
            unc &= unc - 1u;
            const int i = i0 + ii;
            const bool bit = exact_sign_nonneg<D>(v, gh + i * W);
            sbits[i >> 5] = (sbits[i >> 5] & ~(1u << (i & 31))) | ((uint32_t)bit << (i & 31));
        }
    }

    // Stores: nibbles (D/2 B), signs (D/16 B), norm.
    if constexpr (D == 128) {
        uint4 *np = reinterpret_cast<uint4 *>(nibbles + row * (D / 2));
#pragma unroll
        for (int k = 0; k < 4; ++k) np[k] = make_uint4(packed[4 * k], packed[4 * k + 1], packed[4 * k + 2], packed[4 * k + 3]);
        reinterpret_cast<uint2 *>(qjl + row * (D / 16))[0] = make_uint2(sbits[0], sbits[1]);
    } else {
        reinterpret_cast<uint4 *>(nibbles + row * (D / 2))[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
        reinterpret_cast<uint16_t *>(qjl + row * (D / 16))[0] = (uint16_t)(sbits[0] & 0xffffu);
    }
    norms[row] = nrm;
}

// ── omni_dequantize ─────────────────────────────────────────────────────
//
// k_hat_d = fl(cb[code_d] + fl(s_d * fl(norm * c))), c = fp32(sqrt(2/pi)/D),
// s_d = sum_i b+-_i G_h[i][d] = QD - 2 popcount(b ^ Gcol_d)  (an exact integer).

template <int D>
__global__ __launch_bounds__(kRowsPerBlock) void dequant_kernel(
    const uint8_t *nibbles, const uint8_t *qjl, const float *norms, const float *codebooks,
    int per_head, const uint32_t *g_bits, int64_t T, int H, int with_qjl, float *out, float c_alpha) {
    constexpr int QD = D / 2;
    constexpr int W = D / 32;
    __shared__ uint64_t gcol[D];
    const int h = blockIdx.y;
    const int64_t b = blockIdx.z;
    if (with_qjl) {
        // Transpose G_h (QD rows x D bits) into D column masks of QD bits.
        for (int d = threadIdx.x; d < D; d += blockDim.x) {
            uint64_t m = 0;
            for (int i = 0; i < QD; ++i)
                m |= (uint64_t)((g_bits[((int64_t)h * QD + i) * W + (d >> 5)] >> (d & 31)) & 1u) << i;
            gcol[d] = m;
        }
        __syncthreads();
    }
    const int64_t t = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x;
    if (t >= T) return;
    const int64_t row = (b * H + h) * T + t;
    const float *cbp = codebooks + (per_head ? h * 16 : 0);
    float cb[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) cb[k] = cbp[k];

    uint64_t sb = 0;
    float sc = 0.0f;
    if (with_qjl) {
        if constexpr (D == 128) {
            uint2 q2 = reinterpret_cast<const uint2 *>(qjl + row * (D / 16))[0];
            sb = (uint64_t)q2.x | ((uint64_t)q2.y << 32);
        } else {
            sb = reinterpret_cast<const uint16_t *>(qjl + row * (D / 16))[0];
        }
        sc = __fmul_rn(norms[row], c_alpha);
    }
    const uint8_t *np = nibbles + row * (D / 2);
    float *op = out + row * D;
#pragma unroll 4
    for (int m = 0; m < D / 2; ++m) {
        const uint32_t byte = np[m];
        float v0 = cb[byte & 15u], v1 = cb[byte >> 4];
        if (with_qjl) {
            const int d0 = 2 * m, d1 = 2 * m + 1;
            const float s0 = (float)(QD - 2 * (int)__popcll(sb ^ gcol[d0]));
            const float s1 = (float)(QD - 2 * (int)__popcll(sb ^ gcol[d1]));
            v0 = __fadd_rn(v0, __fmul_rn(s0, sc));
            v1 = __fadd_rn(v1, __fmul_rn(s1, sc));
        }
        op[2 * m] = v0;
        op[2 * m + 1] = v1;
    }
}

}  // namespace omni

using namespace omni;

extern "C" int omni_wht_rotate(const void *x, int dtype, int64_t rows, int head_dim,
                               const int8_t *sign_flip, void *out, void *stream) {
    OMNI_CHECK_ARG(dtype_ok(dtype), "omni_wht_rotate: bad dtype %d", dtype);
    OMNI_CHECK_ARG(head_dim_ok(head_dim), "WHT rotation requires last dim = 128 (or 32), got %d", head_dim);
    OMNI_CHECK_ARG(rows >= 0, "omni_wht_rotate: rows < 0");
    OMNI_CHECK_ARG(rows == 0 || (x && out), "omni_wht_rotate: NULL pointer");
    if (rows == 0) return OMNI_OK;
    dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    const float s = inv_sqrt_dim_f32(head_dim);
    if (head_dim == 128)
        hipLaunchKernelGGL(wht_kernel<128>, grid, dim3(kRowsPerBlock), 0, as_stream(stream), x, dtype, rows, sign_flip, out, s);
    else
        hipLaunchKernelGGL(wht_kernel<32>, grid, dim3(kRowsPerBlock), 0, as_stream(stream), x, dtype, rows, sign_flip, out, s);
    OMNI_CHECK_LAUNCH("omni_wht_rotate");
    return OMNI_OK;
}

extern "C" int omni_encode(const void *x, int x_dtype, int64_t B, int H, int64_t T, int head_dim,
                           int rotate, const int8_t *sign_flip, const float *codebooks,
                           int per_head_codebook, const uint32_t *g_bits,
                           uint8_t *nibbles, uint8_t *qjl, float *norms, void *stream) {
    OMNI_CHECK_ARG(dtype_ok(x_dtype), "omni_encode: bad dtype %d", x_dtype);
    OMNI_CHECK_ARG(head_dim_ok(head_dim), "omni_encode: head_dim must be 128 or 32, got %d", head_dim);
    OMNI_CHECK_ARG(B >= 0 && H >= 0 && T >= 0, "omni_encode: negative shape");
    if (B == 0 || H == 0 || T == 0) return OMNI_OK;
    OMNI_CHECK_ARG(x && codebooks && g_bits && nibbles && qjl && norms, "omni_encode: NULL pointer");
    OMNI_CHECK_ARG(B <= 65535 && H <= 65535, "omni_encode: B and H must be <= 65535");
    dim3 grid((unsigned)((T + kRowsPerBlock - 1) / kRowsPerBlock), (unsigned)H, (unsigned)B);
    const float s = inv_sqrt_dim_f32(head_dim);
    if (head_dim == 128)
        hipLaunchKernelGGL(encode_kernel<128>, grid, dim3(kRowsPerBlock), 0, as_stream(stream), x, x_dtype, T, H,
                           rotate, sign_flip, codebooks, per_head_codebook, g_bits, nibbles, qjl, norms, s);
    else
        hipLaunchKernelGGL(encode_kernel<32>, grid, dim3(kRowsPerBlock), 0, as_stream(stream), x, x_dtype, T, H,
                           rotate, sign_flip, codebooks, per_head_codebook, g_bits, nibbles, qjl, norms, s);
    OMNI_CHECK_LAUNCH("omni_encode");
    return OMNI_OK;
}

extern "C" int omni_dequantize(const uint8_t *nibbles, const uint8_t *qjl, const float *norms,
                               const float *codebooks, int per_head_codebook, const uint32_t *g_bits,
                               int64_t B, int H, int64_t T, int head_dim, int with_qjl, float *out,
                               void *stream) {
    OMNI_CHECK_ARG(head_dim_ok(head_dim), "omni_dequantize: head_dim must be 128 or 32, got %d", head_dim);
    OMNI_CHECK_ARG(B >= 0 && H >= 0 && T >= 0, "omni_dequantize: negative shape");
    if (B == 0 || H == 0 || T == 0) return OMNI_OK;
    OMNI_CHECK_ARG(nibbles && codebooks && out, "omni_dequantize: NULL pointer");
    OMNI_CHECK_ARG(!with_qjl || (qjl && norms && g_bits), "omni_dequantize: NULL QJL pointer");
    OMNI_CHECK_ARG(B <= 65535 && H <= 65535, "omni_dequantize: B and H must be <= 65535");
    dim3 grid((unsigned)((T + kRowsPerBlock - 1) / kRowsPerBlock), (unsigned)H, (unsigned)B);
    const float c = (float)(sqrt(2.0 / M_PI) / (double)head_dim);
    if (head_dim == 128)
        hipLaunchKernelGGL(dequant_kernel<128>, grid, dim3(kRowsPerBlock), 0, as_stream(stream), nibbles, qjl,
                           norms, codebooks, per_head_codebook, g_bits, T, H, with_qjl, out, c);
    else
        hipLaunchKernelGGL(dequant_kernel<32>, grid, dim3(kRowsPerBlock), 0, as_stream(stream), nibbles, qjl,
                           norms, codebooks, per_head_codebook, g_bits, T, H, with_qjl, out, c);
    OMNI_CHECK_LAUNCH("omni_dequantize");
    return OMNI_OK;
}
