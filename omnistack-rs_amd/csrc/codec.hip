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

    // ||e||_2: the exact squares (fp32 x fp32 fits fp64) summed in fp64 and
    // rounded once; a sum beyond the fp32 range is +inf, where the
    // reference's fp32 accumulation overflows.
    double ss = 0.0;
    float abs_sum = 0.0f;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const double ed = (double)v[d];
        ss = __builtin_fma(ed, ed, ss);
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

typedef float float4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t cvt_pk_f16(float x, float y) {
    typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
    typedef float f2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2_t){x, y}, h2_t));
}

// ── fast encoder: 16-bit input, D = 128 ─────────────────────────────────
//
// Same contract as encode_kernel, organised for gfx950:
//   * 16 rows per wave-iteration; lane (n, g) holds elements 32 s + 8 g + i
//     (s < 4, i < 8) of row n.  The WHT runs in registers (h = 1, 2, 4, 32,
//     64) and by paired v_permlane16/32_swap butterflies (h = 8, 16), in the
//     reference stage order with the reference's fp32 operations.
//   * Codes come from a 64 KB LDS table indexed by the rotated value's
//     16-bit pattern, built exactly (brute-force first-index argmin with the
//     NaN rule) by code_table_kernel into the caller's workspace.
//   * QJL projections P = E G^T on v_mfma_f32_16x16x32_bf16: each residual
//     is split into two round-to-nearest bf16 parts (the dropped remainder is
//     below 2^-16 |e|), G is exactly +-1, so the products are exact and the
//     error (fp32 accumulation plus the remainder) is bounded by
//     1312 * 2^-24 * sum|e| (+ 2^-100 for flushed denormals).  Signs outside
//     the bound are certain; the rare rest are recomputed in fp64 with
//     compensated sums.  Rows with a non-finite residual take the
//     order-free sign of the reference's fp32 sum (NaN if it meets NaN or
//     both infinities, else the sign of the infinity).
//   * With A = G rows and B = the residual rows, lane (n, g) receives
//     P[n][16 cb + 4 g + i]: every value a lane needs for its row is local
//     or one 4-lane reduction away.

constexpr int kEncWaves = 12;
constexpr int kEncTab = 65536;                            // u8 code table (both nibbles = code)
constexpr int kEncCentOff = kEncTab;                      // f32 centroid by table byte (256 slots)
constexpr int kEncGimgOff = kEncCentOff + 256 * 4;        // [cb][s][lane] uint4: 8 bf16 +-1 of G
constexpr int kEncGbitsOff = kEncGimgOff + 4 * 4 * 64 * 16;   // G rows as bits, 64 x 4 words
constexpr int kEncFlipOff = kEncGbitsOff + 64 * 4 * 4;       // [lane][16] u32: sign-bit xor of the raw 16-bit words
constexpr int kEncStageOff = kEncFlipOff + 64 * 16 * 4;      // [wave][128] f32: one residual row (rare paths)
constexpr int kEncLdsBytes = kEncStageOff + kEncWaves * 128 * 4;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

struct EncArgs {
    const void *x[2];            // one or two tensors of the same shape (blockIdx.z)
    const uint8_t *table;        // n_tables x 65536
    const float *codebooks;
    const uint32_t *g_bits;
    const int8_t *sign_flip;
    uint8_t *nibbles[2], *qjl[2];
    float *norms[2];
    int64_t T, nrows_head, rows_per_block[2];    // per tensor
    int nx0;                                      // paged: blocks of the first tensor
    int H, per_head, rotate;
    float scale;
    // paged output (encode128_kernel<..., true>): row (b, h, t) goes to pool
    // row (page_table[b][p >> page_shift] * H + h) * page_size + p %
    // page_size, p = positions[b] + t; rows whose page is outside the pool
    // (or past the table) are not written; the second tensor (V) writes
    // its codes only
    const int32_t *page_table, *positions;
    int64_t max_pages, n_pages;
    int page_shift;
};

template <int XDT>
__global__ __launch_bounds__(256) void code_table_kernel(const float *codebooks, int per_head, uint8_t *table) {
    const int h = blockIdx.y;
    const uint32_t u = blockIdx.x * 256u + threadIdx.x;
    const float v = XDT == OMNI_BF16 ? bf16_to_f32((uint16_t)u) : f16_to_f32((uint16_t)u);
    const float *cbp = codebooks + (per_head ? h * 16 : 0);
    float cb[16];
    bool cb_nan = false;
#pragma unroll
    for (int k = 0; k < 16; ++k) { cb[k] = cbp[k]; cb_nan |= (cb[k] != cb[k]); }
    float best = fabsf(v - cb[0]);
    int code = 0;
#pragma unroll
    for (int k = 1; k < 16; ++k) {
        const float dk = fabsf(v - cb[k]);
        bool take = dk < best;
        if (cb_nan) take = take || ((dk != dk) && (best == best));
        best = take ? dk : best;
        code = take ? k : code;
    }
    table[(int64_t)h * kEncTab + u] = (uint8_t)(code | (code << 4));
}

// (a, b) <- butterfly with the partner lane across bit 4 (row parity) or 5
// (half): lanes with the bit clear hold the lower element of each pair.
// Two swaps and one add/sub pair cover two elements.
template <int HALF>
__device__ __forceinline__ void xlane_pair_butterfly(float &a, float &b) {
    uint32_t t0, t1, u0, u1;
    if constexpr (HALF == 16) {
        const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
        t0 = t[0]; t1 = t[1];
    } else {
        const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
        t0 = t[0]; t1 = t[1];
    }
    const float lo = __uint_as_float(t0), hi = __uint_as_float(t1);
    const float s = lo + hi, d = lo - hi;
    if constexpr (HALF == 16) {
        const auto u = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(d), false, false);
        u0 = u[0]; u1 = u[1];
    } else {
        const auto u = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(d), false, false);
        u0 = u[0]; u1 = u[1];
    }
    a = __uint_as_float(u0);
    b = __uint_as_float(u1);
}

template <int HALF>
__device__ __forceinline__ double xlane_sum_f64(double v) {
    const uint64_t bits = __builtin_bit_cast(uint64_t, v);
    uint32_t lo = (uint32_t)bits, hi = (uint32_t)(bits >> 32), plo, phi;
    if constexpr (HALF == 16) {
        const auto a = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
        const auto b = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
        const bool odd = (__lane_id() & 16) != 0;
        plo = odd ? a[0] : a[1];
        phi = odd ? b[0] : b[1];
    } else {
        const auto a = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
        const auto b = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
        const bool up = (__lane_id() & 32) != 0;
        plo = up ? a[0] : a[1];
        phi = up ? b[0] : b[1];
    }
    return v + __builtin_bit_cast(double, ((uint64_t)phi << 32) | plo);
}

template <int HALF>
__device__ __forceinline__ uint32_t xlane_u32(uint32_t v) {
    if constexpr (HALF == 16) {
        const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (__lane_id() & 16) ? a[0] : a[1];
    } else {
        const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (__lane_id() & 32) ? a[0] : a[1];
    }
}

__device__ __forceinline__ float xlane_sum_f32(float v) {
    v += __uint_as_float(xlane_u32<16>(__float_as_uint(v)));
    return v + __uint_as_float(xlane_u32<32>(__float_as_uint(v)));
}

// sum_j s_j e_j over one staged residual row (128 floats in LDS) for G row
// `grow` (4 words): each lane takes elements lane and lane + 64 in fp64 and
// the wave reduces (sum, error) pairs with TwoSum, so the result is the exact
// sum up to ~1e-30 relative.  Commutative steps: every lane gets the same
// value.  `fl` collects the order-free classes of the terms (1 NaN, 2 +inf,
// 4 -inf), OR-reduced over the wave.
__device__ __forceinline__ double wave_row_dot(const float *st, const uint32_t *grow, int lane, uint32_t &fl) {
    const float e1 = st[lane], e2 = st[lane + 64];
    const uint32_t b1 = (grow[lane >> 5] >> (lane & 31)) & 1u, b2 = (grow[2 + (lane >> 5)] >> (lane & 31)) & 1u;
    const float f1 = b1 ? e1 : -e1, f2 = b2 ? e2 : -e2;
    uint32_t cls = 0u;
    cls |= (f1 != f1) ? 1u : (f1 == INFINITY ? 2u : (f1 == -INFINITY ? 4u : 0u));
    cls |= (f2 != f2) ? 1u : (f2 == INFINITY ? 2u : (f2 == -INFINITY ? 4u : 0u));
    fl = (__builtin_amdgcn_ballot_w64((cls & 1u) != 0u) ? 1u : 0u) | (__builtin_amdgcn_ballot_w64((cls & 2u) != 0u) ? 2u : 0u) |
         (__builtin_amdgcn_ballot_w64((cls & 4u) != 0u) ? 4u : 0u);
    const double y1 = (double)f1, y2 = (double)f2;
    double s = y1 + y2;
    double bp = s - y1;
    double c = (y1 - (s - bp)) + (y2 - bp);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const double so = __shfl_xor(s, m), co = __shfl_xor(c, m);
        const double t = s + so;
        bp = t - s;
        const double err = (s - (t - bp)) + (so - bp);
        s = t;
        c = (c + co) + err;
    }
    return s + c;
}

template <int XDT, bool ROT, bool PAGED>
__global__ __launch_bounds__(64 * kEncWaves) void encode128_kernel(EncArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[kEncLdsBytes];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int h = blockIdx.y;
    // tensor zb (K or V of one encode_pair call): blockIdx.z, or (paged, where
    // K and V take different block counts) blocks x >= nx0 of one row
    const int zb = PAGED ? (blockIdx.x >= (unsigned)a.nx0 ? 1 : 0) : (int)blockIdx.z;
    const int64_t xb = PAGED && zb ? (int64_t)blockIdx.x - a.nx0 : (int64_t)blockIdx.x;
    const void *const xz = a.x[zb];
    uint8_t *const nibz = a.nibbles[zb];
    uint8_t *const qjlz = a.qjl[zb];
    float *const nrmz = a.norms[zb];
    const int64_t rpb = a.rows_per_block[zb];
    const int64_t v_begin = xb * rpb;
    if (v_begin >= a.nrows_head) return;                     // block-uniform, before any barrier
    const int64_t v_end = v_begin + rpb < a.nrows_head ? v_begin + rpb : a.nrows_head;

    // ── prologue: code table, centroids, G bits and bf16 images ───────
    {
        const uint4 *src = reinterpret_cast<const uint4 *>(a.table + (int64_t)(a.per_head ? h : 0) * kEncTab);
        uint4 *dst = reinterpret_cast<uint4 *>(smem);
        for (int k = tid; k < kEncTab / 16; k += 64 * kEncWaves) dst[k] = src[k];
    }
    const float *cbp = a.codebooks + (a.per_head ? h * 16 : 0);
    if (tid < 16) reinterpret_cast<float *>(smem + kEncCentOff)[tid | (tid << 4)] = cbp[tid];
    const uint32_t *gh = a.g_bits + (int64_t)h * 64 * 4;
    if (tid < 256) reinterpret_cast<uint32_t *>(smem + kEncGbitsOff)[tid] = gh[tid];
    for (int m = tid; m < 4 * 4 * 64; m += 64 * kEncWaves) {
        const int cb = m >> 8, s = (m >> 6) & 3, l = m & 63;
        const uint32_t byte = (gh[(16 * cb + (l & 15)) * 4 + s] >> (8 * (l >> 4))) & 0xffu;
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            w[k] = (((byte >> (2 * k)) & 1u) ? 0x3F80u : 0xBF80u) | ((((byte >> (2 * k + 1)) & 1u) ? 0x3F80u : 0xBF80u) << 16);
        reinterpret_cast<uint4 *>(smem + kEncGimgOff)[m] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    // sign flip as an xor on the raw 16-bit words: word j of chunk (s, g)
    // holds elements 32 s + 8 g + 2 j (low half) and + 1 (high half)
    for (int k = tid; k < 64 * 16; k += 64 * kEncWaves) {
        const int l = k >> 4, q = k & 15, sq = q >> 2, j = q & 3;
        uint32_t m = 0u;
        if (ROT && a.sign_flip) {
            const int e0 = 32 * sq + 8 * (l >> 4) + 2 * j;
            m = (a.sign_flip[e0] < 0 ? 0x8000u : 0u) | (a.sign_flip[e0 + 1] < 0 ? 0x80000000u : 0u);
        }
        reinterpret_cast<uint32_t *>(smem + kEncFlipOff)[k] = m;
    }
    __syncthreads();

    const unsigned char *tab = smem;
    const float *cent = reinterpret_cast<const float *>(smem + kEncCentOff);
    const uint32_t *gbits = reinterpret_cast<const uint32_t *>(smem + kEncGbitsOff);

    // row of lane n in the 16-row group at virtual row v (< v_end): v + n
    // (clamped) -> (b, t) -> memory row
    auto group_bt = [&](int64_t v, int64_t &bq, int64_t &t) {
        const int64_t b0 = v / a.T;                          // uniform
        t = (v - b0 * a.T) + (v + n < v_end ? n : (v_end - 1 - v));
        bq = b0;
        while (t >= a.T) { t -= a.T; ++bq; }                 // at most 16 / T + 1 steps
    };
    auto group_row = [&](int64_t v) {
        int64_t bq, t;
        group_bt(v, bq, t);
        return (bq * a.H + h) * a.T + t;
    };
    // output row of lane n's row: the memory row, or (paged) its pool row,
    // -1 where the page is outside the pool or the position past the table
    auto group_orow = [&](int64_t v, int64_t irow) -> int64_t {
        if constexpr (!PAGED) {
            return irow;
        } else {
            int64_t bq, t;
            group_bt(v, bq, t);
            const int64_t pos = (int64_t)a.positions[bq] + t;
            const int64_t pi = pos >> a.page_shift;
            const int32_t pg = (pos >= 0 && pi < a.max_pages) ? a.page_table[bq * a.max_pages + pi] : -1;
            if (pg < 0 || pg >= a.n_pages) return -1;
            return (((int64_t)pg * a.H + h) << a.page_shift) + (pos & ((1 << a.page_shift) - 1));
        }
    };
    auto load_group = [&](uint4 (&w)[4], int64_t row) {
        const uint4 *src = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(xz) + row * 128);
#pragma unroll
        for (int s = 0; s < 4; ++s) w[s] = src[4 * s + g];
    };
    // One 16-row group: w4 holds lane (n, g)'s four 16-byte chunks of row
    // mrow (virtual row v0 + n).
    auto encode_group = [&](const uint4 (&w4)[4], const int64_t mrow, const int64_t v0) {
        const bool store = v0 + n < v_end && g == 0 && (!PAGED || mrow >= 0);
        // wave priority by phase: the projection MFMAs 2, the rotation 1,
        // the rest 0, so that of a SIMD's three waves the ones in those
        // phases issue first (issue order only: results do not depend on it)
        __builtin_amdgcn_s_setprio(1);

        // flip signs on the raw words (8 x 16-bit per chunk), widen
        float x[4][8];
        uint32_t nib[4];
        double ss = 0.0;
        float as = 0.0f;
        {
            const uint4 *fmk = reinterpret_cast<const uint4 *>(smem + kEncFlipOff) + lane * 4;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const uint4 f = ROT ? fmk[s] : make_uint4(0u, 0u, 0u, 0u);
                const uint32_t w[4] = {w4[s].x ^ f.x, w4[s].y ^ f.y, w4[s].z ^ f.z, w4[s].w ^ f.w};
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t u = (i & 1) ? (w[i >> 1] >> 16) : (w[i >> 1] & 0xffffu);
                    x[s][i] = XDT == OMNI_BF16 ? __uint_as_float(u << 16) : f16_to_f32((uint16_t)u);
                }
            }
        }
        if (ROT) {
            // h = 1, 2, 4 inside each 8-element chunk
#pragma unroll
            for (int hh = 1; hh < 8; hh <<= 1)
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        if (!(i & hh)) {
                            const float u = x[s][i], l = x[s][i + hh];
                            x[s][i] = u + l;
                            x[s][i + hh] = u - l;
                        }
            // h = 8 (lanes l ^ 16), h = 16 (lanes l ^ 32)
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < 8; i += 2) xlane_pair_butterfly<16>(x[s][i], x[s][i + 1]);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < 8; i += 2) xlane_pair_butterfly<32>(x[s][i], x[s][i + 1]);
            // h = 32 (s ^ 1), h = 64 (s ^ 2)
#pragma unroll
            for (int hs = 1; hs < 4; hs <<= 1)
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    if (!(s & hs)) {
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            const float u = x[s][i], l = x[s + hs][i];
                            x[s][i] = u + l;
                            x[s + hs][i] = u - l;
                        }
                    }
        }
        __builtin_amdgcn_s_setprio(0);
        // value bits of each element ((scaled and) rounded to the input dtype)
        uint32_t vb[4][8];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                if (ROT) {
                    const float p = x[s][i] * a.scale, q = x[s][i + 1] * a.scale;
                    uint32_t pk;
                    if (XDT == OMNI_BF16) {
                        typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
                        typedef float f2_t __attribute__((ext_vector_type(2)));
                        pk = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2_t){p, q}, bf2_t));
                        x[s][i] = __uint_as_float(pk << 16);
                        x[s][i + 1] = __uint_as_float(pk & 0xffff0000u);
                    } else {
                        pk = cvt_pk_f16(p, q);
                        x[s][i] = f16_to_f32((uint16_t)(pk & 0xffffu));
                        x[s][i + 1] = f16_to_f32((uint16_t)(pk >> 16));
                    }
                    vb[s][i] = pk & 0xffffu;
                    vb[s][i + 1] = pk >> 16;
                } else if (XDT == OMNI_BF16) {
                    vb[s][i] = __float_as_uint(x[s][i]) >> 16;
                    vb[s][i + 1] = __float_as_uint(x[s][i + 1]) >> 16;
                } else {
                    vb[s][i] = f32_to_f16_rne(x[s][i]);          // exact: the value came from f16
                    vb[s][i + 1] = f32_to_f16_rne(x[s][i + 1]);
                }
            }
        // codes (all table reads issued together), then centroids
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i) vb[s][i] = tab[vb[s][i]];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            uint32_t wn = 0u;
#pragma unroll
            for (int i = 0; i < 8; i += 2)
                wn |= ((vb[s][i] & 0x0Fu) | (vb[s][i + 1] & 0xF0u)) << (4 * i);
            nib[s] = wn;
        }
        if (PAGED && zb == 1) {
            // V in the paged pool: codes only (the attention reads no V
            // residual), so no residual, norm or projection
            if (v0 + n < v_end && mrow >= 0) {
                uint32_t *np = reinterpret_cast<uint32_t *>(nibz + mrow * 64);
#pragma unroll
                for (int s = 0; s < 4; ++s) np[4 * s + g] = nib[s];
            }
            return;
        }
        float cv[4][8];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i) cv[s][i] = cent[vb[s][i]];
        // residuals, norm (fp64 sum of the exact squares) and |e| partial
        // sums, one chain per chunk s (four independent dependency chains)
        double ssp[4] = {0.0, 0.0, 0.0, 0.0};
        float asp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const float e = x[s][i] - cv[s][i];
                x[s][i] = e;
                const double ed = (double)e;
                ssp[s] = __builtin_fma(ed, ed, ssp[s]);
                asp[s] += fabsf(e);
            }
        ss = (ssp[0] + ssp[1]) + (ssp[2] + ssp[3]);
        as = (asp[0] + asp[1]) + (asp[2] + asp[3]);
        ss = xlane_sum_f64<16>(ss);
        ss = xlane_sum_f64<32>(ss);
        as = xlane_sum_f32(as);

        // projections: P^T = G . E^T on MFMA with each residual as two
        // round-to-nearest bf16 parts, e = h + m + l: h = bf16(e), m =
        // bf16(e - h) (e - h is exact), |l| <= 2^-16 |e|.  G is exactly +-1,
        // so the products are exact and the MFMA sum of G (h + m) is within
        // 1024 * 2^-24 * sum(|h| + |m|) <= 1032.1 * 2^-24 * sum|e| of its exact
        // value (fp32 accumulation of 256 terms in any order, rounding to
        // nearest or toward zero); sum|l| adds 256 * 2^-24 * sum|e|, and the
        // fp32 sum `as` is within a relative 127 * 2^-24 of sum|e|:
        // 1312 * 2^-24 * as bounds the total.  Rows with sum|e| >= 2^127
        // (where a part could round to infinity) take the exact path below.
        __builtin_amdgcn_s_setprio(2);
        float4_t acc[4];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[cb] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            uint32_t ph[4], pm[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
                typedef float f2_t __attribute__((ext_vector_type(2)));
                const float e0 = x[s][2 * j], e1 = x[s][2 * j + 1];
                const uint32_t hp = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2_t){e0, e1}, bf2_t));
                const float r0 = e0 - __uint_as_float(hp << 16);
                const float r1 = e1 - __uint_as_float(hp & 0xffff0000u);
                ph[j] = hp;
                pm[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2_t){r0, r1}, bf2_t));
            }
            const bf16x8_t bh = __builtin_bit_cast(bf16x8_t, make_uint4(ph[0], ph[1], ph[2], ph[3]));
            const bf16x8_t bm = __builtin_bit_cast(bf16x8_t, make_uint4(pm[0], pm[1], pm[2], pm[3]));
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                const uint4 gv = reinterpret_cast<const uint4 *>(smem + kEncGimgOff)[(cb * 4 + s) * 64 + lane];
                const bf16x8_t ga = __builtin_bit_cast(bf16x8_t, gv);
                acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ga, bh, acc[cb], 0, 0, 0);
                acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ga, bm, acc[cb], 0, 0, 0);
            }
        }

        __builtin_amdgcn_s_setprio(0);
        // signs: lane (n, g) holds P[n][16 cb + 4 g + i]; cb's four bits go
        // to bits 16 (cb & 1) + 4 g .. + 3 of word cb / 2
        const bool finite_row = as < 0x1p127f;                 // false for inf / NaN
        const float bound = as * 7.82012939453125e-05f + 7.888609052210118e-31f;   // 1312 * 2^-24, 2^-100
        uint32_t slo = 0u, shi = 0u;
        float amin = INFINITY;
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            const uint32_t nb = (acc[cb][0] >= 0.0f ? 1u : 0u) | (acc[cb][1] >= 0.0f ? 2u : 0u) |
                                (acc[cb][2] >= 0.0f ? 4u : 0u) | (acc[cb][3] >= 0.0f ? 8u : 0u);
            const uint32_t w = nb << (16 * (cb & 1) + 4 * g);
            if (cb < 2) slo |= w; else shi |= w;
            amin = fminf(amin, fminf(fminf(fabsf(acc[cb][0]), fabsf(acc[cb][1])), fminf(fabsf(acc[cb][2]), fabsf(acc[cb][3]))));
        }
        // rare: uncertain signs of finite rows (recomputed exactly: the 4
        // lanes of the row each sum their 32 elements, then combine) and
        // rows whose residual is not finite (or whose |e| sum reaches 2^127)
        const bool nf = !finite_row && v0 + n < v_end;
        if (__builtin_amdgcn_ballot_w64((finite_row && !(amin > bound)) || nf)) {
            uint32_t unc = 0u;
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (finite_row && !(fabsf(acc[cb][i]) > bound)) unc |= 1u << (4 * cb + i);
            // one residual row at a time goes through this wave's LDS row
            float *st = reinterpret_cast<float *>(smem + kEncStageOff) + wave * 128;
            int staged = -1;
            auto stage = [&](int r) {
                if (r == staged) return;
                if (n == r) {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int i = 0; i < 8; ++i) st[32 * q + 8 * g + i] = x[q][i];
                }
                staged = r;
            };
            uint64_t pend = __builtin_amdgcn_ballot_w64(unc != 0u);
            while (pend) {
                const int L = __builtin_ctzll(pend);
                const uint32_t uL = __builtin_amdgcn_readlane(unc, L);
                const int item = __builtin_ctz(uL);
                const int o = 16 * (item >> 2) + 4 * (L >> 4) + (item & 3);
                stage(L & 15);
                uint32_t fl;
                const double tot = wave_row_dot(st, gbits + o * 4, lane, fl);
                if (lane == L) {
                    unc &= ~(1u << item);
                    const uint32_t bit = tot >= 0.0 ? 1u : 0u;
                    const int pos = 16 * ((item >> 2) & 1) + 4 * g + (item & 3);
                    if ((item >> 2) < 2) slo = (slo & ~(1u << pos)) | (bit << pos);
                    else shi = (shi & ~(1u << pos)) | (bit << pos);
                }
                pend = __builtin_amdgcn_ballot_w64(unc != 0u);
            }
            uint64_t nfm = __builtin_amdgcn_ballot_w64(nf && g == 0);
            while (nfm) {
                const int r = __builtin_ctzll(nfm);
                nfm &= nfm - 1;
                stage(r);
#pragma unroll 1
                for (int o = 0; o < 64; ++o) {
                    // order-free sign of the fp32 sum: a NaN term or both
                    // infinities -> NaN -> 0; one infinity -> its sign; all
                    // finite (only the |e| sum overflowed) -> exact fp64 sign
                    uint32_t fl;
                    const double tot = wave_row_dot(st, gbits + o * 4, lane, fl);
                    uint32_t bit;
                    if ((fl & 1u) || (fl & 6u) == 6u) bit = 0u;
                    else if (fl & 2u) bit = 1u;
                    else if (fl & 4u) bit = 0u;
                    else bit = tot >= 0.0 ? 1u : 0u;
                    if (n == r && g == ((o & 15) >> 2)) {
                        const int pos = 16 * ((o >> 4) & 1) + 4 * g + (o & 3);
                        if ((o >> 4) < 2) slo = (slo & ~(1u << pos)) | (bit << pos);
                        else shi = (shi & ~(1u << pos)) | (bit << pos);
                    }
                }
            }
        }
        slo |= xlane_u32<16>(slo);
        slo |= xlane_u32<32>(slo);
        shi |= xlane_u32<16>(shi);
        shi |= xlane_u32<32>(shi);

        // stores: nibble dword s of lane (n, g) is bytes 16 s + 4 g .. + 3
        if (v0 + n < v_end && (!PAGED || mrow >= 0)) {
            uint32_t *np = reinterpret_cast<uint32_t *>(nibz + mrow * 64);
#pragma unroll
            for (int s = 0; s < 4; ++s) np[4 * s + g] = nib[s];
        }
        if (store) {
            reinterpret_cast<uint2 *>(qjlz + mrow * 8)[0] = make_uint2(slo, shi);
            nrmz[mrow] = ss > 3.4028234663852886e38 ? INFINITY : (float)sqrt(ss);
        }
    };

    // Groups v0, v0 + 16 nw, ... through a two-slot ring: the next group's
    // rows are requested before the current one is encoded (past the last
    // group, the current group's rows again, so every load is unconditional
    // and the compiler waits only for the slot it consumes).
    constexpr int64_t kStep = 16 * kEncWaves;
    int64_t v0 = v_begin + 16 * wave;
    if (v0 >= v_end) return;                                 // no barrier follows
    uint4 ring0[4], ring1[4];
    int64_t row0 = group_row(v0), row1;
    load_group(ring0, row0);
    for (;;) {
        row1 = v0 + kStep < v_end ? group_row(v0 + kStep) : row0;
        load_group(ring1, row1);
        encode_group(ring0, group_orow(v0, row0), v0);
        v0 += kStep;
        if (v0 >= v_end) break;
        row0 = v0 + kStep < v_end ? group_row(v0 + kStep) : row1;
        load_group(ring0, row0);
        encode_group(ring1, group_orow(v0, row1), v0);
        v0 += kStep;
        if (v0 >= v_end) break;
    }
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

// The table-driven wave kernel serves 16-bit inputs at D = 128 when each head
// has enough rows to amortise its 64 KB table; the rest (f32 inputs, D = 32,
// one-row "heads" of the row-seeded API) take the lane-per-row kernel.
static bool enc_fast(int64_t B, int64_t T, int head_dim, int x_dtype) {
    return head_dim == 128 && (x_dtype == OMNI_BF16 || x_dtype == OMNI_F16) && B * T >= 64;
}

extern "C" size_t omni_encode_workspace_size(int64_t B, int H, int64_t T, int head_dim, int x_dtype,
                                             int per_head_codebook) {
    if (B <= 0 || H <= 0 || T <= 0 || !enc_fast(B, T, head_dim, x_dtype)) return 0;
    return (size_t)(per_head_codebook ? H : 1) * kEncTab;
}

// Value-to-code tables for 16-bit inputs: one 64 KB table per codebook.
static void launch_code_tables(const float *codebooks, int per_head_codebook, int H, int x_dtype, uint8_t *tables,
                               hipStream_t st) {
    const int n_tab = per_head_codebook ? H : 1;
    if (x_dtype == OMNI_BF16)
        hipLaunchKernelGGL(code_table_kernel<OMNI_BF16>, dim3(kEncTab / 256, n_tab), dim3(256), 0, st, codebooks,
                           per_head_codebook, tables);
    else
        hipLaunchKernelGGL(code_table_kernel<OMNI_F16>, dim3(kEncTab / 256, n_tab), dim3(256), 0, st, codebooks,
                           per_head_codebook, tables);
}

// The wave kernel over nz (1 or 2) tensors of one shape, tables built.
// Paged output of the encoder (omni_encode_paged).  V rows there cost less
// (codes only): K takes this share (%) of the blocks.
constexpr int kEncPagedKShare = 55;
struct EncPaged {
    const int32_t *page_table, *positions;
    int64_t max_pages, n_pages;
    int page_shift;
};

static int launch_encode128(const void *const xs[2], int nz, int x_dtype, int64_t B, int H, int64_t T, int rotate,
                            const int8_t *sign_flip, const float *codebooks, int per_head_codebook,
                            const uint32_t *g_bits, const uint8_t *tables, uint8_t *const nib[2],
                            uint8_t *const qjl[2], float *const nrm[2], hipStream_t st,
                            const EncPaged *paged = nullptr) {
    EncArgs a{};
    for (int z = 0; z < 2; ++z) {
        const int zz = z < nz ? z : 0;
        a.x[z] = xs[zz]; a.nibbles[z] = nib[zz]; a.qjl[z] = qjl[zz]; a.norms[z] = nrm[zz];
    }
    a.table = tables; a.codebooks = codebooks; a.g_bits = g_bits; a.sign_flip = sign_flip;
    a.T = T; a.nrows_head = B * T; a.H = H; a.per_head = per_head_codebook; a.rotate = rotate;
    a.scale = inv_sqrt_dim_f32(128);
    // about one block per CU across the tensors and heads; each block a run
    // of rows of one head of one tensor
    const int cus = device_cus();
    // paged K and V: V writes codes only (about 0.4 of K's work per row),
    // so K's rows are spread over more blocks
    const int64_t grp = 16 * kEncWaves;
    const int64_t per_tensor = (cus + (int64_t)H - 1) / H;         // blocks per head over the tensors
    int64_t nxz[2] = {1, 1};
    for (int z = 0; z < 2; ++z) {
        int64_t blocks = (per_tensor + nz - 1) / nz;
        if (paged && nz == 2) blocks = z == 0 ? per_tensor * kEncPagedKShare / 100
                                              : per_tensor - per_tensor * kEncPagedKShare / 100;
        if (blocks < 1) blocks = 1;
        int64_t rpb = (a.nrows_head + blocks - 1) / blocks;
        rpb = (rpb + grp - 1) / grp * grp;
        a.rows_per_block[z] = rpb;
        nxz[z] = (a.nrows_head + rpb - 1) / rpb;
    }
    a.nx0 = (int)nxz[0];
    // paged: one grid row of K's blocks then V's (no empty blocks); else
    // blockIdx.z picks the tensor
    const int64_t nx = paged ? nxz[0] + (nz > 1 ? nxz[1] : 0) : nxz[0];
    OMNI_CHECK_ARG(nx <= 2147483647LL, "omni_encode: grid too large");
    const dim3 eg((unsigned)nx, (unsigned)H, paged ? 1u : (unsigned)nz), eb(64 * kEncWaves);
    if (paged) {
        a.page_table = paged->page_table; a.positions = paged->positions;
        a.max_pages = paged->max_pages; a.n_pages = paged->n_pages; a.page_shift = paged->page_shift;
        if (x_dtype == OMNI_BF16) {
            if (rotate) hipLaunchKernelGGL((encode128_kernel<OMNI_BF16, true, true>), eg, eb, 0, st, a);
            else hipLaunchKernelGGL((encode128_kernel<OMNI_BF16, false, true>), eg, eb, 0, st, a);
        } else {
            if (rotate) hipLaunchKernelGGL((encode128_kernel<OMNI_F16, true, true>), eg, eb, 0, st, a);
            else hipLaunchKernelGGL((encode128_kernel<OMNI_F16, false, true>), eg, eb, 0, st, a);
        }
    } else if (x_dtype == OMNI_BF16) {
        if (rotate) hipLaunchKernelGGL((encode128_kernel<OMNI_BF16, true, false>), eg, eb, 0, st, a);
        else hipLaunchKernelGGL((encode128_kernel<OMNI_BF16, false, false>), eg, eb, 0, st, a);
    } else {
        if (rotate) hipLaunchKernelGGL((encode128_kernel<OMNI_F16, true, false>), eg, eb, 0, st, a);
        else hipLaunchKernelGGL((encode128_kernel<OMNI_F16, false, false>), eg, eb, 0, st, a);
    }
    OMNI_CHECK_LAUNCH("omni_encode");
    return OMNI_OK;
}

// The lane-per-row kernel (f32 inputs, D = 32, few rows per head).
static int launch_encode_rows(const void *x, int x_dtype, int64_t B, int H, int64_t T, int head_dim, int rotate,
                              const int8_t *sign_flip, const float *codebooks, int per_head_codebook,
                              const uint32_t *g_bits, uint8_t *nibbles, uint8_t *qjl, float *norms, hipStream_t st) {
    const float s = inv_sqrt_dim_f32(head_dim);
    dim3 grid((unsigned)((T + kRowsPerBlock - 1) / kRowsPerBlock), (unsigned)H, (unsigned)B);
    if (head_dim == 128)
        hipLaunchKernelGGL(encode_kernel<128>, grid, dim3(kRowsPerBlock), 0, st, x, x_dtype, T, H,
                           rotate, sign_flip, codebooks, per_head_codebook, g_bits, nibbles, qjl, norms, s);
    else
        hipLaunchKernelGGL(encode_kernel<32>, grid, dim3(kRowsPerBlock), 0, st, x, x_dtype, T, H,
                           rotate, sign_flip, codebooks, per_head_codebook, g_bits, nibbles, qjl, norms, s);
    OMNI_CHECK_LAUNCH("omni_encode");
    return OMNI_OK;
}

extern "C" int omni_encode(const void *x, int x_dtype, int64_t B, int H, int64_t T, int head_dim,
                           int rotate, const int8_t *sign_flip, const float *codebooks,
                           int per_head_codebook, const uint32_t *g_bits,
                           uint8_t *nibbles, uint8_t *qjl, float *norms,
                           void *workspace, size_t workspace_bytes, void *stream) {
    OMNI_CHECK_ARG(dtype_ok(x_dtype), "omni_encode: bad dtype %d", x_dtype);
    OMNI_CHECK_ARG(head_dim_ok(head_dim), "omni_encode: head_dim must be 128 or 32, got %d", head_dim);
    OMNI_CHECK_ARG(B >= 0 && H >= 0 && T >= 0, "omni_encode: negative shape");
    if (B == 0 || H == 0 || T == 0) return OMNI_OK;
    OMNI_CHECK_ARG(x && codebooks && g_bits && nibbles && qjl && norms, "omni_encode: NULL pointer");
    OMNI_CHECK_ARG(B <= 65535 && H <= 65535, "omni_encode: B and H must be <= 65535");
    hipStream_t st = as_stream(stream);
    if (enc_fast(B, T, head_dim, x_dtype)) {
        const size_t need = omni_encode_workspace_size(B, H, T, head_dim, x_dtype, per_head_codebook);
        if (workspace == nullptr || workspace_bytes < need) {
            set_error("omni_encode: workspace of %zu bytes required, %zu given", need, workspace_bytes);
            return OMNI_EWORKSPACE;
        }
        uint8_t *table = reinterpret_cast<uint8_t *>(workspace);
        launch_code_tables(codebooks, per_head_codebook, H, x_dtype, table, st);
        OMNI_CHECK_LAUNCH("omni_encode (code table)");
        const void *xs[2] = {x, x};
        uint8_t *nib[2] = {nibbles, nibbles}, *qj[2] = {qjl, qjl};
        float *nr[2] = {norms, norms};
        return launch_encode128(xs, 1, x_dtype, B, H, T, rotate, sign_flip, codebooks, per_head_codebook, g_bits,
                                table, nib, qj, nr, st);
    }
    return launch_encode_rows(x, x_dtype, B, H, T, head_dim, rotate, sign_flip, codebooks, per_head_codebook, g_bits,
                              nibbles, qjl, norms, st);
}

extern "C" size_t omni_encode_tables_size(int H, int per_head_codebook) {
    if (H <= 0) return 0;
    return (size_t)(per_head_codebook ? H : 1) * kEncTab;
}

extern "C" int omni_encode_build_tables(const float *codebooks, int per_head_codebook, int H, int x_dtype,
                                        uint8_t *tables, size_t tables_bytes, void *stream) {
    OMNI_CHECK_ARG(x_dtype == OMNI_BF16 || x_dtype == OMNI_F16,
                   "omni_encode_build_tables: tables serve 16-bit inputs (dtype %d)", x_dtype);
    OMNI_CHECK_ARG(H > 0 && H <= 65535, "omni_encode_build_tables: need 1 <= H <= 65535");
    OMNI_CHECK_ARG(codebooks && tables, "omni_encode_build_tables: NULL pointer");
    const size_t need = omni_encode_tables_size(H, per_head_codebook);
    if (tables_bytes < need) {
        set_error("omni_encode_build_tables: %zu bytes of tables required, %zu given", need, tables_bytes);
        return OMNI_EWORKSPACE;
    }
    launch_code_tables(codebooks, per_head_codebook, H, x_dtype, tables, as_stream(stream));
    OMNI_CHECK_LAUNCH("omni_encode_build_tables");
    return OMNI_OK;
}

extern "C" int omni_encode_pair(const void *x0, const void *x1, int x_dtype, int64_t B, int H, int64_t T,
                                int head_dim, int rotate, const int8_t *sign_flip, const float *codebooks,
                                int per_head_codebook, const uint32_t *g_bits, const uint8_t *tables,
                                size_t tables_bytes, uint8_t *nibbles0, uint8_t *qjl0, float *norms0,
                                uint8_t *nibbles1, uint8_t *qjl1, float *norms1, void *stream) {
    OMNI_CHECK_ARG(dtype_ok(x_dtype), "omni_encode_pair: bad dtype %d", x_dtype);
    OMNI_CHECK_ARG(head_dim_ok(head_dim), "omni_encode_pair: head_dim must be 128 or 32, got %d", head_dim);
    OMNI_CHECK_ARG(B >= 0 && H >= 0 && T >= 0, "omni_encode_pair: negative shape");
    if (B == 0 || H == 0 || T == 0) return OMNI_OK;
    const int nz = x1 ? 2 : 1;
    OMNI_CHECK_ARG(x0 && codebooks && g_bits && nibbles0 && qjl0 && norms0, "omni_encode_pair: NULL pointer");
    OMNI_CHECK_ARG(nz == 1 || (nibbles1 && qjl1 && norms1), "omni_encode_pair: NULL output for the second tensor");
    OMNI_CHECK_ARG(B <= 65535 && H <= 65535, "omni_encode_pair: B and H must be <= 65535");
    hipStream_t st = as_stream(stream);
    if (enc_fast(B, T, head_dim, x_dtype)) {
        const size_t need = omni_encode_tables_size(H, per_head_codebook);
        if (tables == nullptr || tables_bytes < need) {
            set_error("omni_encode_pair: %zu bytes of code tables required, %zu given", need, tables_bytes);
            return OMNI_EWORKSPACE;
        }
        const void *xs[2] = {x0, x1 ? x1 : x0};
        uint8_t *nib[2] = {nibbles0, nz > 1 ? nibbles1 : nibbles0}, *qj[2] = {qjl0, nz > 1 ? qjl1 : qjl0};
        float *nr[2] = {norms0, nz > 1 ? norms1 : norms0};
        return launch_encode128(xs, nz, x_dtype, B, H, T, rotate, sign_flip, codebooks, per_head_codebook, g_bits,
                                tables, nib, qj, nr, st);
    }
    int rc = launch_encode_rows(x0, x_dtype, B, H, T, head_dim, rotate, sign_flip, codebooks, per_head_codebook,
                                g_bits, nibbles0, qjl0, norms0, st);
    if (rc == OMNI_OK && nz > 1)
        rc = launch_encode_rows(x1, x_dtype, B, H, T, head_dim, rotate, sign_flip, codebooks, per_head_codebook,
                                g_bits, nibbles1, qjl1, norms1, st);
    return rc;
}

extern "C" int omni_encode_paged(const void *k, const void *v, int x_dtype, int64_t B, int H, int64_t T,
                                 int rotate, const int8_t *sign_flip, const float *codebooks,
                                 int per_head_codebook, const uint32_t *g_bits, const uint8_t *tables,
                                 size_t tables_bytes, const int32_t *page_table, int64_t max_pages,
                                 const int32_t *positions, int64_t n_pages, int page_size, uint8_t *k_nibbles,
                                 uint8_t *k_qjl, float *k_norms, uint8_t *v_nibbles, void *stream) {
    OMNI_CHECK_ARG(x_dtype == OMNI_BF16 || x_dtype == OMNI_F16, "omni_encode_paged: K and V must be bf16 or f16");
    OMNI_CHECK_ARG(B >= 0 && H >= 0 && T >= 0, "omni_encode_paged: negative shape");
    if (B == 0 || H == 0 || T == 0) return OMNI_OK;
    OMNI_CHECK_ARG(k && codebooks && g_bits && page_table && positions && k_nibbles && k_qjl && k_norms,
                   "omni_encode_paged: NULL pointer");
    OMNI_CHECK_ARG(v == nullptr || v_nibbles, "omni_encode_paged: NULL V pool for a V input");
    OMNI_CHECK_ARG(B <= 65535 && H <= 65535, "omni_encode_paged: B and H must be <= 65535");
    int shift = 4;
    while (shift < 11 && (1 << shift) < page_size) ++shift;
    OMNI_CHECK_ARG(page_size >= 16 && page_size <= 1024 && (1 << shift) == page_size,
                   "omni_encode_paged: page_size must be a power of two in [16, 1024], got %d", page_size);
    OMNI_CHECK_ARG(n_pages >= 1 && max_pages >= 1, "omni_encode_paged: need n_pages >= 1, max_pages >= 1");
    OMNI_CHECK_ARG(n_pages * H * (int64_t)page_size < (int64_t(1) << 40), "omni_encode_paged: pool too large");
    const size_t need = omni_encode_tables_size(H, per_head_codebook);
    if (tables == nullptr || tables_bytes < need) {
        set_error("omni_encode_paged: %zu bytes of code tables required, %zu given", need, tables_bytes);
        return OMNI_EWORKSPACE;
    }
    const int nz = v ? 2 : 1;
    const void *xs[2] = {k, v ? v : k};
    uint8_t *nib[2] = {k_nibbles, v ? v_nibbles : k_nibbles}, *qj[2] = {k_qjl, k_qjl};
    float *nr[2] = {k_norms, k_norms};
    const EncPaged pg{page_table, positions, max_pages, n_pages, shift};
    return launch_encode128(xs, nz, x_dtype, B, H, T, rotate, sign_flip, codebooks, per_head_codebook, g_bits,
                            tables, nib, qj, nr, as_stream(stream), &pg);
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
