// Dense fp32 GQA attention on already dequantized K / V (gfx950).
//
// Reference: reference_attn (omnistack_rs/attention/reference.py:72-177),
// the CPU path's attention: fp32 scores q . k * scale (+ an additive mask
// broadcastable to (B, Hq, T, S)), online softmax over key tiles, fp32
// P . V, output O / l; kv head of q head h = h / (Hq / Hkv) (repeat_kv,
// :49-67) without materialising the repeated K / V.
//
// One block per (64 query rows of one (batch, kv head), kv head, batch):
// four waves of 16 rows (row r = t * G + g of that kv head).  Keys go
// through LDS in tiles of 32; scores and P . V run on
// v_mfma_f32_16x16x4_f32 (fp32 products, fp32 accumulation), the softmax in
// fp32 with expf.  The running-max update is the reference's, made safe for
// tiles whose scores are all -inf (alpha and p are 0 there instead of
// exp(-inf - -inf)); the reference's own result for a row whose whole first
// tile of `first_tile` keys is masked (NaN) is reproduced explicitly, and a
// NaN score makes its row NaN as torch.maximum / amax propagate it.
#include <math.h>

#include "omni_common.h"

namespace omni {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct DenseArgs {
    const float *q, *k, *v, *mask;
    float *out;
    int64_t ms_b, ms_h, ms_t, ms_s;   // mask strides in elements (0: broadcast)
    int64_t T, S, rows, first_tile;
    int Hq, Hkv, G;
    float scale;
};

constexpr int kDnKeys = 32;
constexpr int kDnWaves = 4;
constexpr int kDnRows = 16 * kDnWaves;
constexpr int kDnPStride = kDnKeys + 4;

__device__ __forceinline__ float dn_max16(float v) {
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}
__device__ __forceinline__ float dn_sum16(float v) {
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) v += __shfl_xor(v, m);
    return v;
}

template <int D>
__global__ __launch_bounds__(64 * kDnWaves) void dense_attn_kernel(DenseArgs a) {
    constexpr int DP = D + 4;                     // padded LDS row (floats)
    __shared__ __attribute__((aligned(16))) float ks[kDnKeys * DP];
    __shared__ __attribute__((aligned(16))) float vs[kDnKeys * DP];
    __shared__ float ps[kDnWaves][16 * kDnPStride];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int hk = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int64_t row0 = (int64_t)blockIdx.x * kDnRows + 16 * wave;

    // A operands of the scores: q row (row0 + n), dims 4 s + g
    float qa[D / 4];
    {
        const int64_t r = row0 + n;
        const bool ok = r < a.rows;
        const int64_t t = ok ? r / a.G : 0;
        const int hq = hk * a.G + (ok ? (int)(r % a.G) : 0);
        const float *qrow = a.q + ((b * a.Hq + hq) * a.T + t) * D;
#pragma unroll
        for (int s = 0; s < D / 4; ++s) qa[s] = ok ? qrow[4 * s + g] : 0.0f;
    }
    // this lane's output rows row0 + 4 g + i
    bool rok[4];
    int64_t rt[4];
    int rh[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t r = row0 + 4 * g + i;
        rok[i] = r < a.rows;
        rt[i] = rok[i] ? r / a.G : 0;
        rh[i] = hk * a.G + (rok[i] ? (int)(r % a.G) : 0);
    }

    f32x4_t o[D / 16];
#pragma unroll
    for (int j = 0; j < D / 16; ++j) o[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m[4], l[4];
    bool seen0[4], nan_row[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
        seen0[i] = false;
        nan_row[i] = false;
    }
    const float *kb0 = a.k + ((int64_t)b * a.Hkv + hk) * a.S * D;
    const float *vb0 = a.v + ((int64_t)b * a.Hkv + hk) * a.S * D;
    // waves whose 16 rows are all past the end only help stage K / V
    const bool active = row0 < a.rows;

    // the next tile's K / V sit in registers while the current one is used
    constexpr int kPer = kDnKeys * D / (4 * 64 * kDnWaves);   // float4 per thread per tile
    float4 nk[kPer], nv[kPer];
    auto fetch = [&](int64_t s0) {
#pragma unroll
        for (int c = 0; c < kPer; ++c) {
            const int e = 4 * (tid + c * 64 * kDnWaves);
            const int key = e / D, d = e - key * D;
            nk[c] = nv[c] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (s0 + key < a.S) {
                nk[c] = *reinterpret_cast<const float4 *>(kb0 + (s0 + key) * D + d);
                nv[c] = *reinterpret_cast<const float4 *>(vb0 + (s0 + key) * D + d);
            }
        }
    };
    fetch(0);

    for (int64_t s0 = 0; s0 < a.S; s0 += kDnKeys) {
        __syncthreads();                          // the previous tile is consumed
#pragma unroll
        for (int c = 0; c < kPer; ++c) {
            const int e = 4 * (tid + c * 64 * kDnWaves);
            const int key = e / D, d = e - key * D;
            *reinterpret_cast<float4 *>(ks + key * DP + d) = nk[c];
            *reinterpret_cast<float4 *>(vs + key * DP + d) = nv[c];
        }
        __syncthreads();
        if (s0 + kDnKeys < a.S) fetch(s0 + kDnKeys);
        if (!active) continue;

        // scores: key block kb holds keys s0 + 16 kb + n
        f32x4_t acc[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            acc[kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < D / 4; ++s)
                acc[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[s], ks[(16 * kb + n) * DP + 4 * s + g], acc[kb],
                                                               0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float sc[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int64_t key = s0 + 16 * kb + n;
                float v = acc[kb][i] * a.scale;
                if (key < a.S) {
                    if (a.mask != nullptr && rok[i])
                        v += a.mask[b * a.ms_b + rh[i] * a.ms_h + rt[i] * a.ms_t + key * a.ms_s];
                } else {
                    v = -INFINITY;
                }
                sc[kb] = v;
            }
            // NaN scores poison the row (torch.maximum / amax propagate NaN)
            const float isn = (sc[0] != sc[0] || sc[1] != sc[1]) ? 1.0f : 0.0f;
            nan_row[i] = nan_row[i] || dn_max16(isn) > 0.0f;
            // any finite score among the reference's first tile of keys
            float f0 = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
                if (s0 + 16 * kb + n < a.first_tile) f0 = fmaxf(f0, sc[kb]);
            seen0[i] = seen0[i] || dn_max16(f0) > -INFINITY;

            const float mt = dn_max16(fmaxf(sc[0], sc[1]));
            const float m_new = fmaxf(m[i], mt);
            const float alpha = (m[i] == -INFINITY) ? 0.0f : expf(m[i] - m_new);
            float p[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) p[kb] = (m_new == -INFINITY) ? 0.0f : expf(sc[kb] - m_new);
            const float psum = dn_sum16(p[0] + p[1]);
            l[i] = alpha * l[i] + psum;           // two roundings, as the reference
#pragma unroll
            for (int j = 0; j < D / 16; ++j) o[j][i] *= alpha;
            m[i] = m_new;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) ps[wave][(4 * g + i) * kDnPStride + 16 * kb + n] = p[kb];
        }
        // P goes through this wave's own LDS rows: program order suffices
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float pa[kDnKeys / 4];
#pragma unroll
        for (int s = 0; s < kDnKeys / 4; ++s) pa[s] = ps[wave][n * kDnPStride + 4 * s + g];
#pragma unroll
        for (int j = 0; j < D / 16; ++j)
#pragma unroll
            for (int s = 0; s < kDnKeys / 4; ++s)
                o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[s], vs[(4 * s + g) * DP + 16 * j + n], o[j], 0, 0, 0);
    }

#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (!rok[i]) continue;
        float *orow = a.out + ((b * a.Hq + rh[i]) * a.T + rt[i]) * D;
        const bool nan_out = nan_row[i] || !seen0[i];
#pragma unroll
        for (int j = 0; j < D / 16; ++j) orow[16 * j + n] = nan_out ? __builtin_nanf("") : o[j][i] / l[i];
    }
}

// Few query rows per (batch, kv head) (decode: T * G <= 16): the NW waves
// share one group of 16 rows and split the keys in 16-key chunks (wave w
// takes chunks w, w + NW, ...), each keeping its own online-softmax state;
// the states are merged in LDS at the end (max, then the exp-weighted sums in
// wave order).  K and V go from HBM straight into MFMA operand registers (no
// LDS staging, no block barrier per tile), two chunks in flight per wave.
// Scores: step s's k axis is dims 4 s .. 4 s + 3 (lane group g: dim 4 s + g,
// the summation order of the LDS-staged kernel this replaced); lane (n, g)
// loads 16-byte pieces 16 t + 4 g .. of key n and a 4 x 4 transpose across
// its four lane groups (two permlane swap stages) hands each lane its dims.
// P V: lane (n, g) holds dims (D/16) n .. + D/16 - 1 of keys 4 s + g, so
// output column n of MFMA j is dim (D/16) n + j.
#ifndef OMNI_DN_KS_WAVES
#define OMNI_DN_KS_WAVES 8
#endif
constexpr int kDnKsWaves = OMNI_DN_KS_WAVES;

template <int D>
struct DnChunk {
    float k[D / 4];       // key 16 c + n: k[s] = dim 4 s + g (after the transpose)
    float v[D / 4];       // keys 16 c + 4 s + g (s = 0..3), dims (D/16) n ..: v[s * D/16 + j]
};

// 4 x 4 transpose across the four 16-lane rows: on entry row r of x[c]
// holds M[r][c], on exit M[c][r].
__device__ __forceinline__ void dn_transpose4(float (&x)[4]) {
    auto swap32 = [](float &a, float &b) {
        const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
        a = __uint_as_float(t[0]);
        b = __uint_as_float(t[1]);
    };
    auto swap16 = [](float &a, float &b) {
        const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
        a = __uint_as_float(t[0]);
        b = __uint_as_float(t[1]);
    };
    swap32(x[0], x[2]);
    swap32(x[1], x[3]);
    swap16(x[0], x[1]);
    swap16(x[2], x[3]);
}

template <int D, int NW>
__global__ __launch_bounds__(64 * NW) void dense_attn_ks_kernel(DenseArgs a) {
    constexpr int DQ = D / 4, DV = D / 16, DP = D + 4;
    static_assert(DQ % 4 == 0 && (DV % 4 == 0 || DV == 2), "16- or 8-byte operand loads");
    __shared__ float ps[NW][16 * 20];
    __shared__ float wst[NW][16][4];             // per wave and row: m, l, seen0, nan
    __shared__ __attribute__((aligned(16))) float op[NW * 16 * DP];   // per wave and row: O
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int hk = blockIdx.y;
    const int64_t b = blockIdx.z;

    float qa[DQ];                                 // qa[s] = dim 4 s + g of query row n
    {
        const int64_t r = n;
        const bool ok = r < a.rows;
        const int64_t t = ok ? r / a.G : 0;
        const int hq = hk * a.G + (ok ? (int)(r % a.G) : 0);
        const float *qrow = a.q + ((b * a.Hq + hq) * a.T + t) * D;
#pragma unroll
        for (int s = 0; s < DQ; ++s) qa[s] = ok ? qrow[4 * s + g] : 0.0f;
    }
    // mask offset of row 4 g + i (key 0); rows past the last add nothing
    bool rok[4];
    int64_t mrow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 4 * g + i;
        rok[i] = r < a.rows;
        const int t = rok[i] ? r / a.G : 0;
        const int hq = hk * a.G + (rok[i] ? r % a.G : 0);
        mrow[i] = b * a.ms_b + hq * a.ms_h + t * a.ms_t;
    }
    f32x4_t o[DV];
#pragma unroll
    for (int j = 0; j < DV; ++j) o[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m[4], l[4];
    bool seen0[4], nan_row[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
        seen0[i] = false;
        nan_row[i] = false;
    }
    const float *kb0 = a.k + ((int64_t)b * a.Hkv + hk) * a.S * D;
    const float *vb0 = a.v + ((int64_t)b * a.Hkv + hk) * a.S * D;
    const int S = (int)a.S;                                 // < 2^27 (host check)
    const int nch = (S + 15) / 16;
    // chunk c's operands; keys past S read the last key (a valid address)
    // and their V is zeroed (their P is 0, and 0 * inf would be NaN)
    auto load = [&](DnChunk<D> &R, int c) {
        const int key = 16 * c + n, kk = key < S ? key : S - 1;
        // piece t: dims 16 t + 4 g .. + 3 of key n (transposed at use)
        const float4 *kp = reinterpret_cast<const float4 *>(kb0 + (int64_t)kk * D + 4 * g);
#pragma unroll
        for (int t = 0; t < DQ / 4; ++t) {
            const float4 w = kp[4 * t];
            R.k[4 * t] = w.x; R.k[4 * t + 1] = w.y; R.k[4 * t + 2] = w.z; R.k[4 * t + 3] = w.w;
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int vk = 16 * c + 4 * s + g, vv = vk < S ? vk : S - 1;
            const bool z = vk >= S;
            if constexpr (DV == 2) {
                const float2 w = *reinterpret_cast<const float2 *>(vb0 + (int64_t)vv * D + DV * n);
                R.v[s * DV] = z ? 0.0f : w.x;
                R.v[s * DV + 1] = z ? 0.0f : w.y;
            } else {
                const float4 *vp = reinterpret_cast<const float4 *>(vb0 + (int64_t)vv * D + DV * n);
#pragma unroll
                for (int h = 0; h < DV / 4; ++h) {
                    const float4 w = vp[h];
                    R.v[s * DV + 4 * h] = z ? 0.0f : w.x;
                    R.v[s * DV + 4 * h + 1] = z ? 0.0f : w.y;
                    R.v[s * DV + 4 * h + 2] = z ? 0.0f : w.z;
                    R.v[s * DV + 4 * h + 3] = z ? 0.0f : w.w;
                }
            }
        }
    };
    auto step = [&](const DnChunk<D> &R, int c) {
        // all pieces transposed first: the swaps do not wait on the MFMA chain
        float kx[DQ / 4][4];
#pragma unroll
        for (int t = 0; t < DQ / 4; ++t) {
#pragma unroll
            for (int u = 0; u < 4; ++u) kx[t][u] = R.k[4 * t + u];
            dn_transpose4(kx[t]);                     // kx[t][u] = dim 16 t + 4 u + g
        }
        f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < DQ / 4; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * t + u], kx[t][u], acc, 0, 0, 0);
        const int key = 16 * c + n;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = acc[i] * a.scale;
            if (key < S) {
                if (a.mask != nullptr && rok[i]) v += a.mask[mrow[i] + key * a.ms_s];
            } else {
                v = -INFINITY;
            }
            nan_row[i] = nan_row[i] || dn_max16(v != v ? 1.0f : 0.0f) > 0.0f;
            seen0[i] = seen0[i] || dn_max16(key < a.first_tile ? v : -INFINITY) > -INFINITY;
            const float mt = dn_max16(v);
            const float m_new = fmaxf(m[i], mt);
            const float alpha = (m[i] == -INFINITY) ? 0.0f : expf(m[i] - m_new);
            const float p = (m_new == -INFINITY) ? 0.0f : expf(v - m_new);
            l[i] = alpha * l[i] + dn_sum16(p);
#pragma unroll
            for (int j = 0; j < DV; ++j) o[j][i] *= alpha;
            m[i] = m_new;
            ps[wave][(4 * g + i) * 20 + n] = p;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float pa[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) pa[s] = ps[wave][n * 20 + 4 * s + g];
        // the next chunk's P writes must not pass these reads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int j = 0; j < DV; ++j)
#pragma unroll
            for (int s = 0; s < 4; ++s) o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[s], R.v[s * DV + j], o[j], 0, 0, 0);
    };
    if (wave < nch) {
        // two chunks in flight: loads past the last chunk read valid
        // addresses and are never consumed
        DnChunk<D> r0, r1;
        load(r0, wave);
        for (int c = wave;; c += 2 * NW) {
            load(r1, c + NW);
            step(r0, c);
            if (c + NW >= nch) break;
            load(r0, c + 2 * NW);
            step(r1, c + NW);
            if (c + 2 * NW >= nch) break;
        }
    }

    // merge the waves' states
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < DV; ++j) op[(wave * 16 + 4 * g + i) * DP + DV * n + j] = o[j][i];
        if (n == 0) {
            wst[wave][4 * g + i][0] = m[i];
            wst[wave][4 * g + i][1] = l[i];
            wst[wave][4 * g + i][2] = seen0[i] ? 1.0f : 0.0f;
            wst[wave][4 * g + i][3] = nan_row[i] ? 1.0f : 0.0f;
        }
    }
    __syncthreads();
    for (int e = tid; e < 16 * D; e += 64 * NW) {
        const int r = e / D, d = e - r * D;
        const int64_t row = r;
        if (row >= a.rows) continue;
        float mx = -INFINITY;
        bool s0seen = false, isnan_row = false;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            mx = fmaxf(mx, wst[w][r][0]);
            s0seen = s0seen || wst[w][r][2] != 0.0f;
            isnan_row = isnan_row || wst[w][r][3] != 0.0f;
        }
        float lsum = 0.0f, osum = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float f = (wst[w][r][0] == -INFINITY) ? 0.0f : expf(wst[w][r][0] - mx);
            lsum += f * wst[w][r][1];
            osum += f * op[(w * 16 + r) * DP + d];
        }
        const int64_t t = row / a.G;
        const int hq = hk * a.G + (int)(row % a.G);
        a.out[((b * a.Hq + hq) * a.T + t) * D + d] = (isnan_row || !s0seen) ? __builtin_nanf("") : osum / lsum;
    }
}

}  // namespace omni

using namespace omni;

extern "C" int omni_dense_attn(const float *q, const float *k, const float *v, const float *mask,
                               const int64_t *mask_strides, int64_t B, int Hq, int Hkv, int64_t T, int64_t S,
                               int head_dim, float scale, int64_t first_tile, float *out, void *stream) {
    OMNI_CHECK_ARG(head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256,
                   "omni_dense_attn: head_dim must be 32, 64, 128 or 256, got %d", head_dim);
    OMNI_CHECK_ARG(B >= 0 && Hq > 0 && Hkv > 0 && T >= 0 && S >= 0 && Hq % Hkv == 0,
                   "omni_dense_attn: bad shape");
    OMNI_CHECK_ARG(first_tile >= 1, "omni_dense_attn: first_tile must be >= 1");
    if (B == 0 || T == 0) return OMNI_OK;
    OMNI_CHECK_ARG(q && k && v && out, "omni_dense_attn: NULL pointer");
    OMNI_CHECK_ARG(mask == nullptr || mask_strides != nullptr, "omni_dense_attn: mask without strides");
    OMNI_CHECK_ARG(B <= 65535 && Hkv <= 65535, "omni_dense_attn: grid too large");
    const int G = Hq / Hkv;
    const int64_t rows = T * G;
    const int64_t chunks = (rows + kDnRows - 1) / kDnRows;
    OMNI_CHECK_ARG(chunks <= 2147483647, "omni_dense_attn: too many query rows");
    DenseArgs a;
    a.q = q; a.k = k; a.v = v; a.mask = mask; a.out = out;
    a.ms_b = mask ? mask_strides[0] : 0;
    a.ms_h = mask ? mask_strides[1] : 0;
    a.ms_t = mask ? mask_strides[2] : 0;
    a.ms_s = mask ? mask_strides[3] : 0;
    a.T = T; a.S = S; a.rows = rows; a.first_tile = first_tile < S ? first_tile : S;
    a.Hq = Hq; a.Hkv = Hkv; a.G = G;
    a.scale = scale;
    if (S == 0) a.first_tile = 0;   // no keys: every row is NaN (0 / 0), as the reference
    hipStream_t st = as_stream(stream);
    if (rows <= 16 && head_dim <= 128 && S < (int64_t(1) << 27)) {
        // few rows: the waves split the keys instead of the rows
        const dim3 grid(1u, (unsigned)Hkv, (unsigned)B), block(64 * kDnKsWaves);
        if (head_dim == 32) hipLaunchKernelGGL((dense_attn_ks_kernel<32, kDnKsWaves>), grid, block, 0, st, a);
        else if (head_dim == 64) hipLaunchKernelGGL((dense_attn_ks_kernel<64, kDnKsWaves>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((dense_attn_ks_kernel<128, kDnKsWaves>), grid, block, 0, st, a);
        OMNI_CHECK_LAUNCH("omni_dense_attn");
        return OMNI_OK;
    }
    const dim3 grid((unsigned)chunks, (unsigned)Hkv, (unsigned)B), block(64 * kDnWaves);
    switch (head_dim) {
        case 32: hipLaunchKernelGGL(dense_attn_kernel<32>, grid, block, 0, st, a); break;
        case 64: hipLaunchKernelGGL(dense_attn_kernel<64>, grid, block, 0, st, a); break;
        case 128: hipLaunchKernelGGL(dense_attn_kernel<128>, grid, block, 0, st, a); break;
        default: hipLaunchKernelGGL(dense_attn_kernel<256>, grid, block, 0, st, a); break;
    }
    OMNI_CHECK_LAUNCH("omni_dense_attn");
    return OMNI_OK;
}
