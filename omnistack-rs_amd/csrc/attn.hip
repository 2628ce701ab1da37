// Attention over the packed INT4 + QJL cache on gfx950 (decode: T = 1;
// any T works, rows = query tokens x GQA heads).
//
// Reference semantics: _fused_attn_python + reference_attn
// (omnistack_rs/kernels/fused_attention.py:435-466,
//  omnistack_rs/attention/reference.py:72-177): K_hat with QJL, V INT4
// (same per-head codebook), fp32 online softmax, GQA kv = hq / (Hq/Hkv).
// The QJL term enters as a score correction
//   q . k_hat = q . cb[code] + alpha_s * sum_i b+-_i (G_h q)_i,
//   alpha_s = ||e_s|| sqrt(2/pi) / D,
// with the encoder's per-head G (seed (user % 1024) ^ h).
//
// Work decomposition.  One block streams one (batch, kv head, token split)
// for up to 16 query rows (all GQA heads of the group for one or more query
// tokens), so every cached byte is read once per group, not once per q head.
// Each wave takes 16-token tiles round-robin and runs three MFMA chains
// (v_mfma_f32_16x16x16_f16, tokens on M, query rows on N):
//   S^T  = K16 (16 x D) . (scale log2e Q16)^T, three fp16 passes
//          (K_hi.Q_hi + K_hi.Q_lo + K_lo.Q_hi)         3 * D/16 k-steps
//   C^T  = B+-     (16 x D/2) . (scale log2e G Q)^T      D/32 k-steps
//   O^T += V^T_hi (D x 16)   . P^T ; O^T += V^T_lo . P^T  D/16 row blocks
// Codebook values enter as fp16 hi + fp16 remainder (one 8-byte LDS lookup
// per cache byte gives both halves of two codes); q is split the same way,
// so scores and values keep ~22 bits.  Online softmax in fp32 (exp2 domain) with P rounded to fp16 for
// the PV product; the softmax denominator sums the same rounded P.
#include <math.h>

#include <atomic>
#include <mutex>
#include <new>
#include <type_traits>

#include "omni_common.h"

namespace omni {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kTile = 16;      // tokens per MFMA tile
constexpr int kRows = 16;      // query rows per block (MFMA N)
constexpr int kMaxWaves = 8;

struct AttnArgs {
    const void *q;
    const uint8_t *k_nib;
    const uint8_t *k_qjl;
    const float *k_norms;
    const uint8_t *v_nib;
    const float *codebooks;
    const uint32_t *g_bits;
    const int8_t *sign_flip;
    float *out;
    float *ws;                 // split partials: [unit][split][row][D + 2]
    int64_t T, S, split_len;
    int64_t causal_offset;     // < 0: no mask
    int q_dtype, per_head, Hq, Hkv, G, n_rchunks, splits, ncopy;
    int with_qjl, rotate_q;
    uint64_t g_magic, rch_magic;   // floor(2^32 / d) + 1 for d = G, n_rchunks
    int64_t B;
    // cache sequence of batch entry b: seq_index[b] into a pool of n_seqs
    // sequences (NULL: b itself)
    const int64_t *seq_index;
    int64_t n_seqs;
    int spb;                   // D=128 decode: sequences per block (1, or 2 when T * G <= 4)
    // per-user LoRA on q, fused into the D=128 decode prologue (lora_w_dtype < 0: none)
    const void *lora_x, *lora_a, *lora_b;
    const int32_t *lora_idx;
    int lora_w_dtype, lora_hidden, lora_rank, lora_n;
    float lora_alpha;
    int rows;                  // query rows per block (16: generic kernel, 8: D=128 decode kernel)
    // paged cache (D=128 decode kernel): pool arrays shaped like a contiguous
    // cache with (n_pages, Hkv, page_size); sequence b holds seq_lens[b]
    // tokens in pages page_table[b * max_pages + j] (S = max_pages * page_size)
    const int32_t *page_table;
    const int32_t *seq_lens;
    int64_t max_pages, n_pages;
    int page_size, page_shift;  // page_size = 2^page_shift >= 16
    float qscale;              // scale * log2(e)
    float alpha_c;             // fp32 sqrt(2/pi)/D (the row scale multiplies the whole score)
    float wht_scale;
};

__device__ __forceinline__ int64_t imin64(int64_t x, int64_t y) { return x < y ? x : y; }
__device__ __forceinline__ int64_t imax64(int64_t x, int64_t y) { return x > y ? x : y; }

// Cache sequence read for batch entry b (wave-uniform).  Negative indices
// count from the end of the pool, as tensor indexing does; an index outside
// [-n_seqs, n_seqs) reads sequence 0 and sets `bad` (its rows come out NaN).
__device__ __forceinline__ int64_t cache_seq(const AttnArgs &a, int64_t b, bool &bad) {
    if (a.seq_index == nullptr) {
        bad = false;
        return b;
    }
    int64_t v = a.seq_index[b];
    v = v < 0 ? v + a.n_seqs : v;
    bad = v < 0 || v >= a.n_seqs;
    return bad ? 0 : v;
}

// floor(x / d) for 0 <= x, d < 2^16 as (x * (floor(2^32 / d) + 1)) >> 32:
// the excess x * e / 2^32 (0 < e <= 1) stays below 1/d, so the floor is
// exact.  Branch- and division-free, so the kernel-argument loads are not
// split around a division sequence.
__device__ __forceinline__ int div_small(int x, uint64_t magic) {
    return (int)(((uint64_t)(uint32_t)x * magic) >> 32);
}
__device__ __forceinline__ int imin(int x, int y) { return x < y ? x : y; }
__device__ __forceinline__ int imax(int x, int y) { return x > y ? x : y; }

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    return (uint32_t)f32_to_f16_rne(a) | ((uint32_t)f32_to_f16_rne(b) << 16);
}

__device__ __forceinline__ half4_t as_half4(uint32_t lo, uint32_t hi) {
    uint2 t = make_uint2(lo, hi);
    return __builtin_bit_cast(half4_t, t);
}

__device__ __forceinline__ float wave_max_xor16_32(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}

__device__ __forceinline__ float wave_sum_xor16_32(float v) {
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

// Dynamic LDS layout (bytes):
//   lut   256*ncopy uint2    byte -> (hi pair, lo pair): fp16 hi(cb[lo nib]),
//                            hi(cb[hi nib]) and the fp16 remainders cb - hi
//   qlut  16 uint2           QJL nibble -> four +-1.0 halves
//   qs    kRows*D f32        query rows (fp32, rotated if requested)
//   gq    kRows*D/2 f32      G_h q rows
// The combine phase reuses [0, ...) after the main loop.
template <int D>
struct Lds {
    static constexpr int QD = D / 2;
    __host__ __device__ static size_t lut_bytes(int ncopy) { return (size_t)256 * ncopy * 8 + 16 * 8; }
    __host__ __device__ static size_t comb_bytes(int nw) { (void)nw; return (size_t)(2 * kMaxWaves * kRows + kRows * D) * 4; }
    __host__ __device__ static size_t fixed_bytes() { return (size_t)kRows * (D + QD + 1) * 4; }
    static size_t total(int ncopy, int nw) {
        size_t a = lut_bytes(ncopy), c = comb_bytes(nw);
        return (a > c ? a : c) + fixed_bytes();
    }
};

template <int D>
__global__ __launch_bounds__(64 * kMaxWaves) void attn_kernel(AttnArgs a) {
    constexpr int QD = D / 2;
    constexpr int KSTEPS = D / 16;      // QK k-steps (16 d each)
    constexpr int QSTEPS = QD / 16;     // QJL k-steps (16 signs each) (>= 1)
    constexpr int VB = D / 32;          // V bytes per lane per token
    constexpr int NBLK = 2 * VB;        // PV row blocks (16 d each)

    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int ncopy = a.ncopy;
    uint2 *vlut = reinterpret_cast<uint2 *>(smem);
    uint2 *qlut = reinterpret_cast<uint2 *>(smem + (size_t)256 * ncopy * 8);
    const int nw = blockDim.x >> 6;
    const size_t var_bytes = Lds<D>::lut_bytes(ncopy) > Lds<D>::comb_bytes(nw) ? Lds<D>::lut_bytes(ncopy)
                                                                                 : Lds<D>::comb_bytes(nw);
    float *qs = reinterpret_cast<float *>(smem + var_bytes);
    float *gq = qs + kRows * D;
    float *rsc = gq + kRows * QD;       // per row: scale * log2(e) / 2^k

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int split = blockIdx.x;
    const int hk = blockIdx.y;
    const int64_t bz = blockIdx.z;
    const int64_t b = bz / a.n_rchunks;
    const int rc = (int)(bz % a.n_rchunks);
    const int64_t nrows_total = a.T * a.G;

    // ── prologue: LUTs ────────────────────────────────────────────────
    const float *cbp = a.codebooks + (a.per_head ? hk * 16 : 0);
    for (int s = tid; s < 256 * ncopy; s += blockDim.x) {
        const int e = s / ncopy;
        const float c0 = cbp[e & 15], c1 = cbp[e >> 4];
        const float h0 = f16_to_f32(f32_to_f16_rne(c0)), h1 = f16_to_f32(f32_to_f16_rne(c1));
        vlut[s] = make_uint2(pack_h2(c0, c1), pack_h2(c0 - h0, c1 - h1));
    }
    if (tid < 16) {
        uint32_t w[2];
        for (int k = 0; k < 2; ++k) {
            const uint32_t b0 = (tid >> (2 * k)) & 1u, b1 = (tid >> (2 * k + 1)) & 1u;
            w[k] = (b0 ? 0x3C00u : 0xBC00u) | ((b1 ? 0x3C00u : 0xBC00u) << 16);
        }
        qlut[tid] = make_uint2(w[0], w[1]);
    }

    // ── prologue: query rows (row r <-> flat (t, gh) = rc*16 + r) ─────
    for (int s = tid; s < kRows * D; s += blockDim.x) {
        const int r = s / D, d = s % D;
        const int64_t rho = (int64_t)rc * kRows + r;
        float v = 0.0f;
        if (rho < nrows_total) {
            const int64_t t = rho / a.G;
            const int hq = hk * a.G + (int)(rho % a.G);
            v = load_as_f32(a.q, a.q_dtype, ((b * a.Hq + hq) * a.T + t) * D + d);
        }
        qs[s] = v;
    }
    __syncthreads();
    if (a.rotate_q && tid < kRows) {
        // rotate_queries in-kernel: dtype(WHT(sign_flip * q)), hadamard.py:51-85.
        float *row = qs + tid * D;
        if (a.sign_flip)
            for (int d = 0; d < D; ++d) row[d] = a.sign_flip[d] < 0 ? -row[d] : row[d];
        for (int h = 1; h < D; h <<= 1)
            for (int base = 0; base < D; base += 2 * h)
                for (int i = 0; i < h; ++i) {
                    const float u = row[base + i], l = row[base + h + i];
                    row[base + i] = u + l;
                    row[base + h + i] = u - l;
                }
        for (int d = 0; d < D; ++d) row[d] = round_to_dtype(row[d] * a.wht_scale, a.q_dtype);
    }
    __syncthreads();
    if (tid < kRows) {
        // row max |q| -> 2^k with max * 2^k in [2^14, 2^15): the scaled row
        // and G q stay in fp16 range for any finite q
        float *row = qs + tid * D;
        float m = 0.0f;
        for (int d = 0; d < D; ++d) m = fmaxf(m, fabsf(row[d]));
        int ex = 0;
        if (m > 0.0f && m < INFINITY) frexpf(m, &ex);
        const float sr = ldexpf(1.0f, 15 - imax(ex, -100));
        for (int d = 0; d < D; ++d) row[d] *= sr;
        rsc[tid] = a.qscale / sr;
    }
    __syncthreads();
    if (a.with_qjl) {
        const uint32_t *gh = a.g_bits + (int64_t)hk * QD * (D / 32);
        for (int s = tid; s < kRows * QD; s += blockDim.x) {
            const int r = s / QD, i = s % QD;
            const float *row = qs + r * D;
            float acc = 0.0f;
            for (int j = 0; j < D; ++j) {
                const float g = ((gh[i * (D / 32) + (j >> 5)] >> (j & 31)) & 1u) ? 1.0f : -1.0f;
                acc = __builtin_fmaf(g, row[j], acc);
            }
            gq[s] = acc;
        }
    }
    __syncthreads();

    // ── per-lane MFMA B operands ──────────────────────────────────────
    const int r = lane & 15;          // query row (MFMA column)
    const int g = lane >> 4;          // k-group
    // Q in two fp16 halves (hi + remainder): with the codebook's hi/lo split
    // the score keeps ~22 bits (hi.hi + lo_q.hi + hi.lo_k).
    half4_t qb[KSTEPS], qbl[KSTEPS];
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
        const float *row = qs + r * D + g * (D / 4) + 4 * s;
        float v[4], lo[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[j] = row[j];
            lo[j] = v[j] - f16_to_f32(f32_to_f16_rne(v[j]));
        }
        qb[s] = as_half4(pack_h2(v[0], v[1]), pack_h2(v[2], v[3]));
        qbl[s] = as_half4(pack_h2(lo[0], lo[1]), pack_h2(lo[2], lo[3]));
    }
    // sqrt(2/pi)/D G (2^k q) as fp16 hi + fp16 remainder (|.| <= 2^15 sqrt(2/pi))
    half4_t gb[QSTEPS], gbl[QSTEPS];
#pragma unroll
    for (int s = 0; s < QSTEPS; ++s) {
        if (a.with_qjl) {
            const float *row = gq + r * QD + g * (QD / 4) + 4 * s;
            float gh[4], gl[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                gh[j] = row[j] * a.alpha_c;
                gl[j] = gh[j] - f16_to_f32(f32_to_f16_rne(gh[j]));
            }
            gb[s] = as_half4(pack_h2(gh[0], gh[1]), pack_h2(gh[2], gh[3]));
            gbl[s] = as_half4(pack_h2(gl[0], gl[1]), pack_h2(gl[2], gl[3]));
        } else {
            gb[s] = gbl[s] = as_half4(0u, 0u);
        }
    }
    const float row_scale = rsc[r];

    // Causal limit for this lane's row.
    const int64_t rho = (int64_t)rc * kRows + r;
    const bool row_valid = rho < nrows_total;
    const int64_t key_limit = (a.causal_offset >= 0 && row_valid) ? a.causal_offset + rho / a.G : INT64_MAX;

    // ── main loop ─────────────────────────────────────────────────────
    const int64_t s_begin = (int64_t)split * a.split_len;
    const int64_t s_end = imin64(a.S, s_begin + a.split_len);
    bool seq_bad;
    const int64_t kv_base = (cache_seq(a, b, seq_bad) * a.Hkv + hk) * a.S;   // token row base of this (b, hk)
    const int cmask = ncopy - 1;
    const int cl = lane & cmask;

    float4_t o_acc[NBLK];
#pragma unroll
    for (int k = 0; k < NBLK; ++k) o_acc[k] = float4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f;

    for (int64_t t0 = s_begin + (int64_t)wave * kTile; t0 < s_end; t0 += (int64_t)nw * kTile) {
        // A-operand token for K / QJL: t0 + (lane % 16); output tokens: t0 + 4g + i.
        const int64_t ta = imin64(t0 + r, s_end - 1);
        const int64_t tok_row = kv_base + ta;

        // K nibbles: D/8 bytes per lane.
        uint32_t kw[D / 32];
        if constexpr (D == 128) {
            uint4 t = reinterpret_cast<const uint4 *>(a.k_nib + tok_row * (D / 2))[g];
            kw[0] = t.x; kw[1] = t.y; kw[2] = t.z; kw[3] = t.w;
        } else {
            kw[0] = reinterpret_cast<const uint32_t *>(a.k_nib + tok_row * (D / 2))[g];
        }

        float4_t sacc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
            const uint32_t w = kw[s >> 1];
            const uint32_t b0 = (w >> (16 * (s & 1))) & 0xffu;
            const uint32_t b1 = (w >> (16 * (s & 1) + 8)) & 0xffu;
            const uint2 e0 = vlut[b0 * ncopy + cl], e1 = vlut[b1 * ncopy + cl];
            const half4_t ah = as_half4(e0.x, e1.x), al = as_half4(e0.y, e1.y);
            sacc = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, qb[s], sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, qbl[s], sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_16x16x16f16(al, qb[s], sacc, 0, 0, 0);
        }

        float4_t cacc = float4_t{0.f, 0.f, 0.f, 0.f};
        float4_t nrm4 = float4_t{0.f, 0.f, 0.f, 0.f};
        if (a.with_qjl) {
            uint32_t sb;
            if constexpr (D == 128) {
                sb = reinterpret_cast<const uint16_t *>(a.k_qjl + tok_row * (D / 16))[g];
            } else {
                sb = (reinterpret_cast<const uint16_t *>(a.k_qjl + tok_row * (D / 16))[0] >> (4 * g)) & 0xfu;
            }
#pragma unroll
            for (int s = 0; s < QSTEPS; ++s) {
                const uint2 e = qlut[(sb >> (4 * s)) & 0xfu];
                cacc = __builtin_amdgcn_mfma_f32_16x16x16f16(as_half4(e.x, e.y), gb[s], cacc, 0, 0, 0);
                cacc = __builtin_amdgcn_mfma_f32_16x16x16f16(as_half4(e.x, e.y), gbl[s], cacc, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t tn = imin64(t0 + 4 * g + i, s_end - 1);
                nrm4[i] = a.k_norms[kv_base + tn];
            }
        }

        // Scores (log2 units) with masking.
        float sc[4];
        float mt = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t tn = t0 + 4 * g + i;
            float v = __builtin_fmaf(nrm4[i], cacc[i], sacc[i]) * row_scale;
            if (tn >= s_end || tn > key_limit) v = -INFINITY;
            sc[i] = v;
            mt = fmaxf(mt, v);
        }
        mt = wave_max_xor16_32(mt);
        const float m_new = fmaxf(m_run, mt);
        const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
        const float resc = exp2f(m_run - m_use);
        uint32_t ph[2];
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint16_t p0 = f32_to_f16_rne(exp2f(sc[2 * i] - m_use));
            const uint16_t p1 = f32_to_f16_rne(exp2f(sc[2 * i + 1] - m_use));
            psum += f16_to_f32(p0) + f16_to_f32(p1);
            ph[i] = (uint32_t)p0 | ((uint32_t)p1 << 16);
        }
        l_run = __builtin_fmaf(l_run, resc, psum);
        m_run = m_new;
        const half4_t pb = as_half4(ph[0], ph[1]);
#pragma unroll
        for (int k = 0; k < NBLK; ++k) o_acc[k] *= resc;

        // V: lane row rr = lane % 16 takes byte group rr of tokens t0 + 4g + i.
        uint2 vl[4][VB];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t tn = imin64(t0 + 4 * g + i, s_end - 1);
            const uint8_t *vrow = a.v_nib + (kv_base + tn) * (D / 2);
            uint32_t w;
            if constexpr (D == 128) w = reinterpret_cast<const uint32_t *>(vrow)[r];
            else w = vrow[r];
#pragma unroll
            for (int bb = 0; bb < VB; ++bb) vl[i][bb] = vlut[((w >> (8 * bb)) & 0xffu) * ncopy + cl];
        }
#pragma unroll
        for (int bb = 0; bb < VB; ++bb) {
#pragma unroll
            for (int n = 0; n < 2; ++n) {
                const uint32_t sel = n ? 0x07060302u : 0x05040100u;
                const half4_t ah = as_half4(__builtin_amdgcn_perm(vl[1][bb].x, vl[0][bb].x, sel),
                                            __builtin_amdgcn_perm(vl[3][bb].x, vl[2][bb].x, sel));
                const half4_t al = as_half4(__builtin_amdgcn_perm(vl[1][bb].y, vl[0][bb].y, sel),
                                            __builtin_amdgcn_perm(vl[3][bb].y, vl[2][bb].y, sel));
                o_acc[2 * bb + n] = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, pb, o_acc[2 * bb + n], 0, 0, 0);
                o_acc[2 * bb + n] = __builtin_amdgcn_mfma_f32_16x16x16f16(al, pb, o_acc[2 * bb + n], 0, 0, 0);
            }
        }
    }

    // ── combine waves in LDS (deterministic order) ────────────────────
    l_run = wave_sum_xor16_32(l_run);
    __syncthreads();   // LUTs are dead from here on
    float *wm = reinterpret_cast<float *>(smem);           // [nw][kRows] running max
    float *wl = wm + kMaxWaves * kRows;                     // [nw][kRows] denominators
    float *ob = wl + kMaxWaves * kRows;                     // [kRows][D] merged O
    if (g == 0) {
        wm[wave * kRows + r] = m_run;
        wl[wave * kRows + r] = l_run;
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int w = 0; w < nw; ++w) mx = fmaxf(mx, wm[w * kRows + r]);
    const float mu = (mx == -INFINITY) ? 0.0f : mx;
    const float fw = exp2f(m_run - mu);
    // o_acc[blk][i] holds O^T[d][r] with d = (2*VB) * (4g + i) + blk.
    for (int w = 0; w < nw; ++w) {
        if (wave == w) {
#pragma unroll
            for (int k = 0; k < NBLK; ++k)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float *dst = ob + r * D + (2 * VB) * (4 * g + i) + k;
                    const float v = o_acc[k][i] * fw;
                    *dst = (w == 0) ? v : (*dst + v);
                }
        }
        __syncthreads();
    }

    const int64_t unit = (b * a.Hkv + hk) * a.n_rchunks + rc;
    for (int s = tid; s < kRows * D; s += blockDim.x) {
        const int rr = s / D, d = s % D;
        const int64_t rr_rho = (int64_t)rc * kRows + rr;
        if (rr_rho >= nrows_total) continue;
        float rmx = -INFINITY;
        for (int w = 0; w < nw; ++w) rmx = fmaxf(rmx, wm[w * kRows + rr]);
        const float rmu = (rmx == -INFINITY) ? 0.0f : rmx;
        float lsum = 0.0f;
        for (int w = 0; w < nw; ++w) lsum = __builtin_fmaf(exp2f(wm[w * kRows + rr] - rmu), wl[w * kRows + rr], lsum);
        if (seq_bad) lsum = __builtin_nanf("");
        const float osum = ob[rr * D + d];
        if (a.splits == 1) {
            const int64_t t = rr_rho / a.G;
            const int hq = hk * a.G + (int)(rr_rho % a.G);
            a.out[((b * a.Hq + hq) * a.T + t) * D + d] = osum / lsum;
        } else {
            float *wp = a.ws + ((unit * a.splits + split) * kRows + rr) * (D + 2);
            wp[d] = osum;
            if (d == 0) { wp[D] = rmx; wp[D + 1] = lsum; }
        }
    }
}

template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
    const int hk = blockIdx.y;
    const int64_t bz = blockIdx.z;
    const int64_t b = bz / a.n_rchunks;
    const int rc = (int)(bz % a.n_rchunks);
    const int rows = a.rows;
    const int64_t unit = (b * a.Hkv + hk) * a.n_rchunks + rc;
    const int64_t nrows_total = a.T * a.G;
    for (int s = threadIdx.x; s < rows * D; s += blockDim.x) {
        const int rr = s / D, d = s % D;
        const int64_t rho = (int64_t)rc * rows + rr;
        if (rho >= nrows_total) continue;
        float mx = -INFINITY;
        for (int sp = 0; sp < a.splits; ++sp)
            mx = fmaxf(mx, a.ws[((unit * a.splits + sp) * rows + rr) * (D + 2) + D]);
        const float mu = (mx == -INFINITY) ? 0.0f : mx;
        float lsum = 0.0f, osum = 0.0f;
        for (int sp = 0; sp < a.splits; ++sp) {
            const float *wp = a.ws + ((unit * a.splits + sp) * rows + rr) * (D + 2);
            const float f = exp2f(wp[D] - mu);
            lsum = __builtin_fmaf(f, wp[D + 1], lsum);
            osum = __builtin_fmaf(f, wp[d], osum);
        }
        const int64_t t = rho / a.G;
        const int hq = hk * a.G + (int)(rho % a.G);
        a.out[((b * a.Hq + hq) * a.T + t) * D + d] = osum / lsum;
    }
}

// ── D = 128 decode kernel ───────────────────────────────────────────────
//
// 32-token tiles per wave iteration; v_mfma_f32_16x16x32_f16 throughout.
// Query rows (<= 8) sit in MFMA columns 0-7.
//   K pass   A = K16 (16 tok x 256 slots): each cache byte's LUT entry
//            (hi(c_even), hi(c_odd), lo(c_even), lo(c_odd)) fills four
//            consecutive k-slots as loaded, so B repeats q over the hi and
//            lo slots: columns 0-7 = Q_hi (both slots), columns 8-15 = Q_lo
//            (hi slots only).  S_main(row n) = acc[n] + acc[n+8]
//            = K_hi.Q_hi + K_lo.Q_hi + K_hi.Q_lo.
//   QJL pass A = B+- (16 tok x 64), B = scale log2e sqrt(2/pi)/D G_h q:
//            fp16 in columns 0-7, its fp16 remainder in 8-15, into a second
//            accumulator; t = acc + norm * qacc (norms fp32, quad-broadcast
//            by DPP), score = t[n] + t[n+8].
// One DPP row shift moves columns 8-15 onto 0-7.
// Twelve waves per block (three per SIMD, <= 168 VGPRs) each keep a 2-deep
// ring of tiles in flight; waves 0-7 also own one query row in the prologue.  PV contracts the 32
// tokens of the tile: O^T (128 x 16) += V^T_hi . P^T + V^T_lo . P^T, plus a
// ones row that accumulates the softmax denominator from the same fp16 P.
//
// LDS (static): [0, 64K)       byte LUT, 32 bank-private copies at a
//                              256-byte stride, so one v_perm forms the
//                              LDS address (byte << 8) | (lane % 32) * 8
//               [64K, 68K)     sign byte -> eight +-1.0 halves
//               [68K, 74K)     query rows and G q (prologue)
//               [74K, 86K)     query rows as MFMA operands: (scale q) hi/lo
//                              B images for the scores, q hi/lo A images
//                              for G q
//               [86K, +32)     per-row score scales
//               [+32, +16)     tile counter (dynamic tile claims)
constexpr int kDecRows = 8;
constexpr int kDecWaves = 12;
constexpr int kDecTile = 32;
constexpr int kDecPrefetch = 2;      // tiles in flight per wave (ring depth)
constexpr int kLutOff = 0;
constexpr int kLutBytes = 256 * 256;
constexpr int kSlutOff = kLutBytes;
constexpr int kSlutBytes = 16 * 256;
static_assert((kSlutOff & (kSlutOff - 1)) == 0 && kSlutOff >= kSlutBytes, "sign LUT address is formed with an OR");
constexpr int kDecQsOff = kSlutOff + kSlutBytes;
constexpr int kDecGqStride = 64 + 2;   // G q rows: the pad spreads the rows of one read over the banks
constexpr int kDecBkOff = kDecQsOff + kDecRows * (128 + kDecGqStride) * 4;   // [row][quad][hi, lo] 16 B
constexpr int kDecGaOff = kDecBkOff + kDecRows * 32 * 2 * 16;        // [row][8-dim group][hi, lo] 16 B
constexpr int kDecCscOff = kDecGaOff + kDecRows * 16 * 2 * 16;      // per row: scale * log2(e) / 2^k
// 16-byte chunk c of a row's operand image is stored at c ^ 2 (row % 8): the
// eight rows read by one instruction then fall in different bank groups
// (unswizzled, every row starts on the same bank and one read serializes
// ~32 ways)
__device__ __forceinline__ int dec_chunk(int row, int c) { return c ^ (2 * (row & 7)); }
constexpr int kDecCntOff = kDecCscOff + kDecRows * 4;                // next unclaimed tile of the block
constexpr int kDecLrOff = kDecCntOff + 16;                           // fused LoRA: x A^T of two row groups
constexpr int kDecLdsBytes = kDecLrOff + 2 * 16 * 4;
// Paged cache: the pool row of each 16-token half of the split (half h at
// kDecPtOff + 4 h, the row of token s_begin + 16 h), staged in the prologue
// when the split has at most kDecPtMax halves (the paged plan keeps every
// split within that), so a claimed tile's two rows are one 8-byte LDS read
// away; the variants with the fused LoRA prologue or two sequences per block
// read the page table per tile.  Each wave also records whether its staged
// halves met a page id outside the pool (one word per wave at
// kDecPtFlagOff).
constexpr int kDecPtOff = (kDecLdsBytes + 15) & ~15;
constexpr int kDecPtMax = 6144;
constexpr int kDecPtLoads = kDecPtMax / (64 * kDecWaves);
static_assert(kDecPtLoads * 64 * kDecWaves == kDecPtMax, "page rows staged by a fixed number of loads per thread");
constexpr int kDecPtFlagOff = kDecPtOff + 4 * kDecPtMax;
constexpr int kDecPtLdsBytes = kDecPtFlagOff + 4 * kDecWaves;
// epilogue reuse of [0, 68K): per-wave O slabs (rows padded to 132 floats),
// then per-wave running max and denominator
constexpr int kObStride = 128 + 4;
constexpr int kDecSlabBytes = kDecWaves * kDecRows * kObStride * 4;
static_assert(kDecSlabBytes + 2 * kDecWaves * kDecRows * 4 <= kDecQsOff, "epilogue slabs overlap the query rows");
static_assert(kDecWaves >= kDecRows, "one query row per wave in the prologue");

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ half8_t as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    uint4 t = make_uint4(a, b, c, d);
    return __builtin_bit_cast(half8_t, t);
}

__device__ __forceinline__ half8_t pair_half8(uint2 x, uint2 y) {
    return as_half8(x.x, x.y, y.x, y.y);
}

// Value of lane 4 * (lane / 4) + I (a broadcast within each quad).
template <int I>
__device__ __forceinline__ float dpp_quad_bcast_i(float v) {
    // every source lane exists (no old value needed), so the move can fold
    // into the consuming VOP2 instruction as its DPP operand
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), I * 0x55, 0xf, 0xf, true));
}
__device__ __forceinline__ float dpp_quad_bcast(float v, int i) {
    return i == 0 ? dpp_quad_bcast_i<0>(v) : i == 1 ? dpp_quad_bcast_i<1>(v) : i == 2 ? dpp_quad_bcast_i<2>(v)
                                                                                      : dpp_quad_bcast_i<3>(v);
}

__device__ __forceinline__ float dpp_row_shl8(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x108, 0xf, 0xf, false));
}
// lane i of each 16-lane row reads lane i ^ 8 (rotate by 8).  A row rotate
// reads a valid lane for every lane, so no prior value of the destination is
// kept (no move to initialise it).
__device__ __forceinline__ uint32_t dpp_row_ror8(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xf, 0xf, true);
}

// max(a, b) and max(a, b, c) as single instructions.  fmaxf on values the
// compiler cannot prove canonical (lane moves, selects) first quiets each
// operand with an extra v_max; no signalling NaN reaches these call sites
// (every operand is an arithmetic result or a lane move of one), where the
// plain instruction already returns fmaxf's result.
__device__ __forceinline__ float vmax2(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ float vmax3(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// LDS byte offset of the LUT entry for byte k of w: (byte << 8) | copy offset.
__device__ __forceinline__ uint32_t lut_addr(uint32_t w, uint32_t laneoff, int k) {
    return __builtin_amdgcn_perm(w, laneoff, 0x0C0C0000u | ((uint32_t)(4 + k) << 8));
}

// Sign table: nibble v -> four fp16 halves (+1.0 where bit i of v is set,
// -1.0 elsewhere), 32 bank-private copies at a 256-byte stride like the byte
// LUT, so random nibbles read without bank conflicts.  `slane` is
// kSlutOff | (lane % 32) * 8.
__device__ __forceinline__ void sign_table_store(unsigned char *smem, int t) {
    // thread t < 512 writes copy t % 32 of nibble t / 32
    const uint32_t v = (uint32_t)t >> 5;
    uint32_t w[2];
#pragma unroll
    for (int k = 0; k < 2; ++k)
        w[k] = (((v >> (2 * k)) & 1) ? 0x3C00u : 0xBC00u) | ((((v >> (2 * k + 1)) & 1) ? 0x3C00u : 0xBC00u) << 16);
    *reinterpret_cast<uint2 *>(smem + kSlutOff + v * 256u + ((uint32_t)t & 31u) * 8u) = make_uint2(w[0], w[1]);
}

// Eight +-1.0 halves for bits pos .. pos + 7 of w (bit pos first).
__device__ __forceinline__ half8_t sign_halves(const unsigned char *smem, uint32_t w, uint32_t pos, uint32_t slane) {
    const uint32_t n0 = __builtin_amdgcn_ubfe(w, pos, 4u), n1 = __builtin_amdgcn_ubfe(w, pos + 4u, 4u);
    const uint2 e0 = *reinterpret_cast<const uint2 *>(smem + ((n0 << 8) | slane));
    const uint2 e1 = *reinterpret_cast<const uint2 *>(smem + ((n1 << 8) | slane));
    return as_half8(e0.x, e0.y, e1.x, e1.y);
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
constexpr int kBufWord3 = 0x00020000;   // raw buffer, gfx9 descriptor dword 3

// Buffer descriptors over one (b, kv head) token stream, limited to the
// split's end: reads past it return 0 (those tokens are masked anyway).
struct DecBufs {
    __amdgpu_buffer_rsrc_t kn, vn, kq, kr;
};

// Lane-constant byte offsets; the tile offset is added per tile and the
// sub-tile / token steps go in the instruction's immediate offset.
struct DecOffsets {
    uint32_t k, sg, nr, v;
};

// One 32-token tile as loaded, before any decoding.
struct TileRaw {
    uint4 k[2];        // K nibbles: token t0 + 16u + (lane % 16), bytes 16g .. 16g + 15
    uint2 sg[2];       // sign rows of the same tokens
    float nr[2];       // one norm per lane and half u; which token is set by the offsets
    uint32_t v[8];     // V dword (lane % 16) of tokens t0 + 16(i/4) + 4g + i%4
};

template <bool QJL>
__device__ __forceinline__ void tile_load(TileRaw &R, const DecBufs &P, const DecOffsets &O, int t0) {
    // The tile offset goes into the per-lane offset, which the buffer range
    // check covers: tiles past the split end read as 0 and touch no memory.
    const uint32_t t = (uint32_t)t0;
    const uint32_t vk = O.k + t * 64u, vsg = O.sg + t * 8u, vnr = O.nr + t * 4u, vv = O.v + t * 64u;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const u32x4_t kv4 = __builtin_amdgcn_raw_buffer_load_b128(P.kn, vk + 1024u * u, 0, 0);
        R.k[u] = make_uint4(kv4.x, kv4.y, kv4.z, kv4.w);
        if (QJL) {
            const u32x2_t sv = __builtin_amdgcn_raw_buffer_load_b64(P.kq, vsg + 128u * u, 0, 0);
            R.sg[u] = make_uint2(sv.x, sv.y);
            R.nr[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(P.kr, vnr + 64u * u, 0, 0));
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
        R.v[i] = __builtin_amdgcn_raw_buffer_load_b32(P.vn, vv + 64u * (16 * (i / 4) + (i % 4)), 0, 0);
}

// The same tile from a paged pool: half u (16 tokens) starts at pool row
// rb[u] = (page * Hkv + hk) * page_size + slot; a half never crosses a page
// (page sizes are multiples of 16 and tiles start at multiples of 32).  The
// row offset goes into the per-lane offset, so the descriptor's range check
// (the whole pool) covers it.
template <bool QJL>
__device__ __forceinline__ void tile_load_paged(TileRaw &R, const DecBufs &P, const DecOffsets &O, const uint32_t (&rb)[2]) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const u32x4_t kv4 = __builtin_amdgcn_raw_buffer_load_b128(P.kn, O.k + rb[u] * 64u, 0, 0);
        R.k[u] = make_uint4(kv4.x, kv4.y, kv4.z, kv4.w);
        if (QJL) {
            const u32x2_t sv = __builtin_amdgcn_raw_buffer_load_b64(P.kq, O.sg + rb[u] * 8u, 0, 0);
            R.sg[u] = make_uint2(sv.x, sv.y);
            R.nr[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(P.kr, O.nr + rb[u] * 4u, 0, 0));
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
        R.v[i] = __builtin_amdgcn_raw_buffer_load_b32(P.vn, O.v + rb[i / 4] * 64u + 64u * (i % 4), 0, 0);
}

// Paged cache: pool rows of the two 16-token halves of the tile at token t
// (wave-uniform scalar loads of the page table row `pt_row`).  A page id
// outside the pool reads page 0 and, for a half that holds tokens of the
// sequence (below `s_end`), sets `bad` (the sequence's rows come out NaN);
// past the table's width (tiles past the end) the last entry is read.
__device__ __forceinline__ void paged_page_ids(const AttnArgs &a, const int32_t *pt_row, int t, int32_t (&id)[2]) {
#pragma unroll
    for (int u = 0; u < 2; ++u) id[u] = pt_row[imin((t + 16 * u) >> a.page_shift, (int)a.max_pages - 1)];
}
__device__ __forceinline__ void paged_rows(const AttnArgs &a, const int32_t (&id)[2], int hk, int t, int s_end,
                                           bool &bad, uint32_t (&rb)[2]) {
    const int sh = a.page_shift;
    const uint32_t np = (uint32_t)a.n_pages;                  // < 2^26 (host check)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int th = t + 16 * u;
        const bool ok = (uint32_t)id[u] < np;                     // negative ids wrap past np
        bad = bad || (!ok && th < s_end);
        rb[u] = (((ok ? (uint32_t)id[u] : 0u) * (uint32_t)a.Hkv + (uint32_t)hk) << sh) +
                ((uint32_t)th & ((1u << sh) - 1u));
    }
}
__device__ __forceinline__ void paged_half_rows(const AttnArgs &a, const int32_t *pt_row, int hk, int t, int s_end,
                                                bool &bad, uint32_t (&rb)[2]) {
    int32_t id[2];
    paged_page_ids(a, pt_row, t, id);
    paged_rows(a, id, hk, t, s_end, bad, rb);
}

__device__ __forceinline__ uint32_t cvt_pk_h2(float x, float y) {
    typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
    typedef float f2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2_t){x, y}, h2_t));
}

// max over lanes {l, l^16, l^32, l^48} without LDS (v_permlane16/32_swap).
__device__ __forceinline__ float max_over_groups(float m) {
    auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    m = vmax2(__uint_as_float(t[0]), __uint_as_float(t[1]));
    auto u = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return vmax2(__uint_as_float(u[0]), __uint_as_float(u[1]));
}

// One lane per (d, d + 64) of a 128-wide row: the normalized WHT of
// _wht_torch (hadamard.py:51-85).  Stage h pairs element u (bit h clear)
// with u + h: u <- x[u] + x[u+h], u + h <- x[u] - x[u+h], all fp32; stages
// h = 1..32 cross lanes, h = 64 pairs the two values of a lane.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// fmaxf over the 64 lanes of a wave without LDS: DPP quad permutes and row
// rotates within each 16-lane row, then the row and half-wave swaps
// (max is exact and order-free, so every lane gets the same value as an
// xor-shuffle tree would give)
__device__ __forceinline__ float wave_max(float m) {
    m = fmaxf(m, dpp_mov<0xB1>(m));     // quad_perm [1,0,3,2]
    m = fmaxf(m, dpp_mov<0x4E>(m));     // quad_perm [2,3,0,1]
    m = fmaxf(m, dpp_mov<0x124>(m));    // row_ror:4
    m = fmaxf(m, dpp_mov<0x128>(m));    // row_ror:8
    return max_over_groups(m);
}

// x[lane ^ H] without LDS: DPP quad permutes (H = 1, 2), row rotates
// (H = 4, 8; lane i reads lane i - k mod 16 for row_ror:k) and the gfx950
// row / half-wave swaps (H = 16, 32).
template <int H>
__device__ __forceinline__ float xor_partner(float x, int lane) {
    if constexpr (H == 1) {
        return dpp_mov<0xB1>(x);                                  // quad_perm [1,0,3,2]
    } else if constexpr (H == 2) {
        return dpp_mov<0x4E>(x);                                  // quad_perm [2,3,0,1]
    } else if constexpr (H == 4) {
        const float up = dpp_mov<0x12C>(x), dn = dpp_mov<0x124>(x);  // row_ror:12 / row_ror:4
        return (lane & 4) ? dn : up;
    } else if constexpr (H == 8) {
        return dpp_mov<0x128>(x);                                 // row_ror:8
    } else if constexpr (H == 16) {
        const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return __uint_as_float((lane & 16) ? t[0] : t[1]);
    } else {
        const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return __uint_as_float((lane & 32) ? t[0] : t[1]);
    }
}

template <int H>
__device__ __forceinline__ void wht_stage(float &lo, float &hi, int lane) {
    // element u (bit H clear) <- x[u] + x[u+H]; u + H <- x[u] - x[u+H]
    const float sgn = (lane & H) ? -1.0f : 1.0f;
    lo = __builtin_fmaf(sgn, lo, xor_partner<H>(lo, lane));
    hi = __builtin_fmaf(sgn, hi, xor_partner<H>(hi, lane));
}

// One lane per (d, d + 64) of a 128-wide row: the normalized WHT of
// _wht_torch (hadamard.py:51-85).  Stage h pairs element u (bit h clear)
// with u + h: u <- x[u] + x[u+h], u + h <- x[u] - x[u+h], all fp32 (an fma
// with +-1 rounds exactly as the add / subtract); stages h = 1..32 cross
// lanes, h = 64 pairs the two values of a lane.
__device__ __forceinline__ void wht128_lanes(float &lo, float &hi, int lane) {
    wht_stage<1>(lo, hi, lane);
    wht_stage<2>(lo, hi, lane);
    wht_stage<4>(lo, hi, lane);
    wht_stage<8>(lo, hi, lane);
    wht_stage<16>(lo, hi, lane);
    wht_stage<32>(lo, hi, lane);
    const float a = lo, b = hi;
    lo = a + b;
    hi = a - b;
}

// q_eff = round(q + ((x A_id^T) B_id^T) alpha) for one query row (b, t, hq)
// held as (lo = dim lane, hi = dim 64 + lane), in exactly the operation order
// of lora_kernel (per-lane fma over hidden = lane, lane + 64, ...; xor-tree
// wave sum; sequential fma over the rank), so the fused and the separate
// paths round q_eff identically.  id < 0: unchanged; id >= n: NaN.
// The fused path takes 16-bit adapters of rank 8 or 16 and hidden <= 256
// with a 16-byte aligned B bank (the host sends others to the gather-apply
// kernel); every load is a branch-free buffer load whose range ends at the
// row it serves, B rows as 16-byte loads of eight rank components.
__device__ __forceinline__ float lora_wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}
constexpr int kLoraFusedMaxRank = 16;
constexpr int kLoraFusedMaxHidden = 256;

__device__ __forceinline__ float lora_w16(uint32_t w, bool bf) {
    return bf ? __uint_as_float(w << 16) : f16_to_f32((uint16_t)w);
}

// x row of (b, t) as raw 16-bit values: element 64 kh + lane in xw[kh]
// (0 past `hidden`: the descriptor's range ends there).
__device__ __forceinline__ void lora_x_load(uint32_t (&xw)[4], const AttnArgs &a, int64_t b, int64_t t, int lane) {
    const __amdgpu_buffer_rsrc_t XR = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(reinterpret_cast<const uint16_t *>(a.lora_x) + (b * a.T + t) * a.lora_hidden), (short)0,
        2 * a.lora_hidden, kBufWord3);
#pragma unroll
    for (int kh = 0; kh < 4; ++kh) xw[kh] = __builtin_amdgcn_raw_buffer_load_b16(XR, 2u * (64 * kh + lane), 0, 0);
}

// Rank components 2 s and 2 s + 1 of each 8-block of x A_id^T (s = row slot
// % 4), the lora_row sums, into `dst` (rank <= 16 floats) for the row
// group of four slots that shares the (sequence, token).
__device__ __forceinline__ void lora_rank_share(const AttnArgs &a, int32_t id_raw, const uint32_t (&xw)[4], int slot,
                                                int lane, float *dst) {
    const int32_t id = __builtin_amdgcn_readfirstlane(id_raw);
    const bool active = id >= 0 && id < a.lora_n;
    const int64_t sid = active ? id : 0;
    const bool bf = a.lora_w_dtype == OMNI_BF16;
    const int hidden = a.lora_hidden, rank = a.lora_rank;
    const __amdgpu_buffer_rsrc_t AR = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(reinterpret_cast<const uint16_t *>(a.lora_a) + sid * rank * (int64_t)hidden), (short)0,
        2 * rank * hidden, kBufWord3);
    float xv[4];
#pragma unroll
    for (int kh = 0; kh < 4; ++kh) xv[kh] = lora_w16(xw[kh], bf);
    const int sub = slot & 3;
    for (int j0 = 0; j0 < rank; j0 += 8) {
        uint32_t aw[2][4];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const uint32_t j = j0 + 2 * sub + jj;
#pragma unroll
            for (int kh = 0; kh < 4; ++kh)
                aw[jj][kh] = __builtin_amdgcn_raw_buffer_load_b16(AR, 2u * (j * hidden + 64 * kh + lane), 0, 0);
        }
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            float part = 0.0f;
#pragma unroll
            for (int kh = 0; kh < 4; ++kh) {
                const float f = __builtin_fmaf(xv[kh], lora_w16(aw[jj][kh], bf), part);
                part = 64 * kh + lane < hidden ? f : part;
            }
            const float dr = lora_wave_sum(part);
            if (lane == 0) dst[j0 + 2 * sub + jj] = dr;
        }
    }
}

// `shared`: the rank components from lora_rank_share (NULL: computed here).
__device__ __forceinline__ void lora_row(float &lo, float &hi, const AttnArgs &a, int32_t id_raw,
                                         const uint32_t (&xw)[4], int hq, int lane, const float *shared = nullptr) {
    const int32_t id = __builtin_amdgcn_readfirstlane(id_raw);
    const bool active = id >= 0 && id < a.lora_n, bad = id >= a.lora_n;
    const int64_t sid = active ? id : 0;
    const bool bf = a.lora_w_dtype == OMNI_BF16;
    const int hidden = a.lora_hidden, rank = a.lora_rank;
    // A[sid] (rank x hidden) and this head's 128 rows of B[sid] (128 x rank)
    const __amdgpu_buffer_rsrc_t AR = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(reinterpret_cast<const uint16_t *>(a.lora_a) + sid * rank * (int64_t)hidden), (short)0,
        2 * rank * hidden, kBufWord3);
    const __amdgpu_buffer_rsrc_t BR = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(reinterpret_cast<const uint16_t *>(a.lora_b) + (sid * a.Hq + hq) * 128 * (int64_t)rank), (short)0,
        2 * 128 * rank, kBufWord3);
    float xv[4];
#pragma unroll
    for (int kh = 0; kh < 4; ++kh) xv[kh] = lora_w16(xw[kh], bf);
    float acc_lo = 0.0f, acc_hi = 0.0f;
    for (int j0 = 0; j0 < rank; j0 += 8) {
        // all loads of eight rank components first (one latency); rows past
        // the rank read 0 (A) or are not used (B)
        uint32_t aw[8][4], bl[8], bh[8];
        if (shared == nullptr) {
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const uint32_t j = j0 + jj;
#pragma unroll
                for (int kh = 0; kh < 4; ++kh)
                    aw[jj][kh] = __builtin_amdgcn_raw_buffer_load_b16(AR, 2u * (j * hidden + 64 * kh + lane), 0, 0);
            }
        }
        {
            // B rows lane and 64 + lane, components j0 .. j0 + 7: one 16-byte
            // load each (rank % 8 == 0 and a 16-byte aligned bank)
            const u32x4_t l4 = __builtin_amdgcn_raw_buffer_load_b128(BR, 2u * (lane * rank + j0), 0, 0);
            const u32x4_t h4 = __builtin_amdgcn_raw_buffer_load_b128(BR, 2u * ((64 + lane) * rank + j0), 0, 0);
            const uint32_t lw[4] = {l4.x, l4.y, l4.z, l4.w}, hw[4] = {h4.x, h4.y, h4.z, h4.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                bl[2 * k] = lw[k] & 0xffffu;
                bl[2 * k + 1] = lw[k] >> 16;
                bh[2 * k] = hw[k] & 0xffffu;
                bh[2 * k + 1] = hw[k] >> 16;
            }
        }
        float dr[8];
        if (shared != nullptr) {
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) dr[jj] = shared[j0 + jj];
        } else {
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                float part = 0.0f;
#pragma unroll
                for (int kh = 0; kh < 4; ++kh) {
                    // a select, not a branch: the load must not sink into one
                    const float f = __builtin_fmaf(xv[kh], lora_w16(aw[jj][kh], bf), part);
                    part = 64 * kh + lane < hidden ? f : part;
                }
                dr[jj] = lora_wave_sum(part);
            }
        }
        // B values live in registers here: keeps the compiler from sinking
        // their loads into the (uniform) rank test below
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) asm volatile("" : "+v"(bl[jj]), "+v"(bh[jj]));
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const bool jv = j0 + jj < rank;
            acc_lo = jv ? __builtin_fmaf(dr[jj], lora_w16(bl[jj], bf), acc_lo) : acc_lo;
            acc_hi = jv ? __builtin_fmaf(dr[jj], lora_w16(bh[jj], bf), acc_hi) : acc_hi;
        }
    }
    const float ulo = round_to_dtype(__fadd_rn(lo, __fmul_rn(acc_lo, a.lora_alpha)), a.q_dtype);
    const float uhi = round_to_dtype(__fadd_rn(hi, __fmul_rn(acc_hi, a.lora_alpha)), a.q_dtype);
    lo = active ? ulo : (bad ? __builtin_nanf("") : lo);
    hi = active ? uhi : (bad ? __builtin_nanf("") : hi);
}

// Tile claims from the block's LDS counter: claim_issue() has lane 0 bump
// it and returns the register the old value lands in; claim_value() makes
// it wave-uniform.  The loop reads a claim one step after issuing it, so
// the atomic's latency hides behind that step's LUT traffic (LDS operations
// complete in order) instead of stalling the next tile's loads.
__device__ __forceinline__ int claim_issue(int *cnt, int lane) {
    int v = 0;
    if (lane == 0) v = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return v;
}
__device__ __forceinline__ int claim_value(int v) { return __builtin_amdgcn_readfirstlane(v); }

template <bool QJL, int PF, int SPB, bool LORA, bool PAGED>
__global__ __launch_bounds__(64 * kDecWaves) void attn_decode128_kernel(AttnArgs a) {
    static_assert(SPB == 1 || SPB == 2, "one or two sequences per block");
    constexpr int D = 128, QD = 64;
    constexpr int nw = kDecWaves;
    __shared__ __attribute__((aligned(16))) unsigned char smem[PAGED && !LORA && SPB == 1 ? kDecPtLdsBytes : kDecLdsBytes];
    float *qs = reinterpret_cast<float *>(smem + kDecQsOff);
    float *gq = qs + kDecRows * D;

    // the arguments the prologue needs are requested together with the first
    // kernel-argument loads (the compiler would otherwise fetch some after
    // the cache-index test: one more round trip before the first cache load)
    asm volatile("" ::"s"(a.q), "s"(a.k_nib), "s"(a.k_qjl), "s"(a.k_norms), "s"(a.v_nib), "s"(a.codebooks),
                 "s"(a.g_bits), "s"(a.sign_flip), "s"(a.rotate_q), "s"(a.qscale), "s"(a.alpha_c), "s"(a.wht_scale));
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int split = blockIdx.x, hk = blockIdx.y;
    // (batch, row chunk) from blockIdx.z (< 2^16); with two sequences per
    // block (spb = 2, one row chunk), sequences 2 bz and 2 bz + 1
    const int bz = blockIdx.z;
    const int bzq = div_small(bz, a.rch_magic);
    const int rc = bz - bzq * a.n_rchunks;
    const int b32 = bzq * SPB;
    const int64_t b = b32;
    const int nrows_total = (int)(a.T * a.G);
    const int nseq = (SPB > 1 && b32 + 1 < a.B) ? 2 : 1;
    const int n = lane & 15, g = lane >> 4;
    // row slot r -> (sequence index, flat (t, head) row of that sequence, valid)
    auto row_seq = [&](int r) { return (SPB > 1 && r >= nrows_total) ? 1 : 0; };
    auto row_rho = [&](int r) { return SPB > 1 ? r - row_seq(r) * nrows_total : rc * kDecRows + r; };
    auto row_valid = [&](int r) {
        return SPB > 1 ? (r < 2 * nrows_total && row_seq(r) < nseq) : (rc * kDecRows + r < nrows_total);
    };

    // ── cache stream descriptors ──────────────────────────────────────
    const int s_begin = split * (int)a.split_len;
    // paged: each sequence's length; one outside [0, capacity] reads nothing
    // and its rows come out NaN (with two sequences per block, seq_len1 ..
    // s_end1 are the second's; otherwise they repeat the first's)
    int seq_len = (int)a.S, seq_len1 = (int)a.S;
    bool len_bad = false, len_bad1 = false;
    if constexpr (PAGED) {
        const int32_t L = a.seq_lens[b32];
        len_bad = L < 0 || (int64_t)L > a.S;
        seq_len = len_bad ? 0 : L;
        seq_len1 = seq_len;
        if (SPB > 1 && nseq > 1) {
            const int32_t L1 = a.seq_lens[b32 + 1];
            len_bad1 = L1 < 0 || (int64_t)L1 > a.S;
            seq_len1 = len_bad1 ? 0 : L1;
        }
    }
    const int s_end = imax(s_begin, (int)imin64(seq_len, (int64_t)s_begin + a.split_len));
    const int s_end1 = imax(s_begin, (int)imin64(seq_len1, (int64_t)s_begin + a.split_len));
    // cache sequences of the block's batch entries: with a pool index both
    // indices are requested before either is used (one round trip), and
    // their out-of-pool flags are kept for the epilogue
    int64_t cs0 = b, cs1 = -1;            // cs1 < 0: no pool (the batch entry itself)
    bool cs_bad0 = false, cs_bad1 = false;
    if (!PAGED && a.seq_index != nullptr) {
        const int64_t v0 = a.seq_index[b], v1 = a.seq_index[nseq > 1 ? b + 1 : b];
        auto norm = [&](int64_t v, bool &bad) {
            v = v < 0 ? v + a.n_seqs : v;
            bad = v < 0 || v >= a.n_seqs;
            return bad ? (int64_t)0 : v;
        };
        cs0 = norm(v0, cs_bad0);
        cs1 = norm(v1, cs_bad1);
    }
    auto stream_bufs = [&](int64_t cs) {
        if constexpr (PAGED) {
            // the whole pool (its row count times 64 fits 32 bits: the host checks)
            (void)cs;
            const uint32_t rows = (uint32_t)(a.n_pages * a.Hkv * a.page_size);
            DecBufs Q;
            Q.kn = __builtin_amdgcn_make_buffer_rsrc((void *)a.k_nib, (short)0, rows * 64u, kBufWord3);
            Q.vn = __builtin_amdgcn_make_buffer_rsrc((void *)a.v_nib, (short)0, rows * 64u, kBufWord3);
            Q.kq = __builtin_amdgcn_make_buffer_rsrc((void *)(QJL ? a.k_qjl : a.k_nib), (short)0, QJL ? rows * 8u : 0u,
                                                     kBufWord3);
            Q.kr = __builtin_amdgcn_make_buffer_rsrc((void *)(QJL ? a.k_norms : (const float *)a.k_nib), (short)0,
                                                     QJL ? rows * 4u : 0u, kBufWord3);
            return Q;
        }
        const int64_t kv_base = (cs * a.Hkv + hk) * a.S;
        DecBufs Q;
        Q.kn = __builtin_amdgcn_make_buffer_rsrc((void *)(a.k_nib + kv_base * 64), (short)0, s_end * 64, kBufWord3);
        Q.vn = __builtin_amdgcn_make_buffer_rsrc((void *)(a.v_nib + kv_base * 64), (short)0, s_end * 64, kBufWord3);
        Q.kq = __builtin_amdgcn_make_buffer_rsrc((void *)(QJL ? a.k_qjl + kv_base * 8 : a.k_nib), (short)0,
                                                 QJL ? s_end * 8 : 0, kBufWord3);
        Q.kr = __builtin_amdgcn_make_buffer_rsrc((void *)(QJL ? a.k_norms + kv_base : (const float *)a.k_nib),
                                                 (short)0, QJL ? s_end * 4 : 0, kBufWord3);
        return Q;
    };
    const DecBufs P = stream_bufs(cs0);
    const DecBufs P1 = stream_bufs(cs1 >= 0 ? cs1 : (nseq > 1 ? b + 1 : b));
    // tiles of the split per sequence; claim index i -> sequence (i >= tps)
    const int tps = (s_end - s_begin + kDecTile - 1) / kDecTile;
    const int tps1 = (s_end1 - s_begin + kDecTile - 1) / kDecTile;
    const int ntiles = tps + (nseq > 1 ? tps1 : 0);
    auto make_ofs = [](int l) {
        const int nn = l & 15, gg = l >> 4;
        DecOffsets o;
        o.k = (uint32_t)nn * 64u + 16u * gg;
        o.sg = (uint32_t)nn * 8u;
        o.nr = 16u * gg + 4u * (nn & 3);      // norm of token 4g + n % 4 (of each 16-token half)
        o.v = 256u * gg + 4u * nn;
        return o;
    };
    const DecOffsets OFS = make_ofs(lane);
    // loop-time offsets: with the fused LoRA prologue or two sequences per
    // block (whose registers run short) they are recomputed from an opaque
    // lane id at each use instead of being kept live across the loop
    auto ofs_loop = [&]() {
        if constexpr (LORA || SPB > 1) {
            int l = lane;
            asm volatile("" : "+v"(l));
            return make_ofs(l);
        } else {
            return OFS;
        }
    };

    // Paged cache: pool rows of a tile's two halves; a page id outside the
    // pool marks this wave's state bad (the sequence's rows come out NaN)
    bool page_bad = false, page_bad1 = false;
    const int32_t *pt_row = PAGED ? a.page_table + b * a.max_pages : nullptr;
    const int32_t *pt_row1 = PAGED && SPB > 1 && nseq > 1 ? pt_row + a.max_pages : pt_row;
    auto half_rows = [&](int t, int sq, uint32_t (&rb)[2]) {
        if (SPB > 1 && sq) paged_half_rows(a, pt_row1, hk, t, s_end1, page_bad1, rb);
        else paged_half_rows(a, pt_row, hk, t, s_end, page_bad, rb);
    };
    // the page id of each half of the split (pages pg0 .. pg0 + npg - 1;
    // halves past the split end take its last page, as the page-table path
    // does), requested before the cache prefetch so that waiting for them
    // does not wait for it; converted to pool rows and staged in LDS before
    // the first barrier (not with the fused LoRA prologue, whose scalar
    // registers are full)
    constexpr bool kStage = PAGED && !LORA && SPB == 1;
    const int pg0 = kStage ? (s_begin >> a.page_shift) : 0;
    const int npg = kStage && s_end > s_begin ? ((s_end - 1) >> a.page_shift) - pg0 + 1 : 0;
    const int nh = 2 * tps;
    const bool pt_lds = kStage && nh <= kDecPtMax;
    uint32_t ptv[kStage ? kDecPtLoads : 1];
    if constexpr (kStage) {
        const __amdgpu_buffer_rsrc_t PT = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(pt_row + pg0), (short)0, pt_lds ? npg * 4 : 0, kBufWord3);
#pragma unroll
        for (int k = 0; k < kDecPtLoads; ++k) {
            // halves past the staged count read out of range (0, no memory access)
            const int h = tid + 64 * nw * k;
            const int q = imax(imin(((s_begin + 16 * h) >> a.page_shift) - pg0, npg - 1), 0);
            ptv[k] = __builtin_amdgcn_raw_buffer_load_b32(PT, h < nh ? 4u * (uint32_t)q : 0x80000000u, 0, 0);
        }
    }
    // rows of the two 16-token halves of the tile at token t, in two steps:
    // from the staged rows when the split's halves fit (an LDS read, then
    // its scalar copies), else from the page table (scalar loads, waited for
    // here, before the next claim is issued, so that wait does not also
    // wait for the claim's atomic)
    struct RowReq { uint2 r; uint32_t rb[2]; };
    auto rows_request = [&](int t, int sq, RowReq &q) {
        if (!kStage || !pt_lds) {
            half_rows(t, sq, q.rb);
            asm volatile("" ::"s"(q.rb[0]), "s"(q.rb[1]));
            __builtin_amdgcn_sched_barrier(0);
            return;
        }
        // claims past the split end (prefetched, never consumed) read the
        // last tile's rows
        const int i = imin((t - s_begin) / kDecTile, tps - 1);
        q.r = *reinterpret_cast<const uint2 *>(smem + kDecPtOff + 8 * i);
    };
    auto rows_resolve = [&](const RowReq &q, uint32_t (&rb)[2]) {
        if (!kStage || !pt_lds) {
            rb[0] = q.rb[0];
            rb[1] = q.rb[1];
            return;
        }
        rb[0] = __builtin_amdgcn_readfirstlane(q.r.x);
        rb[1] = __builtin_amdgcn_readfirstlane(q.r.y);
    };

    // ── prologue loads: branch-free buffer loads (an absent input gets a
    //    zero-size descriptor and reads 0), issued before the cache
    //    prefetch so that waiting for them does not wait for the cache ──
    // this wave's query row
    const bool row_ok = row_valid(wave);
    const int rho_c = row_ok ? row_rho(wave) : 0;
    const int64_t b_q = row_ok ? b + row_seq(wave) : b;
    const int t_q = div_small(rho_c, a.g_magic);
    const int hq_q = hk * a.G + (rho_c - t_q * a.G);
    const bool q32 = a.q_dtype == OMNI_F32;
    const int esz = q32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t QR = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(reinterpret_cast<const char *>(a.q) + ((b_q * a.Hq + hq_q) * a.T + t_q) * (int64_t)(D * esz)),
        (short)0, D * esz, kBufWord3);
    const uint32_t q32_lo = __builtin_amdgcn_raw_buffer_load_b32(QR, 4u * lane, 0, 0);
    const uint32_t q32_hi = __builtin_amdgcn_raw_buffer_load_b32(QR, 4u * (64 + lane), 0, 0);
    const uint32_t q16_lo = __builtin_amdgcn_raw_buffer_load_b16(QR, 2u * lane, 0, 0);
    const uint32_t q16_hi = __builtin_amdgcn_raw_buffer_load_b16(QR, 2u * (64 + lane), 0, 0);
    int32_t lora_id = -1;
    uint32_t lora_xw[4] = {0u, 0u, 0u, 0u};
    if constexpr (LORA) {
        if (row_ok && wave < kDecRows) {
            lora_id = a.lora_idx[b_q];
            lora_x_load(lora_xw, a, b_q, t_q, lane);
        }
    }
    const bool use_flip = a.rotate_q && a.sign_flip;
    const __amdgpu_buffer_rsrc_t SF = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(use_flip ? (const void *)a.sign_flip : (const void *)a.codebooks), (short)0, use_flip ? D : 0, kBufWord3);
    const uint32_t sf_lo = __builtin_amdgcn_raw_buffer_load_b8(SF, (uint32_t)lane, 0, 0);
    const uint32_t sf_hi = __builtin_amdgcn_raw_buffer_load_b8(SF, (uint32_t)(64 + lane), 0, 0);
    // codebook entry lane % 16 (threads 0-15 publish it as fp16 hi / remainder)
    const __amdgpu_buffer_rsrc_t CB = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.codebooks + (a.per_head ? hk * 16 : 0)), (short)0, 16 * 4, kBufWord3);
    const float cb_mine = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(CB, 4u * (lane & 15), 0, 0));
    // G rows 16 * wave + n (waves 0-3 compute that 16-column block of G q)
    const __amdgpu_buffer_rsrc_t GB = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.g_bits + (QJL ? (int64_t)hk * QD * 4 : 0)), (short)0, (QJL && wave < QD / 16) ? QD * 16 : 0, kBufWord3);
    const u32x4_t gw = __builtin_amdgcn_raw_buffer_load_b128(GB, (uint32_t)(16 * wave + n) * 16u, 0, 0);

    // ── both ring slots in flight (tiles `wave` and `wave + nw` of the
    //    split) before the prologue's work, so the cache streams while the
    //    prologue runs.  Loads are unconditional (past the split end they
    //    read 0 and touch no memory), so the compiler counts outstanding
    //    loads exactly and waits only for the tile it consumes. ─────────
    TileRaw ring[PF];
    // claim index i -> (sequence, token offset); i >= ntiles is past the end
    auto tile_seq = [&](int i) { return (nseq > 1 && i >= tps) ? 1 : 0; };
    auto tile_tok = [&](int i) { return s_begin + (i - tile_seq(i) * tps) * kDecTile; };
    if constexpr (PAGED) {
        uint32_t rb0[2], rb1[2];
        half_rows(tile_tok(wave), tile_seq(wave), rb0);
        half_rows(tile_tok(wave + nw), tile_seq(wave + nw), rb1);
        tile_load_paged<QJL>(ring[0], P, OFS, rb0);
        tile_load_paged<QJL>(ring[1], P, OFS, rb1);
    } else {
        tile_load<QJL>(ring[0], tile_seq(wave) ? P1 : P, OFS, tile_tok(wave));
        tile_load<QJL>(ring[1], tile_seq(wave + nw) ? P1 : P, OFS, tile_tok(wave + nw));
    }

    // ── centroid lane % 16 as an (fp16 hi, fp16 remainder) pair ────────
    const uint16_t cb_h16 = f32_to_f16_rne(cb_mine);
    const uint32_t cb_pair = (uint32_t)cb_h16 | ((uint32_t)f32_to_f16_rne(cb_mine - f16_to_f32(cb_h16)) << 16);
    // tiles 0 .. 2 nw - 1 are taken statically (two per wave, already in flight)
    if (tid == 0) *reinterpret_cast<int *>(smem + kDecCntOff) = 2 * nw;
    // ── sign table (threads 0..511) ───────────────────────────────────
    if (tid < 512) sign_table_store(smem, tid);
    // fused LoRA with G % 4 == 0: row slots 4 k .. 4 k + 3 hold one
    // (sequence, token), so x A^T is shared: each of the four waves sums a
    // quarter of its rank components, the others read them after a barrier
    // (same per-lane order and lane tree: the same values)
    const bool lora_share = LORA && (a.G & 3) == 0;
    float *lora_dr = reinterpret_cast<float *>(smem + kDecLrOff) + 16 * (wave >> 2);
    if constexpr (LORA) {
        if (lora_share) {
            if (wave < kDecRows && row_ok) lora_rank_share(a, lora_id, lora_xw, wave, lane, lora_dr);
            __syncthreads();
        }
    }
    if (wave >= kDecRows) {
        // ── byte LUT, built by the waves without a query row while the
        //    others rotate theirs: entry e at e * 256, 32 copies of (hi
        //    pair, lo pair); thread t writes 16-byte chunk t % 16 of the
        //    entries with low nibble t / 16 (high nibble i) ──────────────
        static_assert(kDecWaves - kDecRows == 4, "four LUT-building waves (256 threads)");
        const int t = tid - 64 * kDecRows;
        const uint32_t w0 = __shfl(cb_pair, (t >> 4) & 15);      // low nibble's centroid
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t w1 = __builtin_amdgcn_readlane(cb_pair, i);   // high nibble's centroid
            const int e = (t >> 4) + 16 * i;
            const uint32_t hp = __builtin_amdgcn_perm(w1, w0, 0x05040100u);   // (hi c0, hi c1)
            const uint32_t lp = __builtin_amdgcn_perm(w1, w0, 0x07060302u);   // (lo c0, lo c1)
            *reinterpret_cast<uint4 *>(smem + kLutOff + e * 256 + (t & 15) * 16) = make_uint4(hp, lp, hp, lp);
        }
    } else {
        // ── this wave's query row: (sign flip,) WHT, round to the q dtype ──
        {
            float lo, hi;
            if (q32) {
                lo = __uint_as_float(q32_lo);
                hi = __uint_as_float(q32_hi);
            } else if (a.q_dtype == OMNI_BF16) {
                lo = __uint_as_float(q16_lo << 16);
                hi = __uint_as_float(q16_hi << 16);
            } else {
                lo = f16_to_f32((uint16_t)q16_lo);
                hi = f16_to_f32((uint16_t)q16_hi);
            }
            if constexpr (LORA) {
                if (row_ok) lora_row(lo, hi, a, lora_id, lora_xw, hq_q, lane, lora_share ? lora_dr : nullptr);
            }
            lo = (sf_lo & 0x80u) ? -lo : lo;
            hi = (sf_hi & 0x80u) ? -hi : hi;
            if (a.rotate_q) {
                wht128_lanes(lo, hi, lane);
                lo = round_to_dtype(lo * a.wht_scale, a.q_dtype);
                hi = round_to_dtype(hi * a.wht_scale, a.q_dtype);
            }
            // row max |q| -> 2^k with max * 2^k in [2^14, 2^15): the scaled row
            // and G q (|.| <= 128 * 2^15 * sqrt(2/pi) / 128) stay in fp16 range
            // for any finite q; scores take scale * log2(e) * 2^-k
            float m = row_ok ? fmaxf(fabsf(lo), fabsf(hi)) : 0.0f;
            m = wave_max(m);
            int ex = 0;
            if (m > 0.0f && m < INFINITY) frexpf(m, &ex);
            const float sr = ldexpf(1.0f, 15 - imax(ex, -100));     // 2^k stays finite for tiny rows
            // the score scale's sign goes into the staged row (exact), so the
            // row's factor |scale| log2(e) / 2^k >= 0 maps raw scores
            // monotonically.  A factor below 2^-126 is raised to it: raw
            // scores stay below 2^40, so no exponent moves by more than
            // 2^-86, and a masked key's -inf times the factor stays -inf (a
            // zero scale, whose inf x 0 = NaN this would hide, runs another
            // kernel).
            const float ssr = a.qscale < 0.0f ? -sr : sr;
            qs[wave * D + lane] = row_ok ? lo * ssr : 0.0f;
            qs[wave * D + 64 + lane] = row_ok ? hi * ssr : 0.0f;
            const float cf = fabsf(a.qscale) / sr;
            if (lane == 0) reinterpret_cast<float *>(smem + kDecCscOff)[wave] = cf < 0x1p-126f ? 0x1p-126f : cf;
        }
        // MFMA operand images of this row (read back by the same wave):
        //   lanes 0-31, quad j = dims 4j..4j+3 of 2^k q: B slots
        //     hi [h0 h1 h0 h1 h2 h3 h2 h3], lo [l0 l1 0 0 l2 l3 0 0]
        //   lanes 32-47, group j = dims 8j..8j+7 of 2^k q: A slots hi / lo
        if (lane < 32) {
            const float4 v = *reinterpret_cast<const float4 *>(qs + wave * D + 4 * lane);
            const float h[4] = {v.x, v.y, v.z, v.w};
            float l[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) l[j] = h[j] - f16_to_f32(f32_to_f16_rne(h[j]));
            uint4 *dst = reinterpret_cast<uint4 *>(smem + kDecBkOff + dec_chunk(wave, (wave * 32 + lane) * 2) * 16);
            dst[0] = make_uint4(pack_h2(h[0], h[1]), pack_h2(h[0], h[1]), pack_h2(h[2], h[3]), pack_h2(h[2], h[3]));
            dst[1] = make_uint4(pack_h2(l[0], l[1]), 0u, pack_h2(l[2], l[3]), 0u);
        } else if (QJL && lane < 48) {
            const int j = lane - 32;
            const float4 v0 = *reinterpret_cast<const float4 *>(qs + wave * D + 8 * j);
            const float4 v1 = *reinterpret_cast<const float4 *>(qs + wave * D + 8 * j + 4);
            const float x[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                hw[k] = pack_h2(x[2 * k], x[2 * k + 1]);
                lw[k] = pack_h2(x[2 * k] - f16_to_f32(f32_to_f16_rne(x[2 * k])),
                                x[2 * k + 1] - f16_to_f32(f32_to_f16_rne(x[2 * k + 1])));
            }
            uint4 *dst = reinterpret_cast<uint4 *>(smem + kDecGaOff + dec_chunk(wave, (wave * 16 + j) * 2) * 16);
            dst[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
            dst[1] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        }
    }
    if constexpr (kStage) {
        // pool row of each staged half: (page * Hkv + hk) * page_size + slot;
        // a page id outside the pool reads page 0 and, for a half that holds
        // tokens of the sequence, flags the wave (rows come out NaN)
        uint32_t *ptl = reinterpret_cast<uint32_t *>(smem + kDecPtOff);
        const uint32_t np = (uint32_t)a.n_pages;                  // < 2^26 (host check)
        const uint32_t pmask = (1u << a.page_shift) - 1u;
        bool bad = false;
#pragma unroll
        for (int k = 0; k < kDecPtLoads; ++k) {
            const int h = tid + 64 * nw * k;
            const int th = s_begin + 16 * h;
            const bool ok = ptv[k] < np;                          // negative ids wrap past np
            bad = bad || (pt_lds && h < nh && !ok && th < s_end);
            if (pt_lds && h < nh)
                ptl[h] = (((ok ? ptv[k] : 0u) * (uint32_t)a.Hkv + (uint32_t)hk) << a.page_shift) +
                         ((uint32_t)th & pmask);
        }
        const bool wbad = __builtin_amdgcn_ballot_w64(bad) != 0;
        if (lane == 0) reinterpret_cast<uint32_t *>(smem + kDecPtFlagOff)[wave] = wbad ? 1u : 0u;
    }
    __syncthreads();
    if constexpr (kStage) {
        // the split's bad pages poison every wave's denominator (the block
        // merges them all, so this is the sequence's result either way)
        if (pt_lds) {
            const uint32_t *fl = reinterpret_cast<const uint32_t *>(smem + kDecPtFlagOff);
            uint32_t any = 0u;
#pragma unroll
            for (int w = 0; w < kDecWaves; ++w) any |= w < nw ? fl[w] : 0u;
            page_bad = any != 0u;
        }
    }


    if (QJL && wave < QD / 16) {
        // GQ (rows x 64) = Q (rows x 128) . G_h^T on MFMA, one 16-column block
        // per wave: Q as fp16 hi + lo, G rows expanded 8 bits at a time
        // through the sign LUT.
        const int cb = wave;
        half8_t ah[4], al[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            uint4 hv = make_uint4(0u, 0u, 0u, 0u), lv = hv;
            if (n < kDecRows) {
                const uint4 *src = reinterpret_cast<const uint4 *>(smem + kDecGaOff + dec_chunk(n, (n * 16 + 4 * s + g) * 2) * 16);
                hv = src[0];
                lv = src[1];
            }
            ah[s] = as_half8(hv.x, hv.y, hv.z, hv.w);
            al[s] = as_half8(lv.x, lv.y, lv.z, lv.w);
        }
        float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
        const int o = 16 * cb + n;
        const uint32_t gws[4] = {gw.x, gw.y, gw.z, gw.w};
        const uint32_t slane = (uint32_t)kSlutOff | ((uint32_t)(lane & 31) * 8u);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const half8_t bg = sign_halves(smem, gws[s], 8u * g, slane);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[s], bg, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[s], bg, acc, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (4 * g + i < kDecRows) gq[(4 * g + i) * kDecGqStride + o] = acc[i];
    }
    __syncthreads();

    // ── per-lane B operands ───────────────────────────────────────────
    const bool lo_col = n >= kDecRows;           // columns 8-15
    const int rn = lo_col ? n - kDecRows : n;
    half8_t bk[8], bgq[2];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        // quad 8g + s of row rn: columns 0-7 take the hi image, 8-15 the lo image
        const uint4 v = *reinterpret_cast<const uint4 *>(smem + kDecBkOff + (dec_chunk(rn, (rn * 32 + 8 * g + s) * 2) + (lo_col ? 1 : 0)) * 16);
        bk[s] = as_half8(v.x, v.y, v.z, v.w);
    }
    // QJL B operand carries sqrt(2/pi) / D on G (2^k q) (fp16 in columns
    // 0-7, its fp16 remainder in 8-15), so a score needs only
    // norm * (signs . B) on top of the K pass, then the row's scale
    const float gscale = a.alpha_c;
    const float csc = reinterpret_cast<const float *>(smem + kDecCscOff)[rn];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float *row = gq + rn * kDecGqStride + 32 * s + 8 * g + 2 * j;
            float g0 = row[0] * gscale, g1 = row[1] * gscale;
            if (lo_col) {
                g0 -= (float)(_Float16)g0;
                g1 -= (float)(_Float16)g1;
            }
            w[j] = QJL ? pack_h2(g0, g1) : 0u;
        }
        bgq[s] = as_half8(w[0], w[1], w[2], w[3]);
    }
    const int rho_n = row_rho(rn);
    const int seq_n = row_seq(rn);             // this column's sequence
    // causal: query token t sees keys <= coff + t (a paged cache aligns the
    // last query token with the sequence's last key: coff = length - T)
    const bool causal = a.causal_offset >= 0;
    const int64_t coff = PAGED ? (int64_t)(seq_n ? seq_len1 : seq_len) - a.T : a.causal_offset;
    const int64_t key_limit64 = (causal && row_valid(rn)) ? coff + div_small(rho_n, a.g_magic) : INT64_MAX;

    // ── main loop ─────────────────────────────────────────────────────
    const int key_limit = (int)imax64(imin64(key_limit64, (int64_t)0x7fffffff), -1);
    // tiles ending at or below min(s_end, first masked key of any row) need no masks
    const int64_t min_limit64 = causal ? coff + div_small(rc * kDecRows, a.g_magic) : INT64_MAX;
    // two sequences per block: every tile masks the other sequence's columns
    const int full_end = nseq > 1 ? s_begin : (int)imin64((int64_t)s_end, min_limit64 + 1);
    const uint32_t laneoff = (uint32_t)(lane & 31) * 8u;
    const uint32_t slane = (uint32_t)kSlutOff | laneoff;
    // ones in every slot of A row 0: one MFMA sums the P of all 32 tokens of
    // a tile (B holds the two halves' P side by side).  Only output row 0 of
    // that MFMA is read (lanes with n == 0 hold A row 0): the other rows get
    // zeros.  The matrix cores run at a power-limited clock under sustained
    // load, and operands that only feed discarded outputs still cost power
    // when nonzero.
    const uint32_t one2 = n == 0 ? 0x3C003C00u : 0u;
    const half8_t ones = as_half8(one2, one2, one2, one2);
    const unsigned char *lut = smem + kLutOff;

    float4_t oacc[8], lacc_sum;
#pragma unroll
    for (int k = 0; k < 8; ++k) oacc[k] = float4_t{0.f, 0.f, 0.f, 0.f};
    lacc_sum = float4_t{0.f, 0.f, 0.f, 0.f};
    // running max starts at -FLT_MAX rather than -inf, so it can serve as the
    // exponent offset directly: a tile whose keys are all masked (-inf)
    // still gives exp2(-inf - m) = 0, and the first finite maximum replaces
    // it (scaling the empty accumulators by exp2(-FLT_MAX - mt) = 0)
    // Padding row slots (no query row) start at +FLT_MAX instead, so every
    // probability of their columns is exp2(-FLT_MAX) = 0 and the PV operand
    // columns they feed stay zero (their outputs are never read).
    float m_run = row_valid(rn) ? -__FLT_MAX__ : __FLT_MAX__;
    // Exponents are fma(raw, csc, -m_run): exact products against a rounded
    // maximum, which keeps relative weights exact but puts an error of up to
    // half an ulp of m_run on every exponent.  Once any row's |m_run| reaches
    // 2^13 (that error would pass 2^-11) the wave rounds each logit first,
    // as the reference does (wave-uniform, set at most once).
    bool round_first = false;

    // One 32-token tile: scores, online softmax, PV.
    auto tile_step = [&](TileRaw &R, const int tt, const int tseq, auto &&after_k) {
        const bool full = tt + kDecTile <= full_end;
        // wave priority by phase: the K pass 2, masks and maxima 1, the
        // softmax and PV 0 (issue order only: results do not depend on it)
        __builtin_amdgcn_s_setprio(2);

        // scores: lane (n, g) holds tokens tt + 16u + 4g + i
        float sc[8];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f}, qacc = float4_t{0.f, 0.f, 0.f, 0.f};
            const uint32_t kw[4] = {R.k[u].x, R.k[u].y, R.k[u].z, R.k[u].w};
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const uint2 e0 = *reinterpret_cast<const uint2 *>(lut + lut_addr(kw[s >> 1], laneoff, 2 * (s & 1)));
                const uint2 e1 = *reinterpret_cast<const uint2 *>(lut + lut_addr(kw[s >> 1], laneoff, 2 * (s & 1) + 1));
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pair_half8(e0, e1), bk[s], acc, 0, 0, 0);
            }
            if (QJL) {
#pragma unroll
                for (int s = 0; s < 2; ++s)
                    qacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(sign_halves(smem, s ? R.sg[u].y : R.sg[u].x, 8u * g, slane),
                                                                  bgq[s], qacc, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // token 4g + i's norm sits in lane 4 * (n / 4) + i of this row:
                // a quad broadcast.  Columns 8-15 compute finite junk that
                // never reaches columns 0-7 (MFMA columns are independent)
                // nor the output.
                float v = acc[i];
                if (QJL) v = __builtin_fmaf(dpp_quad_bcast(R.nr[u], i), qacc[i], v);
                // columns n and n + 8 (hi and lo parts of row n) both get the
                // raw sum; the row's factor csc >= 0 enters each exponent's fma
                sc[4 * u + i] = v + __uint_as_float(dpp_row_ror8(__float_as_uint(v)));
            }
        }
        __builtin_amdgcn_s_setprio(1);
        after_k();
        if (!full) {
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int tn = tt + 16 * u + 4 * g + i;
                    if (tn >= (tseq ? s_end1 : s_end) || tn > key_limit || seq_n != tseq) sc[4 * u + i] = -INFINITY;
                }
        }

        // online softmax (exp2 domain), lazy rescale.  The scaled maximum of
        // the lane's scores is csc times their raw maximum (rounding is
        // monotonic and csc >= 2^-126, so a fully masked lane gives -inf),
        // so every exponent below is at most 8 plus the rounding of one
        // product.  m_run is the same in the four lane
        // groups of a row (it only ever takes a cross-group maximum), so each
        // lane tests its own maximum and the cross-group maximum is formed
        // only when some lane rescales.
        const float mr = vmax3(vmax3(sc[0], sc[1], sc[2]), vmax3(sc[3], sc[4], sc[5]), vmax2(sc[6], sc[7]));
        float mt = mr * csc;
        __builtin_amdgcn_s_setprio(0);
        if (__builtin_amdgcn_ballot_w64(mt > m_run + 8.0f)) {
            mt = max_over_groups(mt);
            const bool need = mt > m_run + 8.0f;
            const float f = need ? __builtin_amdgcn_exp2f(m_run - mt) : 1.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) oacc[k] *= f;
            lacc_sum *= f;
            // in place (one register for the running maximum on both paths:
            // no copy where no lane rescales)
            const uint64_t nmask = __builtin_amdgcn_ballot_w64(need);
            asm volatile("v_cndmask_b32 %0, %0, %1, %2" : "+v"(m_run) : "v"(mt), "s"(nmask));
            round_first = round_first ||
                          __builtin_amdgcn_ballot_w64(fabsf(m_run) >= 8192.0f && m_run > -__FLT_MAX__ && m_run < __FLT_MAX__);
        }
        const float nm = -m_run;
        // lanes n and n + 8 hold the same scores: columns 0-7 exponentiate the
        // tile's first 16 tokens, columns 8-15 the last 16, and the halves
        // trade places by a row rotation (B columns 8-15 feed output columns
        // that are never read, so what they hold does not matter).  csc >=
        // 2^-126, so masked keys give exp2(-inf) = 0.
        float ex[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) ex[k] = lo_col ? sc[4 + k] : sc[k];
        // the two modes as separate code (no select of the multiplier)
        if (round_first) {
#pragma unroll
            for (int k = 0; k < 4; ++k) ex[k] = ex[k] * csc + nm;
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) ex[k] = __builtin_fmaf(ex[k], csc, nm);
        }
        const uint32_t my01 = cvt_pk_h2(__builtin_amdgcn_exp2f(ex[0]), __builtin_amdgcn_exp2f(ex[1]));
        const uint32_t my23 = cvt_pk_h2(__builtin_amdgcn_exp2f(ex[2]), __builtin_amdgcn_exp2f(ex[3]));
        const uint32_t ot01 = dpp_row_ror8(my01), ot23 = dpp_row_ror8(my23);
        // B columns 8-15 of PV feed output columns that are never read: zero
        // (power, as for the denominator's ones)
        half8_t pb[2];
        {
            const uint32_t a01 = lo_col ? 0u : my01, a23 = lo_col ? 0u : my23;
            const uint32_t b01 = lo_col ? 0u : ot01, b23 = lo_col ? 0u : ot23;
            pb[0] = as_half8(a01, a01, a23, a23);
            pb[1] = as_half8(b01, b01, b23, b23);
            // the denominator: tokens 4g .. 4g + 3 of both halves in one operand
            lacc_sum = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, as_half8(a01, a23, b01, b23), lacc_sum, 0, 0, 0);
        }

        // PV: pair bytes interleave the nibbles of two tokens at one d, so
        // each LUT entry is an MFMA-ready (hi pair, lo pair) for that d.
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            uint32_t ev[2], od[2];
#pragma unroll
            for (int pr = 0; pr < 2; ++pr) {
                const uint32_t va = R.v[4 * u + 2 * pr], vb = R.v[4 * u + 2 * pr + 1];
                ev[pr] = ((vb << 4) & 0xF0F0F0F0u) | (va & 0x0F0F0F0Fu);
                od[pr] = (vb & 0xF0F0F0F0u) | ((va >> 4) & 0x0F0F0F0Fu);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint2 e0 = *reinterpret_cast<const uint2 *>(lut + lut_addr(ev[0], laneoff, j));
                const uint2 e1 = *reinterpret_cast<const uint2 *>(lut + lut_addr(ev[1], laneoff, j));
                oacc[2 * j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pair_half8(e0, e1), pb[u], oacc[2 * j], 0, 0, 0);
                const uint2 f0 = *reinterpret_cast<const uint2 *>(lut + lut_addr(od[0], laneoff, j));
                const uint2 f1 = *reinterpret_cast<const uint2 *>(lut + lut_addr(od[1], laneoff, j));
                oacc[2 * j + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pair_half8(f0, f1), pb[u], oacc[2 * j + 1], 0, 0, 0);
            }
        }
    };

    // Tiles are claimed dynamically from the block's LDS counter: the waves
    // sharing a SIMD do not progress at the same rate (the issue arbiter
    // favours the oldest), and static round-robin tiles would leave the
    // youngest waves running alone at the end.  Each loop step claims the
    // tile after next (its result is needed one step later, so the atomic's
    // latency hides behind the LUT traffic), prefetches the next tile
    // (unconditionally: past the split end it reads 0 and touches no
    // memory) and consumes the current one.  A wave's claims increase, so
    // the first tile past the end means every later one is past it too.
    // The first two tiles (both slots, issued before the prologue) are
    // consumed ahead of the loop, so only one slot is live at its head.
    static_assert(PF == 2, "the dynamic tile loop alternates two ring slots");
    int *tile_cnt = reinterpret_cast<int *>(smem + kDecCntOff);
    int i_cur = wave;
    int c_raw = claim_issue(tile_cnt, lane);
    if (i_cur < ntiles) {
        tile_step(ring[0], tile_tok(i_cur), tile_seq(i_cur), [] {});
        const int i_pre = wave + nw;
        if (i_pre < ntiles && PAGED) {
            // paged: the claimed tile's pool rows are requested before the
            // current tile's K pass and its loads issued right after it, so
            // the row read's latency hides behind the K pass
            RowReq q;
            i_cur = claim_value(c_raw);
            rows_request(tile_tok(i_cur), tile_seq(i_cur), q);
            c_raw = claim_issue(tile_cnt, lane);
            tile_step(ring[1], tile_tok(i_pre), tile_seq(i_pre), [&] {
                uint32_t rb[2];
                rows_resolve(q, rb);
                __builtin_amdgcn_sched_barrier(0);
                tile_load_paged<QJL>(ring[0], P, ofs_loop(), rb);
                __builtin_amdgcn_sched_barrier(0);
            });
            for (;;) {
                if (i_cur >= ntiles) break;
                const int i_nxt = claim_value(c_raw);
                rows_request(tile_tok(i_nxt), tile_seq(i_nxt), q);
                c_raw = claim_issue(tile_cnt, lane);
                tile_step(ring[0], tile_tok(i_cur), tile_seq(i_cur), [&] {
                    uint32_t rb[2];
                    rows_resolve(q, rb);
                    __builtin_amdgcn_sched_barrier(0);
                    tile_load_paged<QJL>(ring[1], P, ofs_loop(), rb);
                    __builtin_amdgcn_sched_barrier(0);
                });
                if (i_nxt >= ntiles) break;
                i_cur = claim_value(c_raw);
                rows_request(tile_tok(i_cur), tile_seq(i_cur), q);
                c_raw = claim_issue(tile_cnt, lane);
                tile_step(ring[1], tile_tok(i_nxt), tile_seq(i_nxt), [&] {
                    uint32_t rb[2];
                    rows_resolve(q, rb);
                    __builtin_amdgcn_sched_barrier(0);
                    tile_load_paged<QJL>(ring[0], P, ofs_loop(), rb);
                    __builtin_amdgcn_sched_barrier(0);
                });
            }
        } else if (i_pre < ntiles) {
            i_cur = claim_value(c_raw);
            c_raw = claim_issue(tile_cnt, lane);
            __builtin_amdgcn_sched_barrier(0);
            tile_load<QJL>(ring[0], tile_seq(i_cur) ? P1 : P, ofs_loop(), tile_tok(i_cur));
            __builtin_amdgcn_sched_barrier(0);
            tile_step(ring[1], tile_tok(i_pre), tile_seq(i_pre), [] {});
            for (;;) {
                if (i_cur >= ntiles) break;
                const int i_nxt = claim_value(c_raw);
                c_raw = claim_issue(tile_cnt, lane);
                __builtin_amdgcn_sched_barrier(0);
                tile_load<QJL>(ring[1], tile_seq(i_nxt) ? P1 : P, ofs_loop(), tile_tok(i_nxt));
                __builtin_amdgcn_sched_barrier(0);
                tile_step(ring[0], tile_tok(i_cur), tile_seq(i_cur), [] {});
                if (i_nxt >= ntiles) break;
                i_cur = claim_value(c_raw);
                c_raw = claim_issue(tile_cnt, lane);
                __builtin_amdgcn_sched_barrier(0);
                tile_load<QJL>(ring[0], tile_seq(i_cur) ? P1 : P, ofs_loop(), tile_tok(i_cur));
                __builtin_amdgcn_sched_barrier(0);
                tile_step(ring[1], tile_tok(i_nxt), tile_seq(i_nxt), [] {});
            }
        }
    }

    // ── combine waves (in wave order) ───────────────────────────────
    __syncthreads();   // LUTs are dead from here on
    float *ob = reinterpret_cast<float *>(smem);                     // [nw][kDecRows][kObStride]
    float *wm = reinterpret_cast<float *>(smem + kDecSlabBytes);     // [nw][kDecRows] running max
    float *wl = wm + kDecWaves * kDecRows;                           // [nw][kDecRows] denominators
    // Each wave's first tile is its own index, so waves at or past the tile
    // count claimed nothing: only the first min(nw, ntiles) slabs (at least
    // one, so an empty split still merges one empty state) hold data.
    const int nw_act = ntiles < 1 ? 1 : (ntiles < nw ? ntiles : nw);
    {
        // lane coordinates recomputed here (opaque), so no address of this
        // step is kept live across the main loop
        int le = lane;
        asm volatile("" : "+v"(le));
        const int ne = le & 15, ge = le >> 4;
        if (ne < kDecRows && wave < nw_act) {
            if (ge == 0) {
                wm[wave * kDecRows + ne] = m_run;
                // a page outside the pool poisons the sequence's denominator
                wl[wave * kDecRows + ne] = (row_seq(ne) ? page_bad1 : page_bad) ? __builtin_nanf("") : lacc_sum[0];
            }
            float *dst = ob + (wave * kDecRows + ne) * kObStride;
#pragma unroll
            for (int k = 0; k < 8; ++k)
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[8 * (4 * ge + i) + k] = oacc[k][i];
        }
    }
    __syncthreads();
    const int64_t unit = (b * a.Hkv + hk) * a.n_rchunks + rc;
    // (max, denominator, output element) of row rr, dim d over the first
    // `cnt` slabs in wave order; a compile-time count unrolls the loops
    auto merge = [&](auto cnt, int rr, int d, float &rmx, float &lsum, float &osum) {
        rmx = -INFINITY;
        for (int w = 0; w < cnt; ++w) rmx = fmaxf(rmx, wm[w * kDecRows + rr]);
        const float rmu = (rmx == -INFINITY) ? 0.0f : rmx;
        lsum = 0.0f;
        osum = 0.0f;
        for (int w = 0; w < cnt; ++w) {
            // merge weights lie in [0, 1]; the hardware exp2 is within 1 ulp
            const float f = __builtin_amdgcn_exp2f(wm[w * kDecRows + rr] - rmu);
            lsum = __builtin_fmaf(f, wl[w * kDecRows + rr], lsum);
            osum = __builtin_fmaf(f, ob[(w * kDecRows + rr) * kObStride + d], osum);
        }
    };
    for (int s = tid; s < kDecRows * D; s += blockDim.x) {
        const int rr = s / D, d = s % D;
        if (!row_valid(rr)) continue;
        const int rr_rho = row_rho(rr);
        const int64_t rr_b = b + row_seq(rr);
        float rmx, lsum, osum;
        if (nw_act == nw) merge(std::integral_constant<int, nw>{}, rr, d, rmx, lsum, osum);
        else merge(nw_act, rr, d, rmx, lsum, osum);
        if (row_seq(rr) ? cs_bad1 : cs_bad0) lsum = __builtin_nanf("");
        if (row_seq(rr) ? len_bad1 : len_bad) lsum = __builtin_nanf("");
        if (a.splits == 1) {
            const int t = div_small(rr_rho, a.g_magic);
            const int hq = hk * a.G + (rr_rho - t * a.G);
            a.out[((rr_b * a.Hq + hq) * a.T + t) * D + d] = osum / lsum;
        } else {
            float *wp = a.ws + ((unit * a.splits + split) * kDecRows + rr) * (D + 2);
            wp[d] = osum;
            if (d == 0) { wp[D] = rmx; wp[D + 1] = lsum; }
        }
    }
}

// ── chunked-prefill kernel (many query rows per (batch, kv head)) ────────
//
// Same math as the decode kernel, organised for T > 1: each wave owns 16 * NCB
// query rows (NCB MFMA column blocks) and streams every key tile for them, so
// each K / V operand decoded from the LUT feeds NCB column blocks; eight
// waves (128 * NCB rows) share one block's LUTs.  q enters the MFMA exactly:
// the rows are bf16 / f16, scaled per row by a power of two into fp16 range,
// and the softmax scale is applied to the fp32 score (score =
// acc * scale / 2^k + norm * (signs . Gq')), so K (fp16 hi + remainder on the
// k axis) and q carry no extra rounding.  f32 queries (QLO) add a second B
// operand with the fp16 remainder of the scaled q.  V is the decode kernel's pair-byte
// (hi, lo) operand.  Rows past T * G, or keys past a row's causal limit,
// are masked.
constexpr int kPreWaves = 8;
constexpr int kPrefillMinRows = 32;                              // T * (Hq / Hkv) above this takes this kernel
constexpr int kPreNcb = 2;                                       // column blocks per wave for 16-bit q (f32 q: 1)
constexpr int kPreCbOff = kSlutOff + kSlutBytes;                 // 16 x (fp16 hi | remainder << 16)
constexpr int kPreStageOff = kPreCbOff + 64;                     // per wave: q rows fp16, then G q fp32
constexpr int kPreQsrOff = kPreStageOff + kPreWaves * 32 * 128 * 2;   // per wave: 32 x f32 score scales
constexpr int kPreLdsBytes = kPreQsrOff + kPreWaves * 32 * 4;

template <bool QJL, int NCB, int PF, bool QLO, bool PAGED>
__global__ __launch_bounds__(64 * kPreWaves) void attn_prefill128_kernel(AttnArgs a) {
    constexpr int D = 128, QD = 64, RW = 16 * NCB;      // rows per wave
    static_assert(!QLO || NCB == 1, "the f32 remainder plane shares the 32-row stage area");
    __shared__ __attribute__((aligned(16))) unsigned char smem[kPreLdsBytes];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int split = blockIdx.x, hk = blockIdx.y;
    const int64_t bz = blockIdx.z;
    const int64_t b = bz / a.n_rchunks;
    const int rc = (int)(bz % a.n_rchunks);
    const int nrows_total = (int)(a.T * a.G);
    const int row0 = rc * a.rows + wave * RW;                  // first flat row of this wave
    unsigned char *stage = smem + kPreStageOff + wave * 32 * 128 * 2;
    float *qsr_l = reinterpret_cast<float *>(smem + kPreQsrOff) + wave * 32;

    // ── LUTs (as the decode kernel) ───────────────────────────────────
    {
        const __amdgpu_buffer_rsrc_t CB = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(a.codebooks + (a.per_head ? hk * 16 : 0)), (short)0, 16 * 4, kBufWord3);
        const float c = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(CB, 4u * (lane & 15), 0, 0));
        const uint16_t h = f32_to_f16_rne(c);
        *reinterpret_cast<uint32_t *>(smem + kPreCbOff + 4 * (lane & 15)) =
            (uint32_t)h | ((uint32_t)f32_to_f16_rne(c - f16_to_f32(h)) << 16);
    }
    sign_table_store(smem, tid);      // 512 threads

    // ── this wave's query rows: (sign flip,) WHT, round; per-row power-of-2
    //    scale into fp16 range; staged as fp16 ───────────────────────────
    {
        const bool use_flip = a.rotate_q && a.sign_flip;
        const bool flip_lo = use_flip && a.sign_flip[lane] < 0, flip_hi = use_flip && a.sign_flip[64 + lane] < 0;
        // the score scale's sign goes into the staged rows (exact), so every
        // row's score scale is >= 0 and the exponent takes it in an fma
        const float ssign = a.qscale < 0.0f ? -1.0f : 1.0f;
        for (int rr = 0; rr < RW; ++rr) {
            const int rho = row0 + rr;
            const bool ok = rho < nrows_total;
            const int rc_ = ok ? rho : nrows_total - 1;
            const int t = rc_ / a.G, hq = hk * a.G + (rc_ - t * a.G);
            const int64_t base = ((b * a.Hq + hq) * a.T + t) * D;
            float lo = load_as_f32(a.q, a.q_dtype, base + lane), hi = load_as_f32(a.q, a.q_dtype, base + 64 + lane);
            lo = flip_lo ? -lo : lo;
            hi = flip_hi ? -hi : hi;
            if (a.rotate_q) {
                wht128_lanes(lo, hi, lane);
                lo = round_to_dtype(lo * a.wht_scale, a.q_dtype);
                hi = round_to_dtype(hi * a.wht_scale, a.q_dtype);
            }
            if (!ok) lo = hi = 0.0f;
            // row max |q| -> 2^k with max * 2^k in [2^14, 2^15)
            float m = fmaxf(fabsf(lo), fabsf(hi));
            m = wave_max(m);
            int ex = 0;
            if (m > 0.0f && m < INFINITY) { frexpf(m, &ex); }
            const float sr = ldexpf(1.0f, 15 - imax(ex, -100));   // m * sr in [2^14, 2^15) unless m < 2^-101
            const float los = ssign * lo * sr, his = ssign * hi * sr;
            const uint16_t l16 = f32_to_f16_rne(los), h16 = f32_to_f16_rne(his);
            reinterpret_cast<uint16_t *>(stage)[rr * D + lane] = l16;
            reinterpret_cast<uint16_t *>(stage)[rr * D + 64 + lane] = h16;
            if constexpr (QLO) {
                // second plane: fp16 remainder of the scaled f32 row
                uint16_t *lop = reinterpret_cast<uint16_t *>(stage) + 16 * D;
                lop[rr * D + lane] = f32_to_f16_rne(los - f16_to_f32(l16));
                lop[rr * D + 64 + lane] = f32_to_f16_rne(his - f16_to_f32(h16));
            }
            // a positive factor is kept >= FLT_MIN (one that underflows
            // leaves every score as good as 0 either way), so a masked
            // score's -inf stays -inf through the maximum and the exponent;
            // a zero scale keeps 0 (inf x 0 = NaN, as the reference forms
            // scale x score) and re-masks the exponents below
            const float q0 = fabsf(a.qscale) / sr;
            if (lane == 0) qsr_l[rr] = (q0 < __FLT_MIN__ && a.qscale != 0.0f) ? __FLT_MIN__ : q0;
        }
    }
    __syncthreads();

    // ── byte LUT (after the codebook table is visible) ───────────────────
    {
        const uint32_t *cbh = reinterpret_cast<const uint32_t *>(smem + kPreCbOff);
        const uint32_t w0 = cbh[(tid >> 4) & 15];
        uint32_t w1[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w1[i] = cbh[(tid >> 8) + 2 * i];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = (tid >> 4) + 32 * i;
            const uint32_t hp = __builtin_amdgcn_perm(w1[i], w0, 0x05040100u);
            const uint32_t lp = __builtin_amdgcn_perm(w1[i], w0, 0x07060302u);
            *reinterpret_cast<uint4 *>(smem + kLutOff + e * 256 + (tid & 15) * 16) = make_uint4(hp, lp, hp, lp);
        }
    }

    // ── per-lane B operands: q (exact fp16) for the scores ───────────────
    half8_t bk[NCB][8], bgq[NCB][2], bgl[NCB][2], bkl[QLO ? NCB : 1][8];
    float qsr[NCB];
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
        const uint16_t *qrow = reinterpret_cast<const uint16_t *>(stage) + (16 * c + n) * D;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint2 w = *reinterpret_cast<const uint2 *>(qrow + 32 * g + 4 * s);
            bk[c][s] = as_half8(w.x, w.x, w.y, w.y);
        }
        qsr[c] = qsr_l[16 * c + n];
        if constexpr (QLO) {
            const uint16_t *lrow = reinterpret_cast<const uint16_t *>(stage) + 16 * D + (16 * c + n) * D;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const uint2 w = *reinterpret_cast<const uint2 *>(lrow + 32 * g + 4 * s);
                bkl[c][s] = as_half8(w.x, w.x, w.y, w.y);
            }
        }
    }
    // G q (staged scale) on MFMA: A = q rows, B = G rows expanded by the sign LUT
    __syncthreads();   // sign LUT visible
    float4_t gacc[NCB][4];
#pragma unroll
    for (int c = 0; c < NCB; ++c)
#pragma unroll
        for (int ob = 0; ob < 4; ++ob) gacc[c][ob] = float4_t{0.f, 0.f, 0.f, 0.f};
    if (QJL) {
        const uint32_t *gh = a.g_bits + (int64_t)hk * QD * 4;
#pragma unroll
        for (int ob = 0; ob < 4; ++ob) {
            const uint4 gw = *reinterpret_cast<const uint4 *>(gh + (16 * ob + n) * 4);
            const uint32_t gws[4] = {gw.x, gw.y, gw.z, gw.w};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const half8_t bg = sign_halves(smem, gws[s], 8u * g, (uint32_t)kSlutOff | ((uint32_t)(lane & 31) * 8u));
#pragma unroll
                for (int c = 0; c < NCB; ++c) {
                    const uint4 qv = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(stage) +
                                                                     (16 * c + n) * D + 32 * s + 8 * g);
                    gacc[c][ob] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(qv.x, qv.y, qv.z, qv.w), bg,
                                                                        gacc[c][ob], 0, 0, 0);
                    if constexpr (QLO) {
                        // the f32 row's fp16 remainder plane
                        const uint4 lv = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(stage) +
                                                                         16 * D + (16 * c + n) * D + 32 * s + 8 * g);
                        gacc[c][ob] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(lv.x, lv.y, lv.z, lv.w), bg,
                                                                            gacc[c][ob], 0, 0, 0);
                    }
                }
            }
        }
    }
    // gacc[c][ob][i] = (staged) G q for row 16 c + 4 g + i, output 16 ob + n:
    // through the stage area (q is no longer needed) into B layout
    float *gqs = reinterpret_cast<float *>(stage);     // [RW][64]
#pragma unroll
    for (int c = 0; c < NCB; ++c)
#pragma unroll
        for (int ob = 0; ob < 4; ++ob)
#pragma unroll
            for (int i = 0; i < 4; ++i) gqs[(16 * c + 4 * g + i) * QD + 16 * ob + n] = gacc[c][ob][i];
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
        // B carries sqrt(2/pi) / D on the staged (2^k-scaled) G q (fp16 hi in
        // bgq, fp16 remainder in bgl); norm * (signs . B) joins K . q in the
        // score accumulator and both take the row's scale * 2^-k
        const float gsc = a.alpha_c;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const float *row = gqs + (16 * c + n) * QD + 32 * s + 8 * g;
            uint32_t w[4], wl[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float g0 = row[2 * j] * gsc, g1 = row[2 * j + 1] * gsc;
                w[j] = QJL ? pack_h2(g0, g1) : 0u;
                wl[j] = QJL ? pack_h2(g0 - (float)(_Float16)g0, g1 - (float)(_Float16)g1) : 0u;
            }
            bgq[c][s] = as_half8(w[0], w[1], w[2], w[3]);
            bgl[c][s] = as_half8(wl[0], wl[1], wl[2], wl[3]);
        }
    }
    // the QJL B operands go back to the stage area as lane-linear images and
    // are read there every tile: held in registers they push the loop past
    // the register file
    {
        uint4 *img = reinterpret_cast<uint4 *>(stage);
#pragma unroll
        for (int c = 0; c < NCB; ++c)
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                img[((c * 2 + s) * 2) * 64 + lane] = __builtin_bit_cast(uint4, bgq[c][s]);
                img[((c * 2 + s) * 2 + 1) * 64 + lane] = __builtin_bit_cast(uint4, bgl[c][s]);
            }
    }
    const uint32_t qimg_off = (uint32_t)(stage - smem) + (uint32_t)lane * 16u;
    __syncthreads();   // byte LUT complete

    // ── key range of this wave: causal limits of its rows ─────────────────
    // paged: the sequence's own length (one outside [0, capacity] reads
    // nothing and its rows come out NaN); a causal chunk ends at that length
    int64_t seq_len = a.S;
    bool len_bad = false;
    if constexpr (PAGED) {
        const int32_t L = a.seq_lens[b];
        len_bad = L < 0 || (int64_t)L > a.S;
        seq_len = len_bad ? 0 : L;
    }
    const bool causal = a.causal_offset >= 0;
    const int64_t coff = PAGED ? seq_len - a.T : a.causal_offset;
    const int s_begin = split * (int)a.split_len;
    int s_end = (int)imin64(seq_len, (int64_t)s_begin + a.split_len);
    const int s_full = imax(s_end, s_begin);     // the split's keys before the causal trim
    int lim[NCB];
    bool rowok[NCB];
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
        const int rho = row0 + 16 * c + n;
        rowok[c] = rho < nrows_total;
        lim[c] = causal ? (int)imax64(imin64(coff + (rowok[c] ? rho : 0) / a.G, 0x7fffffff), -1) : 0x7fffffff;
    }
    int full_end = s_end;
    if (causal) {
        const int rlo = imin(row0, nrows_total - 1), rhi = imin(row0 + RW - 1, nrows_total - 1);
        const int64_t lo_lim = coff + rlo / a.G, hi_lim = coff + rhi / a.G;
        full_end = (int)imin64((int64_t)s_end, lo_lim + 1);
        s_end = (int)imin64((int64_t)s_end, hi_lim + 1);
    }
    s_end = imax(s_end, s_begin);
    full_end = imax(full_end, s_begin);
    bool seq_bad = false;
    DecBufs P;
    if constexpr (PAGED) {
        // the whole pool (its row count times 64 fits 32 bits: the host checks)
        const uint32_t rows = (uint32_t)(a.n_pages * a.Hkv * a.page_size);
        P.kn = __builtin_amdgcn_make_buffer_rsrc((void *)a.k_nib, (short)0, rows * 64u, kBufWord3);
        P.vn = __builtin_amdgcn_make_buffer_rsrc((void *)a.v_nib, (short)0, rows * 64u, kBufWord3);
        P.kq = __builtin_amdgcn_make_buffer_rsrc((void *)(QJL ? a.k_qjl : a.k_nib), (short)0, QJL ? rows * 8u : 0u,
                                                 kBufWord3);
        P.kr = __builtin_amdgcn_make_buffer_rsrc((void *)(QJL ? a.k_norms : (const float *)a.k_nib), (short)0,
                                                 QJL ? rows * 4u : 0u, kBufWord3);
    } else {
        const int64_t kv_base = (cache_seq(a, b, seq_bad) * a.Hkv + hk) * a.S;
        P.kn = __builtin_amdgcn_make_buffer_rsrc((void *)(a.k_nib + kv_base * 64), (short)0, s_end * 64, kBufWord3);
        P.vn = __builtin_amdgcn_make_buffer_rsrc((void *)(a.v_nib + kv_base * 64), (short)0, s_end * 64, kBufWord3);
        P.kq = __builtin_amdgcn_make_buffer_rsrc((void *)(QJL ? a.k_qjl + kv_base * 8 : a.k_nib), (short)0,
                                                 QJL ? s_end * 8 : 0, kBufWord3);
        P.kr = __builtin_amdgcn_make_buffer_rsrc((void *)(QJL ? a.k_norms + kv_base : (const float *)a.k_nib),
                                                 (short)0, QJL ? s_end * 4 : 0, kBufWord3);
    }
    DecOffsets OFS;
    OFS.k = (uint32_t)n * 64u + 16u * g;
    OFS.sg = (uint32_t)n * 8u;
    OFS.nr = 16u * g + 4u * (n & 3);      // norm of token 4g + n % 4 (of each 16-token half)
    OFS.v = 256u * g + 4u * n;
    bool page_bad = false;
    const int32_t *pt_row = PAGED ? a.page_table + b * a.max_pages : nullptr;
    // one tile's loads (paged: from the pool rows of its two halves; tiles
    // are loaded in order, so the next tile's page ids are requested here
    // and waited for only at the next call)
    int32_t pid[2] = {0, 0};
    if constexpr (PAGED) paged_page_ids(a, pt_row, s_begin, pid);
    auto load_tile = [&](TileRaw &R, int t) {
        if constexpr (PAGED) {
            uint32_t rb[2];
            paged_rows(a, pid, hk, t, s_end, page_bad, rb);
            tile_load_paged<QJL>(R, P, OFS, rb);
            paged_page_ids(a, pt_row, t + kDecTile, pid);
        } else {
            tile_load<QJL>(R, P, OFS, t);
        }
    };
    const uint32_t laneoff = (uint32_t)(lane & 31) * 8u;
    const uint32_t slane = (uint32_t)kSlutOff | laneoff;
    // lane (ne, ge) reads denominator row 4 ge: only A rows 0, 4, 8 and 12
    // need the ones (zeros elsewhere save matrix-core power)
    const uint32_t one2 = (n & 3) == 0 ? 0x3C003C00u : 0u;
    const half8_t ones = as_half8(one2, 0u, one2, 0u);
    const unsigned char *lut = smem + kLutOff;

    float4_t oacc[NCB][8], lacc[NCB];
    // running maximum (scaled, log2 domain) from -FLT_MAX: it serves as the
    // exponent offset as is (the first finite maximum replaces it)
    // m_thr: the rescale threshold m_run + 8 in raw score units, (m_run + 8)
    // / qsr (approximate: it only decides when to rescale; a rescale missed
    // by a rounding leaves exponents a hair above 8; at a zero scale it is
    // -inf until the first rescale, then +inf)
    float m_run[NCB], m_thr[NCB], rqsr[NCB], qmul[NCB];
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
#pragma unroll
        for (int k = 0; k < 8; ++k) oacc[c][k] = float4_t{0.f, 0.f, 0.f, 0.f};
        lacc[c] = float4_t{0.f, 0.f, 0.f, 0.f};
        m_run[c] = -__FLT_MAX__;
        m_thr[c] = -INFINITY;
        rqsr[c] = __builtin_amdgcn_rcpf(qsr[c]);
        qmul[c] = qsr[c];
    }
    const int zero_scale = __builtin_amdgcn_readfirstlane(a.qscale == 0.0f ? 1 : 0);
    // exponents are fma(raw, qmul, -m_run) with qmul = qsr: exact products
    // against a rounded maximum, so each carries up to half an ulp of m_run;
    // once any row's |m_run| reaches 2^13 the wave rounds each logit first
    // and qmul becomes 1 (wave-uniform; an int, so it stays a scalar)
    int round_first = 0;

    auto tile_step = [&](TileRaw &R, const int tt) {
        // wave-uniform flags as ints (scalar compares, no lane masks)
        const int full = __builtin_amdgcn_readfirstlane(tt + kDecTile <= full_end ? 1 : 0);
        // wave priority by phase: the K pass 2, the QJL term and the raw
        // maxima 1, the softmax and PV 0, so that of a SIMD's two waves the
        // one feeding the matrix cores issues first and the other's softmax
        // fills the gaps (issue order only: results do not depend on it)
        __builtin_amdgcn_s_setprio(2);
        float4_t acc[NCB][2];
#pragma unroll
        for (int c = 0; c < NCB; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u) acc[c][u] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint32_t kw[4] = {R.k[u].x, R.k[u].y, R.k[u].z, R.k[u].w};
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const uint2 e0 = *reinterpret_cast<const uint2 *>(lut + lut_addr(kw[s >> 1], laneoff, 2 * (s & 1)));
                const uint2 e1 = *reinterpret_cast<const uint2 *>(lut + lut_addr(kw[s >> 1], laneoff, 2 * (s & 1) + 1));
                const half8_t ak = pair_half8(e0, e1);
#pragma unroll
                for (int c = 0; c < NCB; ++c) {
                    acc[c][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, bk[c][s], acc[c][u], 0, 0, 0);
                    if constexpr (QLO) acc[c][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, bkl[c][s], acc[c][u], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_s_setprio(1);
        if (QJL) {
            // signs . (G q as fp16 hi + fp16 remainder), then + norm * that
            // (norm of token 4g + i: a quad broadcast, fp32); the B images
            // are read from the stage area (the opaque offset keeps the
            // reads in the loop), each once for both 16-token halves
            uint32_t qo = qimg_off;
            asm volatile("" : "+v"(qo));
            float4_t qacc[NCB][2];
#pragma unroll
            for (int c = 0; c < NCB; ++c) qacc[c][0] = qacc[c][1] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                half8_t s8[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) s8[u] = sign_halves(smem, s ? R.sg[u].y : R.sg[u].x, 8u * g, slane);
#pragma unroll
                for (int c = 0; c < NCB; ++c) {
                    const half8_t vq = __builtin_bit_cast(half8_t, *reinterpret_cast<const uint4 *>(smem + qo + ((c * 2 + s) * 2) * 1024));
                    const half8_t vl = __builtin_bit_cast(half8_t, *reinterpret_cast<const uint4 *>(smem + qo + ((c * 2 + s) * 2 + 1) * 1024));
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        qacc[c][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(s8[u], vq, qacc[c][u], 0, 0, 0);
                        qacc[c][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(s8[u], vl, qacc[c][u], 0, 0, 0);
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float nri = dpp_quad_bcast(R.nr[u], i);
#pragma unroll
                    for (int c = 0; c < NCB; ++c) acc[c][u][i] = __builtin_fmaf(nri, qacc[c][u][i], acc[c][u][i]);
                }
        }
        // raw scores of both column blocks first (the row scale qsr >= 0
        // enters each exponent's fma); one rescale branch for both, then the
        // exponentials and denominator MFMAs of both as one straight run
        half8_t pb[NCB][2];
        float sc[NCB][8];
#pragma unroll
        for (int c = 0; c < NCB; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i) sc[c][4 * u + i] = acc[c][u][i];
        if (full == 0) {
            // the tile's token, opaque here: the compares stay on this
            // (rare) path instead of being hoisted into every tile
            int tb = tt;
            asm volatile("" : "+s"(tb));
#pragma unroll
            for (int c = 0; c < NCB; ++c)
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int tn = tb + 16 * u + 4 * g + i;
                        if (tn >= s_end || tn > lim[c]) sc[c][4 * u + i] = -INFINITY;
                    }
        }
        // the scaled maximum of a row is the scale times its raw maximum
        // (rounding is monotonic and qsr >= 0; a fully masked lane gives
        // -inf, or NaN at a zero scale, and neither rescales); m_run is the
        // same in the four lane groups of a row, so each lane tests its own
        // raw maximum against the raw threshold and the cross-group maximum
        // is formed only when a lane may rescale
        float mr[NCB];
        bool may = false;
#pragma unroll
        for (int c = 0; c < NCB; ++c) {
            mr[c] = vmax3(vmax3(sc[c][0], sc[c][1], sc[c][2]), vmax3(sc[c][3], sc[c][4], sc[c][5]), vmax2(sc[c][6], sc[c][7]));
            may = may || mr[c] > m_thr[c];
        }
        __builtin_amdgcn_s_setprio(0);
        if (__builtin_amdgcn_ballot_w64(may)) {
#pragma unroll
            for (int c = 0; c < NCB; ++c) {
                if (__builtin_amdgcn_ballot_w64(mr[c] > m_thr[c])) {
                    const float mt = max_over_groups(mr[c] * qsr[c]);
                    const bool need = mt > m_run[c] + 8.0f;
                    const float f = need ? __builtin_amdgcn_exp2f(m_run[c] - mt) : 1.0f;
                    // the old maximum's last use before the new one is formed
                    // (one register for both: no copy on the path without a rescale)
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int k = 0; k < 8; ++k) oacc[c][k] *= f;
                    lacc[c] *= f;
                    m_run[c] = need ? mt : m_run[c];
                    m_thr[c] = (m_run[c] + 8.0f) * rqsr[c];
                    round_first |= __builtin_amdgcn_ballot_w64(fabsf(m_run[c]) >= 8192.0f && m_run[c] > -__FLT_MAX__) ? 1 : 0;
                }
            }
#pragma unroll
            for (int k = 0; k < NCB; ++k) qmul[k] = round_first ? 1.0f : qmul[k];
        }
        if (round_first) {
#pragma unroll
            for (int c = 0; c < NCB; ++c)
#pragma unroll
                for (int k = 0; k < 8; ++k) sc[c][k] = sc[c][k] * qsr[c];
        }
        float ex[NCB][8];
#pragma unroll
        for (int c = 0; c < NCB; ++c)
#pragma unroll
            for (int k = 0; k < 8; ++k) ex[c][k] = __builtin_fmaf(sc[c][k], qmul[c], -m_run[c]);
        // -inf x qmul is -inf unless the scale is 0: then the masked keys'
        // exponents are set again (their tokens tested as above)
        int zr = zero_scale & (full ^ 1);
        asm volatile("" : "+s"(zr));
        if (zr != 0) {
            int tb = tt;
            asm volatile("" : "+s"(tb));
#pragma unroll
            for (int c = 0; c < NCB; ++c)
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int tn = tb + 16 * u + 4 * g + i;
                        if (tn >= s_end || tn > lim[c]) ex[c][4 * u + i] = -INFINITY;
                    }
        }
#pragma unroll
        for (int c = 0; c < NCB; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const uint32_t p01 = cvt_pk_h2(__builtin_amdgcn_exp2f(ex[c][4 * u]), __builtin_amdgcn_exp2f(ex[c][4 * u + 1]));
                const uint32_t p23 = cvt_pk_h2(__builtin_amdgcn_exp2f(ex[c][4 * u + 2]), __builtin_amdgcn_exp2f(ex[c][4 * u + 3]));
                pb[c][u] = as_half8(p01, p01, p23, p23);
                lacc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pb[c][u], lacc[c], 0, 0, 0);
            }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            uint32_t ev[2], od[2];
#pragma unroll
            for (int pr = 0; pr < 2; ++pr) {
                const uint32_t va = R.v[4 * u + 2 * pr], vb = R.v[4 * u + 2 * pr + 1];
                ev[pr] = ((vb << 4) & 0xF0F0F0F0u) | (va & 0x0F0F0F0Fu);
                od[pr] = (vb & 0xF0F0F0F0u) | ((va >> 4) & 0x0F0F0F0Fu);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint2 e0 = *reinterpret_cast<const uint2 *>(lut + lut_addr(ev[0], laneoff, j));
                const uint2 e1 = *reinterpret_cast<const uint2 *>(lut + lut_addr(ev[1], laneoff, j));
                const half8_t ae = pair_half8(e0, e1);
                const uint2 f0 = *reinterpret_cast<const uint2 *>(lut + lut_addr(od[0], laneoff, j));
                const uint2 f1 = *reinterpret_cast<const uint2 *>(lut + lut_addr(od[1], laneoff, j));
                const half8_t ao = pair_half8(f0, f1);
#pragma unroll
                for (int c = 0; c < NCB; ++c) {
                    oacc[c][2 * j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ae, pb[c][u], oacc[c][2 * j], 0, 0, 0);
                    oacc[c][2 * j + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ao, pb[c][u], oacc[c][2 * j + 1], 0, 0, 0);
                }
            }
        }
    };

    // every key tile, in order, with the decode kernel's unconditional ring
    constexpr int stride = kDecTile;
    TileRaw ring[PF];
#pragma unroll
    for (int p = 0; p < PF - 1; ++p) load_tile(ring[p], s_begin + p * stride);
    int tt0 = s_begin;
    for (; tt0 + (PF - 1) * stride < s_end; tt0 += PF * stride) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            __builtin_amdgcn_sched_barrier(0);
            load_tile(ring[(p + PF - 1) % PF], tt0 + (p + PF - 1) * stride);
            __builtin_amdgcn_sched_barrier(0);
            tile_step(ring[p], tt0 + p * stride);
        }
    }
#pragma unroll
    for (int p = 0; p < PF - 1; ++p)
        if (tt0 + p * stride < s_end) tile_step(ring[p], tt0 + p * stride);
    if constexpr (PAGED) {
        // pages of the split past this wave's causal window were never
        // loaded: a page id outside the pool there still makes every row of
        // the sequence NaN (as the decode kernel, which reads every page)
        if (causal && s_full > s_end) {
            const int p_hi = ((s_full - 1) >> a.page_shift) + 1;      // <= max_pages: seq_len <= S
            bool bad = false;
            for (int p = (s_end >> a.page_shift) + lane; p < p_hi; p += 64)
                bad = bad || (uint32_t)pt_row[p] >= (uint32_t)a.n_pages;
            page_bad = page_bad || __builtin_amdgcn_ballot_w64(bad) != 0;
        }
    }

    // ── rows out (or split partials) ──────────────────────────────────────
    const int64_t unit = (b * a.Hkv + hk) * a.n_rchunks + rc;
    // lane coordinates recomputed here (opaque), so no address of this step
    // is kept live across the main loop
    int le = lane;
    asm volatile("" : "+v"(le));
    const int ne = le & 15, ge = le >> 4;
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
        const int rho = row0 + 16 * c + ne;
        if (!rowok[c]) continue;
        const float l = (seq_bad || page_bad || len_bad) ? __builtin_nanf("") : lacc[c][0];
        if (a.splits == 1) {
            const int t = rho / a.G, hq = hk * a.G + (rho - t * a.G);
            float *o = a.out + ((b * a.Hq + hq) * a.T + t) * D;
#pragma unroll
            for (int k = 0; k < 8; ++k)
#pragma unroll
                for (int i = 0; i < 4; ++i) o[8 * (4 * ge + i) + k] = oacc[c][k][i] / l;
        } else {
            const int rr = wave * RW + 16 * c + ne;
            float *wp = a.ws + ((unit * a.splits + split) * a.rows + rr) * (D + 2);
#pragma unroll
            for (int k = 0; k < 8; ++k)
#pragma unroll
                for (int i = 0; i < 4; ++i) wp[8 * (4 * ge + i) + k] = oacc[c][k][i];
            if (ge == 0) { wp[D] = m_run[c]; wp[D + 1] = l; }
        }
    }
}

// ── chunked-prefill kernel at head_dim 32 ────────────────────────────────
//
// The D = 128 prefill scheme for the generalized codec at D = 32 (16-byte
// nibble rows, 2 sign bytes, QJL_DIM 16).  Each wave owns 16 * NCB query rows
// and streams every key tile of its split; per 32-token tile, 16-token half u
// and column block:
//   K pass  2 MFMAs: lane (n, g) holds dword g of token n (dims 8g .. 8g + 7),
//           two cache bytes per k-step through the byte LUT (fp16 hi +
//           remainder slots); B = the exact fp16 q row (per-row 2^k scale)
//   QJL     1 MFMA: A = the token's 16 sign bits as +-1 halves, twice (k-slots
//           0-15 and 16-31), B = sqrt(2/pi)/D (G q) as fp16 hi in slots 0-15
//           and its fp16 remainder in 16-31; the fp32 norm (quad broadcast)
//           scales it into the score
//   PV      2 MFMAs (even and odd dims): lane (n, g) loads byte n of tokens
//           4g .. 4g + 3 and forms pair bytes (two tokens' nibbles at dim 2n
//           or 2n + 1), whose LUT entries are MFMA-ready (hi, lo) pairs
// Online softmax in the exp2 domain with P in fp16, summed by an MFMA
// against ones, as in the other kernels.
#ifndef OMNI_P32_WAVES
#define OMNI_P32_WAVES 8
#endif
constexpr int kP32Waves = OMNI_P32_WAVES;
constexpr int kP32CbOff = kSlutOff + kSlutBytes;                          // 16 x (fp16 hi | remainder << 16)
constexpr int kP32StageOff = kP32CbOff + 64;                               // per wave: q rows fp16 (+ remainder plane), then G q f32
constexpr int kP32StageBytes = 64 * 32 * 2;
constexpr int kP32Ncb = 4;                                                 // column blocks per wave for 16-bit q (f32 q: 2)
constexpr int kP32QsrOff = kP32StageOff + kP32Waves * kP32StageBytes;     // per wave: 64 f32 score scales
constexpr int kP32LdsBytes = kP32QsrOff + kP32Waves * 64 * 4;

// One 32-token tile at D = 32 as loaded.
struct TileRaw32 {
    uint32_t k[2];     // K dword g of token 16u + (lane % 16)
    uint32_t sg[2];    // the 2 sign bytes of the same token
    float4_t nr[2];    // norms of tokens 16u + 4g .. 16u + 4g + 3
    uint32_t v[8];     // V byte (lane % 16) of token 16(i / 4) + 4g + i % 4 (low byte)
};

template <bool QJL>
__device__ __forceinline__ void tile_load32(TileRaw32 &R, const DecBufs &P, int n, int g, int t0) {
    const uint32_t t = (uint32_t)t0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const uint32_t tk = t + 16u * u + (uint32_t)n;
        R.k[u] = __builtin_amdgcn_raw_buffer_load_b32(P.kn, tk * 16u + 4u * g, 0, 0);
        if (QJL) {
            R.sg[u] = __builtin_amdgcn_raw_buffer_load_b16(P.kq, tk * 2u, 0, 0);
            const u32x4_t nv = __builtin_amdgcn_raw_buffer_load_b128(P.kr, (t + 16u * u + 4u * g) * 4u, 0, 0);
            R.nr[u] = float4_t{__uint_as_float(nv.x), __uint_as_float(nv.y), __uint_as_float(nv.z), __uint_as_float(nv.w)};
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
        R.v[i] = __builtin_amdgcn_raw_buffer_load_b8(P.vn, (t + 16u * (i / 4) + 4u * g + (i % 4)) * 16u + (uint32_t)n, 0, 0);
}

// Normalized 32-point WHT of the element (lane % 32) of each half-wave's
// row (_wht_torch order, fp32; an fma with +-1 rounds as the add/subtract).
__device__ __forceinline__ float wht32_lane(float x, int lane) {
    x = __builtin_fmaf((lane & 1) ? -1.0f : 1.0f, x, xor_partner<1>(x, lane));
    x = __builtin_fmaf((lane & 2) ? -1.0f : 1.0f, x, xor_partner<2>(x, lane));
    x = __builtin_fmaf((lane & 4) ? -1.0f : 1.0f, x, xor_partner<4>(x, lane));
    x = __builtin_fmaf((lane & 8) ? -1.0f : 1.0f, x, xor_partner<8>(x, lane));
    x = __builtin_fmaf((lane & 16) ? -1.0f : 1.0f, x, xor_partner<16>(x, lane));
    return x;
}

template <bool QJL, int NCB, bool QLO>
__global__ __launch_bounds__(64 * kP32Waves) void attn_prefill32_kernel(AttnArgs a) {
    constexpr int D = 32, QD = 16, RW = 16 * NCB;       // rows per wave
    static_assert(RW * D * 2 * (QLO ? 2 : 1) <= kP32StageBytes && RW * QD * 4 <= kP32StageBytes,
                  "q rows (and the f32 remainder plane), then G q, fit the wave's stage area");
    __shared__ __attribute__((aligned(16))) unsigned char smem[kP32LdsBytes];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int split = blockIdx.x, hk = blockIdx.y;
    const int64_t bz = blockIdx.z;
    const int64_t b = bz / a.n_rchunks;
    const int rc = (int)(bz % a.n_rchunks);
    const int nrows_total = (int)(a.T * a.G);
    const int row0 = rc * a.rows + wave * RW;
    uint16_t *stage = reinterpret_cast<uint16_t *>(smem + kP32StageOff + wave * kP32StageBytes);
    float *qsr_l = reinterpret_cast<float *>(smem + kP32QsrOff) + wave * 64;

    // ── codebook pairs and the sign table ───────────────────────────────
    {
        const __amdgpu_buffer_rsrc_t CB = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(a.codebooks + (a.per_head ? hk * 16 : 0)), (short)0, 16 * 4, kBufWord3);
        const float c = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(CB, 4u * (lane & 15), 0, 0));
        const uint16_t h = f32_to_f16_rne(c);
        *reinterpret_cast<uint32_t *>(smem + kP32CbOff + 4 * (lane & 15)) =
            (uint32_t)h | ((uint32_t)f32_to_f16_rne(c - f16_to_f32(h)) << 16);
    }
    if (tid < 512) sign_table_store(smem, tid);

    // ── this wave's query rows, two per pass (half-waves): (sign flip,)
    //    WHT, round; per-row power-of-2 scale into fp16 range; fp16 stage.
    //    The score scale's sign goes into the staged rows (exact), so every
    //    row's score scale qsr is >= 0 and the exponent takes it in an fma ──
    {
        const int e = lane & 31, half = lane >> 5;
        const bool flip = a.rotate_q && a.sign_flip && a.sign_flip[e] < 0;
        const float ssign = a.qscale < 0.0f ? -1.0f : 1.0f;
        for (int rp = 0; rp < RW; rp += 2) {
            const int rr = rp + half;
            const int rho = row0 + rr;
            const bool ok = rho < nrows_total;
            const int rcl = ok ? rho : nrows_total - 1;
            const int t = rcl / a.G, hq = hk * a.G + (rcl - t * a.G);
            float x = load_as_f32(a.q, a.q_dtype, ((b * a.Hq + hq) * a.T + t) * D + e);
            x = flip ? -x : x;
            if (a.rotate_q) x = round_to_dtype(wht32_lane(x, lane) * a.wht_scale, a.q_dtype);
            if (!ok) x = 0.0f;
            float m = fabsf(x);
#pragma unroll
            for (int sh = 16; sh >= 1; sh >>= 1) m = fmaxf(m, __shfl_xor(m, sh));
            int ex = 0;
            if (m > 0.0f && m < INFINITY) frexpf(m, &ex);
            const float sr = ldexpf(1.0f, 15 - imax(ex, -100));
            const float xs = ssign * x * sr;
            const uint16_t x16 = f32_to_f16_rne(xs);
            stage[rr * D + e] = x16;
            if constexpr (QLO) stage[RW * D + rr * D + e] = f32_to_f16_rne(xs - f16_to_f32(x16));
            // kept >= FLT_MIN (a positive scale that underflows here leaves
            // every score as good as 0 either way): the softmax below
            // relies on -inf x qsr = -inf.  A zero scale runs elsewhere.
            const float q0 = fabsf(a.qscale) / sr;
            if (e == 0) qsr_l[rr] = q0 < __FLT_MIN__ ? __FLT_MIN__ : q0;
        }
    }
    __syncthreads();

    // ── byte LUT (after the codebook pairs are visible): entry e, 16-byte
    //    chunk k (two of its 32 copies) per item ───────────────────────────
    {
        const uint32_t *cbh = reinterpret_cast<const uint32_t *>(smem + kP32CbOff);
        for (int it = tid; it < 256 * 16; it += 64 * kP32Waves) {
            const int e = it >> 4;
            const uint32_t w0 = cbh[e & 15], w1 = cbh[e >> 4];
            const uint32_t hp = __builtin_amdgcn_perm(w1, w0, 0x05040100u);
            const uint32_t lp = __builtin_amdgcn_perm(w1, w0, 0x07060302u);
            *reinterpret_cast<uint4 *>(smem + kLutOff + e * 256 + (it & 15) * 16) = make_uint4(hp, lp, hp, lp);
        }
    }

    // ── per-lane B operands: q (exact fp16) for the scores ───────────────
    half8_t bk[NCB][2], bkl[QLO ? NCB : 1][2], bgq[NCB];
    float qsr[NCB];
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const uint2 w = *reinterpret_cast<const uint2 *>(stage + (16 * c + n) * D + 8 * g + 4 * s);
            bk[c][s] = as_half8(w.x, w.x, w.y, w.y);
            if constexpr (QLO) {
                const uint2 wl = *reinterpret_cast<const uint2 *>(stage + RW * D + (16 * c + n) * D + 8 * g + 4 * s);
                bkl[c][s] = as_half8(wl.x, wl.x, wl.y, wl.y);
            }
        }
        qsr[c] = qsr_l[16 * c + n];
    }
    __syncthreads();   // sign table visible
    // G q (staged scale) on MFMA: A = q rows (k = the 32 dims), B = G rows
    // expanded by the sign table; lane (n, g) gets row 16 c + 4 g + i,
    // projection n
    float4_t gacc[NCB];
#pragma unroll
    for (int c = 0; c < NCB; ++c) gacc[c] = float4_t{0.f, 0.f, 0.f, 0.f};
    if (QJL) {
        const uint32_t gw = a.g_bits[(int64_t)hk * QD + n];
        const half8_t bg = sign_halves(smem, gw, 8u * g, (uint32_t)kSlutOff | ((uint32_t)(lane & 31) * 8u));
#pragma unroll
        for (int c = 0; c < NCB; ++c) {
            const uint4 qv = *reinterpret_cast<const uint4 *>(stage + (16 * c + n) * D + 8 * g);
            gacc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(qv.x, qv.y, qv.z, qv.w), bg, gacc[c], 0, 0, 0);
            if constexpr (QLO) {
                const uint4 lv = *reinterpret_cast<const uint4 *>(stage + RW * D + (16 * c + n) * D + 8 * g);
                gacc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(lv.x, lv.y, lv.z, lv.w), bg, gacc[c], 0, 0, 0);
            }
        }
    }
    // through the stage area (q is no longer read) into the QJL B layout:
    // column n = row 16 c + n; k-slots 8g .. 8g + 7 = projections 8 (g % 2)
    // .. + 7 as fp16 hi (g < 2) or fp16 remainder (g >= 2)
    float *gqs = reinterpret_cast<float *>(stage);      // [RW][16]
#pragma unroll
    for (int c = 0; c < NCB; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) gqs[(16 * c + 4 * g + i) * QD + n] = gacc[c][i];
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
        const float *row = gqs + (16 * c + n) * QD + 8 * (g & 1);
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float g0 = row[2 * j] * a.alpha_c, g1 = row[2 * j + 1] * a.alpha_c;
            w[j] = !QJL ? 0u : (g < 2 ? pack_h2(g0, g1) : pack_h2(g0 - (float)(_Float16)g0, g1 - (float)(_Float16)g1));
        }
        bgq[c] = as_half8(w[0], w[1], w[2], w[3]);
    }
    __syncthreads();   // byte LUT complete

    // ── key range of this wave: causal limits of its rows ─────────────────
    const int s_begin = split * (int)a.split_len;
    int s_end = (int)imin64(a.S, (int64_t)s_begin + a.split_len);
    int lim[NCB];
    bool rowok[NCB];
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
        const int rho = row0 + 16 * c + n;
        rowok[c] = rho < nrows_total;
        lim[c] = (a.causal_offset >= 0) ? (int)imin64(a.causal_offset + (rowok[c] ? rho : 0) / a.G, 0x7fffffff)
                                        : 0x7fffffff;
    }
    int full_end = s_end;
    if (a.causal_offset >= 0) {
        const int rlo = imin(row0, nrows_total - 1), rhi = imin(row0 + RW - 1, nrows_total - 1);
        const int64_t lo_lim = a.causal_offset + rlo / a.G, hi_lim = a.causal_offset + rhi / a.G;
        full_end = (int)imin64((int64_t)s_end, lo_lim + 1);
        s_end = (int)imin64((int64_t)s_end, hi_lim + 1);
    }
    bool seq_bad;
    const int64_t kv_base = (cache_seq(a, b, seq_bad) * a.Hkv + hk) * a.S;
    DecBufs P;
    P.kn = __builtin_amdgcn_make_buffer_rsrc((void *)(a.k_nib + kv_base * 16), (short)0, s_end * 16, kBufWord3);
    P.vn = __builtin_amdgcn_make_buffer_rsrc((void *)(a.v_nib + kv_base * 16), (short)0, s_end * 16, kBufWord3);
    P.kq = __builtin_amdgcn_make_buffer_rsrc((void *)(QJL ? a.k_qjl + kv_base * 2 : a.k_nib), (short)0,
                                             QJL ? s_end * 2 : 0, kBufWord3);
    P.kr = __builtin_amdgcn_make_buffer_rsrc((void *)(QJL ? a.k_norms + kv_base : (const float *)a.k_nib), (short)0,
                                             QJL ? s_end * 4 : 0, kBufWord3);
    const uint32_t laneoff = (uint32_t)(lane & 31) * 8u;
    const uint32_t slane = (uint32_t)kSlutOff | laneoff;
    // lane (ne, ge) reads denominator row 4 ge: only A rows 0, 4, 8 and 12
    // need the ones (zeros elsewhere save matrix-core power); every k slot
    // of the P operand is a distinct token, so those rows are all ones
    const uint32_t one2 = (n & 3) == 0 ? 0x3C003C00u : 0u;
    const half8_t ones = as_half8(one2, one2, one2, one2);
    const unsigned char *lut = smem + kLutOff;

    float4_t oacc[NCB][2], lacc[NCB];
    // running maximum (scaled, log2 domain) from -FLT_MAX: it serves as the
    // exponent offset as is (the first finite maximum replaces it)
    // m_thr: the rescale threshold m_run + 8 in raw score units, (m_run +
    // 8) / qsr (approximate: it only decides when to rescale; a rescale
    // missed by a rounding leaves exponents a hair above 8)
    float m_run[NCB], m_thr[NCB], rqsr[NCB];
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
        oacc[c][0] = oacc[c][1] = float4_t{0.f, 0.f, 0.f, 0.f};
        lacc[c] = float4_t{0.f, 0.f, 0.f, 0.f};
        m_run[c] = -__FLT_MAX__;
        m_thr[c] = -INFINITY;
        rqsr[c] = __builtin_amdgcn_rcpf(qsr[c]);
    }
    // exponents are fma(raw, qmul, -m_run) with qmul = qsr: exact products
    // against a rounded maximum, so each carries up to half an ulp of m_run;
    // once any row's |m_run| reaches 2^13 the wave rounds each logit first
    // and qmul becomes 1 (wave-uniform; an int, so it stays a scalar)
    int round_first = 0;
    float qmul[NCB];
#pragma unroll
    for (int c = 0; c < NCB; ++c) qmul[c] = qsr[c];

    auto tile_step = [&](TileRaw32 &R, const int tt) {
        // wave-uniform as an int (a scalar compare per use, no lane mask)
        const int full = __builtin_amdgcn_readfirstlane(tt + kDecTile <= full_end ? 1 : 0);
        // wave priority by phase: the K pass and QJL term 2, the PV operand
        // reads and the raw maxima 1, the softmax and PV 0 (as in the
        // head_dim-128 kernel)
        __builtin_amdgcn_s_setprio(2);
        float4_t acc[NCB][2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            // K pass: bytes 2s, 2s + 1 of the lane's dword are dims 8g + 4s .. + 3
            const half8_t ak0 = pair_half8(*reinterpret_cast<const uint2 *>(lut + lut_addr(R.k[u], laneoff, 0)),
                                           *reinterpret_cast<const uint2 *>(lut + lut_addr(R.k[u], laneoff, 1)));
            const half8_t ak1 = pair_half8(*reinterpret_cast<const uint2 *>(lut + lut_addr(R.k[u], laneoff, 2)),
                                           *reinterpret_cast<const uint2 *>(lut + lut_addr(R.k[u], laneoff, 3)));
#pragma unroll
            for (int c = 0; c < NCB; ++c) {
                float4_t ac = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak0, bk[c][0], float4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                if constexpr (QLO) ac = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak0, bkl[c][0], ac, 0, 0, 0);
                ac = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak1, bk[c][1], ac, 0, 0, 0);
                if constexpr (QLO) ac = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak1, bkl[c][1], ac, 0, 0, 0);
                acc[c][u] = ac;
            }
            if (QJL) {
                // k-slots 8g .. 8g + 7 take sign byte g % 2 (projections 8 (g % 2) ..)
                const half8_t s8 = sign_halves(smem, R.sg[u], 8u * (uint32_t)(g & 1), slane);
#pragma unroll
                for (int c = 0; c < NCB; ++c) {
                    const float4_t qacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(s8, bgq[c], float4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[c][u][i] = __builtin_fmaf(R.nr[u][i], qacc[i], acc[c][u][i]);
                }
            }
        }
        // PV operands, read before the softmax so that each column block's
        // PV MFMAs can issue as soon as its probabilities exist (interleaved
        // with the other blocks' exponentials below): pair bytes of tokens (4g, 4g + 1) and (4g + 2, 4g + 3) of each
        // half at dims 2n (low nibbles) and 2n + 1 (high nibbles); a LUT
        // entry is (fp16 hi pair, remainder pair), read as two dwords so the
        // hi and remainder planes are two A operands over the same P
        __builtin_amdgcn_s_setprio(1);
        uint32_t ph[2][4], pl[2][4];      // [dim parity][pair byte]
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint32_t b0 = R.v[4 * u], b1 = R.v[4 * u + 1], b2 = R.v[4 * u + 2], b3 = R.v[4 * u + 3];
            // (only byte 0 of pe reaches the LUT address: the bits above it
            // may hold b1's high nibble, so one bit-field insert forms it)
            const uint32_t pe[2] = {(b0 & 0x0Fu) | ((b1 << 4) & ~0x0Fu), (b2 & 0x0Fu) | ((b3 << 4) & ~0x0Fu)};
            const uint32_t po[2] = {(b0 >> 4) | (b1 & 0xF0u), (b2 >> 4) | (b3 & 0xF0u)};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t ae = lut_addr(pe[h], laneoff, 0), ao = lut_addr(po[h], laneoff, 0);
                // the remainder dwords read as volatile, so that they are not
                // merged with the hi dwords into paired reads (whose results
                // would need register copies to form the two A operands)
                ph[0][2 * u + h] = *reinterpret_cast<const uint32_t *>(lut + ae);
                pl[0][2 * u + h] = *(const volatile __attribute__((address_space(3))) uint32_t *)(lut + ae + 4);
                ph[1][2 * u + h] = *reinterpret_cast<const uint32_t *>(lut + ao);
                pl[1][2 * u + h] = *(const volatile __attribute__((address_space(3))) uint32_t *)(lut + ao + 4);
            }
        }
        half8_t ahv[2], alv[2];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            ahv[p] = as_half8(ph[p][0], ph[p][1], ph[p][2], ph[p][3]);
            alv[p] = as_half8(pl[p][0], pl[p][1], pl[p][2], pl[p][3]);
        }
        // P of the lane's eight tokens (4g .. 4g + 3 of each half) as one
        // B operand: k slot 8g + j holds token 16 (j / 4) + 4g + j % 4.
        // Raw scores of every column block first (the row scale qsr >= 0
        // enters each exponent's fma); one rescale branch for all blocks,
        // then the exponentials and MFMAs of all blocks as one straight run.
        float sc[NCB][8];
#pragma unroll
        for (int c = 0; c < NCB; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int i = 0; i < 4; ++i) sc[c][4 * u + i] = acc[c][u][i];
        if (full == 0) {
            // the tile's token, opaque here: the compares stay on this
            // (rare) path instead of being hoisted into every tile
            int tb = tt;
            asm volatile("" : "+s"(tb));
#pragma unroll
            for (int c = 0; c < NCB; ++c)
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int tn = tb + 16 * u + 4 * g + i;
                        if (tn >= s_end || tn > lim[c]) sc[c][4 * u + i] = -INFINITY;
                    }
        }
        // the scaled maximum of a row is the scale times its raw maximum
        // (rounding is monotonic and qsr > 0, so a fully masked lane gives
        // -inf); m_run is the same in the four lane groups of a row, so each
        // lane tests its own raw maximum against the raw threshold and the
        // cross-group maximum is formed only when a lane may rescale
        float mr[NCB];
        bool may = false;
#pragma unroll
        for (int c = 0; c < NCB; ++c) {
            mr[c] = vmax3(vmax3(sc[c][0], sc[c][1], sc[c][2]), vmax3(sc[c][3], sc[c][4], sc[c][5]), vmax2(sc[c][6], sc[c][7]));
            may = may || mr[c] > m_thr[c];
        }
        __builtin_amdgcn_s_setprio(0);
        if (__builtin_amdgcn_ballot_w64(may)) {
#pragma unroll
            for (int c = 0; c < NCB; ++c) {
                if (__builtin_amdgcn_ballot_w64(mr[c] > m_thr[c])) {
                    const float mt = max_over_groups(mr[c] * qsr[c]);
                    const bool need = mt > m_run[c] + 8.0f;
                    const float f = need ? __builtin_amdgcn_exp2f(m_run[c] - mt) : 1.0f;
                    // the old maximum's last use before the new one is formed
                    // (one register for both: no copy on the path without a rescale)
                    __builtin_amdgcn_sched_barrier(0);
                    oacc[c][0] *= f;
                    oacc[c][1] *= f;
                    lacc[c] *= f;
                    m_run[c] = need ? mt : m_run[c];
                    m_thr[c] = (m_run[c] + 8.0f) * rqsr[c];
                    round_first |= __builtin_amdgcn_ballot_w64(fabsf(m_run[c]) >= 8192.0f && m_run[c] > -__FLT_MAX__) ? 1 : 0;
                }
            }
#pragma unroll
            for (int k = 0; k < NCB; ++k) qmul[k] = round_first ? 1.0f : qmul[k];
        }
        if (round_first) {
#pragma unroll
            for (int c = 0; c < NCB; ++c)
#pragma unroll
                for (int k = 0; k < 8; ++k) sc[c][k] = sc[c][k] * qsr[c];
        }
#pragma unroll
        for (int c = 0; c < NCB; ++c) {
            // a masked score (-inf) gives -inf here: qmul > 0
            const float nm = -m_run[c];
            float ex[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) ex[k] = __builtin_fmaf(sc[c][k], qmul[c], nm);
            uint32_t pw[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                pw[j] = cvt_pk_h2(__builtin_amdgcn_exp2f(ex[2 * j]), __builtin_amdgcn_exp2f(ex[2 * j + 1]));
            const half8_t pb = as_half8(pw[0], pw[1], pw[2], pw[3]);
            lacc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pb, lacc[c], 0, 0, 0);
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                oacc[c][p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahv[p], pb, oacc[c][p], 0, 0, 0);
                oacc[c][p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alv[p], pb, oacc[c][p], 0, 0, 0);
            }
        }
    };

    // every key tile, in order, with a two-slot ring of unconditional loads
    // (past the split end they read 0 and touch no memory)
    constexpr int stride = kDecTile;
    TileRaw32 ring[2];
    tile_load32<QJL>(ring[0], P, n, g, s_begin);
    int tt0 = s_begin;
    for (; tt0 + stride < s_end; tt0 += 2 * stride) {
        __builtin_amdgcn_sched_barrier(0);
        tile_load32<QJL>(ring[1], P, n, g, tt0 + stride);
        __builtin_amdgcn_sched_barrier(0);
        tile_step(ring[0], tt0);
        __builtin_amdgcn_sched_barrier(0);
        tile_load32<QJL>(ring[0], P, n, g, tt0 + 2 * stride);
        __builtin_amdgcn_sched_barrier(0);
        tile_step(ring[1], tt0 + stride);
    }
    if (tt0 < s_end) tile_step(ring[0], tt0);

    // ── rows out (or split partials): oacc[c][p][i] is dim 8g + 2i + p ────
    const int64_t unit = (b * a.Hkv + hk) * a.n_rchunks + rc;
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
        const int rho = row0 + 16 * c + n;
        if (!rowok[c]) continue;
        const float l = seq_bad ? __builtin_nanf("") : lacc[c][0];
        float *o;
        if (a.splits == 1) {
            const int t = rho / a.G, hq = hk * a.G + (rho - t * a.G);
            o = a.out + ((b * a.Hq + hq) * a.T + t) * D;
        } else {
            const int rr = wave * RW + 16 * c + n;
            o = a.ws + ((unit * a.splits + split) * a.rows + rr) * (D + 2);
            if (g == 0) { o[D] = m_run[c]; o[D + 1] = l; }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float e0 = oacc[c][0][i], e1 = oacc[c][1][i];
            if (a.splits == 1) {
                o[8 * g + 2 * i] = e0 / l;
                o[8 * g + 2 * i + 1] = e1 / l;
            } else {
                o[8 * g + 2 * i] = e0;
                o[8 * g + 2 * i + 1] = e1;
            }
        }
    }
}

// ── launch planning ─────────────────────────────────────────────────────

struct Plan {
    bool dec128;       // D == 128: decode kernel with 8 query rows per block
    bool prefill;      // D == 128 with many rows per kv head: prefill kernel
    bool prefill32;    // D == 32 with many rows per kv head: head_dim-32 prefill kernel
    int rows, n_rchunks, splits, nw, ncopy;
    int spb;           // decode kernel: sequences sharing a block's 8 row slots
    int64_t split_len;
    size_t lds, ws_bytes;
};

static int64_t clamp64(int64_t v, int64_t lo, int64_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

// `zero_scale`: a score scale of exactly 0.  The decode and head_dim-32
// prefill kernels need a positive score factor (a masked key's -inf must
// stay -inf through it); a zero scale, where an infinite score gives NaN
// (inf x 0, as the reference forms scale x score), runs the head_dim-128
// prefill kernel or the generic one instead, which keep the factor 0.
static Plan make_plan(int64_t B, int Hq, int Hkv, int64_t T, int64_t S, int D, bool q32, bool paged = false,
                      bool zero_scale = false) {
    Plan p;
    const int G = Hq / Hkv;
    const int cus = device_cus();
    p.prefill = (D == 128) && (T * G > kPrefillMinRows || zero_scale);
    p.prefill32 = (D == 32) && T * G > kPrefillMinRows && !zero_scale;
    p.dec128 = (D == 128) && !p.prefill;
    p.rows = p.prefill ? kPreWaves * 16 * (q32 ? 1 : kPreNcb)
                       : (p.prefill32 ? kP32Waves * 16 * (q32 ? 2 : kP32Ncb) : (p.dec128 ? kDecRows : kRows));
    p.n_rchunks = (int)((T * G + p.rows - 1) / p.rows);
    // Short decode steps of many sequences (more (sequence, kv head) pairs
    // than CUs, at most 4 query rows each): two sequences share a block's 8
    // row slots, halving the blocks (and the per-block prologues) without
    // idling any slot.
    p.spb = (p.dec128 && T * G <= kDecRows / 2 && B >= 2 && B * (int64_t)Hkv > cus) ? 2 : 1;
    const int64_t units = ((B + p.spb - 1) / p.spb) * (int64_t)Hkv * p.n_rchunks;
    if (p.prefill || p.prefill32) {
        const int64_t tiles = (S + kDecTile - 1) / kDecTile;
        int64_t splits = clamp64((cus + units - 1) / (units > 0 ? units : 1), 1, (tiles / 16) > 1 ? tiles / 16 : 1);
        const int64_t tps = (tiles + splits - 1) / splits;
        p.splits = (int)splits;
        p.split_len = tps * kDecTile;
        p.nw = p.prefill ? kPreWaves : kP32Waves;
        p.ncopy = 32;
        p.lds = p.prefill ? kPreLdsBytes : kP32LdsBytes;
    } else if (p.dec128) {
        const int64_t tiles = (S + kDecTile - 1) / kDecTile;
        int64_t splits = clamp64((cus + units - 1) / (units > 0 ? units : 1), 1, (tiles / 16) > 1 ? tiles / 16 : 1);
        if (p.spb > 1) splits = 1;
        // paged: splits short enough for every half's pool row to be staged
        if (paged && p.spb == 1) {
            const int64_t cap = kDecPtMax / 2;
            if (tiles > splits * cap) splits = (tiles + cap - 1) / cap;
        }
        const int64_t tps = (tiles + splits - 1) / splits;
        p.splits = (int)splits;
        p.split_len = tps * kDecTile;
        p.nw = kDecWaves;
        p.ncopy = 32;
        p.lds = kDecLdsBytes;
    } else {
        const int64_t tiles = (S + kTile - 1) / kTile;
        int64_t splits = clamp64((2 * (int64_t)cus + units - 1) / (units > 0 ? units : 1), 1,
                                 tiles / (2 * kMaxWaves) > 1 ? tiles / (2 * kMaxWaves) : 1);
        const int64_t tps = (tiles + splits - 1) / splits;
        p.splits = (int)splits;
        p.split_len = tps * kTile;
        p.nw = (int)clamp64((tps + 1) / 2, 1, kMaxWaves);
        p.ncopy = tps >= 64 ? 16 : (tps >= 8 ? 4 : 1);
        p.lds = D == 128 ? Lds<128>::total(p.ncopy, p.nw) : Lds<32>::total(p.ncopy, p.nw);
    }
    p.ws_bytes = p.splits > 1 ? (size_t)units * p.splits * p.rows * (D + 2) * sizeof(float) : 0;
    return p;
}

// Split-K workspace of a contiguous-cache call, whatever its score scale
// (a zero scale may take another kernel).
static size_t plan_ws_bytes(int64_t B, int Hq, int Hkv, int64_t T, int64_t S, int D, bool q32) {
    const size_t a = make_plan(B, Hq, Hkv, T, S, D, q32).ws_bytes;
    const size_t b = make_plan(B, Hq, Hkv, T, S, D, q32, false, true).ws_bytes;
    return a > b ? a : b;
}

}  // namespace omni

using namespace omni;

extern "C" size_t omni_attn_workspace_size(int64_t B, int Hq, int Hkv, int64_t T, int64_t S, int head_dim) {
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || T <= 0 || S <= 0 || Hq % Hkv || !head_dim_ok(head_dim)) return 0;
    // the prefill plan differs for f32 queries: size for either
    const size_t a = plan_ws_bytes(B, Hq, Hkv, T, S, head_dim, false);
    const size_t b = plan_ws_bytes(B, Hq, Hkv, T, S, head_dim, true);
    return a > b ? a : b;
}

// Per-user LoRA on q (omni_attn_lora).
struct LoraSpec {
    const void *x, *A, *Bw;
    int w_dtype;
    const int32_t *idx;
    int hidden, rank, n_loras;
    float alpha;
};

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

template <bool QJL, int SPB, bool PAGED = false>
static void launch_decode128(bool lora, dim3 grid, dim3 block, hipStream_t s, const AttnArgs &a) {
    if (lora)
        hipLaunchKernelGGL((attn_decode128_kernel<QJL, kDecPrefetch, SPB, true, PAGED>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((attn_decode128_kernel<QJL, kDecPrefetch, SPB, false, PAGED>), grid, block, 0, s, a);
}

// Paged cache of omni_attn_paged.
struct PagedSpec {
    const int32_t *page_table, *seq_lens;
    int64_t max_pages, n_pages;
    int page_size, page_shift;
};

static int attn_run(const void *q, int q_dtype, const uint8_t *k_nib, const uint8_t *k_qjl,
                    const float *k_norms, const uint8_t *v_nib, const float *codebooks,
                    int per_head_codebook, const uint32_t *g_bits, int64_t B, int Hq, int Hkv,
                    int64_t T, int64_t S, int head_dim, float scale, int with_qjl,
                    int64_t causal_offset, int rotate_q, const int8_t *sign_flip, float *out,
                    void *workspace, size_t workspace_bytes, void *stream, const LoraSpec *lora,
                    const int64_t *seq_index, int64_t n_seqs, const PagedSpec *paged = nullptr) {
    OMNI_CHECK_ARG(dtype_ok(q_dtype), "omni_attn: bad q dtype %d", q_dtype);
    OMNI_CHECK_ARG(head_dim_ok(head_dim), "omni_attn: head_dim must be 128 or 32, got %d", head_dim);
    OMNI_CHECK_ARG(B >= 0 && Hq > 0 && Hkv > 0 && T >= 0 && S >= 0, "omni_attn: bad shape");
    OMNI_CHECK_ARG(Hq % Hkv == 0, "omni_attn: n_heads (%d) must be divisible by n_kv_heads (%d)", Hq, Hkv);
    if (B == 0 || T == 0) return OMNI_OK;
    OMNI_CHECK_ARG(S > 0, "omni_attn: empty KV cache (S = 0) has no softmax");
    OMNI_CHECK_ARG(q && k_nib && v_nib && codebooks && out, "omni_attn: NULL pointer");
    OMNI_CHECK_ARG(!with_qjl || (k_qjl && k_norms && g_bits), "omni_attn: NULL QJL pointer");
    OMNI_CHECK_ARG(isfinite(scale), "omni_attn: scale must be finite");
    OMNI_CHECK_ARG(S < (int64_t(1) << 25), "omni_attn: S must be < 2^25 tokens per sequence");
    OMNI_CHECK_ARG(T * (Hq / Hkv) < (int64_t(1) << 31), "omni_attn: T * (n_heads / n_kv_heads) must be < 2^31");
    OMNI_CHECK_ARG(seq_index == nullptr || n_seqs >= 1, "omni_attn: a cache index needs a pool of >= 1 sequences");
    Plan p = make_plan(B, Hq, Hkv, T, S, head_dim, q_dtype == OMNI_F32, paged != nullptr, scale == 0.0f);
    OMNI_CHECK_ARG(paged == nullptr || head_dim == 128, "omni_attn_paged: needs head_dim 128");
    OMNI_CHECK_ARG(Hkv <= 65535 && ((B + p.spb - 1) / p.spb) * p.n_rchunks <= 65535 && p.splits <= 2147483647,
                   "omni_attn: grid too large (batch x row chunks must be <= 65535)");
    // LoRA: fused into the D=128 decode prologue; other kernels read q_eff
    // written by the gather-apply kernel into the workspace tail
    const bool lora_fused = lora != nullptr && p.dec128 && lora->w_dtype != OMNI_F32 &&
                            lora->rank <= kLoraFusedMaxRank && lora->rank % 8 == 0 &&
                            lora->hidden <= kLoraFusedMaxHidden && ((uintptr_t)lora->Bw % 16) == 0;
    const size_t q_bytes = (size_t)B * Hq * T * head_dim * (q_dtype == OMNI_F32 ? 4 : 2);
    const size_t ws_need = (lora != nullptr && !lora_fused) ? align256(p.ws_bytes) + q_bytes : p.ws_bytes;
    if (ws_need > 0 && (workspace == nullptr || workspace_bytes < ws_need)) {
        set_error("omni_attn: workspace of %zu bytes required, %zu given", ws_need, workspace_bytes);
        return OMNI_EWORKSPACE;
    }
    if (lora != nullptr && !lora_fused) {
        void *q_eff = reinterpret_cast<char *>(workspace) + align256(p.ws_bytes);
        const int rc = omni_lora_apply(q, q_dtype, lora->x, lora->A, lora->Bw, lora->w_dtype, lora->idx, B, Hq, T,
                                       head_dim, lora->hidden, lora->rank, lora->n_loras, lora->alpha, q_eff, stream);
        if (rc != OMNI_OK) return rc;
        q = q_eff;
    }
    AttnArgs a;
    a.lora_x = a.lora_a = a.lora_b = nullptr;
    a.lora_idx = nullptr;
    a.lora_w_dtype = -1; a.lora_hidden = a.lora_rank = a.lora_n = 0; a.lora_alpha = 0.0f;
    if (lora_fused) {
        a.lora_x = lora->x; a.lora_a = lora->A; a.lora_b = lora->Bw; a.lora_idx = lora->idx;
        a.lora_w_dtype = lora->w_dtype; a.lora_hidden = lora->hidden; a.lora_rank = lora->rank;
        a.lora_n = lora->n_loras; a.lora_alpha = lora->alpha;
    }
    a.q = q; a.k_nib = k_nib; a.k_qjl = k_qjl; a.k_norms = k_norms; a.v_nib = v_nib;
    a.codebooks = codebooks; a.g_bits = g_bits; a.sign_flip = sign_flip; a.out = out;
    a.ws = reinterpret_cast<float *>(workspace);
    a.T = T; a.S = S; a.split_len = p.split_len; a.causal_offset = causal_offset;
    a.q_dtype = q_dtype; a.per_head = per_head_codebook; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv;
    a.n_rchunks = p.n_rchunks; a.splits = p.splits; a.ncopy = p.ncopy; a.rows = p.rows;
    a.with_qjl = with_qjl; a.rotate_q = rotate_q;
    a.g_magic = ((uint64_t)1 << 32) / (uint64_t)a.G + 1;
    a.rch_magic = ((uint64_t)1 << 32) / (uint64_t)p.n_rchunks + 1;
    const double log2e = 1.4426950408889634;
    a.qscale = (float)((double)scale * log2e);
    a.alpha_c = (float)(sqrt(2.0 / M_PI) / (double)head_dim);
    a.wht_scale = inv_sqrt_dim_f32(head_dim);
    a.B = B;
    a.seq_index = seq_index;
    a.n_seqs = seq_index ? n_seqs : B;
    a.spb = p.spb;
    a.page_table = paged ? paged->page_table : nullptr;
    a.seq_lens = paged ? paged->seq_lens : nullptr;
    a.max_pages = paged ? paged->max_pages : 0;
    a.n_pages = paged ? paged->n_pages : 0;
    a.page_size = paged ? paged->page_size : 0;
    a.page_shift = paged ? paged->page_shift : 0;
    dim3 grid((unsigned)p.splits, (unsigned)Hkv, (unsigned)(((B + p.spb - 1) / p.spb) * p.n_rchunks));
    dim3 block(64 * p.nw);
    if (p.prefill && paged) {
        const bool qlo = q_dtype == OMNI_F32;
        hipStream_t st = as_stream(stream);
        if (with_qjl) {
            if (qlo) hipLaunchKernelGGL((attn_prefill128_kernel<true, 1, 2, true, true>), grid, block, 0, st, a);
            else hipLaunchKernelGGL((attn_prefill128_kernel<true, kPreNcb, 2, false, true>), grid, block, 0, st, a);
        } else {
            if (qlo) hipLaunchKernelGGL((attn_prefill128_kernel<false, 1, 2, true, true>), grid, block, 0, st, a);
            else hipLaunchKernelGGL((attn_prefill128_kernel<false, kPreNcb, 2, false, true>), grid, block, 0, st, a);
        }
    } else if (p.prefill) {
        const bool qlo = q_dtype == OMNI_F32;
        hipStream_t st = as_stream(stream);
        if (with_qjl) {
            if (qlo) hipLaunchKernelGGL((attn_prefill128_kernel<true, 1, 2, true, false>), grid, block, 0, st, a);
            else hipLaunchKernelGGL((attn_prefill128_kernel<true, kPreNcb, 2, false, false>), grid, block, 0, st, a);
        } else {
            if (qlo) hipLaunchKernelGGL((attn_prefill128_kernel<false, 1, 2, true, false>), grid, block, 0, st, a);
            else hipLaunchKernelGGL((attn_prefill128_kernel<false, kPreNcb, 2, false, false>), grid, block, 0, st, a);
        }
    } else if (p.prefill32) {
        const bool qlo = q_dtype == OMNI_F32;
        hipStream_t st = as_stream(stream);
        if (with_qjl) {
            if (qlo) hipLaunchKernelGGL((attn_prefill32_kernel<true, 2, true>), grid, block, 0, st, a);
            else hipLaunchKernelGGL((attn_prefill32_kernel<true, kP32Ncb, false>), grid, block, 0, st, a);
        } else {
            if (qlo) hipLaunchKernelGGL((attn_prefill32_kernel<false, 2, true>), grid, block, 0, st, a);
            else hipLaunchKernelGGL((attn_prefill32_kernel<false, kP32Ncb, false>), grid, block, 0, st, a);
        }
    } else if (p.dec128 && paged) {
        hipStream_t st = as_stream(stream);
        if (with_qjl && p.spb > 1) launch_decode128<true, 2, true>(lora_fused, grid, block, st, a);
        else if (with_qjl) launch_decode128<true, 1, true>(lora_fused, grid, block, st, a);
        else if (p.spb > 1) launch_decode128<false, 2, true>(lora_fused, grid, block, st, a);
        else launch_decode128<false, 1, true>(lora_fused, grid, block, st, a);
    } else if (p.dec128) {
        hipStream_t st = as_stream(stream);
        if (with_qjl && p.spb > 1) launch_decode128<true, 2>(lora_fused, grid, block, st, a);
        else if (with_qjl) launch_decode128<true, 1>(lora_fused, grid, block, st, a);
        else if (p.spb > 1) launch_decode128<false, 2>(lora_fused, grid, block, st, a);
        else launch_decode128<false, 1>(lora_fused, grid, block, st, a);
    } else {
        hipLaunchKernelGGL(attn_kernel<32>, grid, block, p.lds, as_stream(stream), a);
    }
    OMNI_CHECK_LAUNCH("omni_attn");
    if (p.splits > 1) {
        dim3 g2(1, (unsigned)Hkv, (unsigned)(B * p.n_rchunks));
        if (head_dim == 128)
            hipLaunchKernelGGL(attn_combine_kernel<128>, g2, dim3(256), 0, as_stream(stream), a);
        else
            hipLaunchKernelGGL(attn_combine_kernel<32>, g2, dim3(256), 0, as_stream(stream), a);
        OMNI_CHECK_LAUNCH("omni_attn combine");
    }
    return OMNI_OK;
}

extern "C" int omni_attn(const void *q, int q_dtype, const uint8_t *k_nib, const uint8_t *k_qjl,
                         const float *k_norms, const uint8_t *v_nib, const float *codebooks,
                         int per_head_codebook, const uint32_t *g_bits, int64_t B, int Hq, int Hkv,
                         int64_t T, int64_t S, int head_dim, float scale, int with_qjl,
                         int64_t causal_offset, int rotate_q, const int8_t *sign_flip, float *out,
                         void *workspace, size_t workspace_bytes, void *stream) {
    return attn_run(q, q_dtype, k_nib, k_qjl, k_norms, v_nib, codebooks, per_head_codebook, g_bits, B, Hq, Hkv, T,
                    S, head_dim, scale, with_qjl, causal_offset, rotate_q, sign_flip, out, workspace,
                    workspace_bytes, stream, nullptr, nullptr, 0);
}

extern "C" size_t omni_attn_lora_workspace_size(int64_t B, int Hq, int Hkv, int64_t T, int64_t S, int head_dim,
                                                int q_dtype) {
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || T <= 0 || S <= 0 || Hq % Hkv || !head_dim_ok(head_dim) || !dtype_ok(q_dtype))
        return 0;
    const size_t ws = plan_ws_bytes(B, Hq, Hkv, T, S, head_dim, q_dtype == OMNI_F32);
    // room for the gather-apply fallback's q_eff: the adapter's rank and
    // hidden size, which decide between it and the fused path, are not
    // arguments here
    return align256(ws) + (size_t)B * Hq * T * head_dim * (q_dtype == OMNI_F32 ? 4 : 2);
}

extern "C" int omni_attn_lora(const void *q, int q_dtype, const void *x, const void *lora_a, const void *lora_b,
                              int w_dtype, const int32_t *lora_idx, int hidden, int rank, int n_loras,
                              float lora_alpha, const uint8_t *k_nib, const uint8_t *k_qjl, const float *k_norms,
                              const uint8_t *v_nib, const float *codebooks, int per_head_codebook,
                              const uint32_t *g_bits, int64_t B, int Hq, int Hkv, int64_t T, int64_t S,
                              int head_dim, float scale, int with_qjl, int64_t causal_offset, int rotate_q,
                              const int8_t *sign_flip, float *out, void *workspace, size_t workspace_bytes,
                              void *stream) {
    OMNI_CHECK_ARG(dtype_ok(w_dtype), "omni_attn_lora: bad LoRA dtype %d", w_dtype);
    OMNI_CHECK_ARG(hidden > 0 && rank >= 1 && rank <= 64 && n_loras >= 1,
                   "omni_attn_lora: need hidden > 0, 1 <= rank <= 64, n_loras >= 1");
    if (B > 0 && T > 0) OMNI_CHECK_ARG(x && lora_a && lora_b && lora_idx, "omni_attn_lora: NULL LoRA pointer");
    OMNI_CHECK_ARG((int64_t)Hq * head_dim <= (int64_t)1 << 30, "omni_attn_lora: n_heads * head_dim too large");
    const LoraSpec spec{x, lora_a, lora_b, w_dtype, lora_idx, hidden, rank, n_loras, lora_alpha};
    return attn_run(q, q_dtype, k_nib, k_qjl, k_norms, v_nib, codebooks, per_head_codebook, g_bits, B, Hq, Hkv, T,
                    S, head_dim, scale, with_qjl, causal_offset, rotate_q, sign_flip, out, workspace,
                    workspace_bytes, stream, &spec, nullptr, 0);
}

extern "C" int omni_attn_serve(const void *q, int q_dtype, const int64_t *cache_index, int64_t n_cache_seqs,
                               const void *x, const void *lora_a, const void *lora_b, int w_dtype,
                               const int32_t *lora_idx, int hidden, int rank, int n_loras, float lora_alpha,
                               const uint8_t *k_nib, const uint8_t *k_qjl, const float *k_norms,
                               const uint8_t *v_nib, const float *codebooks, int per_head_codebook,
                               const uint32_t *g_bits, int64_t B, int Hq, int Hkv, int64_t T, int64_t S,
                               int head_dim, float scale, int with_qjl, int64_t causal_offset, int rotate_q,
                               const int8_t *sign_flip, float *out, void *workspace, size_t workspace_bytes,
                               void *stream) {
    if (B > 0 && T > 0) OMNI_CHECK_ARG(cache_index != nullptr, "omni_attn_serve: NULL cache index");
    OMNI_CHECK_ARG(n_cache_seqs >= 1, "omni_attn_serve: n_cache_seqs must be >= 1");
    if (lora_a == nullptr)
        return attn_run(q, q_dtype, k_nib, k_qjl, k_norms, v_nib, codebooks, per_head_codebook, g_bits, B, Hq, Hkv,
                        T, S, head_dim, scale, with_qjl, causal_offset, rotate_q, sign_flip, out, workspace,
                        workspace_bytes, stream, nullptr, cache_index, n_cache_seqs);
    OMNI_CHECK_ARG(dtype_ok(w_dtype), "omni_attn_serve: bad LoRA dtype %d", w_dtype);
    OMNI_CHECK_ARG(hidden > 0 && rank >= 1 && rank <= 64 && n_loras >= 1,
                   "omni_attn_serve: need hidden > 0, 1 <= rank <= 64, n_loras >= 1");
    if (B > 0 && T > 0) OMNI_CHECK_ARG(x && lora_b && lora_idx, "omni_attn_serve: NULL LoRA pointer");
    OMNI_CHECK_ARG((int64_t)Hq * head_dim <= (int64_t)1 << 30, "omni_attn_serve: n_heads * head_dim too large");
    const LoraSpec spec{x, lora_a, lora_b, w_dtype, lora_idx, hidden, rank, n_loras, lora_alpha};
    return attn_run(q, q_dtype, k_nib, k_qjl, k_norms, v_nib, codebooks, per_head_codebook, g_bits, B, Hq, Hkv, T,
                    S, head_dim, scale, with_qjl, causal_offset, rotate_q, sign_flip, out, workspace,
                    workspace_bytes, stream, &spec, cache_index, n_cache_seqs);
}

// ── paged cache ──────────────────────────────────────────────────────────
//
// Pool arrays are shaped like a contiguous cache with the batch axis as
// pages: nibbles (n_pages, Hkv, page_size, 64), signs (.., 8), norms
// (n_pages, Hkv, page_size), V (.., 64).  Sequence b holds seq_lens[b] tokens
// in pages page_table[b * max_pages + j], j < ceil(len / page_size); entries
// past that are never read for keys.  D = 128; up to 32 query rows per kv
// head (T * Hq / Hkv) run the decode kernel, more the chunked-prefill kernel.
// causal != 0 aligns query token t with key len - T + t.

static bool paged_args_ok(int64_t B, int Hkv, int64_t n_pages, int page_size, int64_t max_pages, int &shift) {
    shift = 0;
    while (shift < 11 && (1 << shift) < page_size) ++shift;
    if (page_size < 16 || page_size > 1024 || (1 << shift) != page_size) {
        set_error("omni_attn_paged: page_size must be a power of two in [16, 1024], got %d", page_size);
        return false;
    }
    if (n_pages < 1 || max_pages < 1 || B < 0) {
        set_error("omni_attn_paged: need n_pages >= 1, max_pages >= 1");
        return false;
    }
    // every byte offset into the pool fits 32 bits
    if (Hkv < 1 || n_pages * Hkv * (int64_t)page_size >= (int64_t(1) << 26)) {
        set_error("omni_attn_paged: pool too large (n_pages * n_kv_heads * page_size must be < 2^26 tokens)");
        return false;
    }
    if (max_pages * (int64_t)page_size >= (int64_t(1) << 25)) {
        set_error("omni_attn_paged: max_pages * page_size must be < 2^25 tokens per sequence");
        return false;
    }
    return true;
}

extern "C" size_t omni_attn_paged_workspace_size(int64_t B, int Hq, int Hkv, int64_t T, int64_t max_pages,
                                                 int page_size, int q_dtype) {
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || T <= 0 || max_pages <= 0 || page_size <= 0 || Hq % Hkv || !dtype_ok(q_dtype))
        return 0;
    // either plan (a zero score scale runs another kernel), plus room for
    // the gather-apply LoRA fallback's q_eff
    const int64_t S = max_pages * (int64_t)page_size;
    const size_t a = make_plan(B, Hq, Hkv, T, S, 128, q_dtype == OMNI_F32, true).ws_bytes;
    const size_t z = make_plan(B, Hq, Hkv, T, S, 128, q_dtype == OMNI_F32, true, true).ws_bytes;
    return align256(a > z ? a : z) + (size_t)B * Hq * T * 128 * (q_dtype == OMNI_F32 ? 4 : 2);
}

extern "C" int omni_attn_paged(const void *q, int q_dtype, const uint8_t *k_nib, const uint8_t *k_qjl,
                               const float *k_norms, const uint8_t *v_nib, int64_t n_pages, int page_size,
                               const int32_t *page_table, int64_t max_pages, const int32_t *seq_lens,
                               const void *x, const void *lora_a, const void *lora_b, int w_dtype,
                               const int32_t *lora_idx, int hidden, int rank, int n_loras, float lora_alpha,
                               const float *codebooks, int per_head_codebook, const uint32_t *g_bits, int64_t B,
                               int Hq, int Hkv, int64_t T, int head_dim, float scale, int with_qjl, int causal,
                               int rotate_q, const int8_t *sign_flip, float *out, void *workspace,
                               size_t workspace_bytes, void *stream) {
    int shift = 0;
    if (!paged_args_ok(B, Hkv, n_pages, page_size, max_pages, shift)) return OMNI_EINVAL;
    if (B > 0 && T > 0) OMNI_CHECK_ARG(page_table && seq_lens, "omni_attn_paged: NULL page table or lengths");
    const PagedSpec pg{page_table, seq_lens, max_pages, n_pages, page_size, shift};
    const int64_t S = max_pages * (int64_t)page_size;
    const int64_t coff = causal ? 0 : -1;
    if (lora_a == nullptr)
        return attn_run(q, q_dtype, k_nib, k_qjl, k_norms, v_nib, codebooks, per_head_codebook, g_bits, B, Hq, Hkv,
                        T, S, head_dim, scale, with_qjl, coff, rotate_q, sign_flip, out, workspace, workspace_bytes,
                        stream, nullptr, nullptr, 0, &pg);
    OMNI_CHECK_ARG(dtype_ok(w_dtype), "omni_attn_paged: bad LoRA dtype %d", w_dtype);
    OMNI_CHECK_ARG(hidden > 0 && rank >= 1 && rank <= 64 && n_loras >= 1,
                   "omni_attn_paged: need hidden > 0, 1 <= rank <= 64, n_loras >= 1");
    if (B > 0 && T > 0) OMNI_CHECK_ARG(x && lora_b && lora_idx, "omni_attn_paged: NULL LoRA pointer");
    OMNI_CHECK_ARG((int64_t)Hq * head_dim <= (int64_t)1 << 30, "omni_attn_paged: n_heads * head_dim too large");
    const LoraSpec spec{x, lora_a, lora_b, w_dtype, lora_idx, hidden, rank, n_loras, lora_alpha};
    return attn_run(q, q_dtype, k_nib, k_qjl, k_norms, v_nib, codebooks, per_head_codebook, g_bits, B, Hq, Hkv, T,
                    S, head_dim, scale, with_qjl, coff, rotate_q, sign_flip, out, workspace, workspace_bytes, stream,
                    &spec, nullptr, 0, &pg);
}

// ── allocation-free variant of omni_attn ─────────────────────────────────
//
// For callers that cannot allocate device memory (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc): the split-K
// partials live in this file-scope array instead of a caller workspace.
// Each device holds its own copy for the life of the process.  In host code
// `scratch` names a host-side stand-in, never the device memory: its device
// address is looked up once per device (hipGetSymbolAddress, with that
// device current) and only that address is handed to kernels.  Every call on
// a device shares the array, so calls that overlap on one device (several
// streams, several host threads) race; nothing in it needs to start at zero
// (each launch writes every partial it reads back).
namespace omni {

constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kScratchMaxDevices = 64;
static std::atomic<void *> g_scratch_addr[kScratchMaxDevices];
static std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (looked up on the first
// call per device).
static int scratch_address(void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchMaxDevices) {
        set_error("omni_attn_noalloc: no usable current device (%d)", dev);
        return OMNI_ERUNTIME;
    }
    void *p = g_scratch_addr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_addr[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || p == nullptr) {
                set_error("omni_attn_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                          hipGetErrorString(e));
                return OMNI_ERUNTIME;
            }
            g_scratch_addr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return OMNI_OK;
}

}  // namespace omni

extern "C" size_t omni_attn_noalloc_scratch_bytes(void) { return omni::kScratchBytes; }

extern "C" int omni_attn_noalloc(const void *q, int q_dtype, const uint8_t *k_nib, const uint8_t *k_qjl,
                                 const float *k_norms, const uint8_t *v_nib, const float *codebooks,
                                 int per_head_codebook, const uint32_t *g_bits, int64_t B, int Hq, int Hkv,
                                 int64_t T, int64_t S, int head_dim, float scale, int with_qjl,
                                 int64_t causal_offset, int rotate_q, const int8_t *sign_flip, float *out,
                                 void *stream) {
    const size_t need = omni_attn_workspace_size(B, Hq, Hkv, T, S, head_dim);
    if (need > kScratchBytes) {
        set_error("omni_attn_noalloc: this launch needs %zu bytes of split-K scratch, more than the %zu-byte "
                  "static array; call omni_attn with a workspace instead", need, kScratchBytes);
        return OMNI_EWORKSPACE;
    }
    void *ws = nullptr;
    const int rc = scratch_address(&ws);
    if (rc != OMNI_OK) return rc;
    return attn_run(q, q_dtype, k_nib, k_qjl, k_norms, v_nib, codebooks, per_head_codebook, g_bits, B, Hq, Hkv, T,
                    S, head_dim, scale, with_qjl, causal_offset, rotate_q, sign_flip, out, ws, kScratchBytes,
                    stream, nullptr, nullptr, 0);
}

// ── prepared calls (omni_attn_plan_*) ──────────────────────────────────
//
// The static arguments of one attention configuration, stored once, so a
// serving loop's per-step call passes only what changes (q, the LoRA inputs,
// the cache index, the stream).  A run is exactly the omni_attn /
// omni_attn_lora / omni_attn_serve call the stored arguments describe.
struct omni_attn_plan {
    int q_dtype;
    int64_t n_cache_seqs;                 // > 0: a pool indexed per query (omni_attn_serve)
    const void *lora_a, *lora_b;          // lora_a NULL: no adapters
    int w_dtype, hidden, rank, n_loras;
    float lora_alpha;
    const uint8_t *k_nib, *k_qjl;
    const float *k_norms;
    const uint8_t *v_nib;
    const float *codebooks;
    int per_head_codebook;
    const uint32_t *g_bits;
    int64_t B;
    int Hq, Hkv;
    int64_t T, S;
    int head_dim;
    float scale;
    int with_qjl;
    int64_t causal_offset;
    int rotate_q;
    const int8_t *sign_flip;
    float *out;
    void *workspace;
    size_t workspace_bytes;
};

extern "C" int omni_attn_plan_create(int q_dtype, int64_t n_cache_seqs, const void *lora_a, const void *lora_b,
                                     int w_dtype, int hidden, int rank, int n_loras, float lora_alpha,
                                     const uint8_t *k_nib, const uint8_t *k_qjl, const float *k_norms,
                                     const uint8_t *v_nib, const float *codebooks, int per_head_codebook,
                                     const uint32_t *g_bits, int64_t B, int Hq, int Hkv, int64_t T, int64_t S,
                                     int head_dim, float scale, int with_qjl, int64_t causal_offset, int rotate_q,
                                     const int8_t *sign_flip, float *out, void *workspace, size_t workspace_bytes,
                                     omni_attn_plan **plan) {
    OMNI_CHECK_ARG(plan != nullptr, "omni_attn_plan_create: NULL plan pointer");
    *plan = nullptr;
    OMNI_CHECK_ARG(dtype_ok(q_dtype), "omni_attn_plan_create: bad q dtype %d", q_dtype);
    OMNI_CHECK_ARG(head_dim_ok(head_dim), "omni_attn_plan_create: head_dim must be 128 or 32, got %d", head_dim);
    OMNI_CHECK_ARG(n_cache_seqs >= 0, "omni_attn_plan_create: n_cache_seqs must be >= 0");
    OMNI_CHECK_ARG(lora_a == nullptr || dtype_ok(w_dtype), "omni_attn_plan_create: bad LoRA dtype %d", w_dtype);
    omni_attn_plan *p = new (std::nothrow) omni_attn_plan;
    if (p == nullptr) {
        set_error("omni_attn_plan_create: out of host memory");
        return OMNI_ERUNTIME;
    }
    *p = omni_attn_plan{q_dtype, n_cache_seqs, lora_a, lora_b, w_dtype, hidden, rank, n_loras, lora_alpha,
                        k_nib, k_qjl, k_norms, v_nib, codebooks, per_head_codebook, g_bits, B, Hq, Hkv, T, S,
                        head_dim, scale, with_qjl, causal_offset, rotate_q, sign_flip, out, workspace,
                        workspace_bytes};
    *plan = p;
    return OMNI_OK;
}

extern "C" int omni_attn_plan_run(const omni_attn_plan *p, const void *q, const void *x, const int32_t *lora_idx,
                                  const int64_t *cache_index, void *stream) {
    OMNI_CHECK_ARG(p != nullptr, "omni_attn_plan_run: NULL plan");
    if (p->n_cache_seqs > 0)
        return omni_attn_serve(q, p->q_dtype, cache_index, p->n_cache_seqs, x, p->lora_a, p->lora_b, p->w_dtype,
                               lora_idx, p->hidden, p->rank, p->n_loras, p->lora_alpha, p->k_nib, p->k_qjl,
                               p->k_norms, p->v_nib, p->codebooks, p->per_head_codebook, p->g_bits, p->B, p->Hq,
                               p->Hkv, p->T, p->S, p->head_dim, p->scale, p->with_qjl, p->causal_offset,
                               p->rotate_q, p->sign_flip, p->out, p->workspace, p->workspace_bytes, stream);
    OMNI_CHECK_ARG(cache_index == nullptr, "omni_attn_plan_run: a cache index needs a plan over a pool");
    if (p->lora_a != nullptr)
        return omni_attn_lora(q, p->q_dtype, x, p->lora_a, p->lora_b, p->w_dtype, lora_idx, p->hidden, p->rank,
                              p->n_loras, p->lora_alpha, p->k_nib, p->k_qjl, p->k_norms, p->v_nib, p->codebooks,
                              p->per_head_codebook, p->g_bits, p->B, p->Hq, p->Hkv, p->T, p->S, p->head_dim,
                              p->scale, p->with_qjl, p->causal_offset, p->rotate_q, p->sign_flip, p->out,
                              p->workspace, p->workspace_bytes, stream);
    OMNI_CHECK_ARG(x == nullptr && lora_idx == nullptr, "omni_attn_plan_run: LoRA inputs need a plan with a bank");
    return omni_attn(q, p->q_dtype, p->k_nib, p->k_qjl, p->k_norms, p->v_nib, p->codebooks, p->per_head_codebook,
                     p->g_bits, p->B, p->Hq, p->Hkv, p->T, p->S, p->head_dim, p->scale, p->with_qjl,
                     p->causal_offset, p->rotate_q, p->sign_flip, p->out, p->workspace, p->workspace_bytes, stream);
}

extern "C" void omni_attn_plan_destroy(omni_attn_plan *p) { delete p; }

// ── prepared paged call (PagedKVAttention) ───────────────────────────────
//
// The arguments of omni_attn_paged that stay fixed across a serving loop (the
// pool, its geometry, the code tables, the LoRA bank, the shapes, output and
// workspace) stored once, so each call passes the query, the page table,
// the lengths, the LoRA inputs and the stream.  The plan holds pointers only:
// the pool and every buffer it names must outlive it.
struct omni_attn_paged_plan {
    int q_dtype;
    const uint8_t *k_nib, *k_qjl;
    const float *k_norms;
    const uint8_t *v_nib;
    int64_t n_pages;
    int page_size;
    int64_t max_pages;
    const void *lora_a, *lora_b;          // lora_a NULL: no adapters
    int w_dtype, hidden, rank, n_loras;
    float lora_alpha;
    const float *codebooks;
    int per_head_codebook;
    const uint32_t *g_bits;
    int64_t B;
    int Hq, Hkv;
    int64_t T;
    int head_dim;
    float scale;
    int with_qjl, causal, rotate_q;
    const int8_t *sign_flip;
    float *out;
    void *workspace;
    size_t workspace_bytes;
};

extern "C" int omni_attn_paged_plan_create(int q_dtype, const uint8_t *k_nib, const uint8_t *k_qjl,
                                           const float *k_norms, const uint8_t *v_nib, int64_t n_pages,
                                           int page_size, int64_t max_pages, const void *lora_a, const void *lora_b,
                                           int w_dtype, int hidden, int rank, int n_loras, float lora_alpha,
                                           const float *codebooks, int per_head_codebook, const uint32_t *g_bits,
                                           int64_t B, int Hq, int Hkv, int64_t T, int head_dim, float scale,
                                           int with_qjl, int causal, int rotate_q, const int8_t *sign_flip,
                                           float *out, void *workspace, size_t workspace_bytes,
                                           omni_attn_paged_plan **plan) {
    OMNI_CHECK_ARG(plan != nullptr, "omni_attn_paged_plan_create: NULL plan pointer");
    *plan = nullptr;
    OMNI_CHECK_ARG(dtype_ok(q_dtype), "omni_attn_paged_plan_create: bad q dtype %d", q_dtype);
    OMNI_CHECK_ARG(head_dim_ok(head_dim), "omni_attn_paged_plan_create: head_dim must be 128 or 32, got %d", head_dim);
    int shift = 0;
    if (!paged_args_ok(B, Hkv, n_pages, page_size, max_pages, shift)) return OMNI_EINVAL;
    OMNI_CHECK_ARG(lora_a == nullptr || dtype_ok(w_dtype), "omni_attn_paged_plan_create: bad LoRA dtype %d", w_dtype);
    omni_attn_paged_plan *p = new (std::nothrow) omni_attn_paged_plan;
    if (p == nullptr) {
        set_error("omni_attn_paged_plan_create: out of host memory");
        return OMNI_ERUNTIME;
    }
    *p = omni_attn_paged_plan{q_dtype, k_nib, k_qjl, k_norms, v_nib, n_pages, page_size, max_pages, lora_a, lora_b,
                              w_dtype, hidden, rank, n_loras, lora_alpha, codebooks, per_head_codebook, g_bits, B,
                              Hq, Hkv, T, head_dim, scale, with_qjl, causal, rotate_q, sign_flip, out, workspace,
                              workspace_bytes};
    *plan = p;
    return OMNI_OK;
}

extern "C" int omni_attn_paged_plan_run(const omni_attn_paged_plan *p, const void *q, const int32_t *page_table,
                                        const int32_t *seq_lens, const void *x, const int32_t *lora_idx,
                                        void *stream) {
    OMNI_CHECK_ARG(p != nullptr, "omni_attn_paged_plan_run: NULL plan");
    if (p->lora_a == nullptr)
        OMNI_CHECK_ARG(x == nullptr && lora_idx == nullptr, "omni_attn_paged_plan_run: LoRA inputs need a plan with a bank");
    return omni_attn_paged(q, p->q_dtype, p->k_nib, p->k_qjl, p->k_norms, p->v_nib, p->n_pages, p->page_size,
                           page_table, p->max_pages, seq_lens, p->lora_a ? x : nullptr, p->lora_a, p->lora_b,
                           p->w_dtype, p->lora_a ? lora_idx : nullptr, p->hidden, p->rank, p->n_loras,
                           p->lora_alpha, p->codebooks, p->per_head_codebook, p->g_bits, p->B, p->Hq, p->Hkv, p->T,
                           p->head_dim, p->scale, p->with_qjl, p->causal, p->rotate_q, p->sign_flip, p->out,
                           p->workspace, p->workspace_bytes, stream);
}

extern "C" void omni_attn_paged_plan_destroy(omni_attn_paged_plan *p) { delete p; }
