/*
 * omnistack_amd.h — C ABI of the MI355X (gfx950) KV-cache codec and
 * compressed-KV attention library (libomnistack_amd.so).
 *
 * Plain pointers and sizes only: every tensor argument is a device pointer
 * to a contiguous, row-major buffer that the caller allocated; `stream` is a
 * hipStream_t passed as void*.  No entry point synchronizes the host; all
 * device work is enqueued on `stream`.  Return value: OMNI_OK (0) or a
 * negative OMNI_E* code; omni_last_error() returns a message for the
 * calling thread.  The Python wrapper maps OMNI_EINVAL -> ValueError,
 * OMNI_EINDEX -> IndexError, everything else -> RuntimeError.
 *
 * Layouts are the reference's (deepsheth3/Omnistack-RS, Python/torch):
 *   rotated K/V         (B, H, T, D)        f32 | f16 | bf16
 *   nibbles             (B, H, T, D/2)      u8   byte m = c[2m] | c[2m+1] << 4
 *   qjl signs           (B, H, T, D/16)     u8   bit b of byte m = [P_{8m+b} >= 0]
 *   norms               (B, H, T)           f32  ||x - cb[code]||_2
 *   codebooks           (H, 16) or (16,)    f32
 *   QJL G bits          (H, D/2, D/32)      u32  bit j%32 of word j/32 of row i
 *                                                = [G_h[i][j] == +1]
 * D is 128 (the reference's only head_dim) or 32 (generalized codec:
 * QJL_DIM = D/2, alpha = sqrt(2/pi) * ||e|| / D).
 */
#ifndef OMNISTACK_AMD_H
#define OMNISTACK_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum omni_dtype { OMNI_F32 = 0, OMNI_F16 = 1, OMNI_BF16 = 2 };

enum omni_status {
    OMNI_OK = 0,
    OMNI_EINVAL = -1,     /* bad shape / argument   -> ValueError   */
    OMNI_EINDEX = -2,     /* index out of range     -> IndexError   */
    OMNI_ERUNTIME = -3,   /* HIP launch / runtime   -> RuntimeError */
    OMNI_EWORKSPACE = -4  /* workspace too small    -> RuntimeError */
};

/* Message for the last non-OK return on the calling thread. */
const char *omni_last_error(void);

/* Library ABI version (bumped on any signature change). */
int omni_abi_version(void);

/*
 * Host routine (no GPU).  QJL Rademacher matrix for one (user, head) seed,
 * seed = (user_id % 1024) ^ head: row i, column j is +1 iff the low bit of
 * the (D*i + j)-th output of std::mt19937(seed) is 1.  Writes
 * (D/2) * (D/32) words to `out_words`.
 * Replaces the G draw inside _batch_qjl_encode / _batch_qjl_reconstruct
 * (omnistack_rs/kernels/quantize.py:410-414, :443-447) and
 * RademacherQJL._make_G (omnistack_rs/quantization/qjl.py:59-76).
 */
int omni_qjl_g_bits(uint32_t seed, int head_dim, uint32_t *out_words);

/*
 * Normalized Walsh-Hadamard rotation of `rows` vectors of length head_dim:
 * out = dtype(fp32 WHT(sign_flip * x) * fp32(1/sqrt(D))), butterflies in the
 * reference order h = 1, 2, ..., D/2.  sign_flip (length D, +-1) may be NULL.
 * out may alias x.
 * Replaces _wht_torch / _wht_rotate / rotate_queries / rotate_kv_cache
 * (omnistack_rs/kernels/hadamard.py:51-85, :155-191, :196-234).
 */
int omni_wht_rotate(const void *x, int dtype, int64_t rows, int head_dim,
                    const int8_t *sign_flip, void *out, void *stream);

/*
 * Fused KV encoder.  For each row of x (B, H, T, D):
 *   if rotate:  x <- dtype(WHT(sign_flip * x))        (as omni_wht_rotate)
 *   code_d  = argmin_k fp32|x_d - cb_h[k]|  (first index on ties, NaN wins)
 *   e       = x - cb_h[code]   (fp32),   norm = ||e||_2 (fp64 sum, rounded)
 *   bit_i   = [sum_j G_h[i][j] e_j >= 0] (exact sign), packed LSB-first
 * codebooks: (H,16) when per_head_codebook, else (16,).
 * g_bits: (H, D/2, D/32) words for seeds (user_id % 1024) ^ h.
 * workspace: omni_encode_workspace_size(...) bytes of device memory.
 * Replaces quantize_heads (omnistack_rs/kernels/quantize.py:542-590) and,
 * with rotate=1, the bake's _wht_torch + quantize_heads
 * (scripts/run_criteo_benchmark.py:355, :367).
 */
int omni_encode(const void *x, int x_dtype, int64_t B, int H, int64_t T, int head_dim,
                int rotate, const int8_t *sign_flip,
                const float *codebooks, int per_head_codebook,
                const uint32_t *g_bits,
                uint8_t *nibbles, uint8_t *qjl, float *norms,
                void *workspace, size_t workspace_bytes, void *stream);

/*
 * Device workspace bytes omni_encode needs for these arguments (0: none).
 * 16-bit inputs at head_dim 128 use one 64 KB code table per codebook
 * (value bits -> code), rebuilt by every call; OMNI_EWORKSPACE if absent.
 * No reference counterpart (the reference encoder runs on the CPU).
 */
size_t omni_encode_workspace_size(int64_t B, int H, int64_t T, int head_dim, int x_dtype,
                                  int per_head_codebook);

/*
 * The encoder with its code tables built once (serving loops that encode
 * every step's new K and V against a fixed, baked codebook), and K and V of
 * one step in a single launch.  The reference encodes each tensor with its
 * own quantize_heads call (omnistack_rs/kernels/quantize.py:542-590; the
 * bake, scripts/run_criteo_benchmark.py:355-367, calls it for K and for V);
 * these entry points give the same codes, signs and norms.
 *   omni_encode_tables_size: bytes of the tables, (per_head_codebook ? H : 1)
 *     x 64 KB.
 *   omni_encode_build_tables: writes them for 16-bit inputs (x_dtype bf16 or
 *     f16) from `codebooks` (as omni_encode); they stay valid while the
 *     codebooks and the dtype do.
 *   omni_encode_pair: omni_encode of x0 and, when x1 is not NULL, of x1
 *     (same dtype and shape, same G and codebooks) into their own outputs.
 *     16-bit inputs at head_dim 128 with B * T >= 64 read the prebuilt
 *     `tables` (OMNI_EWORKSPACE when missing or short) in one launch; other
 *     inputs take the lane-per-row kernel (tables unused, may be NULL).
 */
size_t omni_encode_tables_size(int H, int per_head_codebook);
int omni_encode_build_tables(const float *codebooks, int per_head_codebook, int H, int x_dtype,
                             uint8_t *tables, size_t tables_bytes, void *stream);
int omni_encode_pair(const void *x0, const void *x1, int x_dtype, int64_t B, int H, int64_t T,
                     int head_dim, int rotate, const int8_t *sign_flip,
                     const float *codebooks, int per_head_codebook, const uint32_t *g_bits,
                     const uint8_t *tables, size_t tables_bytes,
                     uint8_t *nibbles0, uint8_t *qjl0, float *norms0,
                     uint8_t *nibbles1, uint8_t *qjl1, float *norms1, void *stream);

/*
 * Encode one step's new K (and V) tokens straight into the pages of a paged
 * pool (the layout of omni_attn_paged): token t of batch entry b is
 * position p = positions[b] + t of its sequence and goes to slot
 * p % page_size of page page_table[b * max_pages + p / page_size].  K rows
 * get codes, sign bits and norms (as omni_encode_pair), V rows codes only
 * (the attention reads no V residual: fused_attention.py:456-463 passes
 * zero V signs and norms).  16-bit K / V (B, H, T, 128); `tables` from
 * omni_encode_build_tables.  A row whose position is negative or past the
 * table, or whose page id lies outside [0, n_pages), is not written (the
 * host wrapper checks and raises first).  The reference has no paged cache
 * (its bake writes a contiguous one, scripts/run_criteo_benchmark.py:355-367);
 * the codes, signs and norms are those of quantize_heads (quantize.py:542-590).
 */
int omni_encode_paged(const void *k, const void *v, int x_dtype, int64_t B, int H, int64_t T,
                      int rotate, const int8_t *sign_flip, const float *codebooks,
                      int per_head_codebook, const uint32_t *g_bits, const uint8_t *tables,
                      size_t tables_bytes, const int32_t *page_table, int64_t max_pages,
                      const int32_t *positions, int64_t n_pages, int page_size, uint8_t *k_nibbles,
                      uint8_t *k_qjl, float *k_norms, uint8_t *v_nibbles, void *stream);

/*
 * Dequantize packed rows to f32 (B, H, T, D):
 *   out = cb_h[code] + (b+- . G_h) * fp32(norm * fp32(sqrt(2/pi)/D))   (with_qjl)
 *   out = cb_h[code]                                                   (otherwise)
 * b+- . G_h is an integer sum (computed exactly by popcount), so the result
 * is bit-identical to the reference's fp32 path.  qjl / norms / g_bits may
 * be NULL when with_qjl == 0.
 * Replaces dequantize_heads (omnistack_rs/kernels/quantize.py:593-640).
 */
int omni_dequantize(const uint8_t *nibbles, const uint8_t *qjl, const float *norms,
                    const float *codebooks, int per_head_codebook,
                    const uint32_t *g_bits, int64_t B, int H, int64_t T, int head_dim,
                    int with_qjl, float *out, void *stream);

/*
 * Dense fp32 GQA attention on dequantized K / V:
 *   out[b, h, t] = softmax_s(scale * q[b, h, t] . k[b, h / G, s] + mask[b, h, t, s]) . v[b, h / G, s]
 * q (B, Hq, T, D), k and v (B, Hkv, S, D), out (B, Hq, T, D), all f32
 * contiguous; D in {32, 64, 128, 256}.  mask (nullable) is additive, read at
 * b * ms[0] + h * ms[1] + t * ms[2] + s * ms[3] (stride 0 broadcasts).
 * Online softmax in fp32; a row whose first `first_tile` keys are all
 * masked, or that has a NaN score, comes out NaN as the reference's tile
 * loop gives it (first_tile = the reference's tile_size).
 * Replaces reference_attn + repeat_kv (omnistack_rs/attention/reference.py:
 * 49-67, :72-177) on the device.
 */
int omni_dense_attn(const float *q, const float *k, const float *v, const float *mask,
                    const int64_t *mask_strides, int64_t B, int Hq, int Hkv, int64_t T, int64_t S,
                    int head_dim, float scale, int64_t first_tile, float *out, void *stream);

/*
 * Lloyd-Max INT4 codebooks, one per group of samples:
 *   init     16 equal-count bins of the sorted samples (bin size n / 16, the
 *            n % 16 largest in no bin), centroid = bin mean;
 *   iterate  code = first-index argmin_k fp32 |x - c_k|, c_k = mean of its
 *            samples (empty cells keep theirs), until max_iters or the
 *            largest fp32 move < tol;  output sorted ascending (n_groups, 16).
 * Group g's sample e (e < outer * inner) is
 *   x[(e / inner) * outer_stride + g * group_stride + e % inner]
 * (a flat vector: outer = 1; head h of a (B, H, T, D) cache: outer = B,
 * inner = T*D, outer_stride = H*T*D, group_stride = T*D).  Samples must be
 * finite, n >= 16.  Means are taken from fp64 sums in a fixed order
 * (deterministic); the reference's fp32 mean() can differ in the last bits.
 * iters_out (device int32 per group, nullable) receives the steps run.
 * workspace: omni_lloyd_max_workspace_size(...) bytes.
 * Replaces LloydMaxCalibrator.fit / calibrate_codebook / calibrate_per_group
 * (omnistack_rs/quantization/codebook.py:64-108, :129-172) as the bake calls
 * them (scripts/run_criteo_benchmark.py:357-362).
 */
size_t omni_lloyd_max_workspace_size(int n_groups, int64_t outer, int64_t inner);

int omni_lloyd_max(const void *x, int x_dtype, int n_groups, int64_t outer, int64_t inner,
                   int64_t outer_stride, int64_t group_stride, int max_iters, float tol,
                   float *codebooks, int32_t *iters_out, void *workspace, size_t workspace_bytes,
                   void *stream);

/*
 * Per-user LoRA on queries, branchless gather-apply:
 *   q_out[b] = dtype(q[b] + reshape(((x[b] A[id]^T) B[id]^T) * alpha))  if id = idx[b] >= 0
 *   q_out[b] = q[b]                                                      if id < 0
 * (a select, never a multiply-by-zero).  Shapes: q (B, Hq, T, D), x (B, T,
 * hidden), A (n_loras, rank, hidden), Bw (n_loras, Hq*D, rank), idx (B,)
 * int32, rank <= 64; x, A, Bw share `w_dtype`; q_out has q_dtype and may
 * alias q.  An index >= n_loras writes NaN rows (never reads out of bounds);
 * callers that need the reference's IndexError validate indices on the host.
 * Replaces _apply_lora_to_q (omnistack_rs/kernels/fused_attention.py:401-430)
 * and the kernel's LoRA block (:166-191).
 */
int omni_lora_apply(const void *q, int q_dtype, const void *x, const void *A, const void *Bw,
                    int w_dtype, const int32_t *idx, int64_t B, int Hq, int64_t T,
                    int head_dim, int hidden, int rank, int n_loras, float alpha,
                    void *q_out, void *stream);

/*
 * Attention over the packed cache (any T; the decode path is T = 1):
 *   k_hat = cb[code_k] + alpha_s * (b+- G_h),  v_hat = cb[code_v],
 *   out[b, hq, t] = softmax_s(scale * q_eff . k_hat_s + mask) . v_hat
 * with GQA kv head = hq / (Hq / Hkv).  The QJL term is applied as a score
 * correction alpha_s * sum_i b_i (G_h q)_i.  causal_offset < 0: no mask;
 * otherwise query t attends keys s <= causal_offset + t.  rotate_q applies
 * WHT(sign_flip * q) to the query inside the kernel (the K/V cache lives in
 * rotated space); 0 reproduces omni_attn, which takes q as given.
 * Output f32 (B, Hq, T, D).  `workspace` must hold
 * omni_attn_workspace_size(...) bytes (may be 0 -> NULL allowed).
 * Domain: codebook centroids within fp16 range (|c| <= 65504; they are held
 * as fp16 hi + fp16 remainder pairs), S < 2^25; query rows of any finite
 * magnitude (each row is scaled by a power of two in-kernel).
 * Replaces omni_attn / OmniAttention.forward / _fused_attn_triton /
 * _fused_attn_python (omnistack_rs/kernels/fused_attention.py:320-396,
 * :435-466, :471-565).
 */
size_t omni_attn_workspace_size(int64_t B, int Hq, int Hkv, int64_t T, int64_t S, int head_dim);

int omni_attn(const void *q, int q_dtype,
              const uint8_t *k_nib, const uint8_t *k_qjl, const float *k_norms,
              const uint8_t *v_nib, const float *codebooks, int per_head_codebook,
              const uint32_t *g_bits,
              int64_t B, int Hq, int Hkv, int64_t T, int64_t S, int head_dim,
              float scale, int with_qjl, int64_t causal_offset,
              int rotate_q, const int8_t *sign_flip,
              float *out, void *workspace, size_t workspace_bytes, void *stream);

/*
 * omni_attn with the per-user LoRA update of q applied first:
 *   q_eff[b] = dtype(q[b] + ((x[b] A[idx[b]]^T) B[idx[b]]^T) * lora_alpha)
 * (idx < 0: q unchanged; idx >= n_loras: NaN rows), then attention on q_eff
 * exactly as omni_attn.  LoRA shapes and dtypes as omni_lora_apply.  At
 * head_dim 128 with <= 32 query rows per kv head, a nonzero score scale and
 * a 16-bit adapter of rank 8 or 16, hidden <= 256 and a 16-byte aligned
 * lora_b, the update runs inside the attention kernel's prologue (one
 * launch); otherwise the gather-apply kernel writes
 * q_eff into the workspace tail first.  q_eff is rounded
 * exactly as omni_lora_apply rounds it.  `workspace` must hold
 * omni_attn_lora_workspace_size(...) bytes.
 * Replaces omni_attn(..., x, lora_a, lora_b, lora_indices, lora_alpha)
 * (omnistack_rs/kernels/fused_attention.py:537-565) and the Triton kernel's
 * LoRA block (:166-191).
 */
size_t omni_attn_lora_workspace_size(int64_t B, int Hq, int Hkv, int64_t T, int64_t S, int head_dim,
                                     int q_dtype);

int omni_attn_lora(const void *q, int q_dtype,
                   const void *x, const void *lora_a, const void *lora_b, int w_dtype,
                   const int32_t *lora_idx, int hidden, int rank, int n_loras, float lora_alpha,
                   const uint8_t *k_nib, const uint8_t *k_qjl, const float *k_norms,
                   const uint8_t *v_nib, const float *codebooks, int per_head_codebook,
                   const uint32_t *g_bits,
                   int64_t B, int Hq, int Hkv, int64_t T, int64_t S, int head_dim,
                   float scale, int with_qjl, int64_t causal_offset,
                   int rotate_q, const int8_t *sign_flip,
                   float *out, void *workspace, size_t workspace_bytes, void *stream);

/*
 * omni_attn without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * The split-K partials live in a static device array of
 * omni_attn_noalloc_scratch_bytes() bytes (16 MiB) that each device holds
 * until the process ends; a launch needing more
 * (omni_attn_workspace_size(...) > that) returns OMNI_EWORKSPACE without
 * launching.  Calls on one device share the array: calls that overlap on
 * one device (several streams or threads) race.  The first call on a
 * device looks up the array's address (make it outside graph capture).
 * Results are those of omni_attn with the same arguments.
 */
size_t omni_attn_noalloc_scratch_bytes(void);

int omni_attn_noalloc(const void *q, int q_dtype,
                      const uint8_t *k_nib, const uint8_t *k_qjl, const float *k_norms,
                      const uint8_t *v_nib, const float *codebooks, int per_head_codebook,
                      const uint32_t *g_bits,
                      int64_t B, int Hq, int Hkv, int64_t T, int64_t S, int head_dim,
                      float scale, int with_qjl, int64_t causal_offset,
                      int rotate_q, const int8_t *sign_flip,
                      float *out, void *stream);

/*
 * One serving step over a pool of cached sequences: query b attends cache
 * sequence cache_index[b] of a pool of n_cache_seqs (k_nib, k_qjl, k_norms,
 * v_nib are (n_cache_seqs, Hkv, S, ...)); q, x, lora_idx and out have B
 * entries.  Negative indices count from the end of the pool (tensor
 * indexing); an index outside [-n_cache_seqs, n_cache_seqs) gives NaN rows
 * and reads nothing out of bounds.  LoRA as omni_attn_lora when lora_a is
 * not NULL (x, lora_b, lora_idx then required), none when it is NULL.
 * workspace: omni_attn_lora_workspace_size(B, ...) bytes with adapters,
 * omni_attn_workspace_size(B, ...) without.
 * Replaces the serving loop's gather of the batch's caches followed by
 * omni_attn (scripts/run_criteo_benchmark.py:554-557, :593-597): the
 * gather is an index the kernels follow, no copy.
 */
int omni_attn_serve(const void *q, int q_dtype, const int64_t *cache_index, int64_t n_cache_seqs,
                    const void *x, const void *lora_a, const void *lora_b, int w_dtype,
                    const int32_t *lora_idx, int hidden, int rank, int n_loras, float lora_alpha,
                    const uint8_t *k_nib, const uint8_t *k_qjl, const float *k_norms,
                    const uint8_t *v_nib, const float *codebooks, int per_head_codebook,
                    const uint32_t *g_bits,
                    int64_t B, int Hq, int Hkv, int64_t T, int64_t S, int head_dim,
                    float scale, int with_qjl, int64_t causal_offset,
                    int rotate_q, const int8_t *sign_flip,
                    float *out, void *workspace, size_t workspace_bytes, void *stream);

/*
 * Prepared attention: replaces the reference serving loop's per-step
 * omni_attn call (scripts/run_criteo_benchmark.py:684), whose cache,
 * codebooks, adapters and shapes stay fixed from step to step.
 * omni_attn_plan_create stores those static arguments (the pointers are
 * kept, not copied: the buffers must outlive the plan); omni_attn_plan_run
 * then takes only what changes per step and is exactly
 *   n_cache_seqs > 0:        omni_attn_serve(q, ..., cache_index, ..., x, ..., lora_idx, ...)
 *   lora_a != NULL:          omni_attn_lora(q, ..., x, ..., lora_idx, ...)   (cache_index must be NULL)
 *   otherwise:               omni_attn(q, ...)                               (x, lora_idx, cache_index NULL)
 * with the stored arguments, including every argument check.  A plan is
 * read-only once created (runs on several threads or streams may share it,
 * but not its `out` and `workspace`); omni_attn_plan_destroy frees it.
 */
typedef struct omni_attn_plan omni_attn_plan;
int omni_attn_plan_create(int q_dtype, int64_t n_cache_seqs,
                          const void *lora_a, const void *lora_b, int w_dtype,
                          int hidden, int rank, int n_loras, float lora_alpha,
                          const uint8_t *k_nib, const uint8_t *k_qjl, const float *k_norms,
                          const uint8_t *v_nib, const float *codebooks, int per_head_codebook,
                          const uint32_t *g_bits,
                          int64_t B, int Hq, int Hkv, int64_t T, int64_t S, int head_dim,
                          float scale, int with_qjl, int64_t causal_offset,
                          int rotate_q, const int8_t *sign_flip,
                          float *out, void *workspace, size_t workspace_bytes,
                          omni_attn_plan **plan);
int omni_attn_plan_run(const omni_attn_plan *plan, const void *q, const void *x, const int32_t *lora_idx,
                       const int64_t *cache_index, void *stream);
void omni_attn_plan_destroy(omni_attn_plan *plan);

/*
 * The serving step over a page-granular cache.  The reference plans a paged
 * KV cache (MANIFEST.md:211-215; page_size = 16 tokens, config.py:43) but
 * gathers whole sequences instead (scripts/run_criteo_benchmark.py:553-557);
 * this is that gather as page lookups inside the attention kernels (decode
 * for up to 32 query rows per kv head, T * Hq / Hkv; chunked prefill above).
 * Pools (k_nib, k_qjl, k_norms, v_nib) are shaped like a contiguous cache
 * with pages as the batch axis: (n_pages, Hkv, page_size, ...).  Sequence b
 * holds seq_lens[b] tokens; token s sits in page page_table[b * max_pages +
 * s / page_size] at slot s % page_size.  page_size is a power of two in
 * [16, 1024]; n_pages * Hkv * page_size < 2^26; head_dim 128.  causal != 0
 * lets query token t see keys <= seq_lens[b] - T + t (a row with none is
 * NaN).  A page id outside [0, n_pages) among a
 * sequence's pages, or a length outside [0, max_pages * page_size], gives
 * NaN rows for that sequence and reads nothing out of bounds; a length of 0
 * gives NaN rows (no keys).  LoRA as omni_attn_serve (lora_a NULL: none).
 * workspace: omni_attn_paged_workspace_size(...) bytes.
 */
size_t omni_attn_paged_workspace_size(int64_t B, int Hq, int Hkv, int64_t T, int64_t max_pages,
                                      int page_size, int q_dtype);
int omni_attn_paged(const void *q, int q_dtype,
                    const uint8_t *k_nib, const uint8_t *k_qjl, const float *k_norms,
                    const uint8_t *v_nib, int64_t n_pages, int page_size,
                    const int32_t *page_table, int64_t max_pages, const int32_t *seq_lens,
                    const void *x, const void *lora_a, const void *lora_b, int w_dtype,
                    const int32_t *lora_idx, int hidden, int rank, int n_loras, float lora_alpha,
                    const float *codebooks, int per_head_codebook, const uint32_t *g_bits,
                    int64_t B, int Hq, int Hkv, int64_t T, int head_dim,
                    float scale, int with_qjl, int causal, int rotate_q, const int8_t *sign_flip,
                    float *out, void *workspace, size_t workspace_bytes, void *stream);

/*
 * Prepared paged attention: the paged form of omni_attn_plan, for the same
 * per-step call of the reference serving loop (scripts/run_criteo_benchmark.py:684)
 * over the page pool above.  omni_attn_paged_plan_create stores the
 * arguments that stay fixed (pool, geometry, code tables, LoRA bank, shapes,
 * out, workspace; pointers kept, not copied: the buffers must outlive the
 * plan); omni_attn_paged_plan_run(plan, q, page_table, seq_lens, x, lora_idx,
 * stream) is exactly omni_attn_paged with them, including every argument
 * check (x and lora_idx must be NULL for a plan without a bank).  Read-only
 * once created; omni_attn_paged_plan_destroy frees it.
 */
typedef struct omni_attn_paged_plan omni_attn_paged_plan;
int omni_attn_paged_plan_create(int q_dtype,
                                const uint8_t *k_nib, const uint8_t *k_qjl, const float *k_norms,
                                const uint8_t *v_nib, int64_t n_pages, int page_size, int64_t max_pages,
                                const void *lora_a, const void *lora_b, int w_dtype,
                                int hidden, int rank, int n_loras, float lora_alpha,
                                const float *codebooks, int per_head_codebook, const uint32_t *g_bits,
                                int64_t B, int Hq, int Hkv, int64_t T, int head_dim,
                                float scale, int with_qjl, int causal, int rotate_q, const int8_t *sign_flip,
                                float *out, void *workspace, size_t workspace_bytes,
                                omni_attn_paged_plan **plan);
int omni_attn_paged_plan_run(const omni_attn_paged_plan *plan, const void *q, const int32_t *page_table,
                             const int32_t *seq_lens, const void *x, const int32_t *lora_idx, void *stream);
void omni_attn_paged_plan_destroy(omni_attn_paged_plan *plan);

/*
 * Measurement helper with no counterpart in the reference: streams `bytes`
 * (a multiple of 16, 16-byte aligned device buffer) once with n_partials
 * blocks and writes one XOR fold per block to partials[0 .. n_partials),
 * so the XOR of the partials is the XOR of every 32-bit word of `buf`.
 * Its rate is the plain-kernel HBM read bandwidth that the decode
 * kernel's rate is compared with.
 */
int omni_hbm_read_probe(const void *buf, size_t bytes, uint32_t *partials, int n_partials, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* OMNISTACK_AMD_H */
