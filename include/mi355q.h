/*
 * mi355q - gfx950 (MI355X) kernels for llm-compressor's calibration-time
 * quantization path, behind a plain C ABI.
 *
 * Conventions
 *  - Every pointer argument named *_dev is device memory; *_host is host
 *    memory.  The caller owns and allocates all buffers, including the
 *    workspaces sized by the *_workspace_size queries.
 *  - `stream` is a hipStream_t passed as void* (NULL = default stream).
 *    Calls are stream-ordered and never synchronise, except where a
 *    comment says otherwise.
 *  - Matrices are row-major with an explicit leading dimension in elements.
 *  - bf16 data is passed as raw 16-bit patterns (uint16_t / void*).
 *  - Every entry point returns an mi355q_status; on failure a message is
 *    available from mi355q_last_error() (thread-local).
 *  - The library holds no mutable global state: calls on distinct streams
 *    from several host threads are safe.
 *
 * Reference citations are paths inside ANGDL/llm-compressor
 * (src/llmcompressor/...) unless they name compressed-tensors (CT).
 */
#ifndef MI355Q_H
#define MI355Q_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  MI355Q_OK = 0,
  MI355Q_INVALID_ARGUMENT = 1,
  MI355Q_UNSUPPORTED = 2,
  MI355Q_NOT_POSITIVE_DEFINITE = 3,
  MI355Q_HIP_ERROR = 4,
  /* a per-matrix status of the hinv entry points: the factorisation's
     workgroups stopped waiting for each other (results invalid; the caller
     raises instead of falling back) */
  MI355Q_TIMEOUT = 5
} mi355q_status;

typedef enum { MI355Q_BF16 = 0, MI355Q_F32 = 1, MI355Q_F16 = 2 } mi355q_dtype;

/* Quantization strategy, as compressed-tensors QuantizationStrategy. */
typedef enum {
  MI355Q_TENSOR = 0,
  MI355Q_CHANNEL = 1,
  MI355Q_GROUP = 2,
  MI355Q_BLOCK = 3,
  MI355Q_TOKEN = 4
} mi355q_strategy;

/* Value type of a quantized weight (compressed-tensors type + num_bits). */
typedef enum {
  MI355Q_QTYPE_INT = 0,        /* integers, num_bits <= 8 */
  MI355Q_QTYPE_FP8_E4M3 = 1,   /* float8_e4m3fn (FP8 schemes) */
  MI355Q_QTYPE_FP4_E2M1 = 2,   /* fp4 e2m1 (MXFP4, NVFP4) */
  MI355Q_QTYPE_MXFP4_CT = 3,   /* e2m1 with e8m0 group scales, CT rule (MSE searches only) */
  MI355Q_QTYPE_MXFP4_OCP = 4   /* e2m1 with e8m0 group scales, OCP rule (MSE searches only) */
} mi355q_qtype;

/* MXFP4 shared-exponent rule (see mi355q_mxfp4_quantize_pack). */
typedef enum { MI355Q_MX_RULE_CT = 0, MI355Q_MX_RULE_OCP = 1 } mi355q_mx_rule;

const char* mi355q_last_error(void);
int mi355q_version(void);

/* ------------------------------------------------------------------ Hessian
 * H[i][j] += alpha * sum_t x[t][i] * x[t][j] for i <= j (upper triangle,
 * diagonal included).  Elements strictly below the diagonal are never read
 * or written.  x is [n_tokens, d] bf16 with leading dimension ldx; products
 * of bf16 values are exact in fp32 and accumulate in fp32 (MFMA).
 *
 * Replaces: modifiers/gptq/gptq_quantize.py:22-32 (_hessian_update) as
 * called by accumulate_hessian (:63-97); the reference's 2/n scaling is
 * alpha = 2 here plus the division by num_samples in mi355q_gptq_hinv.
 * Requirements: d % 8 == 0, ldx % 8 == 0, x 16-byte aligned.
 */
size_t mi355q_hessian_workspace_size(int64_t n_tokens, int64_t d);
int mi355q_hessian_syrk_bf16(const void* x_dev, int64_t n_tokens, int64_t d, int64_t ldx,
                             float* h_dev, int64_t ldh, float alpha,
                             void* workspace_dev, size_t workspace_bytes, void* stream);

/* H[i][j] = beta * H[i][j] + alpha * sum_t x[t][i] * x[t][j] (i <= j), the
 * scaling of H a rounded multiply of its own; with n_tokens == 0 only the
 * scaling runs.  Workspace as mi355q_hessian_syrk_bf16.
 * Replaces: modifiers/pruning/sparsegpt/sgpt_sparsify.py:48-53 (the running
 * mean H *= n / (n + added); H += (sqrt(2 / n') X)^T (sqrt(2 / n') X), i.e.
 * beta = n / n', alpha = 2 / n'). */
int mi355q_hessian_syrk_scaled_bf16(const void* x_dev, int64_t n_tokens, int64_t d, int64_t ldx,
                                    float* h_dev, int64_t ldh, float alpha, float beta,
                                    void* workspace_dev, size_t workspace_bytes, void* stream);

/* The same for calibration activations of any floating type the reference
 * accepts (it casts the input to fp32, modifiers/gptq/gptq_quantize.py:93,
 * modifiers/pruning/sparsegpt/sgpt_sparsify.py:51): bf16 and fp16 take the
 * 16-bit MFMA kernels above (products exact in fp32), fp32 an fp32 MFMA
 * product over the upper tiles (no workspace).  H = beta * H + alpha * X^T X
 * on the upper triangle, as mi355q_hessian_syrk_scaled_bf16.  x is [n_tokens,
 * d] row-major (ldx); for the 16-bit types d % 8 == 0, ldx % 8 == 0 and x
 * 16-byte aligned.  Workspace: mi355q_hessian_syrk_workspace_size. */
size_t mi355q_hessian_syrk_workspace_size(int64_t n_tokens, int64_t d, mi355q_dtype dtype);
int mi355q_hessian_syrk(const void* x_dev, mi355q_dtype dtype, int64_t n_tokens, int64_t d, int64_t ldx,
                        float* h_dev, int64_t ldh, float alpha, float beta, void* workspace_dev,
                        size_t workspace_bytes, void* stream);

/* The same over the rows of several calls at once, left where the calls
 * put them: H = beta * H + alpha * sum_k X_k^T X_k, X_k = [n_tokens[k], d]
 * at x_devs[k] (host arrays of n_segments device pointers and row counts;
 * every segment with the common row stride ldx; empty segments skipped).
 * The reference's hook (modifiers/gptq/base.py:255-289 calling
 * gptq_quantize.py:22-32, and modifiers/pruning/sparsegpt/base.py with
 * sgpt_sparsify.py:36-59) adds each forward pass to H at once; a caller that
 * holds the activations of its small calls by reference sums them here in
 * one launch per 64 segments instead of copying them into one buffer.  Each
 * segment starts a new 32-row stage, so segments whose row counts are
 * multiples of 32 give bit for bit the sums of one call over their
 * concatenation.  Workspace: mi355q_hessian_syrk_segments_workspace_size
 * (0 for fp32, which runs one fp32 product per segment). */
size_t mi355q_hessian_syrk_segments_workspace_size(const int64_t* n_tokens, int n_segments, int64_t d,
                                                   mi355q_dtype dtype);
int mi355q_hessian_syrk_segments(const void* const* x_devs, const int64_t* n_tokens, int n_segments,
                                 mi355q_dtype dtype, int64_t d, int64_t ldx, float* h_dev, int64_t ldh,
                                 float alpha, float beta, void* workspace_dev, size_t workspace_bytes,
                                 void* stream);

/* Grouped (MoE) variant: expert e accumulates the rows
 * x[rows_dev[k]] for k in [offsets_dev[e], offsets_dev[e+1]) into
 * h_dev + e * h_stride (each d x d, leading dimension d, upper triangle):
 * H_e = beta * H_e + alpha * X_e^T X_e, beta 1 (add) or 0 (H_e's upper
 * triangle is written without being read, zeros for an expert without
 * rows: a freshly allocated stack need not be cleared).  Replaces the per-expert accumulate_hessian
 * calls that modeling/moe/linear_experts.py:244-277 triggers with routed
 * tokens.  x is [n_x, d] (ldx), bf16 or fp16; rows_dev (n_rows int32
 * indices into x) may be NULL when x's rows are already grouped (row k of
 * expert e is x[k]; then n_rows <= n_x).  offsets_dev is int64 [n_experts+1]
 * in device memory, non-decreasing with offsets[n_experts] <= n_rows: the
 * work table is built on the device, so the call never waits for the host
 * (offsets outside that contract are clamped and row indices outside
 * [0, n_x) are clamped; nothing is read or written out of bounds).
 * Workspace: mi355q_hessian_grouped_syrk_workspace_size(n_rows, n_experts,
 * d) bytes. */
size_t mi355q_hessian_grouped_syrk_workspace_size(int64_t n_rows, int n_experts, int64_t d);
int mi355q_hessian_grouped_syrk(const void* x_dev, mi355q_dtype dtype, int64_t n_x, int64_t ldx, int64_t d,
                                const int32_t* rows_dev, int64_t n_rows, const int64_t* offsets_dev,
                                int n_experts, float* h_dev, int64_t h_stride, float alpha, float beta,
                                void* workspace_dev, size_t workspace_bytes, void* stream);

/* Mirror the upper triangle into the lower one (full symmetric matrix). */
int mi355q_symmetrize_upper(float* h_dev, int64_t d, int64_t ldh, void* stream);

/* ------------------------------------------------------------------ GPTQ
 * mi355q_gptq_hinv: from the accumulated upper-triangle Hessian (optionally
 * permuted by perm_dev, may be NULL), computes
 *   H' = H / num_samples (modifiers/gptq/base.py:594),
 *   dead columns: diag(H') == 0 -> H'_ii = 1, dead_dev[i] = 1
 *     (modifiers/gptq/gptq_quantize.py:35-38),
 *   H' += percdamp * mean(diag(H')) * I  (:182-184),
 *   hinv = upper Cholesky factor of inverse(H') (:185-188)
 * using H' = R R^T with R upper (reverse-order Cholesky) and hinv = R^-1.
 * On a non-positive-definite H' the kernels set *status_dev = 3 and hinv
 * holds no meaningful values; the caller then uses the identity (RTN
 * fallback, :189-196).  *status_dev is written with 0 first.
 */
size_t mi355q_gptq_hinv_workspace_size(int64_t d);
int mi355q_gptq_hinv(const float* h_dev, int64_t ldh, int64_t d, const int32_t* perm_dev,
                     float num_samples, float percdamp, float* hinv_dev,
                     int32_t* dead_dev, int32_t* status_dev, void* workspace_dev,
                     size_t workspace_bytes, void* stream);

/* Batched variants.  The reference solves the Hessians of same-shaped modules
 * (the experts of an MoE layer, modeling/moe/linear_experts.py:244-277) one
 * module at a time in compress_module_list (modifiers/gptq/base.py:578-601);
 * these run `batch` independent solves per launch.  Matrix b reads
 * h + b * stride_h and perm + b * stride_perm (stride 0: shared perm),
 * num_samples_dev[b], and writes hinv + b * stride_hinv, dead + b * d and
 * status_dev[b].  Workspace: batch * mi355q_gptq_hinv_workspace_size(d). */
int mi355q_gptq_hinv_batched(const float* h_dev, int64_t ldh, int64_t stride_h, int64_t d,
                             int64_t batch, const int32_t* perm_dev, int64_t stride_perm,
                             const float* num_samples_dev, float percdamp, float* hinv_dev,
                             int64_t stride_hinv, int32_t* dead_dev, int32_t* status_dev,
                             void* workspace_dev, size_t workspace_bytes, void* stream);

/* mi355q_gptq_hinv_fallback: hinv + b * stride_hinv = identity for every b
 * with status_dev[b] != 0 -- the reference's non-positive-definite branch
 * (gptq_quantize.py:189-196: LinAlgError -> Hinv = eye, round-to-nearest)
 * applied on the device, so the solve runs on without reading the flag on
 * the host.  batch <= 65535. */
int mi355q_gptq_hinv_fallback(float* hinv_dev, int64_t d, int64_t stride_hinv, int64_t batch,
                              const int32_t* status_dev, void* stream);

/* mi355q_gptq_load_weight: w_work[r][j] = dead[j] ? 0 : float(w[r][perm[j]])
 * (fp32 working copy, :121,126,142,178).  perm_dev / dead_dev may be NULL. */
int mi355q_gptq_load_weight(const void* w_dev, mi355q_dtype w_dtype, int64_t rows, int64_t cols,
                            int64_t ldw, const int32_t* perm_dev, const int32_t* dead_dev,
                            float* w_work_dev, void* stream);
/* batched: matrix b reads w + b * stride_w (elements), perm + b * stride_perm,
 * dead + b * cols, and writes w_work + b * rows * cols */
int mi355q_gptq_load_weight_batched(const void* w_dev, mi355q_dtype w_dtype, int64_t rows, int64_t cols,
                                    int64_t ldw, int64_t stride_w, int64_t batch,
                                    const int32_t* perm_dev, int64_t stride_perm,
                                    const int32_t* dead_dev, float* w_work_dev, void* stream);

/* mi355q_gptq_sweep: the blocked column sweep of :199-277 over the fp32
 * working copy, in place.  Column j is quantised with
 *   scale = scale_dev[r * ld_scale + sidx(r, j)], zp likewise,
 * where sidx is 0 (TENSOR, ld_scale ignored -> scale_dev[0]), 0 (CHANNEL),
 * g_idx_dev[j] (GROUP) or (BLOCK) (r / block_h) rows and g_idx_dev[j] cols.
 *   q = clamp(rint(w / scale + zp), qmin, qmax)          (CT quantize)
 *   w_q = (q - zp) * scale, rounded to bf16 if dequant_bf16 (CT dequantize
 *         in the bf16 scale dtype)
 *   err = (w - w_q) / hinv[j][j];  losses[r] += (w - w_q)^2 / hinv[j][j]^2 / 2
 *   w[:, j+1:block_end] -= err * hinv[j, j+1:block_end]   (mul, then sub)
 *   after each block: w[:, block_end:] -= Err_block @ hinv[block, block_end:]
 * On return w_work holds the dequantised values, codes_dev[r][j] the integer
 * codes q (int8, working column order) and losses_dev[r] the per-row loss
 * (fp32, accumulated onto its input).  Integer types only (num_bits <= 8);
 * mi355q_gptq_sweep_typed_batched takes the fp8 / fp4 grids.
 * zp_dev may be NULL: zero points 0 (symmetric), a faster kernel variant.
 */
size_t mi355q_gptq_sweep_workspace_size(int64_t rows, int64_t cols, int64_t blocksize);
int mi355q_gptq_sweep(float* w_work_dev, int64_t rows, int64_t cols, const float* hinv_dev,
                      const float* scale_dev, const float* zp_dev, int64_t ld_scale,
                      const int32_t* g_idx_dev, int strategy, int block_h, float qmin, float qmax,
                      int dequant_bf16, int64_t blocksize, int8_t* codes_dev, float* losses_dev,
                      void* workspace_dev, size_t workspace_bytes, void* stream);
/* batched: matrix b uses w_work + b * rows * cols, hinv + b * stride_hinv,
 * scale / zp + b * stride_scale, g_idx + b * stride_gidx (0: shared),
 * codes + b * rows * cols, losses + b * rows.
 * Workspace: batch * mi355q_gptq_sweep_workspace_size(rows, cols, blocksize). */
int mi355q_gptq_sweep_batched(float* w_work_dev, int64_t rows, int64_t cols, int64_t batch,
                              const float* hinv_dev, int64_t stride_hinv, const float* scale_dev,
                              const float* zp_dev, int64_t ld_scale, int64_t stride_scale,
                              const int32_t* g_idx_dev, int64_t stride_gidx, int strategy, int block_h,
                              float qmin, float qmax, int dequant_bf16, int64_t blocksize,
                              int8_t* codes_dev, float* losses_dev, void* workspace_dev,
                              size_t workspace_bytes, void* stream);

/* The sweep for every weight type the reference's GPTQ quantizes
 * (gptq_quantize.py:215-257 call CT fake_quantize with the module's args and
 * global_scale): qtype selects the rounding of x / scale after the clamp to
 * [qmin, qmax] -- rint for integers, the float8_e4m3fn cast (round to
 * nearest even) for FP8, CT's cast_to_fp4 thresholds for fp4 (MXFP4 with its
 * power-of-two group scales; NVFP4 tensor-group with fp8 group scales and a
 * global scale).  global_scale_dev (NULL: none) holds one fp32 value per
 * matrix; the effective scale is scale / global_scale (CT's tensor-group
 * rule).  Float types take no zero point and qmin = -qmax.  codes_dev holds
 * the integer codes (QTYPE_INT), float8_e4m3fn bit patterns (FP8) or e2m1
 * codes sign << 3 | grid index (FP4).  Otherwise as mi355q_gptq_sweep_batched. */
int mi355q_gptq_sweep_typed_batched(float* w_work_dev, int64_t rows, int64_t cols, int64_t batch,
                                    const float* hinv_dev, int64_t stride_hinv, const float* scale_dev,
                                    const float* zp_dev, int64_t ld_scale, int64_t stride_scale,
                                    const int32_t* g_idx_dev, int64_t stride_gidx, int strategy, int block_h,
                                    int qtype, float qmin, float qmax, const float* global_scale_dev,
                                    int dequant_bf16, int64_t blocksize, int8_t* codes_dev, float* losses_dev,
                                    void* workspace_dev, size_t workspace_bytes, void* stream);

/* mi355q_gptq_sweep_noalloc: mi355q_gptq_sweep without a workspace argument
 * and without any allocation, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It has no counterpart in the reference.  The error workspace
 * lives in a 64 MiB device array the library holds on each GPU it runs on
 * until the process ends (mi355q_gptq_sweep_noalloc_max_bytes()): shapes whose
 * mi355q_gptq_sweep_workspace_size (rows * min(1024, cols) fp32) exceeds it
 * are rejected with MI355Q_INVALID_ARGUMENT.  Every call on a GPU shares that
 * GPU's array, so calls that overlap on one GPU (other streams or threads)
 * race; sequential calls need no clearing in between.  Arguments and results
 * otherwise as mi355q_gptq_sweep, bit for bit. */
size_t mi355q_gptq_sweep_noalloc_max_bytes(void);
int mi355q_gptq_sweep_noalloc(float* w_work_dev, int64_t rows, int64_t cols, const float* hinv_dev,
                              const float* scale_dev, const float* zp_dev, int64_t ld_scale,
                              const int32_t* g_idx_dev, int strategy, int block_h, float qmin, float qmax,
                              int dequant_bf16, int64_t blocksize, int8_t* codes_dev, float* losses_dev,
                              void* stream);

/* mi355q_gptq_store_weight: w_out[r][j] = w_work[r][invperm[j]] converted
 * to out_dtype (:279-284); codes are permuted the same way when
 * codes_in/codes_out are non-NULL.  invperm_dev may be NULL. */
int mi355q_gptq_store_weight(const float* w_work_dev, int64_t rows, int64_t cols,
                             const int32_t* invperm_dev, void* w_out_dev, mi355q_dtype out_dtype,
                             int64_t ld_out, const int8_t* codes_in_dev, int8_t* codes_out_dev,
                             void* stream);
/* batched: matrix b reads w_work + b * rows * cols, invperm + b * stride_perm,
 * codes_in + b * rows * cols, writes w_out + b * stride_out, codes_out + b * rows * cols */
int mi355q_gptq_store_weight_batched(const float* w_work_dev, int64_t rows, int64_t cols, int64_t batch,
                                     const int32_t* invperm_dev, int64_t stride_perm, void* w_out_dev,
                                     mi355q_dtype out_dtype, int64_t ld_out, int64_t stride_out,
                                     const int8_t* codes_in_dev, int8_t* codes_out_dev, void* stream);

/* ------------------------------------------------------------------ SparseGPT
 * The solve of modifiers/pruning/sparsegpt/sgpt_sparsify.py:58-213 on a
 * working copy from mi355q_gptq_load_weight (dead columns zeroed) and the
 * upper factor from mi355q_gptq_hinv / _hinv_fallback (the same chain as
 * :97-117, num_samples = 1 since the running-mean Hessian is normalised).
 *
 * mi355q_sparsegpt_base_mask: mask[i] = (w_work[i] == 0), count = number of
 * such entries (device uint32; the caller reads it for the reference's
 * "target sparsity is lower than the sparsity of the base model" check,
 * :122-135).
 *
 * mi355q_sparsegpt_sweep: blocked sweep (:137-206) in place on w_work (fp32
 * [rows, cols]); losses [rows] fp32 accumulate sum_blocks sum (w - q)^2 /
 * d^2 / 2 (zero it first).  prune_n == 0: unstructured, per block every
 * entry whose w^2 / Hinv[c][c]^2 is at or below the k-th smallest of the
 * block, k = int(rows * count * sparsity) (:150-165).  prune_n > 0: N:M
 * groups of prune_m <= 16 columns from each block's start, the prune_n
 * smallest per row pruned, lower column first on equal values (:166-186).
 * mask_dev != NULL: preserve_sparsity_mask with the mask from
 * mi355q_sparsegpt_base_mask (in N:M mode it is updated in place, as the
 * reference's view of it is).  blocksize <= 128 (MI355Q_UNSUPPORTED above);
 * arguments the reference rejects by raising (k out of range, a group
 * narrower than prune_n, mismatched preserved-mask windows) give
 * MI355Q_INVALID_ARGUMENT. */
int mi355q_sparsegpt_base_mask(const float* w_work_dev, int64_t rows, int64_t cols, uint8_t* mask_dev,
                               uint32_t* count_dev, void* stream);
size_t mi355q_sparsegpt_workspace_size(int64_t rows, int64_t cols, int64_t blocksize);
int mi355q_sparsegpt_sweep(float* w_work_dev, int64_t rows, int64_t cols, const float* hinv_dev,
                           double sparsity, int prune_n, int prune_m, int64_t blocksize,
                           uint8_t* mask_dev, float* losses_dev, void* workspace_dev,
                           size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ observers
 * Min/max statistics per strategy (observers/min_max.py:106-110 over
 * observers/helpers.py:63-101 flattening).  Outputs are fp32 holding the
 * exact input-dtype values: TENSOR -> 1, CHANNEL -> rows, GROUP ->
 * rows * ceil(cols / group), BLOCK -> ceil(rows/bh) * ceil(cols/bw)
 * (zero padding included, as the reference pads), TOKEN -> rows.
 */
int mi355q_observe_minmax(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols,
                          int64_t ldx, int strategy, int64_t group_size, int block_h, int block_w,
                          float* min_dev, float* max_dev, void* stream);

/* CT calculate_qparams (observers/base.py:99-123 -> CT) over the quantized
 * range [qmin, qmax] ((-2^(b-1), 2^(b-1)-1) for int, (-448, 448) for fp8):
 * symmetric scale = absmax / ((qmax - qmin) / 2), asymmetric scale =
 * (max - min) / (qmax - qmin) with zp = rint(clamp(qmin - min / scale)),
 * min/max first widened to include 0; every step is rounded to scale_dtype
 * (bf16 = the weight dtype for a bf16 weight); zero scales become the
 * dtype's epsilon.  strict != 0 selects observers/min_max.py:33-55 (fp32
 * absmax / qmax clamped at 1e-8).  scale_out is fp32 holding scale_dtype
 * values; zp_out is fp32 integers. */
int mi355q_calculate_qparams(const float* min_dev, const float* max_dev, int64_t n, float qmin,
                             float qmax, int symmetric, int strict, mi355q_dtype scale_dtype,
                             float* scale_out_dev, float* zp_out_dev, void* stream);

/* MX shared scales from observer statistics: e8m0 byte per group (rule as
 * in mi355q_mxfp4_quantize_pack, absmax = max(|min|, |max|) of bf16
 * values) and the scale 2^(e-127) as fp32.  Either output may be NULL. */
int mi355q_mx_scales(const float* min_dev, const float* max_dev, int64_t n, int rule,
                     uint8_t* e8m0_out_dev, float* scale_out_dev, void* stream);

/* NVFP4 tensor-group qparams from the n groups' min / max statistics (fp32
 * holding values of stats_dtype, bf16 or fp32): the global scale
 * (observers/base.py:78-96 -> CT generate_gparam: 448 * 6 / absmax of the
 * whole weight, computed in stats_dtype, stored as fp32 in global_scale_dev[0])
 * and each group's scale (CT calculate_qparams with that global scale:
 * global * (absmax / 6) clamped to +-448 and cast to float8_e4m3fn, 0 -> the
 * fp8 epsilon 0.125) as fp32 values (scale_out_dev) and / or e4m3 bits. */
int mi355q_nvfp4_qparams(const float* min_dev, const float* max_dev, int64_t n, mi355q_dtype stats_dtype,
                         float* global_scale_dev, float* scale_out_dev, uint8_t* e4m3_out_dev, void* stream);

/* MSE observer grid search (observers/mse_quant.py:48-130,244-273; the
 * memoryless_mse / mse observers of observers/mse.py:12-98).  x [rows, cols]
 * (bf16 or fp32, leading dimension ldx) is split into cells of cell_rows x
 * cell_cols (clipped at the edges, row-major; a group is 1 x group_size, a
 * channel 1 x cols, the tensor rows x cols, a block its block shape); min_dev /
 * max_dev hold each cell's min / max.  For candidate i < total_steps
 * (= int(maxshrink * grid)) the min / max are scaled by p = 1 - i / grid,
 * qparams computed as calculate_qparams does in the observed dtype, and the
 * error is sum |fake_quantize(x) - x|^norm in that dtype (for bf16 with the
 * exponent rounded to bf16, as torch's pow does); each cell keeps its
 * first best candidate over the steps before the first run of `patience`
 * steps without an improvement in any cell.  Writes the chosen min / max
 * (float values of the observed dtype) to min_out / max_out.  qtype
 * MI355Q_QTYPE_INT: the integer grid (rint); MI355Q_QTYPE_FP8_E4M3: the fp8
 * e4m3 grid (symmetric, qmin = -qmax <= 448; round to nearest even after the
 * clamp, as the cast to float8_e4m3fn in CT round_to_quantized_type does);
 * MI355Q_QTYPE_FP4_E2M1: the e2m1 grid (symmetric, qmin = -qmax <= 6; CT
 * cast_to_fp4).  The candidates' scales are calculate_qparams' without a
 * global scale (observers/mse_quant.py:255-262); MI355Q_QTYPE_MXFP4_CT /
 * _OCP: the e2m1 grid with each candidate's scale 2^(e - 127), e the e8m0
 * exponent of max(|min|, |max|) by that rule (as mi355q_mx_scales). */
size_t mi355q_observe_mse_workspace_size(int64_t rows, int64_t cols, int64_t cell_rows, int64_t cell_cols,
                                         int total_steps);
int mi355q_observe_mse(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols, int64_t ldx,
                       int64_t cell_rows, int64_t cell_cols, float qmin, float qmax, int symmetric, int qtype,
                       int total_steps, int patience, double grid, float norm, const float* min_dev,
                       const float* max_dev, float* min_out_dev, float* max_out_dev, void* workspace_dev,
                       size_t workspace_bytes, void* stream);

/* The imatrix observer's search (observers/imatrix.py:289-440): as
 * mi355q_observe_mse with total_steps = max(1, int(maxshrink * grid)) + 1,
 * the error |fq(x) - x|^norm computed and summed in fp32 (fq in the observed
 * dtype) and weighted by importance_dev[column] (fp32 [cols], normalised E[x^2];
 * NULL: uniform), and no early stop when patience is 0. */
int mi355q_observe_imatrix_mse(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols, int64_t ldx,
                               int64_t cell_rows, int64_t cell_cols, float qmin, float qmax, int symmetric,
                               int qtype, int total_steps, int patience, double grid, float norm,
                               const float* importance_dev, const float* min_dev, const float* max_dev,
                               float* min_out_dev, float* max_out_dev, void* workspace_dev,
                               size_t workspace_bytes, void* stream);

/* sum_dev[c] += sum_r x[r][c]^2 in fp32 (fixed summation order): the imatrix
 * observer's per-input-channel accumulation (observers/imatrix.py:92-121).
 * Workspace from mi355q_column_sumsq_workspace_size. */
size_t mi355q_column_sumsq_workspace_size(int64_t rows, int64_t cols);
int mi355q_column_sumsq(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols, int64_t ldx,
                        float* sum_dev, void* workspace_dev, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ quantize / pack
 * Integer quantize of a whole weight with the scale indexing of
 * mi355q_gptq_sweep (g_idx may be NULL: column / group_size):
 *   codes = clamp(rint(x / scale + zp), qmin, qmax), division in
 *   div_dtype (bf16 rounds the quotient, as CT does for a bf16 weight with
 *   a bf16 scale).  Replaces CT quantize inside the compressors called at
 *   transformers/compression/compressed_tensors_utils.py:172-191.
 */
int mi355q_quantize_int(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols,
                        int64_t ldx, const float* scale_dev, const float* zp_dev,
                        int64_t ld_scale, const int32_t* g_idx_dev, int strategy,
                        int64_t group_size, int block_h, int block_w, int num_bits,
                        mi355q_dtype div_dtype, int8_t* codes_dev, void* stream);

/* CT pack_quantized (pack_to_int32): 4-bit codes -> int32 words, eight per
 * word, element k of a word at bits 4k, stored offset-binary (q + 8).
 * cols % 8 == 0.  out is [rows, cols/8]. */
int mi355q_pack_int4_int32(const int8_t* codes_dev, int64_t rows, int64_t cols,
                           int32_t* out_dev, void* stream);

/* The same layout for num_bits in {2, 4, 8}: 32 / num_bits codes per word,
 * element e at bits num_bits * e, offset-binary (q + 2^(num_bits-1)); out is
 * [rows, ceil(cols * num_bits / 32)] and positions past a row's end are 0.
 * Replaces CT pack_to_int32 for pack-quantized W4 / W8 checkpoints (the
 * compressor call at transformers/compression/compressed_tensors_utils.py:191). */
int mi355q_pack_int32(const int8_t* codes_dev, int64_t rows, int64_t cols, int num_bits,
                      int32_t* out_dev, void* stream);

/* utils/pack_int4_to_int8.py:13-28: out[r][k] = (c[r][2k+1] & 15) << 4 |
 * (c[r][2k] & 15).  cols must be even. */
int mi355q_pack_int4_int8(const int8_t* codes_dev, int64_t rows, int64_t cols,
                          int8_t* out_dev, void* stream);

/* MXFP4 (W4A4 / MXFP4 preset): per row, groups of 32 along columns share
 * an e8m0 exponent e (scale 2^(e-127)); elements are rounded to e2m1
 * (ties to even, saturating at 6, negative values rounding to zero keep the
 * sign bit), code = sign<<3 | index in {0,.5,1,1.5,2,3,4,6}; two codes per
 * byte, even column in the low nibble.  codes [rows, cols/2] uint8, scales
 * [rows, cols/32] uint8.  cols % 32 == 0.  Rule MI355Q_MX_RULE_CT follows
 * CT's generate_mx_scales (bf16 absmax rounded up to a power of two at
 * 1.75, exponent - 2); MI355Q_MX_RULE_OCP is OCP MX v1.0 floor(log2)-2.
 * Replaces the observer + CT mxfp4_pack_quantized path
 * (modifiers/quantization/calibration.py:86-157 and the compressor call at
 * compressed_tensors_utils.py:191). */
int mi355q_mxfp4_quantize_pack(const void* x_dev, int64_t rows, int64_t cols, int64_t ldx,
                               int rule, uint8_t* codes_dev, uint8_t* scales_dev, void* stream);
int mi355q_mxfp4_dequantize(const uint8_t* codes_dev, const uint8_t* scales_dev, int64_t rows,
                            int64_t cols, void* out_dev, void* stream);

/* fp4 e2m1 quantize + pack with given group scales (the NVFP4 weight of
 * an nvfp4-pack-quantized checkpoint, docs/guides/compression_schemes.md:57-64):
 * q = e2m1(x / (scale[r][c / group_size] / global_scale)), the effective
 * scale and the quotient in fp32 as CT's quantize forms them (no global
 * scale: NULL), e2m1 rounding, codes and byte layout as
 * mi355q_mxfp4_quantize_pack.  scale is fp32 [rows, >= ceil(cols /
 * group_size)] (ld_scale), codes [rows, cols / 2] uint8, cols even.
 * Replaces the CT nvfp4_pack_quantized compressor at save
 * (transformers/compression/compressed_tensors_utils.py:191). */
int mi355q_fp4_quantize_pack(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols, int64_t ldx,
                             const float* scale_dev, int64_t ld_scale, int64_t group_size,
                             const float* global_scale_dev, uint8_t* codes_dev, void* stream);

/* fp8 e4m3 (float8_e4m3fn) quantize: q = fp8_rne(clamp(x / scale, -448,
 * 448)) with the scale indexing of mi355q_quantize_int; division in
 * div_dtype.  Output bytes are e4m3fn bit patterns. */
int mi355q_quantize_fp8(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols,
                        int64_t ldx, const float* scale_dev, int64_t ld_scale, int strategy,
                        int64_t group_size, mi355q_dtype div_dtype, uint8_t* out_dev,
                        void* stream);

/* Dynamic per-token int8 (W8A8 activations, CT TOKEN strategy): per row
 * scale = bf16(absmax / 127.5) (epsilon if zero), codes = clamp(rint(bf16(x
 * / scale)), -128, 127).  scale_out is bf16 bits [rows]. */
int mi355q_quantize_int8_per_token(const void* x_dev, int64_t rows, int64_t cols, int64_t ldx,
                                   int8_t* codes_dev, uint16_t* scale_out_dev, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MI355Q_H */
