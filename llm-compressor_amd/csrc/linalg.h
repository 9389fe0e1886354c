// fp32 MFMA GEMM used by the Cholesky chain and the GPTQ trailing update.
#pragma once

#include "common.h"

namespace mi355q {

struct GemmArgs {
  const float* A;  // [M x K] row-major (lda)
  const float* B;  // [K x N] row-major (ldb), or [N x K] when b_trans
  float* C;        // [M x N] row-major (ldc)
  int64_t lda, ldb, ldc;
  int64_t strideA, strideB, strideC;  // batch strides (elements)
  // optional second batch level: batch index z = b1 + inner * b2 with
  // b1 < inner; element offsets b1 * stride + b2 * stride2 (inner = 0: one level)
  int64_t inner;
  int64_t strideA2, strideB2, strideC2;
  int64_t M, N, K;
  float alpha, beta;  // C = beta * C + alpha * (A op(B)); beta == 0 never reads C
  int lower_only;     // only C elements with row >= col (tiles fully above skipped)
  int upper_only;     // only C elements with row <= col (tiles fully below skipped)
  int a_trans;        // A stored as [K x M] row-major (lda); general kernel only
  // triangular operands (general kernel): A lower (A[i][k] = 0 for k > i) or
  // B lower (B[k][j] = 0 for k < j) limits each tile's K range to where the
  // operand can be nonzero
  int a_lower, b_lower;
  // C is A itself (same rows, ldc == lda): every workgroup must own whole
  // rows of C, so N fits one column tile and B is transposed
  int in_place;
  // fp32-accurate product on the bf16 MFMA (each operand split into three
  // bf16 parts, six products per 16-deep slice) where the large-K kernel
  // takes it: 1 for K >= 256 (the GPTQ / SparseGPT lazy updates, the blocked
  // Cholesky's rank-512 updates and the triangular inverse's doubling
  // products; the sweep's K = 128 updates stay on the fp32 MFMA, as the
  // sweep kernel computes the ones it pulls), 2 also for K = 128 (the
  // blocked Cholesky's inner updates)
  int x6;
};

// Whether products asking for x6 take it (MI355Q_GEMM_X6=0 turns it off).
bool x6_enabled();

// Launches the batched GEMM (batch = total number of products) on `stream`;
// returns a status code.
int gemm_f32(const GemmArgs& g, bool b_trans, int batch, hipStream_t stream);

// H[i][j] = beta * H[i][j] + alpha * sum_t x[t][i] x[t][j] for i <= j, x
// [n, d] fp32 row-major (ldx): the fp32 MFMA product of the general kernel
// with A = x transposed, upper tiles only.
int syrk_f32_upper(const float* x, int64_t n, int64_t d, int64_t ldx, float* h, int64_t ldh, float alpha,
                   float beta, hipStream_t stream);

}  // namespace mi355q
