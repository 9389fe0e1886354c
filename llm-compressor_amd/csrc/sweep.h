// Pieces shared by the blocked column sweeps (GPTQ and SparseGPT): the lane
// layout of a row, the packed Hinv block in LDS, the correctly rounded
// quotient from a reciprocal, and the three-level lazy-update schedule.
#pragma once

#include "linalg.h"

namespace mi355q {
namespace sweep {

constexpr int SW_G = 16;                 // lanes per row
constexpr int SW_ROWS = 16;              // rows per workgroup
constexpr int SW_NT = SW_G * SW_ROWS;    // 256 threads
constexpr int MAXB = 128;                // largest block one sweep launch holds
constexpr int SW_T = MAXB / SW_G;        // columns per lane
constexpr int SUPER = 1024;              // columns per lazy-update super-block
constexpr int MID = 512;                 // columns per lazy-update mid-block
constexpr int HPK = MAXB * (MAXB + 1) / 2;  // packed upper triangle of a Hinv block

// Row i of the block's upper triangle starts at hrow(i) in the packed LDS copy
// (element (i, j), j >= i, at hrow(i) + j - i): 33 KB instead of 64 KB, so four
// workgroups fit in a CU's LDS.
__host__ __device__ constexpr int hrow(int i) { return i * MAXB - i * (i - 1) / 2; }

// a / b correctly rounded, from rb = 1 / b correctly rounded: q0 = a rb,
// then one FMA residual correction (Markstein's theorem: with a correctly
// rounded reciprocal the corrected quotient is the correctly rounded one, in
// the absence of overflow and underflow, as for every scale and Hinv diagonal
// here).  Three dependent operations on the sweep's serial chain instead of
// the ten of a full IEEE division; a probe found no difference from a / b in
// 2^32 random and near-half-integer quotients.
__device__ __forceinline__ float div_by_recip(float a, float b, float rb) {
  const float q0 = a * rb;
  const float r = fmaf(-b, q0, a);
  return fmaf(r, rb, q0);
}

// Broadcast lane `L` of every 16-lane row to the whole row (DPP row_newbcast).
template <int L>
__device__ __forceinline__ float row_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + L, 0xF, 0xF, false));
}

// The Hinv values step I of a sweep uses (diagonal, its reciprocal, and row I
// at the lane's columns from slot I / SW_G on), read from LDS two steps ahead
// so that the reads' latency stays off the serial chain.
struct StepH {
  float dd, rd, h[SW_T];
};

template <int I>
__device__ __forceinline__ void load_step(StepH& p, const float* h1, const float* rdg, int g) {
  if constexpr (I < MAXB) {
    constexpr int TO = I / SW_G;
    p.dd = h1[hrow(I)];
    p.rd = rdg[I];
    // (col < I reads a neighbouring entry, in bounds, and is never taken)
#pragma unroll
    for (int t = TO; t < SW_T; ++t) p.h[t] = h1[hrow(I) - I + SW_G * t + g];
  }
}

// Loads Hinv[i1 + i][i1 + j] (j >= i, i, j < count) into the packed LDS
// triangle h1 with all SW_NT threads (16-byte loads for a whole aligned block).
__device__ __forceinline__ void load_hinv_block(float* h1, const float* __restrict__ hinv, int64_t cols,
                                                int64_t i1, int count, int tid) {
  if (count == MAXB && (cols & 3) == 0 && (reinterpret_cast<uintptr_t>(hinv) & 15) == 0) {
    f32x4_t hv[MAXB * MAXB / 4 / SW_NT];
#pragma unroll
    for (int v = 0; v < MAXB * MAXB / 4 / SW_NT; ++v) {
      const int e = v * SW_NT + tid;
      hv[v] = *reinterpret_cast<const f32x4_t*>(hinv + (i1 + (e >> 5)) * cols + i1 + (e & 31) * 4);
    }
#pragma unroll
    for (int v = 0; v < MAXB * MAXB / 4 / SW_NT; ++v) {
      const int e = v * SW_NT + tid;
      const int i = e >> 5, j0 = (e & 31) * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (j0 + q >= i) h1[hrow(i) + j0 + q - i] = hv[v][q];
    }
  } else {
    for (int e = tid; e < count * count; e += SW_NT) {
      const int i = e / count, j = e % count;
      if (j >= i) h1[hrow(i) + j - i] = hinv[(i1 + i) * cols + (i1 + j)];
    }
  }
}

// Columns of the error buffer: one super-block of whole blocks, or all columns.
inline int64_t err_cols(int64_t cols, int64_t blocksize) {
  const int64_t B = blocksize < MAXB ? blocksize : MAXB;
  const int64_t sup = (SUPER / B) * B;
  return sup < cols ? sup : cols;
}

// W[:, c0:c1] -= Err[:, k0:k1] Hinv[k0:k1, c0:c1] for the errors of the
// super-block starting at s0 (Err holds them from column s0 on, leading
// dimension lde): the product is rounded once, then subtracted.
inline int lazy_update(float* w, int64_t rows, int64_t cols, int64_t batch, const float* hinv,
                       int64_t stride_hinv, const float* err, int64_t lde, int64_t k0, int64_t k1, int64_t s0,
                       int64_t c0, int64_t c1, hipStream_t st) {
  GemmArgs g{};
  g.A = err + (k0 - s0); g.lda = lde; g.strideA = rows * lde;
  g.B = hinv + k0 * cols + c0; g.ldb = cols; g.strideB = stride_hinv;
  g.C = w + c0; g.ldc = cols; g.strideC = rows * cols;
  g.M = rows; g.N = c1 - c0; g.K = k1 - k0;
  g.alpha = -1.f; g.beta = 1.f;
  g.x6 = 1;
  return gemm_f32(g, false, (int)batch, st);
}

// The blocked sweep's order of work over cols columns in blocks of B <= MAXB:
// block(i1, i2, s0) sweeps columns [i1, i2) (s0: start of its super-block);
// lazy(k0, k1, s0, c0, c1) applies the errors of columns [k0, k1) to columns
// [c0, c1).  Lazy updates are three-level: inside a mid-block of MID columns
// each block's errors update the rest of the mid-block (K = B, as in the
// reference); the rest of the super-block (SUPER columns) receives a
// mid-block's errors in one product (K up to MID), and the columns past the
// super-block all its errors in one product (K up to SUPER).  The far columns
// thus get Sum_b Err_b Hinv[b, far] rounded once per mid- or super-block
// instead of once per block, an fp32 rounding-order difference of the same
// kind as a GEMM's summation order; most of the multiply-adds run at the
// large-K GEMM's rate instead of the K = 128 kernel's.  Block
// boundaries stay those of the reference (whole blocks per mid- and
// super-block).  Returns the first nonzero status.
template <class Block, class Lazy>
int blocked_schedule(int64_t cols, int64_t B, Block block, Lazy lazy) {
  const int64_t sup = (SUPER / B) * B, mid = (MID / B) * B;
  for (int64_t s0 = 0; s0 < cols; s0 += sup) {
    const int64_t s1 = s0 + sup < cols ? s0 + sup : cols;
    for (int64_t m0 = s0; m0 < s1; m0 += mid) {
      const int64_t m1 = m0 + mid < s1 ? m0 + mid : s1;
      for (int64_t i1 = m0; i1 < m1; i1 += B) {
        const int64_t i2 = (i1 + B < m1) ? i1 + B : m1;
        int rc = block(i1, i2, s0);
        if (rc) return rc;
        if (i2 < m1 && (rc = lazy(i1, i2, s0, i2, m1))) return rc;
      }
      if (m1 < s1) {
        const int rc = lazy(m0, m1, s0, m1, s1);
        if (rc) return rc;
      }
    }
    if (s1 < cols) {
      const int rc = lazy(s0, s1, s0, s1, cols);
      if (rc) return rc;
    }
  }
  return MI355Q_OK;
}

// blocked_schedule for a sweep that applies the K = B updates inside a
// mid-block itself: when the mid-block's blocks are all whole (B == MAXB),
// its block q runs as block(i1, i2, s0, q, m0) and first applies the errors
// of the q blocks before it, in block order, to its own columns, in place of
// the products lazy(i1, i2, s0, i2, m1) after each of those blocks; other
// mid-blocks, and all of them without can_pull, run as in blocked_schedule
// (with q = 0).
template <class Block, class Lazy>
int blocked_schedule_pull(int64_t cols, int64_t B, bool can_pull, Block block, Lazy lazy) {
  const int64_t sup = (SUPER / B) * B, mid = (MID / B) * B;
  for (int64_t s0 = 0; s0 < cols; s0 += sup) {
    const int64_t s1 = s0 + sup < cols ? s0 + sup : cols;
    for (int64_t m0 = s0; m0 < s1; m0 += mid) {
      const int64_t m1 = m0 + mid < s1 ? m0 + mid : s1;
      const bool pull = can_pull && B == MAXB && (m1 - m0) % MAXB == 0;
      for (int64_t i1 = m0; i1 < m1; i1 += B) {
        const int64_t i2 = (i1 + B < m1) ? i1 + B : m1;
        int rc = block(i1, i2, s0, pull ? (int)((i1 - m0) / B) : 0, m0);
        if (rc) return rc;
        if (!pull && i2 < m1 && (rc = lazy(i1, i2, s0, i2, m1))) return rc;
      }
      if (m1 < s1) {
        const int rc = lazy(m0, m1, s0, m1, s1);
        if (rc) return rc;
      }
    }
    if (s1 < cols) {
      const int rc = lazy(s0, s1, s0, s1, cols);
      if (rc) return rc;
    }
  }
  return MI355Q_OK;
}

}  // namespace sweep
}  // namespace mi355q
