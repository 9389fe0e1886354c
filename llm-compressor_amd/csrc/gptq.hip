// GPTQ blocked column sweep on gfx950.
//
// Replaces modifiers/gptq/gptq_quantize.py:199-277.  Rows of W are
// independent given Hinv and the (static) scales, so the serial column loop
// runs for all rows at once: a workgroup holds 16 rows, each row is shared by
// 16 lanes, and lane g owns the block columns j = 16 t + g (t = 0..7) in
// registers.  For column i the owner's value is broadcast to its 16 lanes,
// every lane quantises it (CT quantize/dequantize arithmetic), and each lane
// applies err * Hinv[i][j] to its own later columns as a rounded multiply
// followed by a rounded subtract (the reference's outer-product matmul and
// in-place subtract).  Hinv's diagonal block sits in LDS.  After each block
// the lazy update W[:, i2:] -= Err @ Hinv[i1:i2, i2:] runs as an fp32 MFMA
// GEMM whose output is rounded once and then subtracted, as in the reference.
#include "linalg.h"

#pragma clang fp contract(off)

namespace mi355q {
namespace {

constexpr int SW_G = 16;                 // lanes per row
constexpr int SW_ROWS = 16;              // rows per workgroup
constexpr int SW_NT = SW_G * SW_ROWS;    // 256 threads
constexpr int MAXB = 128;                // largest supported block size
constexpr int SW_T = MAXB / SW_G;        // columns per lane

__device__ __forceinline__ int64_t sidx(int strategy, int64_t r, int64_t c, int64_t ld_scale,
                                        const int32_t* g_idx, int block_h) {
  switch (strategy) {
    case MI355Q_TENSOR: return 0;
    case MI355Q_CHANNEL: return r * ld_scale;
    case MI355Q_GROUP: return r * ld_scale + g_idx[c];
    case MI355Q_BLOCK: return (r / block_h) * ld_scale + g_idx[c];
  }
  return 0;
}

__global__ __launch_bounds__(SW_NT) void sweep_block_kernel(
    float* __restrict__ W, int64_t rows, int64_t cols, const float* __restrict__ hinv, int64_t i1,
    int count, const float* __restrict__ scale, const float* __restrict__ zp, int64_t ld_scale,
    const int32_t* __restrict__ g_idx, int strategy, int block_h, float qmin, float qmax, int dq_bf16,
    int8_t* __restrict__ codes, float* __restrict__ losses, float* __restrict__ err_out) {
  __shared__ float h1[MAXB * MAXB];
  const int tid = threadIdx.x;
  if (count == MAXB && (cols & 3) == 0 && (reinterpret_cast<uintptr_t>(hinv) & 15) == 0) {
    // 16 independent 16-byte loads per thread (lower-triangle chunks skipped)
#pragma unroll
    for (int v = 0; v < MAXB * MAXB / 4 / SW_NT; ++v) {
      const int e = v * SW_NT + tid;
      const int i = e >> 5, j4 = (e & 31) * 4;
      if (j4 + 3 >= i)
        *reinterpret_cast<f32x4_t*>(h1 + i * MAXB + j4) =
            *reinterpret_cast<const f32x4_t*>(hinv + (i1 + i) * cols + i1 + j4);
    }
  } else {
    for (int e = tid; e < count * count; e += SW_NT) {
      const int i = e / count, j = e % count;
      if (j >= i) h1[i * MAXB + j] = hinv[(i1 + i) * cols + (i1 + j)];
    }
  }
  __syncthreads();

  const int g = tid & (SW_G - 1);
  const int64_t r = (int64_t)blockIdx.x * SW_ROWS + (tid / SW_G);
  const bool live = r < rows;

  float w[SW_T], s[SW_T], z[SW_T], q[SW_T], er[SW_T];
  int cq[SW_T];
#pragma unroll
  for (int t = 0; t < SW_T; ++t) {
    const int col = SW_G * t + g;
    w[t] = 0.f; s[t] = 1.f; z[t] = 0.f; q[t] = 0.f; er[t] = 0.f; cq[t] = 0;
    if (live && col < count) {
      const int64_t c = i1 + col;
      w[t] = W[r * cols + c];
      const int64_t si = sidx(strategy, r, c, ld_scale, g_idx, block_h);
      s[t] = scale[si];
      z[t] = zp ? zp[si] : 0.f;
    }
  }

  float loss = 0.f;
  // column i = SW_G * to + go; `to` is a compile-time register slot (outer
  // loop unrolled), `go` the owner lane (inner loop, runtime), so no
  // register array is ever indexed dynamically
#pragma unroll
  for (int to = 0; to < SW_T; ++to) {
  for (int go = 0; go < SW_G; ++go) {
    const int i = SW_G * to + go;
    if (i >= count) break;
    const float x = __shfl(w[to], go, SW_G);
    const float sc = __shfl(s[to], go, SW_G);
    const float zz = __shfl(z[to], go, SW_G);
    const float dd = h1[i * MAXB + i];
    float qq = x / sc + zz;
    qq = rintf(fminf(fmaxf(qq, qmin), qmax));
    float deq = (qq - zz) * sc;
    if (dq_bf16) deq = round_to_bf16(deq);
    const float diff = x - deq;
    const float err = diff / dd;
    if (g == go) {
      q[to] = deq;
      cq[to] = (int)qq;
      er[to] = err;
      loss = loss + diff * diff / (dd * dd);
    }
#pragma unroll
    for (int t = to; t < SW_T; ++t) {
      const int col = SW_G * t + g;
      if (col > i && col < count) w[t] = w[t] - err * h1[i * MAXB + col];
    }
  }
  }

  if (live) {
#pragma unroll
    for (int t = 0; t < SW_T; ++t) {
      const int col = SW_G * t + g;
      if (col < count) {
        const int64_t c = i1 + col;
        W[r * cols + c] = q[t];
        codes[r * cols + c] = (int8_t)cq[t];
        err_out[r * MAXB + col] = er[t];
      }
    }
  }
#pragma unroll
  for (int o = 1; o < SW_G; o <<= 1) loss += __shfl_xor(loss, o, SW_G);
  if (live && g == 0) losses[r] = losses[r] + loss / 2.f;
}

__global__ void load_weight_kernel(const void* w, mi355q_dtype dt, int64_t rows, int64_t cols, int64_t ldw,
                                   const int32_t* perm, const int32_t* dead, float* out) {
  const int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cols, j = i % cols;
    const int64_t src = perm ? perm[j] : j;
    float v = dt == MI355Q_BF16 ? bf16_bits_to_f32(static_cast<const uint16_t*>(w)[r * ldw + src])
                                : static_cast<const float*>(w)[r * ldw + src];
    if (dead && dead[j]) v = 0.f;
    out[i] = v;
  }
}

__global__ void store_weight_kernel(const float* w, int64_t rows, int64_t cols, const int32_t* invperm,
                                    void* out, mi355q_dtype dt, int64_t ld_out, const int8_t* cin,
                                    int8_t* cout) {
  const int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cols, j = i % cols;
    const int64_t src = r * cols + (invperm ? invperm[j] : j);
    const float v = w[src];
    if (dt == MI355Q_BF16)
      static_cast<uint16_t*>(out)[r * ld_out + j] = f32_to_bf16_bits(v);
    else
      static_cast<float*>(out)[r * ld_out + j] = v;
    if (cin && cout) cout[i] = cin[src];
  }
}

inline unsigned grid1d(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace
}  // namespace mi355q

using namespace mi355q;

extern "C" int mi355q_gptq_load_weight(const void* w_dev, mi355q_dtype w_dtype, int64_t rows, int64_t cols,
                                       int64_t ldw, const int32_t* perm_dev, const int32_t* dead_dev,
                                       float* w_work_dev, void* stream) {
  MQ_CHECK_ARG(w_dev && w_work_dev, "gptq_load_weight: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && ldw >= cols, "gptq_load_weight: bad shape");
  hipLaunchKernelGGL(load_weight_kernel, dim3(grid1d(rows * cols)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), w_dev, w_dtype, rows, cols, ldw, perm_dev, dead_dev,
                     w_work_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" size_t mi355q_gptq_sweep_workspace_size(int64_t rows, int64_t cols, int64_t blocksize) {
  (void)cols;
  (void)blocksize;
  return rows > 0 ? (size_t)rows * MAXB * sizeof(float) : 0;
}

extern "C" int mi355q_gptq_sweep(float* w_work_dev, int64_t rows, int64_t cols, const float* hinv_dev,
                                 const float* scale_dev, const float* zp_dev, int64_t ld_scale,
                                 const int32_t* g_idx_dev, int strategy, int block_h, float qmin, float qmax,
                                 int dequant_bf16, int64_t blocksize, int8_t* codes_dev, float* losses_dev,
                                 void* workspace_dev, size_t workspace_bytes, void* stream) {
  MQ_CHECK_ARG(w_work_dev && hinv_dev && scale_dev && codes_dev && losses_dev, "gptq_sweep: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0, "gptq_sweep: bad shape");
  MQ_CHECK_ARG(blocksize > 0, "gptq_sweep: blocksize must be positive");
  MQ_CHECK_ARG(strategy == MI355Q_TENSOR || strategy == MI355Q_CHANNEL || strategy == MI355Q_GROUP ||
                   strategy == MI355Q_BLOCK,
               "Quantization strategy is not supported for GPTQ: %d", strategy);
  MQ_CHECK_ARG((strategy != MI355Q_GROUP && strategy != MI355Q_BLOCK) || g_idx_dev,
               "gptq_sweep: group/block strategies need g_idx");
  MQ_CHECK_ARG(strategy != MI355Q_BLOCK || block_h > 0, "gptq_sweep: block_h must be positive");
  MQ_CHECK_ARG(qmin < qmax && qmin >= -128.f && qmax <= 127.f, "gptq_sweep: integer range must fit int8");
  const size_t need = mi355q_gptq_sweep_workspace_size(rows, cols, blocksize);
  MQ_CHECK_ARG(workspace_dev && workspace_bytes >= need, "gptq_sweep: workspace too small");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  float* err = static_cast<float*>(workspace_dev);
  // the sweep kernel holds at most MAXB columns; larger reference block
  // sizes give the same result up to fp32 rounding of the lazy update, so
  // they are processed in MAXB-wide sub-blocks
  const int64_t B = blocksize < MAXB ? blocksize : MAXB;
  const unsigned nwg = (unsigned)((rows + SW_ROWS - 1) / SW_ROWS);
  for (int64_t i1 = 0; i1 < cols; i1 += B) {
    const int64_t i2 = (i1 + B < cols) ? i1 + B : cols;
    const int count = (int)(i2 - i1);
    hipLaunchKernelGGL(sweep_block_kernel, dim3(nwg), dim3(SW_NT), 0, st, w_work_dev, rows, cols, hinv_dev, i1,
                       count, scale_dev, zp_dev, ld_scale, g_idx_dev, strategy, block_h, qmin, qmax,
                       dequant_bf16, codes_dev, losses_dev, err);
    MQ_LAUNCH_CHECK();
    if (i2 < cols) {
      GemmArgs g{};
      g.A = err; g.lda = MAXB;
      g.B = hinv_dev + i1 * cols + i2; g.ldb = cols;
      g.C = w_work_dev + i2; g.ldc = cols;
      g.M = rows; g.N = cols - i2; g.K = count;
      g.alpha = -1.f; g.beta = 1.f;
      int rc = gemm_f32(g, false, 1, st);
      if (rc) return rc;
    }
  }
  return MI355Q_OK;
}

extern "C" int mi355q_gptq_store_weight(const float* w_work_dev, int64_t rows, int64_t cols,
                                        const int32_t* invperm_dev, void* w_out_dev, mi355q_dtype out_dtype,
                                        int64_t ld_out, const int8_t* codes_in_dev, int8_t* codes_out_dev,
                                        void* stream) {
  MQ_CHECK_ARG(w_work_dev && w_out_dev, "gptq_store_weight: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && ld_out >= cols, "gptq_store_weight: bad shape");
  MQ_CHECK_ARG(codes_out_dev != codes_in_dev || !codes_in_dev, "gptq_store_weight: codes must not alias");
  hipLaunchKernelGGL(store_weight_kernel, dim3(grid1d(rows * cols)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), w_work_dev, rows, cols, invperm_dev, w_out_dev,
                     out_dtype, ld_out, codes_in_dev, codes_out_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}
