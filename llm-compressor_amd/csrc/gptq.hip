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
#include "gptq_sweep.h"

#include <mutex>

#pragma clang fp contract(off)

namespace mi355q {
namespace {

// One row per blockIdx.y, four consecutive output columns per thread.
// (matrix blockIdx.z of a batch: w + z sw elements, perm + z sp, dead + z cols,
// out + z rows cols)
__global__ void load_weight_kernel(const void* w, mi355q_dtype dt, int64_t rows, int64_t cols, int64_t ldw,
                                   const int32_t* perm, const int32_t* dead, float* out, int64_t sw, int64_t sp) {
  const int64_t z = blockIdx.z;
  w = dt == MI355Q_BF16 ? (const void*)(static_cast<const uint16_t*>(w) + z * sw)
                        : (const void*)(static_cast<const float*>(w) + z * sw);
  if (perm) perm += z * sp;
  if (dead) dead += z * cols;
  out += z * rows * cols;
  const int64_t r = blockIdx.y;
  // whole rows of bf16 without a permutation: 8-byte loads of four values
  const bool vec = !perm && dt == MI355Q_BF16 && (cols & 3) == 0 && (ldw & 3) == 0 &&
                   (reinterpret_cast<uintptr_t>(w) & 7) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(dead) & 15) == 0;
  for (int64_t j4 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; j4 < cols;
       j4 += (int64_t)gridDim.x * blockDim.x * 4) {
    f32x4_t v;
    if (vec) {
      const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(w) + r * ldw + j4);
      v[0] = __uint_as_float(u.x << 16);
      v[1] = __uint_as_float(u.x & 0xffff0000u);
      v[2] = __uint_as_float(u.y << 16);
      v[3] = __uint_as_float(u.y & 0xffff0000u);
      if (dead) {
        const int4 dd = *reinterpret_cast<const int4*>(dead + j4);
        if (dd.x) v[0] = 0.f;
        if (dd.y) v[1] = 0.f;
        if (dd.z) v[2] = 0.f;
        if (dd.w) v[3] = 0.f;
      }
      *reinterpret_cast<f32x4_t*>(out + r * cols + j4) = v;
      continue;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t j = j4 + e < cols ? j4 + e : cols - 1;
      const int64_t src = perm ? perm[j] : j;
      float x = dt == MI355Q_BF16 ? bf16_bits_to_f32(static_cast<const uint16_t*>(w)[r * ldw + src])
                                  : static_cast<const float*>(w)[r * ldw + src];
      v[e] = (dead && dead[j]) ? 0.f : x;
    }
    float* o = out + r * cols + j4;
    if ((cols & 3) == 0) {
      *reinterpret_cast<f32x4_t*>(o) = v;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (j4 + e < cols) o[e] = v[e];
    }
  }
}

// (matrix blockIdx.z: w, cin, cout + z rows cols; invperm + z sp; out + z so)
__global__ void store_weight_kernel(const float* w, int64_t rows, int64_t cols, const int32_t* invperm,
                                    void* out, mi355q_dtype dt, int64_t ld_out, const int8_t* cin,
                                    int8_t* cout, int64_t sp, int64_t so) {
  const int64_t z = blockIdx.z;
  w += z * rows * cols;
  if (invperm) invperm += z * sp;
  out = dt == MI355Q_BF16 ? (void*)(static_cast<uint16_t*>(out) + z * so) : (void*)(static_cast<float*>(out) + z * so);
  if (cin) cin += z * rows * cols;
  if (cout) cout += z * rows * cols;
  const int64_t r = blockIdx.y;
  // whole rows to bf16 without a permutation: 16-byte loads, 8-byte stores
  const bool vec = !invperm && dt == MI355Q_BF16 && (cols & 3) == 0 && (ld_out & 3) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 7) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(cin) & 3) == 0 && (reinterpret_cast<uintptr_t>(cout) & 3) == 0;
  for (int64_t j4 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; j4 < cols;
       j4 += (int64_t)gridDim.x * blockDim.x * 4) {
    if (vec) {
      const f32x4_t v = *reinterpret_cast<const f32x4_t*>(w + r * cols + j4);
      uint2 u;
      u.x = f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16);
      u.y = f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + r * ld_out + j4) = u;
      if (cin && cout)
        *reinterpret_cast<uint32_t*>(cout + r * cols + j4) = *reinterpret_cast<const uint32_t*>(cin + r * cols + j4);
      continue;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t j = j4 + e;
      if (j >= cols) break;
      const int64_t src = r * cols + (invperm ? invperm[j] : j);
      const float v = w[src];
      if (dt == MI355Q_BF16)
        static_cast<uint16_t*>(out)[r * ld_out + j] = f32_to_bf16_bits(v);
      else
        static_cast<float*>(out)[r * ld_out + j] = v;
      if (cin && cout) cout[r * cols + j] = cin[src];
    }
  }
}

inline dim3 grid_rows(int64_t rows, int64_t cols, int64_t batch = 1) {
  int64_t gx = (cols / 4 + 255) / 256;
  if (gx < 1) gx = 1;
  if (gx > 64) gx = 64;
  return dim3((unsigned)gx, (unsigned)rows, (unsigned)batch);
}

}  // namespace
}  // namespace mi355q

using namespace mi355q;
using namespace mi355q::sweep;
using mi355q::gsw::QK_INT;
using mi355q::gsw::QK_FP8;
using mi355q::gsw::QK_FP4;
using mi355q::gsw::SweepBatch;

extern "C" int mi355q_gptq_load_weight_batched(const void* w_dev, mi355q_dtype w_dtype, int64_t rows,
                                               int64_t cols, int64_t ldw, int64_t stride_w, int64_t batch,
                                               const int32_t* perm_dev, int64_t stride_perm,
                                               const int32_t* dead_dev, float* w_work_dev, void* stream) {
  MQ_CHECK_ARG(w_dev && w_work_dev, "gptq_load_weight: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && ldw >= cols && batch > 0, "gptq_load_weight: bad shape");
  MQ_CHECK_ARG(w_dtype == MI355Q_BF16 || w_dtype == MI355Q_F32, "gptq_load_weight: dtype must be bf16 or fp32");
  MQ_CHECK_ARG(rows <= 65535 && batch <= 65535, "gptq_load_weight: at most 65535 rows and matrices");
  MQ_CHECK_ARG(batch == 1 || stride_w >= rows * ldw, "gptq_load_weight: matrices overlap");
  hipLaunchKernelGGL(load_weight_kernel, grid_rows(rows, cols, batch), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), w_dev, w_dtype, rows, cols, ldw, perm_dev, dead_dev,
                     w_work_dev, stride_w, stride_perm);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" int mi355q_gptq_load_weight(const void* w_dev, mi355q_dtype w_dtype, int64_t rows, int64_t cols,
                                       int64_t ldw, const int32_t* perm_dev, const int32_t* dead_dev,
                                       float* w_work_dev, void* stream) {
  return mi355q_gptq_load_weight_batched(w_dev, w_dtype, rows, cols, ldw, 0, 1, perm_dev, 0, dead_dev,
                                         w_work_dev, stream);
}

extern "C" size_t mi355q_gptq_sweep_workspace_size(int64_t rows, int64_t cols, int64_t blocksize) {
  if (rows <= 0 || cols <= 0 || blocksize <= 0) return 0;
  return (size_t)rows * err_cols(cols, blocksize) * sizeof(float);
}

extern "C" int mi355q_gptq_sweep_typed_batched(float* w_work_dev, int64_t rows, int64_t cols, int64_t batch,
                                               const float* hinv_dev, int64_t stride_hinv, const float* scale_dev,
                                               const float* zp_dev, int64_t ld_scale, int64_t stride_scale,
                                               const int32_t* g_idx_dev, int64_t stride_gidx, int strategy,
                                               int block_h, int qtype, float qmin, float qmax,
                                               const float* global_scale_dev, int dequant_bf16, int64_t blocksize,
                                               int8_t* codes_dev, float* losses_dev, void* workspace_dev,
                                               size_t workspace_bytes, void* stream) {
  MQ_CHECK_ARG(w_work_dev && hinv_dev && scale_dev && codes_dev && losses_dev, "gptq_sweep: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && batch > 0 && batch <= 65535, "gptq_sweep: bad shape");
  MQ_CHECK_ARG(blocksize > 0, "gptq_sweep: blocksize must be positive");
  MQ_CHECK_ARG(strategy == MI355Q_TENSOR || strategy == MI355Q_CHANNEL || strategy == MI355Q_GROUP ||
                   strategy == MI355Q_BLOCK,
               "Quantization strategy is not supported for GPTQ: %d", strategy);
  MQ_CHECK_ARG((strategy != MI355Q_GROUP && strategy != MI355Q_BLOCK) || g_idx_dev,
               "gptq_sweep: group/block strategies need g_idx");
  MQ_CHECK_ARG(strategy != MI355Q_BLOCK || block_h > 0, "gptq_sweep: block_h must be positive");
  MQ_CHECK_ARG(qtype == MI355Q_QTYPE_INT || qtype == MI355Q_QTYPE_FP8_E4M3 || qtype == MI355Q_QTYPE_FP4_E2M1,
               "gptq_sweep: unknown value type %d", qtype);
  if (qtype == MI355Q_QTYPE_INT)
    MQ_CHECK_ARG(qmin < qmax && qmin >= -128.f && qmax <= 127.f, "gptq_sweep: integer range must fit int8");
  else
    MQ_CHECK_ARG(!zp_dev && qmin == -qmax && qmax <= (qtype == MI355Q_QTYPE_FP8_E4M3 ? 448.f : 6.f) && qmax > 0.f,
                 "gptq_sweep: float types are symmetric within the type's range");
  MQ_CHECK_ARG(batch == 1 || stride_hinv >= cols * cols, "gptq_sweep: Hinv matrices overlap");
  const size_t need = mi355q_gptq_sweep_workspace_size(rows, cols, blocksize) * (size_t)batch;
  MQ_CHECK_ARG(workspace_dev && workspace_bytes >= need, "gptq_sweep: workspace too small");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  float* err = static_cast<float*>(workspace_dev);
  const int64_t lde = err_cols(cols, blocksize);
  SweepBatch sb{rows * cols, stride_hinv, stride_scale, stride_gidx, rows * cols, rows, rows * lde};
  const int qk = qtype == MI355Q_QTYPE_FP8_E4M3 ? QK_FP8 : qtype == MI355Q_QTYPE_FP4_E2M1 ? QK_FP4 : QK_INT;
  // the sweep kernel holds at most MAXB columns; larger reference block
  // sizes give the same result up to fp32 rounding of the lazy update, so
  // they are processed in MAXB-wide sub-blocks
  const int64_t B = blocksize < MAXB ? blocksize : MAXB;
  const unsigned nwg = (unsigned)((rows + SW_ROWS - 1) / SW_ROWS);
  int dev = 0, ncu = 0;
  MQ_CHECK_HIP(hipGetDevice(&dev));
  MQ_CHECK_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
  // Whole integer blocks with symmetric scales of grids with at least eight
  // 16-lane workgroups per CU take the 4-lane sweep (instruction issue, not
  // latency, bounds the 16-lane sweep there).
  const bool wide = (int64_t)nwg * batch >= 8 * (int64_t)ncu;
  // (npre > 0 only for whole blocks: the schedule pulls only in mid-blocks of whole blocks)
  auto block = [&](int64_t i1, int64_t i2, int64_t s0, int npre, int64_t m0) {
    const int count = (int)(i2 - i1);
    MQ_CHECK_ARG(npre == 0 || (count == MAXB && qk == QK_INT), "gptq_sweep: pulled updates need whole integer blocks");
    const gsw::SweepLaunch a{w_work_dev, rows, cols, hinv_dev, i1, count, scale_dev, zp_dev, ld_scale, g_idx_dev,
                             strategy, block_h, qmin, qmax, global_scale_dev, codes_dev, losses_dev, err, lde,
                             (int)(i1 - s0), npre, m0, (int)(m0 - s0), sb};
    const bool bf16 = dequant_bf16 != 0;
    const dim3 grid(nwg, (unsigned)batch);
    if (qk != QK_INT)
      gsw::launch_sweep_float(qk, count == MAXB, bf16, grid, st, a);
    else if (npre > 0)
      gsw::launch_sweep_pull(bf16, zp_dev != nullptr, grid, st, a);
    else if (wide && count == MAXB && !zp_dev)
      gsw::launch_sweep4(bf16, dim3((unsigned)((rows + gsw::W4_ROWS - 1) / gsw::W4_ROWS), (unsigned)batch), st, a);
    else
      gsw::launch_sweep_int(count == MAXB, bf16, zp_dev != nullptr, grid, st, a);
    MQ_LAUNCH_CHECK();
    return MI355Q_OK;
  };
  auto lazy = [&](int64_t k0, int64_t k1, int64_t s0, int64_t c0, int64_t c1) {
    return lazy_update(w_work_dev, rows, cols, batch, hinv_dev, stride_hinv, err, lde, k0, k1, s0, c0, c1, st);
  };
  // The sweep workgroups apply a mid-block's K = 128 updates themselves for
  // integer values when the sweep leaves the CUs room for it (at most two of
  // its workgroups per CU; with more, the separate products use the CUs
  // better) and the error tile can be read in 16-byte pieces.
  const bool can_pull = qk == QK_INT && (int64_t)nwg * batch <= 2 * (int64_t)ncu && lde % 4 == 0 &&
                        (reinterpret_cast<uintptr_t>(err) & 15) == 0;
  return blocked_schedule_pull(cols, B, can_pull, block, lazy);
}

extern "C" int mi355q_gptq_sweep_batched(float* w_work_dev, int64_t rows, int64_t cols, int64_t batch,
                                         const float* hinv_dev, int64_t stride_hinv, const float* scale_dev,
                                         const float* zp_dev, int64_t ld_scale, int64_t stride_scale,
                                         const int32_t* g_idx_dev, int64_t stride_gidx, int strategy, int block_h,
                                         float qmin, float qmax, int dequant_bf16, int64_t blocksize,
                                         int8_t* codes_dev, float* losses_dev, void* workspace_dev,
                                         size_t workspace_bytes, void* stream) {
  return mi355q_gptq_sweep_typed_batched(w_work_dev, rows, cols, batch, hinv_dev, stride_hinv, scale_dev, zp_dev,
                                         ld_scale, stride_scale, g_idx_dev, stride_gidx, strategy, block_h,
                                         MI355Q_QTYPE_INT, qmin, qmax, nullptr, dequant_bf16, blocksize, codes_dev,
                                         losses_dev, workspace_dev, workspace_bytes, stream);
}

extern "C" int mi355q_gptq_sweep(float* w_work_dev, int64_t rows, int64_t cols, const float* hinv_dev,
                                 const float* scale_dev, const float* zp_dev, int64_t ld_scale,
                                 const int32_t* g_idx_dev, int strategy, int block_h, float qmin, float qmax,
                                 int dequant_bf16, int64_t blocksize, int8_t* codes_dev, float* losses_dev,
                                 void* workspace_dev, size_t workspace_bytes, void* stream) {
  return mi355q_gptq_sweep_batched(w_work_dev, rows, cols, 1, hinv_dev, 0, scale_dev, zp_dev, ld_scale, 0,
                                   g_idx_dev, 0, strategy, block_h, qmin, qmax, dequant_bf16, blocksize,
                                   codes_dev, losses_dev, workspace_dev, workspace_bytes, stream);
}

extern "C" int mi355q_gptq_store_weight_batched(const float* w_work_dev, int64_t rows, int64_t cols,
                                                int64_t batch, const int32_t* invperm_dev, int64_t stride_perm,
                                                void* w_out_dev, mi355q_dtype out_dtype, int64_t ld_out,
                                                int64_t stride_out, const int8_t* codes_in_dev,
                                                int8_t* codes_out_dev, void* stream) {
  MQ_CHECK_ARG(w_work_dev && w_out_dev, "gptq_store_weight: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && ld_out >= cols && batch > 0, "gptq_store_weight: bad shape");
  MQ_CHECK_ARG(out_dtype == MI355Q_BF16 || out_dtype == MI355Q_F32, "gptq_store_weight: dtype must be bf16 or fp32");
  MQ_CHECK_ARG(codes_out_dev != codes_in_dev || !codes_in_dev, "gptq_store_weight: codes must not alias");
  MQ_CHECK_ARG(rows <= 65535 && batch <= 65535, "gptq_store_weight: at most 65535 rows and matrices");
  MQ_CHECK_ARG(batch == 1 || stride_out >= rows * ld_out, "gptq_store_weight: matrices overlap");
  hipLaunchKernelGGL(store_weight_kernel, grid_rows(rows, cols, batch), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), w_work_dev, rows, cols, invperm_dev, w_out_dev,
                     out_dtype, ld_out, codes_in_dev, codes_out_dev, stride_perm, stride_out);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" int mi355q_gptq_store_weight(const float* w_work_dev, int64_t rows, int64_t cols,
                                        const int32_t* invperm_dev, void* w_out_dev, mi355q_dtype out_dtype,
                                        int64_t ld_out, const int8_t* codes_in_dev, int8_t* codes_out_dev,
                                        void* stream) {
  return mi355q_gptq_store_weight_batched(w_work_dev, rows, cols, 1, invperm_dev, 0, w_out_dev, out_dtype,
                                          ld_out, 0, codes_in_dev, codes_out_dev, stream);
}

// ---------------------------------------------------------------- sweep without allocation
// The sweep's error workspace in a device array the library holds: one copy
// per GPU (each device's own address, from hipGetSymbolAddress with that
// device current, looked up once per device), alive until the process ends.
// Every call on a GPU shares that GPU's array, so calls that overlap on one
// GPU (different streams or threads) race; the sweep writes each error
// column before any product reads it, so nothing needs clearing between calls.
static constexpr size_t kSweepScratchBytes = size_t(64) << 20;
static __device__ __align__(256) float scratch[kSweepScratchBytes / sizeof(float)];

namespace {
struct ScratchSlot {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t err = hipSuccess;
};
constexpr int kMaxDevices = 64;
ScratchSlot g_scratch_slot[kMaxDevices];

int sweep_scratch(void** out) {
  int dev = 0;
  MQ_CHECK_HIP(hipGetDevice(&dev));
  MQ_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "gptq_sweep_noalloc: device index %d out of range", dev);
  ScratchSlot& s = g_scratch_slot[dev];
  std::call_once(s.once, [&s] { s.err = hipGetSymbolAddress(&s.ptr, HIP_SYMBOL(scratch)); });
  if (s.err != hipSuccess || s.ptr == nullptr) {
    set_error("gptq_sweep_noalloc: hipGetSymbolAddress of the scratch array failed on device %d: %s", dev,
              hipGetErrorString(s.err));
    return MI355Q_HIP_ERROR;
  }
  *out = s.ptr;
  return MI355Q_OK;
}
}  // namespace

extern "C" size_t mi355q_gptq_sweep_noalloc_max_bytes(void) { return kSweepScratchBytes; }

extern "C" int mi355q_gptq_sweep_noalloc(float* w_work_dev, int64_t rows, int64_t cols, const float* hinv_dev,
                                         const float* scale_dev, const float* zp_dev, int64_t ld_scale,
                                         const int32_t* g_idx_dev, int strategy, int block_h, float qmin, float qmax,
                                         int dequant_bf16, int64_t blocksize, int8_t* codes_dev, float* losses_dev,
                                         void* stream) {
  MQ_CHECK_ARG(rows > 0 && cols > 0 && blocksize > 0, "gptq_sweep_noalloc: bad shape");
  const size_t need = mi355q_gptq_sweep_workspace_size(rows, cols, blocksize);
  MQ_CHECK_ARG(need <= kSweepScratchBytes,
               "gptq_sweep_noalloc: the error workspace of %lld x %lld needs %zu bytes, above the %zu-byte scratch "
               "array (rows * min(1024, cols) fp32); use mi355q_gptq_sweep with a caller workspace",
               (long long)rows, (long long)cols, need, kSweepScratchBytes);
  void* ws = nullptr;
  const int rc = sweep_scratch(&ws);
  if (rc) return rc;
  return mi355q_gptq_sweep(w_work_dev, rows, cols, hinv_dev, scale_dev, zp_dev, ld_scale, g_idx_dev, strategy, block_h,
                           qmin, qmax, dequant_bf16, blocksize, codes_dev, losses_dev, ws, kSweepScratchBytes, stream);
}
