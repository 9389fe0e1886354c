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
#include "sweep.h"

#include <mutex>

#pragma clang fp contract(off)

namespace mi355q {
namespace {

using namespace sweep;

// Per-lane state of the sweep: lane g of a row holds block columns
// SW_G * t + g, t = 0..SW_T-1.
struct SweepState {
  float w[SW_T];   // working values (final once their column is reached)
  float s[SW_T];   // scale of each column
  float rs[SW_T];  // 1 / scale, correctly rounded
  float z[SW_T];   // zero point of each column
};

// bf16 round-to-nearest-even of a finite fp32 value (the gfx950 conversion
// instruction: two operations on the sweep's serial chain instead of four).
__device__ __forceinline__ float bf16_rne(float f) { return (float)(__bf16)f; }

// Value types of the sweep: integers, or the float grids of compressed-
// tensors' round_to_quantized_type (float8_e4m3fn, fp4 e2m1).
enum { QK_INT = 0, QK_FP8 = 1, QK_FP4 = 2 };

// CT quantize / dequantize of one value: qq = round_to_type(clamp(x / s + z)),
// deq = (qq - z) * s, rounded to bf16 when the scale is bf16 (BF16).  For
// QK_INT, qq is the integer code; for the float grids it is the grid value
// (no zero point).  ZP: a zero point (asymmetric); without one, z = 0 and the
// additions drop out (x + 0 = x, and the sign of a zero quotient changes
// neither the code nor the error).
template <bool BF16, bool ZP, int QK>
__device__ __forceinline__ void quant1(float x, float s, float rs, float z, float qmin, float qmax, float& qq,
                                       float& deq) {
  qq = div_by_recip(x, s, rs);
  if (ZP) qq = qq + z;
  qq = fminf(fmaxf(qq, qmin), qmax);
  if (QK == QK_INT) qq = rintf(qq);
  if (QK == QK_FP8) qq = fp8e4m3_rne(qq);
  if (QK == QK_FP4) qq = fp4e2m1_round(qq);
  deq = (ZP ? qq - z : qq) * s;
  if (BF16) deq = bf16_rne(deq);
}

template <int QK>
__device__ __forceinline__ int8_t code_of(float qq) {
  if (QK == QK_FP8) return (int8_t)fp8e4m3_bits(qq);
  if (QK == QK_FP4) return (int8_t)fp4e2m1_bits(qq);
  return (int8_t)qq;
}

// One column of the sweep: column I = SW_G * TO + GO, owned by lane GO of
// each row.  Every lane quantises its own slot TO (only the owner's value is
// column I; the others are discarded), the owner's error is broadcast within
// the row, and each lane updates its later columns.  A lane's slot is final
// from its own step on, so its code, dequantised value and error are
// recomputed once after the sweep instead of being selected at every step.
// The update of the slot holding column I + 1 comes first and ends the
// step's scheduling region: the other updates then interleave with the next
// step's chain, and the reads issued with them (two steps ahead) cannot sink
// into the step that uses them.
template <int TO, int GO, bool FULL, bool BF16, bool ZP, int QK>
__device__ __forceinline__ void sweep_step(SweepState& S, const StepH& p, int g, int count, float qmin,
                                           float qmax) {
  constexpr int I = SW_G * TO + GO;
  if (!FULL && I >= count) return;
  constexpr int TN = GO == SW_G - 1 ? TO + 1 : TO;  // slot of column I + 1
  const float x = S.w[TO];
  float qq, deq;
  quant1<BF16, ZP, QK>(x, S.s[TO], S.rs[TO], S.z[TO], qmin, qmax, qq, deq);
  const float err = div_by_recip(x - deq, p.dd, p.rd);
  const float e = row_bcast<GO>(err);
  auto update = [&](int t) __attribute__((always_inline)) {
    const int col = SW_G * t + g;
    const float upd = S.w[t] - e * p.h[t];
    if (t == TO)
      S.w[t] = g > GO ? upd : S.w[t];
    else if (FULL)
      S.w[t] = upd;
    else
      S.w[t] = col < count ? upd : S.w[t];
  };
  if (TN < SW_T) update(TN);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = TO; t < SW_T; ++t)
    if (t != TN) update(t);
}

// cur: the values of step I, nxt: those of step I + 1
template <int I, bool FULL, bool BF16, bool ZP, int QK>
struct SweepSteps {
  static __device__ __forceinline__ void run(SweepState& S, const float* h1, const float* rdg, int g, int count,
                                             float qmin, float qmax, const StepH& cur, const StepH& nxt) {
    StepH nn;
    load_step<I + 2>(nn, h1, rdg, g);
    sweep_step<I / SW_G, I % SW_G, FULL, BF16, ZP, QK>(S, cur, g, count, qmin, qmax);
    SweepSteps<I + 1, FULL, BF16, ZP, QK>::run(S, h1, rdg, g, count, qmin, qmax, nxt, nn);
  }
};
template <bool FULL, bool BF16, bool ZP, int QK>
struct SweepSteps<MAXB, FULL, BF16, ZP, QK> {
  static __device__ __forceinline__ void run(SweepState&, const float*, const float*, int, int, float, float,
                                             const StepH&, const StepH&) {}
};

// The K = 128 lazy updates of a block's columns from the npre earlier
// blocks of its mid-block, applied by the block's own sweep workgroups
// before the sweep: for p = 0 .. npre-1 in order,
//   W[rows, i1 : i1 + 128] += -(Err[rows, block p] Hinv[block p, i1 : i1 + 128]),
// each product formed as the separate K = 128 GEMM forms it (fp32 MFMA
// 32x32x2, k pairs (4j, 4j+1) on one accumulator and (4j+2, 4j+3) on a
// second, the two added, negated, then added to W), so the result is the
// one the lazy products would give.  The workgroup's 16 rows fill half of
// the MFMA's 32 (rows 16..31 are zero); each wave forms 32 columns.  The
// error tile and the product pass through LDS (the space the Hinv block
// fills afterwards); the Hinv panel goes from global memory straight into
// the B operand.  Rows past the matrix's end hold copies of its last row.
constexpr int PLD = MAXB + 1;  // LDS row stride of the error and product tiles

__device__ __forceinline__ void pull_updates(SweepState& S, float* lds, const float* __restrict__ err, int64_t lde,
                                             int err_col0, const float* __restrict__ hinv, int64_t cols,
                                             int64_t k0, int64_t i1, int64_t row0, int64_t rows, int tid,
                                             int npre) {
  float* ea = lds;             // [32][PLD] error tile, rows 16..31 zero
  float* pt = lds + 32 * PLD;  // [16][PLD] product tile
  const int lane = tid & 63, wave = tid >> 6;
  const int g = tid & (SW_G - 1), rw = tid / SW_G;
  for (int e = tid; e < 16 * PLD; e += SW_NT) ea[16 * PLD + e] = 0.f;
  for (int p = 0; p < npre; ++p) {
    f32x4_t ev[2];
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int e = v * SW_NT + tid, m = e >> 5, c4 = 4 * (e & 31);
      const int64_t r = row0 + m < rows ? row0 + m : rows - 1;
      ev[v] = *reinterpret_cast<const f32x4_t*>(err + r * lde + err_col0 + MAXB * p + c4);
    }
    // B operand: b[j] = Hinv[k0 + 128 p + 2 j + lane / 32][i1 + 32 wave + lane % 32]
    const float* hb = hinv + (k0 + MAXB * p + (lane >> 5)) * cols + i1 + 32 * wave + (lane & 31);
    float b[MAXB / 2];
#pragma unroll
    for (int j = 0; j < MAXB / 2; ++j) b[j] = hb[2 * j * cols];
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int e = v * SW_NT + tid, m = e >> 5, c4 = 4 * (e & 31);
#pragma unroll
      for (int q = 0; q < 4; ++q) ea[m * PLD + c4 + q] = ev[v][q];
    }
    __syncthreads();
    f32x16_t acc0, acc1;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc0[r] = acc1[r] = 0.f;
    const float* pa = ea + (lane & 31) * PLD + (lane >> 5);
#pragma unroll
    for (int kk = 0; kk < MAXB / 2; kk += 2) {
      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(pa[2 * kk], b[kk], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(pa[2 * kk + 2], b[kk + 1], acc1, 0, 0, 0);
    }
    // rows 0..15 of the product: registers r < 8
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int m = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      pt[m * PLD + 32 * wave + (lane & 31)] = -1.f * (acc0[r] + acc1[r]);
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < SW_T; ++t) S.w[t] = 1.f * S.w[t] + pt[rw * PLD + SW_G * t + g];
    __syncthreads();
  }
}

// Element strides between the matrices of a batch (blockIdx.y); zero for a
// shared operand.
struct SweepBatch {
  int64_t w, hinv, scale, gidx, codes, losses, err;
};

// FULL: a whole MAXB-column block; BF16: dequantise in bf16; ZP: zero
// points; QK: value type; PULL: the block first applies the updates from
// the npre earlier blocks of its mid-block (a separate variant: its
// prologue needs more registers than the plain sweep's).  gscale (NULL: 1):
// per-matrix global scale, the effective scale being scale / gscale (CT's
// tensor-group scales).
template <bool FULL, bool BF16, bool ZP, int QK, bool PULL = false>
__global__ __launch_bounds__(SW_NT, 4) void sweep_block_kernel(
    float* __restrict__ W, int64_t rows, int64_t cols, const float* __restrict__ hinv, int64_t i1,
    int count, const float* __restrict__ scale, const float* __restrict__ zp, int64_t ld_scale,
    const int32_t* __restrict__ g_idx, int strategy, int block_h, float qmin, float qmax,
    const float* __restrict__ gscale, int8_t* __restrict__ codes, float* __restrict__ losses,
    float* __restrict__ err_out, int64_t lde, int err_col, int npre, int64_t pre_k0, int pre_err_col,
    SweepBatch sb) {
  __shared__ float h1[HPK];
  __shared__ float rdg[MAXB];  // 1 / Hinv[i][i], correctly rounded
  __shared__ int gsh[MAXB];
  {
    const int64_t b = blockIdx.y;
    W += b * sb.w;
    hinv += b * sb.hinv;
    scale += b * sb.scale;
    if (zp) zp += b * sb.scale;
    if (g_idx) g_idx += b * sb.gidx;
    codes += b * sb.codes;
    losses += b * sb.losses;
    err_out += b * sb.err;
  }
  const int tid = threadIdx.x;
  const int g = tid & (SW_G - 1);
  const int64_t r = (int64_t)blockIdx.x * SW_ROWS + (tid / SW_G);
  const bool live = r < rows;
  const int64_t rr = live ? r : rows - 1;  // clamped row: every address below is in bounds
  const float gsc = gscale ? gscale[blockIdx.y] : 1.f;

  SweepState S;
  // every global load is issued before the first LDS store: the row's
  // working values, this thread's diagonal element and group index, then
  // the block of Hinv (the diagonal and g_idx loads would otherwise wait
  // behind the block's stores, a second memory round trip)
#pragma unroll
  for (int t = 0; t < SW_T; ++t) {
    const int col = min(SW_G * t + g, count - 1);
    S.w[t] = W[rr * cols + i1 + col];
  }
  const bool uses_gidx = strategy == MI355Q_GROUP || strategy == MI355Q_BLOCK;
  const int dcol = tid < count ? tid : count - 1;
  const float diag = hinv[(i1 + dcol) * cols + i1 + dcol];
  const int gval = uses_gidx ? g_idx[i1 + dcol] : 0;
  if constexpr (FULL && PULL)
    if (npre > 0)
      pull_updates(S, h1, err_out, lde, pre_err_col, hinv, cols, pre_k0, i1, (int64_t)blockIdx.x * SW_ROWS, rows,
                   tid, npre);
  load_hinv_block(h1, hinv, cols, i1, count, tid);
  if (tid < MAXB) gsh[tid] = tid < count ? gval : 0;
  if (tid < MAXB) rdg[tid] = tid < count ? 1.f / diag : 1.f;
  __syncthreads();

  int64_t sbase = 0;
  if (strategy == MI355Q_CHANNEL || strategy == MI355Q_GROUP) sbase = rr * ld_scale;
  if (strategy == MI355Q_BLOCK) sbase = (rr / block_h) * ld_scale;
#pragma unroll
  for (int t = 0; t < SW_T; ++t) {
    const int col = min(SW_G * t + g, count - 1);
    const int64_t si = sbase + gsh[col];
    S.s[t] = scale[si] / gsc;   // exact for gsc == 1
    S.rs[t] = 1.f / S.s[t];
    S.z[t] = ZP ? zp[si] : 0.f;
  }

  StepH p0, p1;
  load_step<0>(p0, h1, rdg, g);
  load_step<1>(p1, h1, rdg, g);
  SweepSteps<0, FULL, BF16, ZP, QK>::run(S, h1, rdg, g, count, qmin, qmax, p0, p1);

  // each slot is final: its code, dequantised value, error and loss
  float loss = 0.f;
#pragma unroll
  for (int t = 0; t < SW_T; ++t) {
    const int col = SW_G * t + g;
    const int cc = min(col, count - 1);
    const float dd = h1[hrow(cc)];
    float qq, deq;
    quant1<BF16, ZP, QK>(S.w[t], S.s[t], S.rs[t], S.z[t], qmin, qmax, qq, deq);
    const float diff = S.w[t] - deq;
    const float err = div_by_recip(diff, dd, rdg[cc]);
    if (col < count) {
      loss = loss + diff * diff / (dd * dd);
      if (live) {
        const int64_t c = i1 + col;
        W[r * cols + c] = deq;
        codes[r * cols + c] = code_of<QK>(qq);
        err_out[r * lde + err_col + col] = err;
      }
    }
  }
#pragma unroll
  for (int o = 1; o < SW_G; o <<= 1) loss += __shfl_xor(loss, o, SW_G);
  if (live && g == 0) losses[r] = losses[r] + loss / 2.f;
}

// ---------------------------------------------------------------- wide sweep
// The same sweep with 4 lanes per row (lane g holds block columns 4 t + g,
// t = 0..31) and 64 rows per workgroup, for batches large enough to keep
// every SIMD busy several times over (the MoE projections: 98304 rows and
// more per launch).  There the 16-lane sweep is bound by instruction issue:
// every lane of a row repeats the owner's quantisation, 8 VALU instructions
// per row and column against about 3 here.  Each element sees the same
// operations in the same order as in the 16-lane sweep (quantise, error,
// rounded product, rounded subtract), so the results are the same bits.
// Symmetric scales only: a zero point per slot would not fit the registers
// of three waves per SIMD, which the chain needs to hide its latency.
constexpr int W4_G = 4;                  // lanes per row
constexpr int W4_T = MAXB / W4_G;        // columns per lane
constexpr int W4_ROWS = SW_NT / W4_G;    // rows per workgroup

struct Sweep4State {
  float w[W4_T], s[W4_T], rs[W4_T];
};

struct StepH4 {
  float dd, rd, h[W4_T];
};

template <int I>
__device__ __forceinline__ void load_step4(StepH4& p, const float* h1, const float* rdg, int g) {
  if constexpr (I < MAXB) {
    constexpr int TO = I / W4_G;
    p.dd = h1[hrow(I)];
    p.rd = rdg[I];
    // (col < I reads a neighbouring entry, in bounds, and is never taken)
#pragma unroll
    for (int t = TO; t < W4_T; ++t) p.h[t] = h1[hrow(I) - I + W4_G * t + g];
  }
}

// Broadcast lane L of every group of 4 lanes to the group (DPP quad_perm).
template <int L>
__device__ __forceinline__ float quad_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), L * 0x55, 0xF, 0xF, false));
}

template <int TO, int GO, bool BF16>
__device__ __forceinline__ void sweep4_step(Sweep4State& S, const StepH4& p, int g, float qmin, float qmax) {
  constexpr int TN = GO == W4_G - 1 ? TO + 1 : TO;  // slot of column I + 1
  const float x = S.w[TO];
  float qq, deq;
  quant1<BF16, false, QK_INT>(x, S.s[TO], S.rs[TO], 0.f, qmin, qmax, qq, deq);
  const float err = div_by_recip(x - deq, p.dd, p.rd);
  const float e = quad_bcast<GO>(err);
  auto update = [&](int t) __attribute__((always_inline)) {
    const float upd = S.w[t] - e * p.h[t];
    S.w[t] = t == TO ? (g > GO ? upd : S.w[t]) : upd;
  };
  if (TN < W4_T) update(TN);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = TO; t < W4_T; ++t)
    if (t != TN) update(t);
}

// cur: the Hinv values of step I (read one step ahead: two, as in the
// 16-lane sweep, would leave registers for only two waves per SIMD)
template <int I, bool BF16>
struct Sweep4Steps {
  static __device__ __forceinline__ void run(Sweep4State& S, const float* h1, const float* rdg, int g, float qmin,
                                             float qmax, const StepH4& cur) {
    StepH4 nn;
    load_step4<I + 1>(nn, h1, rdg, g);
    sweep4_step<I / W4_G, I % W4_G, BF16>(S, cur, g, qmin, qmax);
    Sweep4Steps<I + 1, BF16>::run(S, h1, rdg, g, qmin, qmax, nn);
  }
};
template <bool BF16>
struct Sweep4Steps<MAXB, BF16> {
  static __device__ __forceinline__ void run(Sweep4State&, const float*, const float*, int, float, float,
                                             const StepH4&) {}
};

// Whole MAXB-column blocks of integer values with symmetric scales;
// arguments as sweep_block_kernel.
template <bool BF16>
__global__ __launch_bounds__(SW_NT, 3) void sweep4_block_kernel(
    float* __restrict__ W, int64_t rows, int64_t cols, const float* __restrict__ hinv, int64_t i1,
    const float* __restrict__ scale, int64_t ld_scale,
    const int32_t* __restrict__ g_idx, int strategy, int block_h, float qmin, float qmax,
    const float* __restrict__ gscale, int8_t* __restrict__ codes, float* __restrict__ losses,
    float* __restrict__ err_out, int64_t lde, int err_col, SweepBatch sb) {
  __shared__ float h1[HPK];
  __shared__ float rdg[MAXB];
  __shared__ int gsh[MAXB];
  {
    const int64_t b = blockIdx.y;
    W += b * sb.w;
    hinv += b * sb.hinv;
    scale += b * sb.scale;
    if (g_idx) g_idx += b * sb.gidx;
    codes += b * sb.codes;
    losses += b * sb.losses;
    err_out += b * sb.err;
  }
  const int tid = threadIdx.x;
  const int g = tid & (W4_G - 1);
  const int64_t r = (int64_t)blockIdx.x * W4_ROWS + (tid / W4_G);
  const bool live = r < rows;
  const int64_t rr = live ? r : rows - 1;
  const float gsc = gscale ? gscale[blockIdx.y] : 1.f;

  Sweep4State S;
#pragma unroll
  for (int t = 0; t < W4_T; ++t) S.w[t] = W[rr * cols + i1 + W4_G * t + g];
  const bool uses_gidx = strategy == MI355Q_GROUP || strategy == MI355Q_BLOCK;
  const float diag = hinv[(i1 + (tid & (MAXB - 1))) * cols + i1 + (tid & (MAXB - 1))];
  const int gval = uses_gidx ? g_idx[i1 + (tid & (MAXB - 1))] : 0;
  load_hinv_block(h1, hinv, cols, i1, MAXB, tid);
  if (tid < MAXB) gsh[tid] = gval;
  if (tid < MAXB) rdg[tid] = 1.f / diag;
  __syncthreads();

  int64_t sbase = 0;
  if (strategy == MI355Q_CHANNEL || strategy == MI355Q_GROUP) sbase = rr * ld_scale;
  if (strategy == MI355Q_BLOCK) sbase = (rr / block_h) * ld_scale;
#pragma unroll
  for (int t = 0; t < W4_T; ++t) {
    const int64_t si = sbase + gsh[W4_G * t + g];
    S.s[t] = scale[si] / gsc;
    S.rs[t] = 1.f / S.s[t];
  }

  StepH4 p0;
  load_step4<0>(p0, h1, rdg, g);
  Sweep4Steps<0, BF16>::run(S, h1, rdg, g, qmin, qmax, p0);

  float loss = 0.f;
#pragma unroll
  for (int t = 0; t < W4_T; ++t) {
    const int col = W4_G * t + g;
    const float dd = h1[hrow(col)];
    float qq, deq;
    quant1<BF16, false, QK_INT>(S.w[t], S.s[t], S.rs[t], 0.f, qmin, qmax, qq, deq);
    const float diff = S.w[t] - deq;
    const float err = div_by_recip(diff, dd, rdg[col]);
    loss = loss + diff * diff / (dd * dd);
    if (live) {
      const int64_t c = i1 + col;
      W[r * cols + c] = deq;
      codes[r * cols + c] = code_of<QK_INT>(qq);
      err_out[r * lde + err_col + col] = err;
    }
  }
#pragma unroll
  for (int o = 1; o < W4_G; o <<= 1) loss += __shfl_xor(loss, o, W4_G);
  if (live && g == 0) losses[r] = losses[r] + loss / 2.f;
}

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

// the kernel variant for (whole block, bf16 dequantisation, zero points,
// pulled updates: integer values only)
template <class... A>
void launch_sweep(bool full, bool bf16, bool zp, int qk, bool pull, dim3 grid, hipStream_t st, A... args) {
  auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(SW_NT), 0, st, args...); };
  if (qk == QK_INT) {
    if (full && pull) {
      if (bf16) zp ? go(sweep_block_kernel<true, true, true, QK_INT, true>) : go(sweep_block_kernel<true, true, false, QK_INT, true>);
      else      zp ? go(sweep_block_kernel<true, false, true, QK_INT, true>) : go(sweep_block_kernel<true, false, false, QK_INT, true>);
    } else if (full) {
      if (bf16) zp ? go(sweep_block_kernel<true, true, true, QK_INT>) : go(sweep_block_kernel<true, true, false, QK_INT>);
      else      zp ? go(sweep_block_kernel<true, false, true, QK_INT>) : go(sweep_block_kernel<true, false, false, QK_INT>);
    } else {
      if (bf16) zp ? go(sweep_block_kernel<false, true, true, QK_INT>) : go(sweep_block_kernel<false, true, false, QK_INT>);
      else      zp ? go(sweep_block_kernel<false, false, true, QK_INT>) : go(sweep_block_kernel<false, false, false, QK_INT>);
    }
  } else if (qk == QK_FP8) {
    if (full) bf16 ? go(sweep_block_kernel<true, true, false, QK_FP8>) : go(sweep_block_kernel<true, false, false, QK_FP8>);
    else      bf16 ? go(sweep_block_kernel<false, true, false, QK_FP8>) : go(sweep_block_kernel<false, false, false, QK_FP8>);
  } else {
    if (full) bf16 ? go(sweep_block_kernel<true, true, false, QK_FP4>) : go(sweep_block_kernel<true, false, false, QK_FP4>);
    else      bf16 ? go(sweep_block_kernel<false, true, false, QK_FP4>) : go(sweep_block_kernel<false, false, false, QK_FP4>);
  }
}

}  // namespace
}  // namespace mi355q

using namespace mi355q;
using namespace mi355q::sweep;

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
    if (wide && count == MAXB && qk == QK_INT && !zp_dev && npre == 0) {
      const dim3 grid4((unsigned)((rows + W4_ROWS - 1) / W4_ROWS), (unsigned)batch);
      auto go4 = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid4, dim3(SW_NT), 0, st, w_work_dev, rows, cols, hinv_dev, i1, scale_dev,
                           ld_scale, g_idx_dev, strategy, block_h, qmin, qmax, global_scale_dev, codes_dev,
                           losses_dev, err, lde, (int)(i1 - s0), sb);
      };
      dequant_bf16 ? go4(sweep4_block_kernel<true>) : go4(sweep4_block_kernel<false>);
      MQ_LAUNCH_CHECK();
      return MI355Q_OK;
    }
    launch_sweep(count == MAXB, dequant_bf16 != 0, zp_dev != nullptr, qk, npre > 0, dim3(nwg, (unsigned)batch), st,
                 w_work_dev, rows, cols, hinv_dev, i1, count, scale_dev, zp_dev, ld_scale, g_idx_dev, strategy,
                 block_h, qmin, qmax, global_scale_dev, codes_dev, losses_dev, err, lde, (int)(i1 - s0), npre, m0,
                 (int)(m0 - s0), sb);
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
