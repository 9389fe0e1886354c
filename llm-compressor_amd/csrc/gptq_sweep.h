// GPTQ column sweep kernels (shared by the translation units that
// instantiate them: the 16-lane integer sweep, the sweep that first pulls a
// mid-block's updates, the float-grid sweeps and the 4-lane sweep, each
// compiled on its own so the kernel variants build in parallel).
#pragma once

#include "sweep.h"

#pragma clang fp contract(off)

namespace mi355q {
namespace gsw {

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
// (as a pair (0, f): the conversion leaves bf16(f) in the high half, which is
// its fp32 value, without a separate shift)
__device__ __forceinline__ float bf16_rne(float f) {
  typedef float f32x2v_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
  const f32x2v_t pair = {0.f, f};
  return __builtin_bit_cast(float, __builtin_convertvector(pair, bf16x2v_t));
}

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
  qq = __builtin_amdgcn_fmed3f(qq, qmin, qmax);  // clamp (qmin <= qmax) in one operation
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
// x: the lane's value of slot TO as the previous step's update left it (the
// owner's, column I, is S.w[TO]; the other lanes' values are not used), and
// on return the same for column I + 1, so the owner select stays off the
// serial chain.
template <int TO, int GO, bool FULL, bool BF16, bool ZP, int QK>
__device__ __forceinline__ void sweep_step(SweepState& S, const StepH& p, float& x, int g, int count, float qmin,
                                           float qmax) {
  constexpr int I = SW_G * TO + GO;
  if (!FULL && I >= count) return;
  constexpr int TN = GO == SW_G - 1 ? TO + 1 : TO;  // slot of column I + 1
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
    return upd;
  };
  if (TN < SW_T) x = update(TN);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = TO; t < SW_T; ++t)
    if (t != TN) update(t);
}

// cur: the values of step I, nxt: those of step I + 1
template <int I, bool FULL, bool BF16, bool ZP, int QK>
struct SweepSteps {
  static __device__ __forceinline__ void run(SweepState& S, const float* h1, const float* rdg, int g, int count,
                                             float qmin, float qmax, const StepH& cur, const StepH& nxt, float x) {
    StepH nn;
    load_step<I + 2>(nn, h1, rdg, g);
    sweep_step<I / SW_G, I % SW_G, FULL, BF16, ZP, QK>(S, cur, x, g, count, qmin, qmax);
    SweepSteps<I + 1, FULL, BF16, ZP, QK>::run(S, h1, rdg, g, count, qmin, qmax, nxt, nn, x);
  }
};
template <bool FULL, bool BF16, bool ZP, int QK>
struct SweepSteps<MAXB, FULL, BF16, ZP, QK> {
  static __device__ __forceinline__ void run(SweepState&, const float*, const float*, int, int, float, float,
                                             const StepH&, const StepH&, float) {}
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
  SweepSteps<0, FULL, BF16, ZP, QK>::run(S, h1, rdg, g, count, qmin, qmax, p0, p1, S.w[0]);

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
__device__ __forceinline__ void sweep4_step(Sweep4State& S, const StepH4& p, float& x, int g, float qmin,
                                            float qmax) {
  constexpr int TN = GO == W4_G - 1 ? TO + 1 : TO;  // slot of column I + 1 (x: as in sweep_step)
  float qq, deq;
  quant1<BF16, false, QK_INT>(x, S.s[TO], S.rs[TO], 0.f, qmin, qmax, qq, deq);
  const float err = div_by_recip(x - deq, p.dd, p.rd);
  const float e = quad_bcast<GO>(err);
  auto update = [&](int t) __attribute__((always_inline)) {
    const float upd = S.w[t] - e * p.h[t];
    S.w[t] = t == TO ? (g > GO ? upd : S.w[t]) : upd;
    return upd;
  };
  if (TN < W4_T) x = update(TN);
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
                                             float qmax, const StepH4& cur, float x) {
    StepH4 nn;
    load_step4<I + 1>(nn, h1, rdg, g);
    sweep4_step<I / W4_G, I % W4_G, BF16>(S, cur, x, g, qmin, qmax);
    Sweep4Steps<I + 1, BF16>::run(S, h1, rdg, g, qmin, qmax, nn, x);
  }
};
template <bool BF16>
struct Sweep4Steps<MAXB, BF16> {
  static __device__ __forceinline__ void run(Sweep4State&, const float*, const float*, int, float, float,
                                             const StepH4&, float) {}
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
  Sweep4Steps<0, BF16>::run(S, h1, rdg, g, qmin, qmax, p0, S.w[0]);

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

// Arguments of one block sweep launch (the kernels' parameters).
struct SweepLaunch {
  float* W;
  int64_t rows, cols;
  const float* hinv;
  int64_t i1;
  int count;
  const float* scale;
  const float* zp;
  int64_t ld_scale;
  const int32_t* g_idx;
  int strategy, block_h;
  float qmin, qmax;
  const float* gscale;
  int8_t* codes;
  float* losses;
  float* err;
  int64_t lde;
  int err_col;
  int npre;
  int64_t pre_k0;
  int pre_err_col;
  SweepBatch sb;
};

// 16-lane integer sweeps (whole or partial block, bf16 dequantisation, zero points)
void launch_sweep_int(bool full, bool bf16, bool zp, dim3 grid, hipStream_t st, const SweepLaunch& a);
// 16-lane integer sweeps of whole blocks that first apply a.npre earlier blocks' updates
void launch_sweep_pull(bool bf16, bool zp, dim3 grid, hipStream_t st, const SweepLaunch& a);
// 16-lane sweeps on the fp8 e4m3 / fp4 e2m1 grids (no zero points)
void launch_sweep_float(int qk, bool full, bool bf16, dim3 grid, hipStream_t st, const SweepLaunch& a);
// 4-lane integer sweeps of whole blocks, symmetric scales
void launch_sweep4(bool bf16, dim3 grid, hipStream_t st, const SweepLaunch& a);

}  // namespace gsw
}  // namespace mi355q
