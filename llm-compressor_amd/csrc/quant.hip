// Observers, qparams, quantize and pack kernels (HBM-bound) for gfx950.
//
// Reference behaviour: observers/min_max.py:16-110 (min/max statistics),
// observers/helpers.py:63-131 (per-strategy flattening),
// modifiers/quantization/calibration.py:86-157 (observe / update_qparams),
// utils/pack_int4_to_int8.py:13-28 (nibble pack) and the compressed-tensors
// quantize / pack_to_int32 / MXFP4 / fp8 arithmetic those call.  Every
// kernel reads its input once with 16-byte loads where the layout allows.
#include "common.h"

#pragma clang fp contract(off)

namespace mi355q {
namespace {

constexpr int NT = 256;

// ---------------------------------------------------------------- helpers
__device__ __forceinline__ float load_elem(const void* x, mi355q_dtype dt, int64_t i) {
  return dt == MI355Q_BF16 ? bf16_bits_to_f32(static_cast<const uint16_t*>(x)[i])
                           : static_cast<const float*>(x)[i];
}

// Total order on floats as signed ints, for atomic min/max.
__device__ __forceinline__ int f2ord(float f) {
  int i = __float_as_int(f);
  return i >= 0 ? i : i ^ 0x7fffffff;
}
__device__ __forceinline__ float ord2f(int i) { return __int_as_float(i >= 0 ? i : i ^ 0x7fffffff); }

__device__ __forceinline__ float warp_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float warp_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Scale index for element (r, c) under a strategy.
__device__ __forceinline__ int64_t scale_index(int strategy, int64_t r, int64_t c, int64_t ld_scale,
                                               const int32_t* g_idx, int64_t group_size, int bh,
                                               int bw) {
  switch (strategy) {
    case MI355Q_TENSOR: return 0;
    case MI355Q_CHANNEL:
    case MI355Q_TOKEN: return r * ld_scale;
    case MI355Q_GROUP: return r * ld_scale + (g_idx ? (int64_t)g_idx[c] : c / group_size);
    case MI355Q_BLOCK: return (r / bh) * ld_scale + (g_idx ? (int64_t)g_idx[c] : c / bw);
  }
  return 0;
}

// ---------------------------------------------------------------- min / max
// One workgroup per row (CHANNEL / TOKEN) or the whole tensor (TENSOR, via
// ordered-int atomics on pre-initialised outputs).
__global__ void minmax_rows_kernel(const void* x, mi355q_dtype dt, int64_t rows, int64_t cols,
                                   int64_t ldx, float* mn_out, float* mx_out, int tensor_mode) {
  __shared__ float smn[NT / 64], smx[NT / 64];
  const int64_t r = blockIdx.x;
  if (r >= rows) return;
  float mn = INFINITY, mx = -INFINITY;
  const int64_t base = r * ldx;
  const bool vec = dt == MI355Q_BF16 && (cols % 8 == 0) && (ldx % 8 == 0) &&
                   ((reinterpret_cast<uintptr_t>(x) & 15) == 0);
  if (vec) {
    const u32x4_t* p = reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(x) + base);
    for (int64_t c = threadIdx.x; c < cols / 8; c += NT) {
      u32x4_t v = p[c];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float a = __uint_as_float(v[q] << 16), b = __uint_as_float(v[q] & 0xffff0000u);
        mn = fminf(mn, fminf(a, b));
        mx = fmaxf(mx, fmaxf(a, b));
      }
    }
  } else {
    for (int64_t c = threadIdx.x; c < cols; c += NT) {
      float v = load_elem(x, dt, base + c);
      mn = fminf(mn, v);
      mx = fmaxf(mx, v);
    }
  }
  mn = warp_min(mn);
  mx = warp_max(mx);
  if ((threadIdx.x & 63) == 0) {
    smn[threadIdx.x >> 6] = mn;
    smx[threadIdx.x >> 6] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < NT / 64; ++w) {
      mn = fminf(mn, smn[w]);
      mx = fmaxf(mx, smx[w]);
    }
    if (tensor_mode) {
      atomicMin(reinterpret_cast<int*>(mn_out), f2ord(mn));
      atomicMax(reinterpret_cast<int*>(mx_out), f2ord(mx));
    } else {
      mn_out[r] = mn;
      mx_out[r] = mx;
    }
  }
}

__global__ void minmax_init_kernel(float* mn, float* mx) {
  reinterpret_cast<int*>(mn)[0] = f2ord(INFINITY);
  reinterpret_cast<int*>(mx)[0] = f2ord(-INFINITY);
}
__global__ void minmax_finish_kernel(float* mn, float* mx) {
  mn[0] = ord2f(reinterpret_cast<int*>(mn)[0]);
  mx[0] = ord2f(reinterpret_cast<int*>(mx)[0]);
}

// Groups along columns, vector path: LPG lanes x 8 elements per group.
template <int LPG>
__global__ void minmax_group_vec_kernel(const uint16_t* x, int64_t rows, int64_t cols, int64_t ldx,
                                        float* mn_out, float* mx_out) {
  const int64_t chunks_per_row = cols / 8;
  const int64_t total = rows * chunks_per_row;
  const int64_t ngroups = cols / (8 * LPG);
  for (int64_t c = (int64_t)blockIdx.x * NT + threadIdx.x; c - (threadIdx.x & (LPG - 1)) < total;
       c += (int64_t)gridDim.x * NT) {
    float mn = INFINITY, mx = -INFINITY;
    if (c < total) {
      const int64_t r = c / chunks_per_row, k = c % chunks_per_row;
      u32x4_t v = *reinterpret_cast<const u32x4_t*>(x + r * ldx + 8 * k);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float a = __uint_as_float(v[q] << 16), b = __uint_as_float(v[q] & 0xffff0000u);
        mn = fminf(mn, fminf(a, b));
        mx = fmaxf(mx, fmaxf(a, b));
      }
    }
#pragma unroll
    for (int o = 1; o < LPG; o <<= 1) {
      mn = fminf(mn, __shfl_xor(mn, o));
      mx = fmaxf(mx, __shfl_xor(mx, o));
    }
    if (c < total && (threadIdx.x & (LPG - 1)) == 0) {
      const int64_t r = c / chunks_per_row, k = c % chunks_per_row;
      const int64_t g = k / LPG;
      mn_out[r * ngroups + g] = mn;
      mx_out[r * ngroups + g] = mx;
    }
  }
}

// Generic groups / blocks: one thread per output cell, zero padding counted.
__global__ void minmax_cells_kernel(const void* x, mi355q_dtype dt, int64_t rows, int64_t cols,
                                    int64_t ldx, int64_t cell_h, int64_t cell_w, int64_t ncr,
                                    int64_t ncc, float* mn_out, float* mx_out) {
  const int64_t cell = (int64_t)blockIdx.x * NT + threadIdx.x;
  if (cell >= ncr * ncc) return;
  const int64_t cr = cell / ncc, cc = cell % ncc;
  float mn = INFINITY, mx = -INFINITY;
  for (int64_t i = 0; i < cell_h; ++i) {
    const int64_t r = cr * cell_h + i;
    for (int64_t j = 0; j < cell_w; ++j) {
      const int64_t c = cc * cell_w + j;
      float v = (r < rows && c < cols) ? load_elem(x, dt, r * ldx + c) : 0.f;
      mn = fminf(mn, v);
      mx = fmaxf(mx, v);
    }
  }
  mn_out[cell] = mn;
  mx_out[cell] = mx;
}

// ---------------------------------------------------------------- qparams
__device__ __forceinline__ float rnd(float v, bool bf16) { return bf16 ? round_to_bf16(v) : v; }

// CT calculate_qparams of one (min, max) pair in the statistics dtype (b:
// bf16, every operation rounded to it) or fp32.
__device__ __forceinline__ void qparams_one(float mn, float mx, float qmin, float qmax, bool symmetric, bool strict,
                                            bool b, float& scale, float& zp) {
  mn = fminf(mn, 0.f);
  mx = fmaxf(mx, 0.f);
  zp = 0.f;
  if (strict) {
    float mvp = fmaxf(fabsf(mn), fabsf(mx));
    scale = fmaxf(mvp / qmax, 1e-8f);
    scale = rnd(scale, b);
  } else if (symmetric) {
    float mvp = fmaxf(fabsf(mn), fabsf(mx));
    scale = rnd(mvp / ((qmax - qmin) / 2.f), b);
  } else {
    scale = rnd(rnd(mx - mn, b) / (qmax - qmin), b);
    zp = rnd(qmin - rnd(mn / scale, b), b);
    zp = fminf(fmaxf(zp, qmin), qmax);
    zp = rintf(zp);
  }
  if (!strict && scale == 0.f) scale = b ? 0.0078125f : 1.1920928955078125e-07f;
}

__global__ void qparams_kernel(const float* mn_in, const float* mx_in, int64_t n, float qmin, float qmax,
                               int symmetric, int strict, int bf16_scale, float* scale_out,
                               float* zp_out) {
  const int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x;
  if (i >= n) return;
  float scale, zp;
  qparams_one(mn_in[i], mx_in[i], qmin, qmax, symmetric != 0, strict != 0, bf16_scale != 0, scale, zp);
  scale_out[i] = scale;
  zp_out[i] = zp;
}

// e8m0 exponent byte of an MX group scale from the group absmax (rule:
// MI355Q_MX_RULE_CT / _OCP)
__device__ __forceinline__ int mx_exponent(float amax, int rule) {
  // amax is a bf16 value (exact in fp32), >= 0
  if (amax == 0.f) return 0;
  int e;
  if (rule == MI355Q_MX_RULE_CT) {
    uint32_t bits = (__float_as_uint(amax) >> 16) & 0xffffu;
    bits = (bits + 32u) & 0xff80u;
    e = (int)((bits >> 7) & 0xffu) - 127;
  } else {
    uint32_t u = __float_as_uint(amax);
    int ef = (int)((u >> 23) & 0xffu);
    if (ef == 0) {  // fp32 subnormal (not reachable from bf16 normal data)
      e = -127 - __clz(u & 0x7fffffu) + 9 - 1;
    } else {
      e = ef - 127;
    }
  }
  int e8 = e + 127 - 2;
  return e8 < 0 ? 0 : (e8 > 254 ? 254 : e8);
}

// ---------------------------------------------------------------- MSE observer
// observers/mse_quant.py:48-130,244-273.  A matrix is split into cells of
// cell_rows x cell_cols (clipped at the edges, row-major) - a group, a channel,
// a block or the whole tensor.  Candidate i < T shrinks the cell's min / max by
// p = 1 - i / grid; its error is sum |fq(x) - x|^norm with every operation in
// the observed dtype (bf16: rounded after each op, the sum accumulated in fp32
// and rounded once).  The first candidate with the smallest error wins, over
// the steps before the first run of `patience` steps in which no cell
// improved.
struct MseArgs {
  const void* x;
  int64_t rows, cols, ldx;
  int64_t ch, cw, ncr, ncc;
  float qmin, qmax;
  int T;
  double grid;
  float norm;
  const float* mn;
  const float* mx;
  const float* imp;  // weighted (imatrix) mode: per-column importance, or NULL
  int mx_rule;       // MX candidate scales (FQ == 3): the e8m0 rule
};

// bf16 rounding (hardware round-to-nearest-even) when the observed dtype is bf16
template <bool B>
__device__ __forceinline__ float rb(float v) { return B ? (float)(__bf16)v : v; }

// torch's pow(tensor, scalar) in the tensor's dtype: 2 as a product, 3 as two
// products (each rounded to bf16 for a bf16 tensor), 0.5 as a square root;
// otherwise pow with the exponent first cast to the tensor's dtype (a bf16
// tensor raises to bf16(norm), e.g. 2.40625 for 2.4).  The caller rounds the
// result to the dtype.
template <bool B>
__device__ __forceinline__ float pow_norm(float a, float norm) {
  if (norm == 2.f) return a * a;
  if (norm == 3.f) return B ? rb<true>(a * a) * a : a * a * a;
  if (norm == 0.5f) return sqrtf(a);
  return powf(a, B ? rb<true>(norm) : norm);
}

// A bf16 error |fq(x) - x| takes one of 2^15 non-negative bf16 values, so its
// rounded power is read from a table of all of them (bf16 bits, 64 KB, held
// in LDS) built once per call with pow_norm.
constexpr int POW_TAB = 1 << 15;

__global__ void mse_pow_table_kernel(float norm, uint16_t* tab) {
  const int i = blockIdx.x * NT + threadIdx.x;
  if (i < POW_TAB) tab[i] = f32_to_bf16_bits(pow_norm<true>(__uint_as_float((uint32_t)i << 16), norm));
}

__device__ __forceinline__ float shrink_p(int i, double grid) { return (float)(1.0 - (double)i / grid); }

// |fq(x) - x|^norm of one value with CT fake_quantize (per-token scale s,
// zero point z; rs = 1 / s correctly rounded), each step in the observed
// dtype.  bf16: the quotient from the reciprocal with one FMA residual step
// (the correctly rounded fp32 quotient, then rounded to bf16 as torch does)
// and the power from the LDS table.
// IM (imatrix observer): |fq(x) - x| and its power in fp32 (fq in the
// observed dtype), times the column's importance w.
// FQ: the value grid after the clamp: 0 integers (rint), 1 fp8 e4m3 (round
// to nearest even, as the cast to float8_e4m3fn does), 2 fp4 e2m1 (CT
// cast_to_fp4's nearest value, ties to even), 3 e2m1 with MX (power of two)
// scales.
template <bool B, bool ZP, bool IM, int FQ = 0>
__device__ __forceinline__ float mse_term(float v, float s, float rs, float z, float qmin, float qmax, float norm,
                                          const uint16_t* tab, float w) {
  float t;
  if (B) {
    const float q0 = v * rs;
    t = rb<true>(fmaf(fmaf(-s, q0, v), rs, q0));
  } else {
    t = v / s;
  }
  if (ZP) t = rb<B>(t + z);
  t = fminf(fmaxf(t, qmin), qmax);
  t = FQ == 1 ? fp8e4m3_rne(t) : FQ >= 2 ? fp4e2m1_round(t) : rintf(t);
  if (ZP) t = rb<B>(t - z);
  if (IM) return pow_norm<false>(fabsf(rb<B>(t * s) - v), norm) * w;
  const float d = fabsf(rb<B>(rb<B>(t * s) - v));
  if (B) return __uint_as_float((uint32_t)tab[__float_as_uint(d) >> 16] << 16);
  return pow_norm<false>(d, norm);
}

// A candidate's scale and zero point from its shrunk min / max: CT
// calculate_qparams in the observed dtype, or for MX the power of two of the
// e8m0 exponent of max(|min|, |max|) (as a bf16 value for the CT rule).
template <bool B, bool ZP, int FQ>
__device__ __forceinline__ void cand_qparams(const MseArgs& a, float mn, float mx, float& s, float& z) {
  if constexpr (FQ == 3) {
    const float amax = fmaxf(fabsf(fminf(mn, 0.f)), fmaxf(mx, 0.f));
    const int e8 = mx_exponent(a.mx_rule == MI355Q_MX_RULE_CT ? round_to_bf16(amax) : amax, a.mx_rule);
    s = e8 > 0 ? __uint_as_float((uint32_t)e8 << 23) : __uint_as_float(0x00400000u);  // 2^(e8 - 127)
    z = 0.f;
  } else {
    qparams_one(mn, mx, a.qmin, a.qmax, !ZP, false, B, s, z);
  }
}

__device__ __forceinline__ void cell_geom(const MseArgs& a, int64_t cell, int64_t& r0, int64_t& c0, int64_t& cwe,
                                          int64_t& n) {
  const int64_t cr = cell / a.ncc, cq = cell % a.ncc;
  r0 = cr * a.ch;
  c0 = cq * a.cw;
  cwe = min(a.cw, a.cols - c0);
  n = cwe * min(a.ch, a.rows - r0);
}

template <bool B>
__device__ __forceinline__ void load_pow_table(uint16_t* tab, const uint16_t* table) {
  if (B) {
    for (int i = threadIdx.x; i < POW_TAB / 8; i += NT)
      reinterpret_cast<uint4*>(tab)[i] = reinterpret_cast<const uint4*>(table)[i];
    __syncthreads();
  }
}

// Cells of at most 8 * LG <= 512 values: LG lanes per cell, 8 values per
// lane; workgroups loop over the cells (the table is loaded once each).
template <bool B, bool ZP, bool IM, int FQ = 0>
__global__ __launch_bounds__(NT) void mse_err_small_kernel(MseArgs a, int lg_log2, const uint16_t* table,
                                                           float* err) {
  constexpr bool TAB = B && !IM;
  __shared__ uint16_t tab[TAB ? POW_TAB : 8];
  load_pow_table<TAB>(tab, table);
  const int LG = 1 << lg_log2, per_wg = NT >> lg_log2;
  const int64_t ncells = a.ncr * a.ncc;
  const int l = threadIdx.x & (LG - 1);
  for (int64_t base = (int64_t)blockIdx.x * per_wg; base < ncells; base += (int64_t)gridDim.x * per_wg) {
    const int64_t cell_raw = base + (threadIdx.x >> lg_log2);
    const bool live = cell_raw < ncells;
    const int64_t cell = live ? cell_raw : ncells - 1;
    int64_t r0, c0, cwe, n;
    cell_geom(a, cell, r0, c0, cwe, n);
    float v[8], w[8];
    bool ok[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t e = l + (int64_t)k * LG;
      ok[k] = e < n;
      const int64_t ee = ok[k] ? e : 0;
      v[k] = load_elem(a.x, B ? MI355Q_BF16 : MI355Q_F32, (r0 + ee / cwe) * a.ldx + c0 + ee % cwe);
      w[k] = (IM && a.imp) ? a.imp[c0 + ee % cwe] : 1.f;
    }
    const float mn = a.mn[cell], mx = a.mx[cell];
    for (int i = 0; i < a.T; ++i) {
      const float p = shrink_p(i, a.grid);
      float s, z;
      cand_qparams<B, ZP, FQ>(a, rb<B>(mn * p), rb<B>(mx * p), s, z);
      const float rs = 1.f / s;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (ok[k]) acc += mse_term<B, ZP, IM, FQ>(v[k], s, rs, z, a.qmin, a.qmax, a.norm, tab, w[k]);
      for (int o = 1; o < LG; o <<= 1) acc += __shfl_xor(acc, o, LG);
      if (live && l == 0) err[cell * a.T + i] = IM ? acc : rb<B>(acc);
    }
  }
}

// Larger cells: chunks of 16 * NT values, one fp32 partial sum per chunk and
// candidate (summed in chunk order by mse_flags_kernel); workgroups loop over
// the (cell, chunk) items.
template <bool B, bool ZP, bool IM, int FQ = 0>
__global__ __launch_bounds__(NT) void mse_err_large_kernel(MseArgs a, int64_t nchunk, const uint16_t* table,
                                                           float* part) {
  constexpr bool TAB = B && !IM;
  __shared__ uint16_t tab[TAB ? POW_TAB : 8];
  __shared__ float red[NT / 64];
  load_pow_table<TAB>(tab, table);
  const int tid = threadIdx.x;
  const int64_t nitems = a.ncr * a.ncc * nchunk;
  for (int64_t item = blockIdx.x; item < nitems; item += gridDim.x) {
    const int64_t cell = item / nchunk, chunk = item % nchunk;
    int64_t r0, c0, cwe, n;
    cell_geom(a, cell, r0, c0, cwe, n);
    float v[16], w[16];
    bool ok[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int64_t e = chunk * (16 * NT) + (int64_t)k * NT + tid;
      ok[k] = e < n;
      const int64_t ee = ok[k] ? e : 0;
      v[k] = load_elem(a.x, B ? MI355Q_BF16 : MI355Q_F32, (r0 + ee / cwe) * a.ldx + c0 + ee % cwe);
      w[k] = (IM && a.imp) ? a.imp[c0 + ee % cwe] : 1.f;
    }
    const float mn = a.mn[cell], mx = a.mx[cell];
    for (int i = 0; i < a.T; ++i) {
      const float p = shrink_p(i, a.grid);
      float s, z;
      cand_qparams<B, ZP, FQ>(a, rb<B>(mn * p), rb<B>(mx * p), s, z);
      const float rs = 1.f / s;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < 16; ++k)
        if (ok[k]) acc += mse_term<B, ZP, IM, FQ>(v[k], s, rs, z, a.qmin, a.qmax, a.norm, tab, w[k]);
      for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
      if ((tid & 63) == 0) red[tid >> 6] = acc;
      __syncthreads();
      if (tid == 0) part[(cell * nchunk + chunk) * a.T + i] = ((red[0] + red[1]) + red[2]) + red[3];
      __syncthreads();
    }
  }
}

// Per cell: the errors (from the chunk partials when nchunk > 0) and, for
// every step, whether any cell improved its best error at it.
// round_sum: the error sums are rounded to bf16 (the uniform MSE observer on
// bf16 values); best0: the largest value of the error dtype.
__global__ void mse_flags_kernel(const float* part, int64_t nchunk, float* err, int64_t ncells, int T, int* any,
                                 int round_sum, float best0) {
  const int64_t cell_raw = (int64_t)blockIdx.x * NT + threadIdx.x;
  const bool live = cell_raw < ncells;
  const int64_t cell = live ? cell_raw : ncells - 1;
  float best = best0;
  for (int i = 0; i < T; ++i) {
    float e;
    if (nchunk > 0) {
      float acc = 0.f;
      for (int64_t c = 0; c < nchunk; ++c) acc += part[(cell * nchunk + c) * T + i];
      e = round_sum ? rb<true>(acc) : acc;
      if (live) err[cell * T + i] = e;
    } else {
      e = err[cell * T + i];
    }
    const bool imp = live && e < best;
    if (imp) best = e;
    if (__any(imp) && (threadIdx.x & 63) == 0) any[i] = 1;
  }
}

// The steps the reference evaluates end at the first run of `patience`
// steps without an improvement anywhere (never when stop_zero_never and
// patience == 0, as the imatrix observer); each cell takes its first best
// candidate among them.
template <bool B>
__global__ void mse_select_kernel(const float* err, const int* any, int64_t ncells, int T, int patience,
                                  int stop_zero_never, float best0, double grid, const float* mn, const float* mx,
                                  float* mn_out, float* mx_out) {
  const int64_t cell = (int64_t)blockIdx.x * NT + threadIdx.x;
  if (cell >= ncells) return;
  int last = T - 1, cnt = 0;
  if (!(stop_zero_never && patience == 0)) {
    for (int i = 0; i < T; ++i) {
      if (any[i]) {
        cnt = 0;
      } else if (++cnt >= patience) {
        last = i;
        break;
      }
    }
  }
  float best = best0;
  int bi = -1;
  for (int i = 0; i <= last; ++i) {
    const float e = err[cell * T + i];
    if (e < best) {
      best = e;
      bi = i;
    }
  }
  if (bi >= 0) {
    const float p = shrink_p(bi, grid);
    mn_out[cell] = rb<B>(mn[cell] * p);
    mx_out[cell] = rb<B>(mx[cell] * p);
  } else {
    mn_out[cell] = mn[cell];
    mx_out[cell] = mx[cell];
  }
}

__global__ void fill_i32_kernel(int* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

struct MsePlan {
  int64_t ncells, nchunk;
  int lg_log2;        // small path: log2 lanes per cell; -1: large path
  size_t off_part, off_any, off_tab, total;
};

MsePlan plan_mse(int64_t rows, int64_t cols, int64_t ch, int64_t cw, int T) {
  MsePlan pl{};
  pl.ncells = ((rows + ch - 1) / ch) * ((cols + cw - 1) / cw);
  const int64_t nmax = min(ch, rows) * min(cw, cols);
  pl.lg_log2 = -1;
  for (int lg = 0; lg <= 6; ++lg)
    if (8 * (int64_t(1) << lg) >= nmax) {
      pl.lg_log2 = lg;
      break;
    }
  pl.nchunk = pl.lg_log2 >= 0 ? 0 : (nmax + 16 * NT - 1) / (16 * NT);
  auto align = [](size_t v) { return (v + 255) & ~(size_t)255; };
  size_t off = align((size_t)pl.ncells * T * sizeof(float));
  pl.off_part = off;
  off = align(off + (size_t)pl.ncells * pl.nchunk * T * sizeof(float));
  pl.off_any = off;
  off = align(off + (size_t)T * sizeof(int));
  pl.off_tab = off;
  pl.total = align(off + (size_t)POW_TAB * sizeof(uint16_t));
  return pl;
}

// ---------------------------------------------------------------- int quantize
__global__ void quantize_int_kernel(const void* x, mi355q_dtype dt, int64_t rows, int64_t cols,
                                    int64_t ldx, const float* scale, const float* zp,
                                    int64_t ld_scale, const int32_t* g_idx, int strategy,
                                    int64_t group_size, int bh, int bw, float qmin, float qmax,
                                    int div_bf16, int8_t* out) {
  const int64_t total = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x; i < total; i += (int64_t)gridDim.x * NT) {
    const int64_t r = i / cols, c = i % cols;
    const int64_t si = scale_index(strategy, r, c, ld_scale, g_idx, group_size, bh, bw);
    float v = load_elem(x, dt, r * ldx + c);
    float q = v / scale[si];
    if (div_bf16) q = round_to_bf16(q);
    if (zp) {
      q = q + zp[si];
      if (div_bf16) q = round_to_bf16(q);
    }
    q = fminf(fmaxf(q, qmin), qmax);
    out[r * cols + c] = (int8_t)rintf(q);
  }
}

// ---------------------------------------------------------------- packs
__global__ void pack_int4_int32_kernel(const int8_t* codes, int64_t rows, int64_t cols,
                                       int32_t* out) {
  const int64_t words = rows * (cols / 8);
  for (int64_t w = (int64_t)blockIdx.x * NT + threadIdx.x; w < words; w += (int64_t)gridDim.x * NT) {
    const int64_t r = w / (cols / 8), k = w % (cols / 8);
    const uint2 raw = *reinterpret_cast<const uint2*>(codes + r * cols + 8 * k);
    uint32_t acc = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint32_t byte = ((e < 4 ? raw.x : raw.y) >> (8 * (e & 3))) & 0xffu;
      acc |= ((byte + 8u) & 0xfu) << (4 * e);
    }
    out[w] = (int32_t)acc;
  }
}

// General form: 32 / bits codes per word, element e of a word at bits
// bits * e, offset-binary (q + 2^(bits-1)); words past the row's end read 0.
__global__ void pack_int32_kernel(const int8_t* codes, int64_t rows, int64_t cols, int bits, int64_t wpr,
                                  int32_t* out) {
  const int pf = 32 / bits;
  const uint32_t off = 1u << (bits - 1), mask = (1u << bits) - 1u;
  const int64_t words = rows * wpr;
  for (int64_t w = (int64_t)blockIdx.x * NT + threadIdx.x; w < words; w += (int64_t)gridDim.x * NT) {
    const int64_t r = w / wpr, k = w % wpr;
    uint32_t acc = 0;
    for (int e = 0; e < pf; ++e) {
      const int64_t c = k * pf + e;
      if (c < cols) acc |= (((uint32_t)((int)codes[r * cols + c] + (int)off)) & mask) << (bits * e);
    }
    out[w] = (int32_t)acc;
  }
}

__global__ void pack_int4_int8_kernel(const int8_t* codes, int64_t rows, int64_t cols, int8_t* out) {
  const int64_t n = rows * (cols / 2);
  for (int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * NT) {
    const int64_t r = i / (cols / 2), k = i % (cols / 2);
    const int lo = codes[r * cols + 2 * k] & 0x0f, hi = codes[r * cols + 2 * k + 1] & 0x0f;
    out[i] = (int8_t)((hi << 4) | lo);
  }
}

// ---------------------------------------------------------------- MXFP4

__device__ __forceinline__ float exp2i(int k) {  // 2^k for k in [-149, 127]
  if (k >= -126) return __uint_as_float((uint32_t)(k + 127) << 23);
  return __uint_as_float(1u << (k + 149));
}

constexpr int MX_U = 4;  // chunks per lane, loads issued together

__global__ __launch_bounds__(NT) void mxfp4_quantize_pack_kernel(const uint16_t* __restrict__ x,
                                                                  int64_t rows, int64_t cols,
                                                                  int64_t ldx, int rule,
                                                                  uint32_t* __restrict__ codes,
                                                                  uint8_t* __restrict__ scales) {
  // chunk = 8 bf16 (16 B); four consecutive lanes hold one 32-element group.
  // Workgroup b owns chunks [b NT U, (b+1) NT U); lane t takes chunks
  // b NT U + u NT + t, so every load instruction is fully coalesced.  A group's
  // four lanes are live or dead together (cols / 8 is a multiple of 4).
  const int64_t cpr = cols / 8;
  const int64_t total = rows * cpr;
  const int64_t c0 = (int64_t)blockIdx.x * NT * MX_U + threadIdx.x;
  const bool dense = ldx == cols;
  u32x4_t v[MX_U];
#pragma unroll
  for (int u = 0; u < MX_U; ++u) {
    const int64_t c = c0 + (int64_t)u * NT;
    const int64_t cc = c < total ? c : total - 1;
    int64_t off = 8 * cc;
    if (!dense) {
      const int64_t r = cc / cpr;
      off = r * ldx + 8 * (cc - r * cpr);
    }
    v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(x + off));
  }
#pragma unroll
  for (int u = 0; u < MX_U; ++u) {
    const int64_t c = c0 + (int64_t)u * NT;
    uint32_t am = 0;  // max |x| as bf16 bits (order-preserving for non-negative)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = v[u][q] & 0x7fffu, hi = (v[u][q] >> 16) & 0x7fffu;
      am = max(am, max(lo, hi));
    }
    am = max(am, (uint32_t)__shfl_xor((int)am, 1));
    am = max(am, (uint32_t)__shfl_xor((int)am, 2));
    const int e8 = mx_exponent(__uint_as_float(am << 16), rule);
    // e8 in [0, 254]: dividing by 2^(e8-127) is an exact multiply by 2^(127-e8)
    const float inv = exp2i(127 - e8);
    // gfx950's fp4 conversion rounds to nearest-even on the e2m1 grid and
    // saturates at 6, which is the cast_to_fp4 rule; it takes the sign from
    // the sign bit, so -0.0 is turned into +0.0 first (the rule sets the sign
    // only for v < 0).  The scale operand is 1: x is pre-multiplied by the
    // exact power of two 1 / 2^(e8 - 127).
    uint32_t word = 0;
    word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, __uint_as_float(v[u][0] << 16) * inv + 0.f,
                                                   __uint_as_float(v[u][0] & 0xffff0000u) * inv + 0.f, 1.f, 0);
    word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, __uint_as_float(v[u][1] << 16) * inv + 0.f,
                                                   __uint_as_float(v[u][1] & 0xffff0000u) * inv + 0.f, 1.f, 1);
    word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, __uint_as_float(v[u][2] << 16) * inv + 0.f,
                                                   __uint_as_float(v[u][2] & 0xffff0000u) * inv + 0.f, 1.f, 2);
    word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, __uint_as_float(v[u][3] << 16) * inv + 0.f,
                                                   __uint_as_float(v[u][3] & 0xffff0000u) * inv + 0.f, 1.f, 3);
    if (c < total) {
      // dense outputs: codes [rows][cols / 8] words, scales [rows][cols / 32]
      __builtin_nontemporal_store(word, codes + c);
      if ((threadIdx.x & 3) == 0) scales[c >> 2] = (uint8_t)e8;
    }
  }
}

__global__ void mx_scales_kernel(const float* mn, const float* mx, int64_t n, int rule, uint8_t* e8_out,
                                 float* scale_out) {
  const int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x;
  if (i >= n) return;
  const float amax = round_to_bf16(fmaxf(fabsf(fminf(mn[i], 0.f)), fabsf(fmaxf(mx[i], 0.f))));
  const int e8 = mx_exponent(amax, rule);
  if (e8_out) e8_out[i] = (uint8_t)e8;
  if (scale_out) scale_out[i] = exp2i(e8 - 127);
}

__global__ void mxfp4_dequant_kernel(const uint8_t* codes, const uint8_t* scales, int64_t rows,
                                     int64_t cols, uint16_t* out) {
  const int64_t n = rows * cols;
  const float lut[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
  for (int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * NT) {
    const int64_t r = i / cols, c = i % cols;
    const uint32_t byte = codes[r * (cols / 2) + c / 2];
    const uint32_t code = (c & 1) ? (byte >> 4) : (byte & 15u);
    const int e8 = scales[r * (cols / 32) + c / 32];
    float v = lut[code & 7u];
    if (code & 8u) v = -v;
    float s = exp2i(e8 - 127 < -149 ? -149 : e8 - 127);
    out[i] = f32_to_bf16_bits(v * s);
  }
}

// ---------------------------------------------------------------- fp4 with given scales
// e2m1 codes of x / (scale / global_scale) for group scales computed
// elsewhere (NVFP4: fp8 group scales and an fp32 global scale), the
// effective scale and the quotient formed in fp32 as CT's quantize forms
// them; two codes per byte, even column in the low nibble.  The gfx950 fp4
// conversion rounds to nearest-even on the e2m1 grid and saturates at 6
// (CT's cast_to_fp4); -0.0 becomes +0.0 first, so only values below zero
// carry the sign bit.  One thread per output byte.
__global__ void fp4_quantize_pack_kernel(const void* x, mi355q_dtype dt, int64_t rows, int64_t cols, int64_t ldx,
                                         const float* scale, int64_t ld_scale, int64_t group_size,
                                         const float* gscale, uint8_t* out) {
  const int64_t half = cols / 2, total = rows * half;
  const float gs = gscale ? gscale[0] : 1.f;
  for (int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x; i < total; i += (int64_t)gridDim.x * NT) {
    const int64_t r = i / half, c = 2 * (i - r * half);
    const float s0 = scale[r * ld_scale + c / group_size] / gs;
    const float s1 = scale[r * ld_scale + (c + 1) / group_size] / gs;
    const float v0 = load_elem(x, dt, r * ldx + c) / s0, v1 = load_elem(x, dt, r * ldx + c + 1) / s1;
    const uint32_t w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, v0 + 0.f, v1 + 0.f, 1.f, 0);
    out[i] = (uint8_t)(w & 0xffu);
  }
}

// ---------------------------------------------------------------- fp8 e4m3fn
__device__ __forceinline__ uint8_t f32_to_e4m3fn(float v) {
  const uint32_t sign = (__float_as_uint(v) >> 31) << 7;
  float a = fabsf(v);  // caller clamps to <= 448
  uint32_t out;
  if (a >= 0.015625f) {  // normal range 2^-6 and up
    uint32_t u = __float_as_uint(a);
    u += 0x7ffffu + ((u >> 20) & 1u);  // RNE to 3 mantissa bits
    const int e = (int)((u >> 23) & 0xffu) - 127 + 7;
    out = ((uint32_t)e << 3) | ((u >> 20) & 7u);
  } else {
    out = (uint32_t)rintf(a * 512.f);  // subnormals m * 2^-9 (8 -> min normal)
  }
  return (uint8_t)(sign | out);
}

__global__ void quantize_fp8_kernel(const void* x, mi355q_dtype dt, int64_t rows, int64_t cols,
                                    int64_t ldx, const float* scale, int64_t ld_scale, int strategy,
                                    int64_t group_size, int div_bf16, uint8_t* out) {
  const int64_t total = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x; i < total; i += (int64_t)gridDim.x * NT) {
    const int64_t r = i / cols, c = i % cols;
    const int64_t si = scale_index(strategy, r, c, ld_scale, nullptr, group_size, 1, 1);
    float q = load_elem(x, dt, r * ldx + c) / scale[si];
    if (div_bf16) q = round_to_bf16(q);
    q = fminf(fmaxf(q, -448.f), 448.f);
    out[r * cols + c] = f32_to_e4m3fn(q);
  }
}

// ---------------------------------------------------------------- per-token int8
__global__ __launch_bounds__(NT) void int8_per_token_kernel(const uint16_t* x, int64_t rows,
                                                            int64_t cols, int64_t ldx, int8_t* codes,
                                                            uint16_t* scale_out) {
  __shared__ float smx[NT / 64];
  const int64_t r = blockIdx.x;
  const uint16_t* row = x + r * ldx;
  float mx = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += NT) mx = fmaxf(mx, fabsf(bf16_bits_to_f32(row[c])));
  mx = warp_max(mx);
  if ((threadIdx.x & 63) == 0) smx[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = smx[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) mx = fmaxf(mx, smx[w]);
  float s = round_to_bf16(mx / 127.5f);
  if (s == 0.f) s = 0.0078125f;
  if (threadIdx.x == 0) scale_out[r] = f32_to_bf16_bits(s);
  for (int64_t c = threadIdx.x; c < cols; c += NT) {
    float q = round_to_bf16(bf16_bits_to_f32(row[c]) / s);
    q = fminf(fmaxf(q, -128.f), 127.f);
    codes[r * cols + c] = (int8_t)rintf(q);
  }
}

// Vectorised variant (16-byte rows, cols % 8 == 0, cols <= 8 NT CPT): each
// thread keeps its CPT chunks of 8 elements in registers, so the row is read
// once; the max |x| is reduced on the bf16 bit patterns (order-preserving for
// non-negative values), and each chunk is written as 8 int8 codes (8 bytes).
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

// Eight bf16 values (one 16-byte chunk) -> eight int8 codes of x / s:
// the quotient by reciprocal and one FMA residual correction (Markstein):
// the refined quotient is exact when x / s is representable and within one
// fp32 ulp otherwise.  Rounded to bf16 it equals the rounded IEEE quotient:
// x / s with 8-bit significands is either a bf16 midpoint exactly or at
// least 2^-17 (relative) away from every midpoint.  Scales below 2^-100
// (rows of denormal-sized values, refine false) take the IEEE division.
// Codes of 8 bf16 values: rint(clamp(bf16(x / s), -128, 127)).  The clamp,
// the round to nearest even and the byte packing are one v_cvt_pk_u8_f32 of
// q + 128 (saturating to [0, 255]; adding the even integer 128 to the bf16
// quotient is exact wherever it can change the rounded result and keeps
// ties on the same side), and the xor with 0x80 per byte restores the sign.
__device__ __forceinline__ void int8_chunk(const u32x4_t& v, float s, float rs, bool refine, uint32_t w[2]) {
  w[0] = w[1] = 0u;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t bits = e & 1 ? (v[e >> 1] & 0xffff0000u) : (v[e >> 1] << 16);
    const float xv = __uint_as_float(bits);
    float q;
    if (refine) {
      const float q0 = xv * rs;
      q = fmaf(fmaf(-q0, s, xv), rs, q0);
    } else {
      q = xv / s;
    }
    q = round_to_bf16(q);
    w[e >> 2] = __builtin_amdgcn_cvt_pk_u8_f32(q + 128.f, e & 3, w[e >> 2]);
  }
  w[0] ^= 0x80808080u;
  w[1] ^= 0x80808080u;
}

// Per-token scale of one row from its absmax bit pattern: bf16(amax / 127.5),
// 2^-7 for an all-zero row.
__device__ __forceinline__ float int8_token_scale(uint32_t am) {
  float s = round_to_bf16(__uint_as_float(am << 16) / 127.5f);
  return s == 0.f ? 0.0078125f : s;
}

// One wave per row (rows of at most 64 CPL 16-byte chunks): every lane keeps
// CPL chunks in flight, the absmax reduction stays inside the wave, and a
// workgroup of NT threads finishes NT / 64 rows.
template <int CPL>
__global__ __launch_bounds__(NT) void int8_per_token_wave_kernel(const uint16_t* __restrict__ x, int64_t rows,
                                                                 int64_t cols, int64_t ldx,
                                                                 int8_t* __restrict__ codes,
                                                                 uint16_t* __restrict__ scale_out) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int nch = (int)(cols / 8);
  const u32x4_t* row = reinterpret_cast<const u32x4_t*>(x + r * ldx);
  u32x4_t v[CPL];
  uint32_t am = 0;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    v[i] = __builtin_nontemporal_load(row + (c < nch ? c : nch - 1));
    if (c >= nch) v[i] = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int q = 0; q < 4; ++q) am = max(am, max(v[i][q] & 0x7fffu, (v[i][q] >> 16) & 0x7fffu));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) am = max(am, (uint32_t)__shfl_xor((int)am, o));
  const float s = int8_token_scale(am);
  if (lane == 0) scale_out[r] = f32_to_bf16_bits(s);
  const bool refine = s >= 0x1p-100f;
  const float rs = __builtin_amdgcn_rcpf(s);
  uint32_t* out = reinterpret_cast<uint32_t*>(codes + r * cols);
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      uint32_t w[2];
      int8_chunk(v[i], s, rs, refine, w);
      __builtin_nontemporal_store(u32x2_t{w[0], w[1]}, reinterpret_cast<u32x2_t*>(out) + c);
    }
  }
}

template <int CPT>
__global__ __launch_bounds__(NT) void int8_per_token_vec_kernel(const uint16_t* __restrict__ x, int64_t cols,
                                                                int64_t ldx, int8_t* __restrict__ codes,
                                                                uint16_t* __restrict__ scale_out) {
  __shared__ uint32_t smx[NT / 64];
  const int64_t r = blockIdx.x;
  const int nch = (int)(cols / 8);
  const u32x4_t* row = reinterpret_cast<const u32x4_t*>(x + r * ldx);
  u32x4_t v[CPT];
  uint32_t am = 0;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + i * NT;
    v[i] = __builtin_nontemporal_load(row + (c < nch ? c : nch - 1));
    if (c >= nch) v[i] = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int q = 0; q < 4; ++q) am = max(am, max(v[i][q] & 0x7fffu, (v[i][q] >> 16) & 0x7fffu));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) am = max(am, (uint32_t)__shfl_xor((int)am, o));
  if ((threadIdx.x & 63) == 0) smx[threadIdx.x >> 6] = am;
  __syncthreads();
  am = smx[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) am = max(am, smx[w]);
  const float s = int8_token_scale(am);
  if (threadIdx.x == 0) scale_out[r] = f32_to_bf16_bits(s);
  const bool refine = s >= 0x1p-100f;
  const float rs = __builtin_amdgcn_rcpf(s);
  uint32_t* out = reinterpret_cast<uint32_t*>(codes + r * cols);
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + i * NT;
    if (c < nch) {
      uint32_t w[2];
      int8_chunk(v[i], s, rs, refine, w);
      __builtin_nontemporal_store(u32x2_t{w[0], w[1]}, reinterpret_cast<u32x2_t*>(out) + c);
    }
  }
}

// NVFP4 (tensor-group fp4) qparams from min / max statistics (fp32 holding
// values of the statistics' dtype; bf16 rounding of every step when stats16):
// the global scale is CT generate_gparam over the whole weight's absmax
// (observers/base.py:78-96): 448 * 6 / absmax in the statistics' dtype, then
// fp32; each group's scale is CT calculate_qparams with that global scale:
// global * (absmax_g / 6), clamped to +-448, cast to float8_e4m3fn (round to
// nearest even), zero replaced by the fp8 epsilon 0.125.
__global__ __launch_bounds__(1024) void nvfp4_global_kernel(const float* __restrict__ mn,
                                                            const float* __restrict__ mx, int64_t n, int stats16,
                                                            float* __restrict__ gscale) {
  __shared__ float red[1024];
  float a = -INFINITY;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) a = fmaxf(a, fmaxf(mx[i], -mn[i]));
  red[threadIdx.x] = a;
  __syncthreads();
  for (int o = blockDim.x / 2; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const float g = red[0];
    const float mvp = fmaxf(fabsf(fminf(-g, 0.f)), fabsf(fmaxf(g, 0.f)));
    // CT writes fp8_max * fp4_max / absmax with a Python scalar over a tensor,
    // which torch evaluates as reciprocal(absmax) * 2688, each result rounded
    // to the statistics' dtype
    float r = 1.f / mvp;
    if (stats16) r = round_to_bf16(r);
    const float gs = 2688.f * r;
    gscale[0] = stats16 ? round_to_bf16(gs) : gs;
  }
}

__global__ void nvfp4_scales_kernel(const float* __restrict__ mn, const float* __restrict__ mx, int64_t n,
                                    int stats16, const float* __restrict__ gscale, float* __restrict__ scale_out,
                                    uint8_t* __restrict__ bits_out) {
  const float g = gscale[0];
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float mvp = fmaxf(fabsf(fminf(mn[i], 0.f)), fabsf(fmaxf(mx[i], 0.f)));
    float q = mvp / 6.f;
    if (stats16) q = round_to_bf16(q);
    float sc = fp8e4m3_rne(fminf(fmaxf(g * q, -448.f), 448.f));
    if (sc == 0.f) sc = 0.125f;
    if (scale_out) scale_out[i] = sc;
    if (bits_out) bits_out[i] = (uint8_t)fp8e4m3_bits(sc);
  }
}

inline unsigned grid_for(int64_t n, int64_t per_block = NT, unsigned cap = 65536u) {
  int64_t g = (n + per_block - 1) / per_block;
  if (g < 1) g = 1;
  return (unsigned)(g > cap ? cap : g);
}

}  // namespace
}  // namespace mi355q

using namespace mi355q;

extern "C" int mi355q_observe_minmax(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols,
                                     int64_t ldx, int strategy, int64_t group_size, int block_h,
                                     int block_w, float* min_dev, float* max_dev, void* stream) {
  MQ_CHECK_ARG(x_dev && min_dev && max_dev, "observe_minmax: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && ldx >= cols, "observe_minmax: bad shape");
  MQ_CHECK_ARG(dtype == MI355Q_BF16 || dtype == MI355Q_F32, "observe_minmax: bad dtype");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (strategy) {
    case MI355Q_TENSOR:
      hipLaunchKernelGGL(minmax_init_kernel, dim3(1), dim3(1), 0, st, min_dev, max_dev);
      hipLaunchKernelGGL(minmax_rows_kernel, dim3((unsigned)rows), dim3(NT), 0, st, x_dev, dtype, rows,
                         cols, ldx, min_dev, max_dev, 1);
      hipLaunchKernelGGL(minmax_finish_kernel, dim3(1), dim3(1), 0, st, min_dev, max_dev);
      break;
    case MI355Q_CHANNEL:
    case MI355Q_TOKEN:
      hipLaunchKernelGGL(minmax_rows_kernel, dim3((unsigned)rows), dim3(NT), 0, st, x_dev, dtype, rows,
                         cols, ldx, min_dev, max_dev, 0);
      break;
    case MI355Q_GROUP: {
      MQ_CHECK_ARG(group_size > 0, "observe_minmax: group_size must be > 0");
      MQ_CHECK_ARG(cols % group_size == 0, "observe_minmax: columns (%lld) not divisible by group_size (%lld)",
                   (long long)cols, (long long)group_size);
      const bool vec = dtype == MI355Q_BF16 && ldx % 8 == 0 && aligned16(x_dev);
      const int64_t lpg = group_size / 8;
      const int64_t chunks = rows * (cols / 8);
      const unsigned g = grid_for(chunks, NT, 1u << 20);
      const uint16_t* xb = static_cast<const uint16_t*>(x_dev);
      if (vec && group_size % 8 == 0 && lpg == 4)
        hipLaunchKernelGGL(minmax_group_vec_kernel<4>, dim3(g), dim3(NT), 0, st, xb, rows, cols, ldx, min_dev, max_dev);
      else if (vec && group_size % 8 == 0 && lpg == 8)
        hipLaunchKernelGGL(minmax_group_vec_kernel<8>, dim3(g), dim3(NT), 0, st, xb, rows, cols, ldx, min_dev, max_dev);
      else if (vec && group_size % 8 == 0 && lpg == 16)
        hipLaunchKernelGGL(minmax_group_vec_kernel<16>, dim3(g), dim3(NT), 0, st, xb, rows, cols, ldx, min_dev, max_dev);
      else if (vec && group_size % 8 == 0 && lpg == 2)
        hipLaunchKernelGGL(minmax_group_vec_kernel<2>, dim3(g), dim3(NT), 0, st, xb, rows, cols, ldx, min_dev, max_dev);
      else {
        const int64_t ng = cols / group_size;
        hipLaunchKernelGGL(minmax_cells_kernel, dim3(grid_for(rows * ng, NT, 1u << 30)), dim3(NT), 0, st,
                           x_dev, dtype, rows, cols, ldx, (int64_t)1, group_size, rows, ng, min_dev, max_dev);
      }
      break;
    }
    case MI355Q_BLOCK: {
      MQ_CHECK_ARG(block_h > 0 && block_w > 0, "observe_minmax: bad block structure");
      const int64_t ncr = (rows + block_h - 1) / block_h, ncc = (cols + block_w - 1) / block_w;
      hipLaunchKernelGGL(minmax_cells_kernel, dim3(grid_for(ncr * ncc, NT, 1u << 30)), dim3(NT), 0, st,
                         x_dev, dtype, rows, cols, ldx, (int64_t)block_h, (int64_t)block_w, ncr, ncc,
                         min_dev, max_dev);
      break;
    }
    default:
      set_error("observe_minmax: unknown strategy %d", strategy);
      return MI355Q_INVALID_ARGUMENT;
  }
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" int mi355q_calculate_qparams(const float* min_dev, const float* max_dev, int64_t n, float qmin,
                                        float qmax, int symmetric, int strict, mi355q_dtype scale_dtype,
                                        float* scale_out_dev, float* zp_out_dev, void* stream) {
  MQ_CHECK_ARG(min_dev && max_dev && scale_out_dev && zp_out_dev, "calculate_qparams: null pointer");
  MQ_CHECK_ARG(qmin < 0.f && qmax > 0.f, "calculate_qparams: range must straddle zero");
  MQ_CHECK_ARG(!strict || symmetric, "calculate_qparams: strict requires symmetric");
  MQ_CHECK_ARG(scale_dtype == MI355Q_BF16 || scale_dtype == MI355Q_F32, "calculate_qparams: scale dtype must be bf16 or fp32");
  if (n <= 0) return MI355Q_OK;
  hipLaunchKernelGGL(qparams_kernel, dim3(grid_for(n, NT, 1u << 30)), dim3(NT), 0,
                     reinterpret_cast<hipStream_t>(stream), min_dev, max_dev, n, qmin, qmax, symmetric,
                     strict, scale_dtype == MI355Q_BF16 ? 1 : 0, scale_out_dev, zp_out_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" size_t mi355q_observe_mse_workspace_size(int64_t rows, int64_t cols, int64_t cell_rows,
                                                   int64_t cell_cols, int total_steps) {
  if (rows <= 0 || cols <= 0 || cell_rows <= 0 || cell_cols <= 0 || total_steps <= 0) return 0;
  return plan_mse(rows, cols, cell_rows, cell_cols, total_steps).total;
}

namespace mi355q {
namespace {
// Both MSE observers: im = the imatrix observer's mode (fp32 error sums,
// weighted by imp when given, patience 0 = no early stop).
int observe_mse_impl(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols, int64_t ldx,
                     int64_t cell_rows, int64_t cell_cols, float qmin, float qmax, int symmetric, int qtype,
                     int total_steps,
                     int patience, double grid, float norm, bool im, const float* imp, const float* min_dev,
                     const float* max_dev, float* min_out_dev, float* max_out_dev, void* workspace_dev,
                     size_t workspace_bytes, void* stream) {
  MQ_CHECK_ARG(x_dev && min_dev && max_dev && min_out_dev && max_out_dev, "observe_mse: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && ldx >= cols, "observe_mse: bad shape");
  MQ_CHECK_ARG(cell_rows > 0 && cell_cols > 0, "observe_mse: bad cell shape");
  MQ_CHECK_ARG(dtype == MI355Q_BF16 || dtype == MI355Q_F32, "observe_mse: dtype must be bf16 or fp32");
  MQ_CHECK_ARG(qmin < 0.f && qmax > 0.f, "observe_mse: range must straddle zero");
  const bool mx = qtype == MI355Q_QTYPE_MXFP4_CT || qtype == MI355Q_QTYPE_MXFP4_OCP;
  MQ_CHECK_ARG(qtype == MI355Q_QTYPE_INT ||
                   (qtype == MI355Q_QTYPE_FP8_E4M3 && symmetric && qmin == -qmax && qmax <= 448.f) ||
                   ((qtype == MI355Q_QTYPE_FP4_E2M1 || mx) && symmetric && qmin == -qmax && qmax <= 6.f),
               "observe_mse: value type must be integer, or fp8 e4m3 / fp4 e2m1 symmetric within their range");
  const int fq = qtype == MI355Q_QTYPE_FP8_E4M3 ? 1 : qtype == MI355Q_QTYPE_FP4_E2M1 ? 2 : mx ? 3 : 0;
  MQ_CHECK_ARG(total_steps >= 0 && grid != 0.0, "observe_mse: bad search grid");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t ncells = ((rows + cell_rows - 1) / cell_rows) * ((cols + cell_cols - 1) / cell_cols);
  if (total_steps == 0) {
    MQ_CHECK_HIP(hipMemcpyAsync(min_out_dev, min_dev, ncells * sizeof(float), hipMemcpyDeviceToDevice, st));
    MQ_CHECK_HIP(hipMemcpyAsync(max_out_dev, max_dev, ncells * sizeof(float), hipMemcpyDeviceToDevice, st));
    return MI355Q_OK;
  }
  const MsePlan pl = plan_mse(rows, cols, cell_rows, cell_cols, total_steps);
  MQ_CHECK_ARG(workspace_dev && workspace_bytes >= pl.total, "observe_mse: workspace too small (%zu < %zu)",
               workspace_bytes, pl.total);
  char* ws = static_cast<char*>(workspace_dev);
  float* err = reinterpret_cast<float*>(ws);
  float* part = reinterpret_cast<float*>(ws + pl.off_part);
  int* any = reinterpret_cast<int*>(ws + pl.off_any);
  uint16_t* tab = reinterpret_cast<uint16_t*>(ws + pl.off_tab);
  MseArgs a{x_dev, rows, cols, ldx, cell_rows, cell_cols, (rows + cell_rows - 1) / cell_rows,
            (cols + cell_cols - 1) / cell_cols, qmin, qmax, total_steps, grid, norm, min_dev, max_dev,
            im ? imp : nullptr, qtype == MI355Q_QTYPE_MXFP4_OCP ? MI355Q_MX_RULE_OCP : MI355Q_MX_RULE_CT};
  const bool b = dtype == MI355Q_BF16, zp = symmetric == 0;
  hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(NT), 0, st, any, total_steps);
  MQ_LAUNCH_CHECK();
  if (b && !im) {
    hipLaunchKernelGGL(mse_pow_table_kernel, dim3(POW_TAB / NT), dim3(NT), 0, st, norm, tab);
    MQ_LAUNCH_CHECK();
  }
  constexpr int64_t kMaxWg = 1024;  // persistent workgroups (each loads the power table once)
  // kernel variant for (bf16, zero points, imatrix mode)
  // (the float grids: symmetric only; f00 .. f11 (fp8) and h00 .. h11 (fp4)
  // are their (bf16, imatrix) variants)
  auto pick = [&](auto k000, auto k001, auto k010, auto k011, auto k100, auto k101, auto k110, auto k111,
                  auto f00, auto f01, auto f10, auto f11, auto h00, auto h01, auto h10, auto h11, auto m00,
                  auto m01, auto m10, auto m11, auto&& go) {
    if (fq == 3) {
      if (b) im ? go(m11) : go(m10); else im ? go(m01) : go(m00);
    } else if (fq == 1) {
      if (b) im ? go(f11) : go(f10); else im ? go(f01) : go(f00);
    } else if (fq == 2) {
      if (b) im ? go(h11) : go(h10); else im ? go(h01) : go(h00);
    } else if (b) {
      if (zp) im ? go(k111) : go(k110); else im ? go(k101) : go(k100);
    } else {
      if (zp) im ? go(k011) : go(k010); else im ? go(k001) : go(k000);
    }
  };
  if (pl.lg_log2 >= 0) {
    const int64_t per_wg = NT >> pl.lg_log2;
    const dim3 g((unsigned)min((ncells + per_wg - 1) / per_wg, kMaxWg));
    pick(mse_err_small_kernel<false, false, false>, mse_err_small_kernel<false, false, true>,
         mse_err_small_kernel<false, true, false>, mse_err_small_kernel<false, true, true>,
         mse_err_small_kernel<true, false, false>, mse_err_small_kernel<true, false, true>,
         mse_err_small_kernel<true, true, false>, mse_err_small_kernel<true, true, true>,
         mse_err_small_kernel<false, false, false, 1>, mse_err_small_kernel<false, false, true, 1>,
         mse_err_small_kernel<true, false, false, 1>, mse_err_small_kernel<true, false, true, 1>,
         mse_err_small_kernel<false, false, false, 2>, mse_err_small_kernel<false, false, true, 2>,
         mse_err_small_kernel<true, false, false, 2>, mse_err_small_kernel<true, false, true, 2>,
         mse_err_small_kernel<false, false, false, 3>, mse_err_small_kernel<false, false, true, 3>,
         mse_err_small_kernel<true, false, false, 3>, mse_err_small_kernel<true, false, true, 3>,
         [&](auto kernel) { hipLaunchKernelGGL(kernel, g, dim3(NT), 0, st, a, pl.lg_log2, tab, err); });
  } else {
    const dim3 g((unsigned)min(ncells * pl.nchunk, kMaxWg));
    pick(mse_err_large_kernel<false, false, false>, mse_err_large_kernel<false, false, true>,
         mse_err_large_kernel<false, true, false>, mse_err_large_kernel<false, true, true>,
         mse_err_large_kernel<true, false, false>, mse_err_large_kernel<true, false, true>,
         mse_err_large_kernel<true, true, false>, mse_err_large_kernel<true, true, true>,
         mse_err_large_kernel<false, false, false, 1>, mse_err_large_kernel<false, false, true, 1>,
         mse_err_large_kernel<true, false, false, 1>, mse_err_large_kernel<true, false, true, 1>,
         mse_err_large_kernel<false, false, false, 2>, mse_err_large_kernel<false, false, true, 2>,
         mse_err_large_kernel<true, false, false, 2>, mse_err_large_kernel<true, false, true, 2>,
         mse_err_large_kernel<false, false, false, 3>, mse_err_large_kernel<false, false, true, 3>,
         mse_err_large_kernel<true, false, false, 3>, mse_err_large_kernel<true, false, true, 3>,
         [&](auto kernel) { hipLaunchKernelGGL(kernel, g, dim3(NT), 0, st, a, pl.nchunk, tab, part); });
  }
  MQ_LAUNCH_CHECK();
  const bool round_sum = b && !im;
  const float best0 = round_sum ? 3.3895313892515355e38f : 3.4028234663852886e38f;
  const dim3 gc((unsigned)((ncells + NT - 1) / NT));
  hipLaunchKernelGGL(mse_flags_kernel, gc, dim3(NT), 0, st, part, pl.nchunk, err, ncells, total_steps, any,
                     round_sum ? 1 : 0, best0);
  MQ_LAUNCH_CHECK();
  if (b) hipLaunchKernelGGL(mse_select_kernel<true>, gc, dim3(NT), 0, st, err, any, ncells, total_steps, patience,
                            im ? 1 : 0, best0, grid, min_dev, max_dev, min_out_dev, max_out_dev);
  else   hipLaunchKernelGGL(mse_select_kernel<false>, gc, dim3(NT), 0, st, err, any, ncells, total_steps, patience,
                            im ? 1 : 0, best0, grid, min_dev, max_dev, min_out_dev, max_out_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

// Column sums of squares over a row range, one partial per (row chunk,
// column); the partials are added in chunk order into the output.
constexpr int SQ_ROWS = 512;  // rows per chunk

__global__ void column_sumsq_part_kernel(const void* x, mi355q_dtype dt, int64_t rows, int64_t cols, int64_t ldx,
                                         float* part) {
  const int64_t c = (int64_t)blockIdx.x * NT + threadIdx.x;
  if (c >= cols) return;
  const int64_t r0 = (int64_t)blockIdx.y * SQ_ROWS, r1 = min(r0 + SQ_ROWS, rows);
  float acc = 0.f;
  for (int64_t r = r0; r < r1; ++r) {
    const float v = load_elem(x, dt, r * ldx + c);
    acc += v * v;
  }
  part[(int64_t)blockIdx.y * cols + c] = acc;
}

__global__ void column_sumsq_add_kernel(const float* part, int64_t nchunk, int64_t cols, float* out) {
  const int64_t c = (int64_t)blockIdx.x * NT + threadIdx.x;
  if (c >= cols) return;
  float acc = 0.f;
  for (int64_t k = 0; k < nchunk; ++k) acc += part[k * cols + c];
  out[c] = out[c] + acc;
}
}  // namespace
}  // namespace mi355q

extern "C" int mi355q_observe_mse(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols, int64_t ldx,
                                  int64_t cell_rows, int64_t cell_cols, float qmin, float qmax, int symmetric,
                                  int qtype, int total_steps, int patience, double grid, float norm, const float* min_dev,
                                  const float* max_dev, float* min_out_dev, float* max_out_dev,
                                  void* workspace_dev, size_t workspace_bytes, void* stream) {
  return observe_mse_impl(x_dev, dtype, rows, cols, ldx, cell_rows, cell_cols, qmin, qmax, symmetric, qtype,
                          total_steps, patience, grid, norm, false, nullptr, min_dev, max_dev, min_out_dev, max_out_dev,
                          workspace_dev, workspace_bytes, stream);
}

extern "C" int mi355q_observe_imatrix_mse(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols,
                                          int64_t ldx, int64_t cell_rows, int64_t cell_cols, float qmin, float qmax,
                                          int symmetric, int qtype, int total_steps, int patience, double grid,
                                          float norm,
                                          const float* importance_dev, const float* min_dev, const float* max_dev,
                                          float* min_out_dev, float* max_out_dev, void* workspace_dev,
                                          size_t workspace_bytes, void* stream) {
  return observe_mse_impl(x_dev, dtype, rows, cols, ldx, cell_rows, cell_cols, qmin, qmax, symmetric, qtype,
                          total_steps, patience, grid, norm, true, importance_dev, min_dev, max_dev, min_out_dev, max_out_dev,
                          workspace_dev, workspace_bytes, stream);
}

extern "C" size_t mi355q_column_sumsq_workspace_size(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return (size_t)((rows + SQ_ROWS - 1) / SQ_ROWS) * cols * sizeof(float);
}

extern "C" int mi355q_column_sumsq(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols, int64_t ldx,
                                   float* sum_dev, void* workspace_dev, size_t workspace_bytes, void* stream) {
  MQ_CHECK_ARG(sum_dev, "column_sumsq: null output");
  MQ_CHECK_ARG(rows >= 0 && cols > 0 && ldx >= cols, "column_sumsq: bad shape");
  MQ_CHECK_ARG(dtype == MI355Q_BF16 || dtype == MI355Q_F32, "column_sumsq: dtype must be bf16 or fp32");
  if (rows == 0) return MI355Q_OK;
  MQ_CHECK_ARG(x_dev, "column_sumsq: null input");
  const int64_t nchunk = (rows + SQ_ROWS - 1) / SQ_ROWS;
  MQ_CHECK_ARG(nchunk <= 65535, "column_sumsq: at most 65535 * 512 rows");
  MQ_CHECK_ARG(workspace_dev && workspace_bytes >= mi355q_column_sumsq_workspace_size(rows, cols),
               "column_sumsq: workspace too small");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace_dev);
  hipLaunchKernelGGL(column_sumsq_part_kernel, dim3((unsigned)((cols + NT - 1) / NT), (unsigned)nchunk), dim3(NT), 0,
                     st, x_dev, dtype, rows, cols, ldx, part);
  MQ_LAUNCH_CHECK();
  hipLaunchKernelGGL(column_sumsq_add_kernel, dim3((unsigned)((cols + NT - 1) / NT)), dim3(NT), 0, st, part, nchunk,
                     cols, sum_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" int mi355q_mx_scales(const float* min_dev, const float* max_dev, int64_t n, int rule,
                                uint8_t* e8m0_out_dev, float* scale_out_dev, void* stream) {
  MQ_CHECK_ARG(min_dev && max_dev, "mx_scales: null pointer");
  MQ_CHECK_ARG(rule == MI355Q_MX_RULE_CT || rule == MI355Q_MX_RULE_OCP, "mx_scales: unknown rule");
  if (n <= 0) return MI355Q_OK;
  hipLaunchKernelGGL(mx_scales_kernel, dim3(grid_for(n, NT, 1u << 30)), dim3(NT), 0,
                     reinterpret_cast<hipStream_t>(stream), min_dev, max_dev, n, rule, e8m0_out_dev,
                     scale_out_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" int mi355q_nvfp4_qparams(const float* min_dev, const float* max_dev, int64_t n, mi355q_dtype stats_dtype,
                                    float* global_scale_dev, float* scale_out_dev, uint8_t* e4m3_out_dev,
                                    void* stream) {
  MQ_CHECK_ARG(min_dev && max_dev && global_scale_dev, "nvfp4_qparams: null pointer");
  MQ_CHECK_ARG(n > 0, "nvfp4_qparams: no statistics");
  MQ_CHECK_ARG(stats_dtype == MI355Q_BF16 || stats_dtype == MI355Q_F32, "nvfp4_qparams: bad statistics dtype");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int s16 = stats_dtype == MI355Q_BF16 ? 1 : 0;
  hipLaunchKernelGGL(nvfp4_global_kernel, dim3(1), dim3(1024), 0, st, min_dev, max_dev, n, s16, global_scale_dev);
  MQ_LAUNCH_CHECK();
  hipLaunchKernelGGL(nvfp4_scales_kernel, dim3(grid_for(n, NT, 1u << 16)), dim3(NT), 0, st, min_dev, max_dev, n, s16,
                     global_scale_dev, scale_out_dev, e4m3_out_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" int mi355q_quantize_int(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols,
                                   int64_t ldx, const float* scale_dev, const float* zp_dev,
                                   int64_t ld_scale, const int32_t* g_idx_dev, int strategy,
                                   int64_t group_size, int block_h, int block_w, int num_bits,
                                   mi355q_dtype div_dtype, int8_t* codes_dev, void* stream) {
  MQ_CHECK_ARG(x_dev && scale_dev && codes_dev, "quantize_int: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && ldx >= cols, "quantize_int: bad shape");
  MQ_CHECK_ARG((dtype == MI355Q_BF16 || dtype == MI355Q_F32) && (div_dtype == MI355Q_BF16 || div_dtype == MI355Q_F32),
               "quantize_int: dtypes must be bf16 or fp32");
  MQ_CHECK_ARG(num_bits >= 2 && num_bits <= 8, "quantize_int: num_bits must be in [2, 8]");
  MQ_CHECK_ARG(strategy != MI355Q_GROUP || group_size > 0 || g_idx_dev, "quantize_int: group_size");
  MQ_CHECK_ARG(strategy != MI355Q_BLOCK || (block_h > 0 && block_w > 0), "quantize_int: block");
  const float qmin = -(float)(1 << (num_bits - 1)), qmax = (float)((1 << (num_bits - 1)) - 1);
  hipLaunchKernelGGL(quantize_int_kernel, dim3(grid_for(rows * cols, NT, 1u << 16)), dim3(NT), 0,
                     reinterpret_cast<hipStream_t>(stream), x_dev, dtype, rows, cols, ldx, scale_dev,
                     zp_dev, ld_scale, g_idx_dev, strategy, group_size, block_h, block_w, qmin, qmax,
                     div_dtype == MI355Q_BF16 ? 1 : 0, codes_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" int mi355q_pack_int4_int32(const int8_t* codes_dev, int64_t rows, int64_t cols,
                                      int32_t* out_dev, void* stream) {
  MQ_CHECK_ARG(codes_dev && out_dev, "pack_int4_int32: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && cols % 8 == 0, "pack_int4_int32: cols must be a multiple of 8");
  MQ_CHECK_ARG((reinterpret_cast<uintptr_t>(codes_dev) & 7) == 0, "pack_int4_int32: codes must be 8-byte aligned");
  hipLaunchKernelGGL(pack_int4_int32_kernel, dim3(grid_for(rows * cols / 8, NT, 1u << 16)), dim3(NT), 0,
                     reinterpret_cast<hipStream_t>(stream), codes_dev, rows, cols, out_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" int mi355q_pack_int32(const int8_t* codes_dev, int64_t rows, int64_t cols, int num_bits,
                                 int32_t* out_dev, void* stream) {
  MQ_CHECK_ARG(codes_dev && out_dev, "pack_int32: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0, "pack_int32: bad shape");
  MQ_CHECK_ARG(num_bits == 2 || num_bits == 4 || num_bits == 8, "pack_int32: num_bits must be 2, 4 or 8");
  const int64_t wpr = (cols + 32 / num_bits - 1) / (32 / num_bits);
  hipLaunchKernelGGL(pack_int32_kernel, dim3(grid_for(rows * wpr, NT, 1u << 16)), dim3(NT), 0,
                     reinterpret_cast<hipStream_t>(stream), codes_dev, rows, cols, num_bits, wpr, out_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" int mi355q_pack_int4_int8(const int8_t* codes_dev, int64_t rows, int64_t cols,
                                     int8_t* out_dev, void* stream) {
  MQ_CHECK_ARG(codes_dev && out_dev, "pack_int4_int8: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0, "pack_int4_int8: bad shape");
  MQ_CHECK_ARG(cols % 2 == 0, "Expected even number of columns for int4 packing, got %lld", (long long)cols);
  hipLaunchKernelGGL(pack_int4_int8_kernel, dim3(grid_for(rows * cols / 2, NT, 1u << 16)), dim3(NT), 0,
                     reinterpret_cast<hipStream_t>(stream), codes_dev, rows, cols, out_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" int mi355q_mxfp4_quantize_pack(const void* x_dev, int64_t rows, int64_t cols, int64_t ldx,
                                          int rule, uint8_t* codes_dev, uint8_t* scales_dev,
                                          void* stream) {
  MQ_CHECK_ARG(x_dev && codes_dev && scales_dev, "mxfp4: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && cols % 32 == 0, "mxfp4: cols must be a positive multiple of 32");
  MQ_CHECK_ARG(ldx >= cols && ldx % 8 == 0 && aligned16(x_dev), "mxfp4: x must be 16-byte aligned rows");
  MQ_CHECK_ARG((reinterpret_cast<uintptr_t>(codes_dev) & 3) == 0, "mxfp4: codes must be 4-byte aligned");
  MQ_CHECK_ARG(rule == MI355Q_MX_RULE_CT || rule == MI355Q_MX_RULE_OCP, "mxfp4: unknown rule");
  const int64_t chunks = rows * (cols / 8);
  MQ_CHECK_ARG((chunks + (int64_t)NT * MX_U - 1) / ((int64_t)NT * MX_U) < (int64_t(1) << 31), "mxfp4: too large");
  const unsigned g = (unsigned)((chunks + (int64_t)NT * MX_U - 1) / ((int64_t)NT * MX_U));
  hipLaunchKernelGGL(mxfp4_quantize_pack_kernel, dim3(g), dim3(NT), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x_dev), rows, cols, ldx, rule,
                     reinterpret_cast<uint32_t*>(codes_dev), scales_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" int mi355q_mxfp4_dequantize(const uint8_t* codes_dev, const uint8_t* scales_dev, int64_t rows,
                                       int64_t cols, void* out_dev, void* stream) {
  MQ_CHECK_ARG(codes_dev && scales_dev && out_dev, "mxfp4_dequantize: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && cols % 32 == 0, "mxfp4_dequantize: bad shape");
  hipLaunchKernelGGL(mxfp4_dequant_kernel, dim3(grid_for(rows * cols, NT, 1u << 16)), dim3(NT), 0,
                     reinterpret_cast<hipStream_t>(stream), codes_dev, scales_dev, rows, cols,
                     static_cast<uint16_t*>(out_dev));
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" int mi355q_quantize_fp8(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols,
                                   int64_t ldx, const float* scale_dev, int64_t ld_scale, int strategy,
                                   int64_t group_size, mi355q_dtype div_dtype, uint8_t* out_dev,
                                   void* stream) {
  MQ_CHECK_ARG(x_dev && scale_dev && out_dev, "quantize_fp8: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && ldx >= cols, "quantize_fp8: bad shape");
  MQ_CHECK_ARG((dtype == MI355Q_BF16 || dtype == MI355Q_F32) && (div_dtype == MI355Q_BF16 || div_dtype == MI355Q_F32),
               "quantize_fp8: dtypes must be bf16 or fp32");
  MQ_CHECK_ARG(strategy == MI355Q_TENSOR || strategy == MI355Q_CHANNEL || strategy == MI355Q_TOKEN ||
                   (strategy == MI355Q_GROUP && group_size > 0),
               "quantize_fp8: unsupported strategy");
  hipLaunchKernelGGL(quantize_fp8_kernel, dim3(grid_for(rows * cols, NT, 1u << 16)), dim3(NT), 0,
                     reinterpret_cast<hipStream_t>(stream), x_dev, dtype, rows, cols, ldx, scale_dev, ld_scale,
                     strategy, group_size, div_dtype == MI355Q_BF16 ? 1 : 0, out_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" int mi355q_fp4_quantize_pack(const void* x_dev, mi355q_dtype dtype, int64_t rows, int64_t cols,
                                        int64_t ldx, const float* scale_dev, int64_t ld_scale, int64_t group_size,
                                        const float* global_scale_dev, uint8_t* codes_dev, void* stream) {
  MQ_CHECK_ARG(x_dev && scale_dev && codes_dev, "fp4_quantize_pack: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && cols % 2 == 0 && ldx >= cols, "fp4_quantize_pack: bad shape (cols even)");
  MQ_CHECK_ARG(dtype == MI355Q_BF16 || dtype == MI355Q_F32, "fp4_quantize_pack: dtype must be bf16 or fp32");
  MQ_CHECK_ARG(group_size > 0 && ld_scale >= (cols + group_size - 1) / group_size,
               "fp4_quantize_pack: group_size and ld_scale must cover the columns");
  hipLaunchKernelGGL(fp4_quantize_pack_kernel, dim3(grid_for(rows * (cols / 2), NT, 1u << 16)), dim3(NT), 0,
                     reinterpret_cast<hipStream_t>(stream), x_dev, dtype, rows, cols, ldx, scale_dev, ld_scale,
                     group_size, global_scale_dev, codes_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" int mi355q_quantize_int8_per_token(const void* x_dev, int64_t rows, int64_t cols, int64_t ldx,
                                              int8_t* codes_dev, uint16_t* scale_out_dev, void* stream) {
  MQ_CHECK_ARG(x_dev && codes_dev && scale_out_dev, "int8_per_token: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && ldx >= cols, "int8_per_token: bad shape");
  MQ_CHECK_ARG(rows < (int64_t(1) << 31), "int8_per_token: too many rows");
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const uint16_t* x = static_cast<const uint16_t*>(x_dev);
  const int64_t nch = cols / 8;
  const bool vec = cols % 8 == 0 && ldx % 8 == 0 && aligned16(x_dev) &&
                   (reinterpret_cast<uintptr_t>(codes_dev) & 7) == 0;
  const unsigned wave_grid = (unsigned)((rows + NT / 64 - 1) / (NT / 64));
  if (vec && nch <= 64 * 4)
    hipLaunchKernelGGL(int8_per_token_wave_kernel<4>, dim3(wave_grid), dim3(NT), 0, st, x, rows, cols, ldx,
                       codes_dev, scale_out_dev);
  else if (vec && nch <= 64 * 8)
    hipLaunchKernelGGL(int8_per_token_wave_kernel<8>, dim3(wave_grid), dim3(NT), 0, st, x, rows, cols, ldx,
                       codes_dev, scale_out_dev);
  else if (vec && nch <= NT)
    hipLaunchKernelGGL(int8_per_token_vec_kernel<1>, dim3((unsigned)rows), dim3(NT), 0, st, x, cols, ldx, codes_dev,
                       scale_out_dev);
  else if (vec && nch <= 2 * NT)
    hipLaunchKernelGGL(int8_per_token_vec_kernel<2>, dim3((unsigned)rows), dim3(NT), 0, st, x, cols, ldx, codes_dev,
                       scale_out_dev);
  else if (vec && nch <= 4 * NT)
    hipLaunchKernelGGL(int8_per_token_vec_kernel<4>, dim3((unsigned)rows), dim3(NT), 0, st, x, cols, ldx, codes_dev,
                       scale_out_dev);
  else if (vec && nch <= 8 * NT)
    hipLaunchKernelGGL(int8_per_token_vec_kernel<8>, dim3((unsigned)rows), dim3(NT), 0, st, x, cols, ldx, codes_dev,
                       scale_out_dev);
  else
    hipLaunchKernelGGL(int8_per_token_kernel, dim3((unsigned)rows), dim3(NT), 0, st, x, rows, cols, ldx, codes_dev,
                       scale_out_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}
