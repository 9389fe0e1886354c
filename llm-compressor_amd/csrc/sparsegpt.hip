// SparseGPT pruning solve on gfx950.
//
// Replaces modifiers/pruning/sparsegpt/sgpt_sparsify.py:119-206, the mask
// selection and blocked sweep.  The Hessian, dead columns and the Cholesky
// chain (:97-117) are the GPTQ ones (the same chain as
// gptq_quantize.py:178-196) and come from mi355q_gptq_hinv.
//
// Unstructured masks (:150-165): per block the threshold is the k-th smallest
// (k = int(numel * sparsity)) of tmp = W1^2 / diag(Hinv1)^2 over every row
// of the block.  tmp >= 0, so its fp32 bit patterns order like its values and
// a three-pass radix select finds the exact k-th key: pass 0 counts the
// exponent (bits 30..23, 256 bins), pass 1 bits 22..12 of the keys in the
// selected bin (2048 bins), pass 2 bits 11..0 of the keys left (4096 bins).
// The sweep kernel reads the threshold key off the three histograms, prunes
// tmp <= threshold (every value tied with the k-th as well, as the
// reference), and clears the other of two histogram sets for the next block.
//
// N:M masks (:166-186): at every m-th column of a block the n smallest tmp of
// each row's next m columns (their values at that moment) are pruned.  The
// group's values sit in at most two of a lane's register slots, so the 16
// lanes of a row rank them among themselves with DPP broadcasts; on equal
// values the lower column is pruned first (torch.topk leaves that order
// unspecified).  m <= 16.
//
// preserve_sparsity_mask (:122-135, :151-161, :181-182, :201-204): entries that
// are zero on entry stay pruned.  The reference's lazy update skips them, so
// they are exactly zero when their block starts; the sweep zeroes them when it
// loads a block, which lets the lazy update run as a plain GEMM.  In N:M mode
// the reference weighs the group starting at block column j by the live mask
// of matrix columns [j, j + m) (it indexes the whole-matrix mask with the
// block-relative column) and scatters its choices into the mask; both are
// reproduced: the sweep writes its block's mask back and reads the multiplier
// from columns [j, j + m).
//
// The sweep has the GPTQ sweep's layout (16 lanes per row, lane g owns the
// block columns 16 t + g in registers, Hinv's block in LDS) with "quantise"
// replaced by "keep or zero": err = (w - q) / d with q = 0 for a pruned entry
// and q = w otherwise, and the same rounded multiply and subtract updates.
#include "sweep.h"

#pragma clang fp contract(off)

namespace mi355q {
namespace {

using namespace sweep;

// Select workspace: two sets of histograms (block b uses set b % 2), each
// three histograms and the base-mask count (uint32 words).
constexpr int NB0 = 256, NB1 = 2048, NB2 = 4096;
constexpr int H0 = 0, H1 = NB0, H2 = NB0 + NB1, HCNT = NB0 + NB1 + NB2, SET_WORDS = HCNT + 64;
constexpr int SEL_WORDS = 2 * SET_WORDS;
constexpr int SEL_NT = 256;
constexpr int SEL_ROWS = 16;  // rows per select workgroup: 2 rows x 128 columns per round
constexpr int SEL_IT = SEL_ROWS / 2;

// The bin holding the k-th (0-based) counted key: the smallest b whose
// cumulative count exceeds k, and k minus the count of the bins before b.
// All 256 threads of the workgroup call it; sh holds 8 words of LDS.
__device__ void find_bin(const unsigned* __restrict__ h, int nb, unsigned k, unsigned* sh, unsigned& bin,
                         unsigned& rem) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = nb / SEL_NT;
  unsigned v = 0;
  for (int j = 0; j < per; ++j) v += h[tid * per + j];
  unsigned x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const unsigned y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) sh[wave] = x;
  __syncthreads();
  unsigned incl = x;
  for (int w = 0; w < wave; ++w) incl += sh[w];
  const unsigned ex = incl - v;
  if (ex <= k && k < incl) {
    unsigned acc = ex;
    for (int j = 0; j < per; ++j) {
      const unsigned c = h[tid * per + j];
      if (k < acc + c) {
        sh[4] = (unsigned)(tid * per + j);
        sh[5] = k - acc;
        break;
      }
      acc += c;
    }
  }
  __syncthreads();
  bin = sh[4];
  rem = sh[5];
  __syncthreads();
}

// tmp of one entry: +0 where the preserved mask holds it, else w^2 / d^2
// (two rounded squares and a correctly rounded division, as the reference's
// W1 ** 2 / diag ** 2).
__device__ __forceinline__ float saliency(float w, float dd2, bool masked) { return masked ? 0.f : (w * w) / dd2; }

// Radix key of a saliency: its bit pattern (sign cleared, so that a NaN from
// a non-finite weight still lands in a bin)
__device__ __forceinline__ unsigned skey(float tmp) { return __float_as_uint(tmp) & 0x7fffffffu; }

// One radix pass over the block's keys into the histograms of set hs.
__global__ __launch_bounds__(SEL_NT) void sgpt_select_kernel(const float* __restrict__ W, int64_t rows, int64_t cols,
                                                             const float* __restrict__ hinv, int64_t i1, int count,
                                                             const uint8_t* __restrict__ mask,
                                                             unsigned* __restrict__ hs, int pass, unsigned k) {
  __shared__ unsigned lh[NB2];
  __shared__ float dd2[MAXB];
  __shared__ unsigned sh[8];
  const int tid = threadIdx.x;
  const int nb = pass == 0 ? NB0 : pass == 1 ? NB1 : NB2;
  for (int b = tid; b < nb; b += SEL_NT) lh[b] = 0u;
  if (tid < count) {
    const float d = hinv[(i1 + tid) * cols + i1 + tid];
    dd2[tid] = d * d;
  }
  unsigned b0 = 0, b1 = 0, rem = k;
  if (pass >= 1) find_bin(hs + H0, NB0, k, sh, b0, rem);
  if (pass >= 2) find_bin(hs + H1, NB1, rem, sh, b1, rem);
  __syncthreads();
  const int c = tid & (MAXB - 1);
  const int64_t r0 = (int64_t)blockIdx.x * SEL_ROWS + (tid >> 7);
  float w[SEL_IT];
  bool mk[SEL_IT];
#pragma unroll
  for (int it = 0; it < SEL_IT; ++it) {   // every load issued before the first use
    const int64_t r = r0 + 2 * it;
    const bool ok = c < count && r < rows;
    const int64_t idx = (ok ? r : 0) * cols + i1 + (ok ? c : 0);
    w[it] = W[idx];
    mk[it] = ok && mask && mask[idx];
  }
  unsigned nmask = 0;
#pragma unroll
  for (int it = 0; it < SEL_IT; ++it) {
    if (!(c < count && r0 + 2 * it < rows)) continue;
    nmask += mk[it];
    const unsigned key = skey(saliency(w[it], dd2[c], mk[it]));
    if (pass == 0)
      atomicAdd(&lh[key >> 23], 1u);
    else if (pass == 1) {
      if ((key >> 23) == b0) atomicAdd(&lh[(key >> 12) & (NB1 - 1)], 1u);
    } else if ((key >> 12) == ((b0 << 11) | b1)) {
      atomicAdd(&lh[key & (NB2 - 1)], 1u);
    }
  }
  __syncthreads();
  unsigned* out = hs + (pass == 0 ? H0 : pass == 1 ? H1 : H2);
  for (int b = tid; b < nb; b += SEL_NT)
    if (lh[b]) atomicAdd(&out[b], lh[b]);
  if (pass == 0 && mask) {
    for (int o = 32; o > 0; o >>= 1) nmask += __shfl_xor(nmask, o);
    if ((tid & 63) == 0 && nmask) atomicAdd(&hs[HCNT], nmask);
  }
}

__global__ void fill_u32_kernel(unsigned* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// Per-lane state: working values, pruned bits of the lane's slots and (N:M
// with a preserved mask) the multiplier bits read from columns [j, j + m).
struct PruneState {
  float w[SW_T];
  unsigned bits;
  unsigned qbits;
};

// Number of the group's lanes with rotated index U..m-1 (lane (I + U) % 16
// of the row) whose broadcast (v, rotated index) orders before this lane's
// (v, t): smaller v, or equal v and smaller index.  Only the m lanes a group
// can hold are visited (m is uniform); members past the block's end
// broadcast +inf and have rotated indices past every real member's, so they
// never order before one.
template <int I, int U>
struct RankBefore {
  static __device__ __forceinline__ int run(float v, int t, int m) {
    const float sv = row_bcast<(I + U) & (SW_G - 1)>(v);
    const int here = (sv < v || (sv == v && U < t)) ? 1 : 0;
    return here + (U + 1 < m ? RankBefore<I, U + 1>::run(v, t, m) : 0);
  }
};
template <int I>
struct RankBefore<I, SW_G> {
  static __device__ __forceinline__ int run(float, int, int) { return 0; }
};

// N:M choice of the group that starts at block column I (I % m == 0) and
// ends at we (m <= 16): its columns are I .. we-1, held by lanes
// (I + t) % 16 for t = 0 .. we-I-1 (slot TO, then slot TO + 1 past the row's
// end), so the rotated lane index t orders them by column.  Each member
// ranks its tmp among the group's (lower column first on equal values) and is
// pruned when fewer than n rank before it.
template <int TO, int GO, bool PRESERVE>
__device__ __forceinline__ void nm_select(PruneState& S, const float* dd2, int g, int we, int n, int m) {
  constexpr int I = SW_G * TO + GO;
  const int t = (g - I) & (SW_G - 1);
  const bool member = t < we - I;
  const bool in_a = g >= (I & (SW_G - 1));  // the member's column is in slot TO
  float v = S.w[TO];
  if constexpr (TO + 1 < SW_T)
    if (!in_a) v = S.w[TO + 1];
  const int slot = in_a ? TO : TO + 1;
  const int col = I + t;
  const bool q = PRESERVE && ((S.qbits >> slot) & 1u);
  float tmp = saliency(v, dd2[min(col, MAXB - 1)], q);
  if (!member) tmp = __builtin_inff();
  const int rank = RankBefore<I, 0>::run(tmp, t, m);
  if (member && rank < n) S.bits |= 1u << slot;
}

// One column of the sweep: column I = SW_G * TO + GO, owned by lane GO.  The
// update of the slot holding column I + 1 comes first and ends the step's
// scheduling region, so the Hinv reads issued before it (two steps ahead)
// cannot sink into the step that uses them.
template <int TO, int GO, bool NM, bool PRESERVE, int MC>
__device__ __forceinline__ void prune_step(PruneState& S, const StepH& p, const float* dd2, int g, int count, int n,
                                           int m, int& next_group) {
  // MC > 0: the group width known at compile time (groups start at I % MC == 0)
  constexpr int I = SW_G * TO + GO;
  constexpr bool start_known = MC > 0;
  if (NM && (start_known ? I % (MC > 0 ? MC : 1) == 0 : I == next_group) && I < count) {
    const int mm = MC > 0 ? MC : m;
    next_group += mm;
    nm_select<TO, GO, PRESERVE>(S, dd2, g, min(I + mm, count), n, mm);
  }
  constexpr int TN = GO == SW_G - 1 ? TO + 1 : TO;  // slot of column I + 1
  const float x = S.w[TO];
  const float diff = ((S.bits >> TO) & 1u) ? x : 0.f;  // w - q
  const float err = div_by_recip(diff, p.dd, p.rd);
  const float e = row_bcast<GO>(err);
  auto update = [&](int t) __attribute__((always_inline)) {
    const float upd = S.w[t] - e * p.h[t];
    if (t == TO)
      S.w[t] = g > GO ? upd : S.w[t];
    else
      S.w[t] = upd;
  };
  if (TN < SW_T) update(TN);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = TO; t < SW_T; ++t)
    if (t != TN) update(t);
  // The updated values are materialised here: without this the compiler sinks
  // each slot's updates past the N:M and mask branches into one chain at the
  // slot's next use, keeping every earlier step's error alive (and spilled).
#pragma unroll
  for (int t = TO; t < SW_T; ++t) asm volatile("" : "+v"(S.w[t]));
}

// cur: the Hinv values of step I, nxt: those of step I + 1
template <int I, bool NM, bool PRESERVE, int MC>
struct PruneSteps {
  static __device__ __forceinline__ void run(PruneState& S, const float* h1, const float* rdg, const float* dd2,
                                             int g, int count, int n, int m, int& next_group, const StepH& cur,
                                             const StepH& nxt) {
    StepH nn;
    load_step<I + 2>(nn, h1, rdg, g);
    prune_step<I / SW_G, I % SW_G, NM, PRESERVE, MC>(S, cur, dd2, g, count, n, m, next_group);
    PruneSteps<I + 1, NM, PRESERVE, MC>::run(S, h1, rdg, dd2, g, count, n, m, next_group, nxt, nn);
  }
};
template <bool NM, bool PRESERVE, int MC>
struct PruneSteps<MAXB, NM, PRESERVE, MC> {
  static __device__ __forceinline__ void run(PruneState&, const float*, const float*, const float*, int, int, int,
                                             int, int&, const StepH&, const StepH&) {}
};

// NM: N:M groups (else the unstructured threshold in sel); PRESERVE: mask
// holds the entries to keep pruned.  Every launch runs all MAXB steps: in a
// block of count < MAXB columns the slots past count hold copies and LDS
// entries that are never written back, and a step only updates later
// columns, so they never reach the count columns that are.
template <bool NM, bool PRESERVE, int MC = 0>
__global__ __launch_bounds__(SW_NT, 4) void sgpt_sweep_kernel(float* __restrict__ W, int64_t rows, int64_t cols,
                                                              const float* __restrict__ hinv, int64_t i1, int count,
                                                              uint8_t* __restrict__ mask,
                                                              const unsigned* __restrict__ hs,
                                                              unsigned* __restrict__ hs_next, unsigned k, int n,
                                                              int m, float* __restrict__ losses,
                                                              float* __restrict__ err_out, int64_t lde,
                                                              int err_col) {
  __shared__ float h1[HPK];
  __shared__ float rdg[MAXB];  // 1 / Hinv[i][i], correctly rounded
  __shared__ float dd2[MAXB];  // Hinv[i][i]^2
  __shared__ unsigned sh[8];
  const int tid = threadIdx.x;
  const int g = tid & (SW_G - 1);
  const int64_t r = (int64_t)blockIdx.x * SW_ROWS + (tid / SW_G);
  const bool live = r < rows;
  const int64_t rr = live ? r : rows - 1;  // clamped row: every address below is in bounds

  PruneState S;
  S.bits = 0u;
  S.qbits = 0u;
#pragma unroll
  for (int t = 0; t < SW_T; ++t) {
    const int col = min(SW_G * t + g, count - 1);
    S.w[t] = W[rr * cols + i1 + col];
    if (PRESERVE) {
      if (mask[rr * cols + i1 + col]) {
        S.bits |= 1u << t;
        S.w[t] = 0.f;
      }
      if (NM && mask[rr * cols + col]) S.qbits |= 1u << t;
    }
  }
  const int dcol = tid < count ? tid : count - 1;
  const float diag = hinv[(i1 + dcol) * cols + i1 + dcol];
  load_hinv_block(h1, hinv, cols, i1, count, tid);
  if (tid < MAXB) {
    rdg[tid] = tid < count ? 1.f / diag : 1.f;
    dd2[tid] = diag * diag;
  }
  __syncthreads();

  if (!NM) {
    // the block's threshold key from the three histograms; the other set is
    // cleared for the next block (its last reader, the previous block's
    // sweep, has finished)
    unsigned b0, b1, b2, rem;
    find_bin(hs + H0, NB0, k, sh, b0, rem);
    find_bin(hs + H1, NB1, rem, sh, b1, rem);
    find_bin(hs + H2, NB2, rem, sh, b2, rem);
    const unsigned thresh = (b0 << 23) | (b1 << 12) | b2;
    if (blockIdx.x == 0)
      for (int i = tid; i < SET_WORDS; i += SW_NT) hs_next[i] = 0u;
    if (!PRESERVE || k > hs[HCNT]) {
#pragma unroll
      for (int t = 0; t < SW_T; ++t) {
        const int col = min(SW_G * t + g, count - 1);
        const float tmp = saliency(S.w[t], dd2[col], (S.bits >> t) & 1u);
        if (skey(tmp) <= thresh) S.bits |= 1u << t;
      }
    }
  }

  int next_group = 0;
  StepH p0, p1;
  load_step<0>(p0, h1, rdg, g);
  load_step<1>(p1, h1, rdg, g);
  PruneSteps<0, NM, PRESERVE, MC>::run(S, h1, rdg, dd2, g, count, n, m, next_group, p0, p1);

  // each slot is final: kept or zeroed value, error, loss
  float loss = 0.f;
#pragma unroll
  for (int t = 0; t < SW_T; ++t) {
    const int col = SW_G * t + g;
    const int cc = min(col, count - 1);
    const float dd = h1[hrow(cc)];
    const bool pr = (S.bits >> t) & 1u;
    const float x = S.w[t];
    const float diff = pr ? x : 0.f;
    const float err = div_by_recip(diff, dd, rdg[cc]);
    if (col < count) {
      loss = loss + diff * diff / (dd * dd);
      if (live) {
        const int64_t c = i1 + col;
        W[r * cols + c] = pr ? 0.f : x;
        err_out[r * lde + err_col + col] = err;
        if (NM && PRESERVE) mask[r * cols + c] = pr ? 1 : 0;
      }
    }
  }
#pragma unroll
  for (int o = 1; o < SW_G; o <<= 1) loss += __shfl_xor(loss, o, SW_G);
  if (live && g == 0) losses[r] = losses[r] + loss / 2.f;
}

template <class... A>
void launch_prune(bool nm, bool preserve, int prune_m, dim3 grid, hipStream_t st, A... args) {
  auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(SW_NT), 0, st, args...); };
  // 2:4 and other groups of four columns: the group starts and the rank
  // loop's length known at compile time
  if (nm && prune_m == 4) preserve ? go(sgpt_sweep_kernel<true, true, 4>) : go(sgpt_sweep_kernel<true, false, 4>);
  else if (nm) preserve ? go(sgpt_sweep_kernel<true, true>) : go(sgpt_sweep_kernel<true, false>);
  else    preserve ? go(sgpt_sweep_kernel<false, true>) : go(sgpt_sweep_kernel<false, false>);
}

__global__ void base_mask_kernel(const float* __restrict__ w, int64_t n, uint8_t* __restrict__ mask,
                                 unsigned* __restrict__ count) {
  unsigned c = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const bool z = w[i] == 0.f;
    mask[i] = z ? 1 : 0;
    c += z;
  }
  for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o);
  if ((threadIdx.x & 63) == 0 && c) atomicAdd(count, c);
}

size_t sel_offset(int64_t rows, int64_t cols, int64_t blocksize) {
  return ((size_t)rows * err_cols(cols, blocksize) * sizeof(float) + 255) & ~(size_t)255;
}

// k = int(numel * sparsity) as Python evaluates it (double product, truncated)
int64_t kth(int64_t numel, double sparsity) { return (int64_t)((double)numel * sparsity); }

}  // namespace
}  // namespace mi355q

using namespace mi355q;
using namespace mi355q::sweep;

extern "C" int mi355q_sparsegpt_base_mask(const float* w_work_dev, int64_t rows, int64_t cols, uint8_t* mask_dev,
                                          uint32_t* count_dev, void* stream) {
  MQ_CHECK_ARG(w_work_dev && mask_dev && count_dev, "sparsegpt_base_mask: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0 && rows * cols < (int64_t(1) << 32),
               "sparsegpt_base_mask: bad shape (at most 2^32 - 1 elements)");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, st, count_dev, 1);
  MQ_LAUNCH_CHECK();
  const int64_t n = rows * cols;
  int64_t nb = (n + 255) / 256;
  if (nb > 2048) nb = 2048;
  hipLaunchKernelGGL(base_mask_kernel, dim3((unsigned)nb), dim3(256), 0, st, w_work_dev, n, mask_dev, count_dev);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}

extern "C" size_t mi355q_sparsegpt_workspace_size(int64_t rows, int64_t cols, int64_t blocksize) {
  if (rows <= 0 || cols <= 0 || blocksize <= 0) return 0;
  return sel_offset(rows, cols, blocksize) + SEL_WORDS * sizeof(unsigned);
}

extern "C" int mi355q_sparsegpt_sweep(float* w_work_dev, int64_t rows, int64_t cols, const float* hinv_dev,
                                      double sparsity, int prune_n, int prune_m, int64_t blocksize,
                                      uint8_t* mask_dev, float* losses_dev, void* workspace_dev,
                                      size_t workspace_bytes, void* stream) {
  MQ_CHECK_ARG(w_work_dev && hinv_dev && losses_dev, "sparsegpt_sweep: null pointer");
  MQ_CHECK_ARG(rows > 0 && cols > 0, "sparsegpt_sweep: bad shape");
  MQ_CHECK_ARG(rows * MAXB < (int64_t(1) << 32), "sparsegpt_sweep: too many rows");
  if (blocksize > MAXB) {
    set_error("sparsegpt_sweep: block sizes above %d are not supported", MAXB);
    return MI355Q_UNSUPPORTED;
  }
  MQ_CHECK_ARG(blocksize > 0, "sparsegpt_sweep: blocksize must be positive");
  MQ_CHECK_ARG(prune_n >= 0, "sparsegpt_sweep: prune_n must be >= 0");
  const bool nm = prune_n > 0;
  const bool preserve = mask_dev != nullptr;
  if (nm) {
    MQ_CHECK_ARG(prune_m > 0, "sparsegpt_sweep: prune_m must be positive with prune_n > 0");
    if (prune_m > SW_G) {
      set_error("sparsegpt_sweep: N:M groups wider than %d columns are not supported", SW_G);
      return MI355Q_UNSUPPORTED;
    }
  } else {
    MQ_CHECK_ARG(sparsity >= 0.0, "sparsegpt_sweep: sparsity must be >= 0");
  }
  const int64_t B = blocksize;
  for (int64_t i1 = 0; i1 < cols; i1 += B) {
    const int64_t count = (i1 + B < cols ? i1 + B : cols) - i1;
    if (nm) {
      const int64_t j = ((count - 1) / prune_m) * prune_m;  // the block's last group
      MQ_CHECK_ARG(count - j >= prune_n && prune_m >= prune_n, "sparsegpt_sweep: selected index k out of range");
      const int64_t mw = (j + prune_m < cols ? j + prune_m : cols) - j;
      MQ_CHECK_ARG(!preserve || mw == count - j,
                   "sparsegpt_sweep: the N:M group at block column %lld spans %lld columns but its preserved-mask "
                   "window %lld (the reference fails to broadcast these)",
                   (long long)j, (long long)(count - j), (long long)mw);
    } else {
      MQ_CHECK_ARG(kth(rows * count, sparsity) < rows * count,
                   "sparsegpt_sweep: index %lld is out of bounds for a block of %lld values",
                   (long long)kth(rows * count, sparsity), (long long)(rows * count));
    }
  }
  const size_t need = mi355q_sparsegpt_workspace_size(rows, cols, blocksize);
  MQ_CHECK_ARG(workspace_dev && workspace_bytes >= need, "sparsegpt_sweep: workspace too small");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  float* err = static_cast<float*>(workspace_dev);
  unsigned* sel = reinterpret_cast<unsigned*>(static_cast<char*>(workspace_dev) + sel_offset(rows, cols, blocksize));
  int nblock = 0;  // blocks swept so far: block b counts into set b % 2
  const int64_t lde = err_cols(cols, blocksize);
  if (!nm) {
    hipLaunchKernelGGL(fill_u32_kernel, dim3(4), dim3(256), 0, st, sel, SEL_WORDS);
    MQ_LAUNCH_CHECK();
  }
  const unsigned nwg = (unsigned)((rows + SW_ROWS - 1) / SW_ROWS);
  const unsigned nsel = (unsigned)((rows + SEL_ROWS - 1) / SEL_ROWS);
  auto block = [&](int64_t i1, int64_t i2, int64_t s0) {
    const int count = (int)(i2 - i1);
    unsigned* hs = sel + (nblock & 1) * SET_WORDS;
    unsigned* hs_next = sel + ((nblock + 1) & 1) * SET_WORDS;
    ++nblock;
    const unsigned k = nm ? 0u : (unsigned)kth(rows * count, sparsity);
    if (!nm) {
      for (int pass = 0; pass < 3; ++pass) {
        hipLaunchKernelGGL(sgpt_select_kernel, dim3(nsel), dim3(SEL_NT), 0, st, w_work_dev, rows, cols, hinv_dev,
                           i1, count, mask_dev, hs, pass, k);
        MQ_LAUNCH_CHECK();
      }
    }
    launch_prune(nm, preserve, prune_m, dim3(nwg), st, w_work_dev, rows, cols, hinv_dev, i1, count, mask_dev,
                 (const unsigned*)hs, hs_next, k, prune_n, prune_m, losses_dev, err, lde, (int)(i1 - s0));
    MQ_LAUNCH_CHECK();
    return MI355Q_OK;
  };
  auto lazy = [&](int64_t k0, int64_t k1, int64_t s0, int64_t c0, int64_t c1) {
    return lazy_update(w_work_dev, rows, cols, 1, hinv_dev, (int64_t)0, err, lde, k0, k1, s0, c0, c1, st);
  };
  return blocked_schedule(cols, B, block, lazy);
}
