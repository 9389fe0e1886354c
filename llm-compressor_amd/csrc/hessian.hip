// Hessian accumulation H += alpha * X^T X (upper triangle) on gfx950.
//
// Replaces modifiers/gptq/gptq_quantize.py:22-32 (fp32 GEMM over the full
// d x d matrix) with a syrk that computes and writes only the tiles on or
// above the diagonal.  X rows are tokens (bf16, feature-contiguous); the
// contraction runs over tokens, so both MFMA operands need token-contiguous
// fragments.  bf16 x bf16 products are exact in fp32 and accumulate in fp32
// (v_mfma_f32_32x32x16_bf16).
//
// Two tile kernels share the work decomposition below:
//  * syrk_stream_kernel (d >= 512, and every grouped call): 256 x 256 tiles
//    streamed global -> LDS by LDS-DMA in token-major layout and read back
//    with the transposing LDS load (details at the kernel); for per-expert
//    Hessians the DMA gathers the routed rows itself;
//  * syrk_bf16_kernel (dense X with d < 512): each thread loads an 8-token
//    x 8-feature block with eight 16-byte loads and transposes it in
//    registers (v_perm) before the LDS store; the transposed stores map
//    lane -> (feature block, token block) with the token block fastest,
//    which keeps 16 consecutive lanes on distinct LDS banks (row stride
//    144 B = 9 x 16 B).
// Tiles are TM x TM (TM = 256 for d >= 512, else 128).  syrk_bf16_kernel runs
// them on a 2 x 2 grid of waves, each owning a (TM/2)^2 block of 32 x 32 MFMA
// tiles; the streaming kernel on a 2 x 4 grid of 8 waves (two per SIMD, so
// one wave's waits are covered by the other's MFMAs), each owning 128 x 64.
// syrk_bf16_kernel writes partial tiles in its fragment order (one 16-float
// run per thread and block); the streaming kernel in 1 KB chunks of one
// float4 per lane, which its own reduction reads back coalesced, or, for a
// single split, adds its tile to H through LDS one 1 KB row at a time.
//
// Dense work decomposition: a work item is (upper tile t, token split s).
// Token splits are assigned by blockIdx % S, and workgroups are dispatched
// round-robin over the 8 XCDs, so with S = 8 each XCD streams only its own
// eighth of X through its L2.  With S > 1 each item writes its partial tile
// to the workspace and a second kernel sums the partials in split order and
// updates H, so results are deterministic.
//
// Grouped (per-expert) decomposition: each expert's routed tokens are cut
// into chunks of kChunkTokens; a work item is (chunk, upper tile).  The
// chunk table is built on the device from the expert offsets, so a call
// never waits for the host.  The first chunk of an expert adds its tile to
// H directly; later chunks write partial slots that a second kernel adds in
// chunk order afterwards (deterministic).  Items are laid out chunk-major
// and each XCD takes a contiguous eighth of them, so the tiles of one chunk
// run on one XCD and share its rows through that XCD's L2.
#include <vector>

#include "common.h"
#include "linalg.h"

namespace mi355q {

namespace {

constexpr int BK = 64;           // tokens per LDS stage
constexpr int NT = 256;          // threads per workgroup (4 waves, 2x2)
constexpr int LDS_ROW = BK + 8;  // bf16 elements per feature row, +16 B pad

struct Matrix {            // one Hessian being accumulated
  int64_t row_begin;       // first index into rows[] (or first token)
  int64_t row_count;       // tokens for this matrix
  float* h;                // d x d, leading dimension ldh
};

constexpr int kChunkTokens = 4096;  // tokens per grouped work chunk (its row indices fit in LDS)

struct GChunk {            // one chunk of one expert's tokens (device-built table)
  int e;                   // expert
  int count;               // tokens, 1 .. kChunkTokens
  int64_t tok_begin;       // first token: index into rows[] (or into x without rows)
  int64_t sbase;           // partial slot of tile 0 (tile t -> sbase + t); -1: add to H directly
};

struct GReduce {           // the later chunks of one expert, added to H in chunk order
  int e;
  int nslots;              // chunks after the first
  int64_t sbase;           // slot of tile 0 of the second chunk; chunk k at sbase + (k - 1) T
};

struct SyrkParams {
  const uint16_t* x;
  int64_t ldx;
  int64_t d;
  int64_t ldh;
  int nt;                  // tiles per edge
  float alpha;
  float beta;              // H = beta * H + alpha * X^T X (beta == 1: H += ...)
  Matrix single;           // dense mode
  int S;
  // dense tail: tiles t >= tail_start run as tail_f parts per split (see
  // plan_dense); tail_start = number of tiles when there is no tail
  int tail_start, tail_f;
  float* ws;               // partial tiles
  // grouped mode
  const int32_t* rows;     // token -> row of x (nullptr: x rows are already grouped)
  int64_t n_x;             // rows of x (gathered indices are clamped into [0, n_x))
  const GChunk* chunks;
  const int* gcounts;      // [0] chunks, [1] reduce items (written by the planner)
  int* queues;             // 8 work-queue counters (zeroed by the planner)
  int T;                   // upper tiles per matrix
  float* h0;               // H of expert 0 (leading dimension d)
  int64_t h_stride;
};

// Dense syrk over rows held in separate buffers (the calls a Hessian hook
// keeps by reference until it flushes): segment k has rows[k] > 0 rows at
// x[k], all with the call's ldx, and takes stages stage0[k] .. stage0[k + 1]
// - 1 of the concatenated stage sequence (its last stage zero-padded past
// rows[k]).  Passed by value as a kernel argument.
constexpr int kMaxSegments = 64;
struct SegTable {
  int n;
  int64_t stage0[kMaxSegments + 1];
  int64_t rows[kMaxSegments];
  const uint16_t* x[kMaxSegments];
};

// The t-th tile on or above the diagonal, in super-block order: super-blocks
// of SBK x SBK tiles (I <= J, row-major), tiles inside row-major.  Workgroups
// of one XCD run consecutive t together, so a round of concurrent tiles
// touches about 2 SBK feature slices of X instead of all of them, and the
// slices it streams are shared through that XCD's L2.
// beta * h as its own rounded multiply (the reference scales H before adding
// the product); beta == 1 leaves h as it is
__device__ __forceinline__ float scaled(float h, float beta) { return beta == 1.f ? h : h * beta; }

__device__ __forceinline__ void tile_coords(int t, int nt, int& ti, int& tj) {
  constexpr int SBK = 8;
  const int nb = (nt + SBK - 1) / SBK;
  for (int I = 0; I < nb; ++I) {
    const int i0 = I * SBK, i1 = min(nt, i0 + SBK);
    for (int J = I; J < nb; ++J) {
      const int j0 = J * SBK, j1 = min(nt, j0 + SBK);
      const int m = i1 - i0, w = j1 - j0;
      const int cnt = I == J ? m * (m + 1) / 2 : m * w;
      if (t < cnt) {
        if (I == J) {
          int r = 0, rowlen = m;
          while (t >= rowlen) {
            t -= rowlen;
            ++r;
            --rowlen;
          }
          ti = i0 + r;
          tj = i0 + r + t;
        } else {
          ti = i0 + t / w;
          tj = j0 + t % w;
        }
        return;
      }
      t -= cnt;
    }
  }
  ti = tj = 0;  // t >= nt (nt + 1) / 2 is never launched
}

__device__ __forceinline__ unsigned perm_lo(unsigned a, unsigned b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);  // lo16(a) | lo16(b) << 16
}
__device__ __forceinline__ unsigned perm_hi(unsigned a, unsigned b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);  // hi16(a) | hi16(b) << 16
}

// 32 x 32 x 16 MFMA on 16-bit operands: bf16, or fp16 (F16) -- both form
// exact products in fp32; the operand bits move through the same registers.
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
template <bool F16>
__device__ __forceinline__ f32x16_t mfma16(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                  c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Load one 8 (tokens) x 8 (features) block into r[8] (4 dwords each): tokens
// stage0 + lt0 + 0..7 of the matrix, features f..f+7.  Branch-free:
// out-of-range tokens / features read a clamped in-range address, and the
// returned mask (bit tt = token tt valid) zeroes them when the block is
// stored, so the eight loads issue back to back and nothing waits for them
// before the MFMAs of the current stage.  X is addressed as a wave-uniform
// stage base plus a 32-bit lane offset.
__device__ __forceinline__ unsigned load_block(const SyrkParams& p, int64_t stage0, int lt0, int64_t tok_end,
                                               int64_t row_base, int64_t f, u32x4_t r[8]) {
  const bool fin = f < p.d;
  const int64_t fc = fin ? f : 0;
  const int64_t rem = tok_end - stage0;           // >= 1 for a stage in range
  const int lim = rem < BK ? (int)rem : BK;
  const char* base = reinterpret_cast<const char*>(p.x + (row_base + stage0) * p.ldx);
#pragma unroll
  for (int tt = 0; tt < 8; ++tt) {
    const int lt = lt0 + tt;
    const int ltc = lt < lim ? lt : lim - 1;
    const uint32_t off = (uint32_t)(ltc * p.ldx + fc) * 2u;
    r[tt] = *reinterpret_cast<const u32x4_t*>(base + off);
  }
  const int nv = lim - lt0;
  return !fin || nv <= 0 ? 0u : (nv >= 8 ? 0xffu : (1u << nv) - 1u);
}

// Transpose r (token-major) and store 8 feature rows of 8 tokens to LDS;
// tokens whose mask bit is clear are stored as zeros.
__device__ __forceinline__ void store_block(uint16_t* lds, int fb, int kb, const u32x4_t r[8], unsigned mask) {
  u32x4_t z[8];
#pragma unroll
  for (int tt = 0; tt < 8; ++tt) {
    const unsigned m = (mask >> tt) & 1u ? 0xffffffffu : 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) z[tt][j] = r[tt][j] & m;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {     // feature pair (2j, 2j+1)
    u32x4_t lo, hi;
#pragma unroll
    for (int q = 0; q < 4; ++q) {   // token pair (2q, 2q+1)
      lo[q] = perm_lo(z[2 * q][j], z[2 * q + 1][j]);
      hi[q] = perm_hi(z[2 * q][j], z[2 * q + 1][j]);
    }
    *reinterpret_cast<u32x4_t*>(lds + (8 * fb + 2 * j) * LDS_ROW + 8 * kb) = lo;
    *reinterpret_cast<u32x4_t*>(lds + (8 * fb + 2 * j + 1) * LDS_ROW + 8 * kb) = hi;
  }
}

template <int TM>
struct Cfg {
  static constexpr int W = TM / 2;            // wave tile edge
  static constexpr int NB = W / 32;           // 32x32 MFMA blocks per wave edge
  static constexpr int ACC = NB * NB * 16;    // accumulator floats per lane
  static constexpr int BLK = TM / 128;        // 8x8 load blocks per thread per operand
  static constexpr int OPLDS = TM * LDS_ROW;  // bf16 elements per operand buffer
  static constexpr int TILE = TM * TM;
};

template <int TM, bool F16 = false>
__global__ __launch_bounds__(NT, TM == 128 ? 2 : 1) void syrk_bf16_kernel(SyrkParams p) {
  using C = Cfg<TM>;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][2][C::OPLDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int S = p.S;
  const int s = blockIdx.x % S;
  const int t = blockIdx.x / S;
  const Matrix mat = p.single;
  const int64_t slot = (S > 1) ? (int64_t)t * S + s : -1;
  int ti, tj;
  tile_coords(t, p.nt, ti, tj);

  // token range of this split, rounded to whole stages
  const int64_t n = mat.row_count;
  const int64_t nst_total = (n + BK - 1) / BK;
  const int64_t st_per = (nst_total + S - 1) / S;
  const int64_t st_begin = (int64_t)s * st_per;
  int64_t st_end = st_begin + st_per;
  if (st_end > nst_total) st_end = nst_total;
  const int64_t nst = st_end > st_begin ? st_end - st_begin : 0;

  // loader roles: (operand, block u) -> feature block u / 8, token block u % 8
  int op[C::BLK > 1 ? 2 : 1], fbk[C::BLK > 1 ? 2 : 1], kbk[C::BLK > 1 ? 2 : 1];
  int64_t fbase[C::BLK > 1 ? 2 : 1];
  constexpr int NL = C::BLK > 1 ? 2 : 1;
#pragma unroll
  for (int b = 0; b < NL; ++b) {
    const int u = (TM == 128) ? (tid & 127) : tid;
    op[b] = (TM == 128) ? (tid >> 7) : b;
    fbk[b] = u >> 3;
    kbk[b] = u & 7;
    fbase[b] = (int64_t)(op[b] ? tj : ti) * TM + 8 * fbk[b];
  }

  f32x16_t acc[C::NB][C::NB];
#pragma unroll
  for (int a = 0; a < C::NB; ++a)
#pragma unroll
    for (int b = 0; b < C::NB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  u32x4_t regs[NL][8];
  unsigned vmask[NL];
  if (nst > 0) {
#pragma unroll
    for (int b = 0; b < NL; ++b)
      vmask[b] = load_block(p, st_begin * BK, 8 * kbk[b], n, mat.row_begin, fbase[b], regs[b]);
#pragma unroll
    for (int b = 0; b < NL; ++b) store_block(lds[0][op[b]], fbk[b], kbk[b], regs[b], vmask[b]);
  }
  __syncthreads();

  for (int64_t st = 0; st < nst; ++st) {
    const int buf = st & 1;
    const bool more = st + 1 < nst;
    if (more) {
#pragma unroll
      for (int b = 0; b < NL; ++b)
        vmask[b] = load_block(p, (st_begin + st + 1) * BK, 8 * kbk[b], n, mat.row_begin, fbase[b], regs[b]);
    }
    const uint16_t* la = lds[buf][0];
    const uint16_t* lb = lds[buf][1];
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int koff = kk * 16 + 8 * (lane >> 5);
      bf16x8_t fa[C::NB], fbv[C::NB];
#pragma unroll
      for (int bm = 0; bm < C::NB; ++bm)
        fa[bm] = *reinterpret_cast<const bf16x8_t*>(la + (wm * C::W + bm * 32 + (lane & 31)) * LDS_ROW + koff);
#pragma unroll
      for (int bn = 0; bn < C::NB; ++bn)
        fbv[bn] = *reinterpret_cast<const bf16x8_t*>(lb + (wn * C::W + bn * 32 + (lane & 31)) * LDS_ROW + koff);
#pragma unroll
      for (int bm = 0; bm < C::NB; ++bm)
#pragma unroll
        for (int bn = 0; bn < C::NB; ++bn)
          acc[bm][bn] = mfma16<F16>(fa[bm], fbv[bn], acc[bm][bn]);
    }
    if (more) {
#pragma unroll
      for (int b = 0; b < NL; ++b) store_block(lds[buf ^ 1][op[b]], fbk[b], kbk[b], regs[b], vmask[b]);
    }
    __syncthreads();
  }

  if (slot >= 0) {
    float* dst = p.ws + (slot * NT + tid) * C::ACC;
#pragma unroll
    for (int bm = 0; bm < C::NB; ++bm)
#pragma unroll
      for (int bn = 0; bn < C::NB; ++bn)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          f32x4_t v = {acc[bm][bn][4 * q], acc[bm][bn][4 * q + 1], acc[bm][bn][4 * q + 2],
                       acc[bm][bn][4 * q + 3]};
          *reinterpret_cast<f32x4_t*>(dst + (bm * C::NB + bn) * 16 + 4 * q) = v;
        }
    return;
  }

  // direct update of the upper triangle, one 32 x 32 block at a time (the
  // scheduling barrier keeps the blocks' loads from being hoisted together,
  // which would need more registers than the accumulators leave free)
  const bool diag = ti == tj;
#pragma unroll
  for (int bm = 0; bm < C::NB; ++bm)
#pragma unroll
    for (int bn = 0; bn < C::NB; ++bn) {
      const int mb = wm * C::W + bm * 32, nb = wn * C::W + bn * 32;
      const int64_t gib = (int64_t)ti * TM + mb, gjb = (int64_t)tj * TM + nb;
      float* hb = mat.h + gib * p.ldh + gjb;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int mi = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3), nj = lane & 31;
        if (gib + mi < p.d && gjb + nj < p.d && (!diag || mb + mi <= nb + nj)) {
          float* hp = hb + (int64_t)mi * p.ldh + nj;
          *hp = scaled(*hp, p.beta) + p.alpha * acc[bm][bn][r];
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
}

// ---------------------------------------------------------------- streaming syrk
// Dense X, 256 x 256 tiles.  Tiles of X are copied global -> LDS by the
// gfx950 LDS-DMA load (global_load_lds_dwordx4: no registers, no VALU) in
// their natural token-major layout, through a ring of NSTG stages of SK
// tokens, so the loads of stage s + NSTG - 1 are in flight while stage s is
// multiplied.  The MFMA operands (8 consecutive tokens of one feature per
// lane) are read with the transposing LDS load ds_read_b64_tr_b16: for lane
// L = 16 g + 4 q + r it returns element r of the 8-byte rows supplied by
// lanes 16 g + 4 e + q, e = 0..3.  Each token row (256 features, 512 B) is
// stored with its 16-byte chunks XOR-swizzled by 4 (row & 3), which keeps
// both the DMA writes and the transposed reads free of bank conflicts.
constexpr int SK = 32;           // tokens per stage
constexpr int NSTG = 4;          // stages in the LDS ring
constexpr int SROW = 512;        // bytes per token row of a 256-feature operand
constexpr int SOP = SK * SROW;   // bytes per operand per stage
// Waves of the streaming kernel.  The 4-wave layout (128 x 128 per wave, a
// third fewer LDS reads per MFMA, one wave per SIMD) gives the same results
// bit for bit and was measured slower on heavy-tailed activations: 2.14
// against 2.11 ms at 131072 x 4096, 76 against 59 us at 2048 tokens, 105.0
// against 101.5 ms at 524288 x 14336 (four token splits), 202.5 against
// 197.9 ms at 262144 x 28672; it won only on Gaussian inputs at 524288 x
// 14336 (93.9 against 97.4 ms, two splits), where the chip ran more
// power-limited.
constexpr int kStreamWaves = 8;
constexpr int SNT = 64 * kStreamWaves;             // its threads

typedef short v4s16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s16_t lds_v4s16_t;
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __attribute__((aligned(16))) const uint32_t kZeroChunk[4] = {0u, 0u, 0u, 0u};

__device__ __forceinline__ bf16x8_t tr_pair(const char* lds, int off0, int off1) {
  const v4s16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s16_t*)(lds + off0));
  const v4s16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s16_t*)(lds + off1));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

enum StreamMode { kDense = 0, kGrouped = 1, kGroupedGather = 2, kDenseSeg = 3 };

// One work item of the streaming kernel: tile t of matrix `mat` over token
// split s (and part `part` of `nparts` for dense tail tiles), into partial
// slot `slot` (-1: H directly).  `ring` is the workgroup's 128 KiB LDS ring,
// `ridx` its row-index cache (gathered chunks); `sg` the segment table of
// kDenseSeg (whose `mat` counts the padded stages' rows).
template <bool F16, int MODE, int WAVES>
__device__ __forceinline__ void stream_item(const SyrkParams& p, char* ring, int* ridx, int t, int s, int part,
                                            int nparts, int S, int64_t slot, Matrix mat,
                                            const SegTable* sg = nullptr) {
  // WAVES = 8: a 2 x 4 grid of waves (two per SIMD), each 4 x 2 MFMA blocks
  // (128 rows x 64 columns); WAVES = 4: a 2 x 2 grid (one per SIMD), each
  // 4 x 4 blocks (128 x 128), a third fewer LDS reads per MFMA
  constexpr int MB = 4, NBN = WAVES == 8 ? 2 : 4;
  constexpr int NTH = 64 * WAVES;
  constexpr int RPW = 32 / WAVES;   // token rows per operand and stage each wave copies
  constexpr int NJ = RPW / 2;       // DMA instructions per operand and stage (two rows each)
  constexpr int NDMA = 2 * NJ;
  using C = Cfg<256>;
  constexpr int TM = 256;
  // LDS ring: operand A in stages 0..3, then operand B; after the loop it
  // holds half an fp32 tile for the direct update of H
  char* const a0 = ring;
  char* const a1 = ring + SOP;
  char* const a2 = ring + 2 * SOP;
  char* const a3 = ring + 3 * SOP;
  char* const b0 = ring + 4 * SOP;
  char* const b1 = ring + 5 * SOP;
  char* const b2 = ring + 6 * SOP;
  char* const b3 = ring + 7 * SOP;

  // the thread index through an opaque copy: in the grouped kernel's item
  // loop nothing derived from it is hoisted out of the loop and kept live
  // across items (which spilled the loop's registers to scratch)
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int wm = WAVES == 8 ? wave >> 2 : wave >> 1, wn = WAVES == 8 ? wave & 3 : wave & 1;
  int ti, tj;
  tile_coords(t, p.nt, ti, tj);

  const int64_t n = mat.row_count;
  const int64_t nst_total = (n + SK - 1) / SK;
  const int64_t st_per = (nst_total + S - 1) / S;
  int64_t st_begin = (int64_t)s * st_per;
  int64_t st_end = st_begin + st_per;
  if (st_end > nst_total) st_end = nst_total;
  if (nparts > 1 && st_end > st_begin) {
    const int64_t per = (st_end - st_begin + nparts - 1) / nparts;
    const int64_t b2 = st_begin + part * per;
    const int64_t e2 = b2 + per < st_end ? b2 + per : st_end;
    st_begin = b2;
    st_end = e2;
  }
  const int64_t nst = st_end > st_begin ? st_end - st_begin : 0;

  if constexpr (MODE == kGroupedGather) {
    for (int i = tid; i < (int)n; i += NTH) {
      const int64_t r = p.rows[mat.row_begin + i];
      ridx[i] = (int)(r < 0 ? 0 : (r >= p.n_x ? p.n_x - 1 : r));
    }
    __syncthreads();
  }

  // DMA roles: wave w copies token rows RPW w .. RPW w + RPW - 1 of each
  // operand, two rows (1 KB) per instruction j; lane L fills LDS position
  // L & 31 of row RPW w + 2 j + L / 32 with global chunk (L & 31) ^ 4 (row & 3).
  const int64_t fa0 = (int64_t)ti * TM, fb0 = (int64_t)tj * TM;
  const bool edge = fa0 + TM > p.d || fb0 + TM > p.d;
  uint32_t doff[NJ];    // lane byte offsets from the stage's first token row
  int drow[NJ], dchunk[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int row = RPW * wave + 2 * j + (lane >> 5);
    const int chunk = (lane & 31) ^ (4 * (row & 3));
    drow[j] = row;
    dchunk[j] = chunk;
    doff[j] = (uint32_t)(row * p.ldx + 8 * chunk) * 2u;
  }
  // The DMA is issued from inline asm so that the compiler does not treat
  // every later LDS read as dependent on it (it cannot tell the ring slots
  // apart and would wait for all DMA in flight); completion is tracked
  // explicitly with vmcnt before each barrier and after the loop.  Whole
  // stages use the scalar-base form (stage base in SGPRs + the lane's 32-bit
  // offset); partial stages, edge tiles and gathered rows use per-lane 64-bit
  // addresses, with lanes past n or d sent to a zero chunk.  M0 (the LDS
  // destination of the wave's 1 KB) is formed in scalar registers.
  auto lds_u32 = [](const char* ptr) { return (uint32_t)reinterpret_cast<uintptr_t>((lds_void_t*)ptr); };
  const uint32_t wave_lds = (uint32_t)wave * (RPW * SROW);
  const uint32_t sa[4] = {lds_u32(a0) + wave_lds, lds_u32(a1) + wave_lds, lds_u32(a2) + wave_lds,
                          lds_u32(a3) + wave_lds};
  const uint32_t sb[4] = {lds_u32(b0) + wave_lds, lds_u32(b1) + wave_lds, lds_u32(b2) + wave_lds,
                          lds_u32(b3) + wave_lds};
  auto dma_s = [&](uint32_t off, const char* base, uint32_t m0) __attribute__((always_inline)) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m0)
                 : "memory", "m0");
  };
  auto dma_v = [&](const void* gaddr, uint32_t m0) __attribute__((always_inline)) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gaddr), "s"(m0) : "memory", "m0");
  };
  const char* xbase = reinterpret_cast<const char*>(p.x + (mat.row_begin + st_begin * SK) * p.ldx);
  const int64_t sbytes = (int64_t)SK * p.ldx * 2;  // bytes per stage
  const bool fast_ok = MODE != kGroupedGather && !edge;
  // kDenseSeg: a cursor over the segment table, kept in scalar registers.
  // Stages are asked for in non-decreasing order (issue, then dma_addrs of
  // stage + 3), so it only moves forward; a binary search places it on the
  // segment of the item's first stage.
  int sk = 0;
  const char* seg_x = nullptr;
  int64_t seg_b = 0, seg_e = 0, seg_rows = 0;
  auto seg_load = [&]() __attribute__((always_inline)) {
    seg_x = reinterpret_cast<const char*>(sg->x[sk]);
    seg_b = sg->stage0[sk];
    seg_e = sg->stage0[sk + 1];
    seg_rows = sg->rows[sk];
  };
  if constexpr (MODE == kDenseSeg) {
    int lo = 0, hi = sg->n - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (sg->stage0[mid] <= st_begin) lo = mid; else hi = mid - 1;
    }
    sk = lo;
    seg_load();
  }
  // stage sc of this item: its first token row and how many of its SK rows
  // exist (>= SK: a whole stage)
  auto stage_rows = [&](int64_t sc, const char*& xs, int64_t& avail) __attribute__((always_inline)) {
    if constexpr (MODE == kDenseSeg) {
      const int64_t G = st_begin + sc;
      while (G >= seg_e && sk + 1 < sg->n) {
        ++sk;
        seg_load();
      }
      const int64_t l = G - seg_b;
      xs = seg_x + l * sbytes;
      avail = seg_rows - l * SK;
    } else {
      xs = xbase + sc * sbytes;
      avail = n - (st_begin + sc) * SK;
    }
  };
  // Per-lane global addresses of the NDMA DMAs of a stage (A0, B0, A1, B1, ...):
  // lanes past n or d read the zero chunk.
  auto dma_addrs = [&](int64_t stage, const void** ad) __attribute__((always_inline)) {
    const int64_t sc = stage < nst ? stage : nst - 1;
    if constexpr (MODE == kGroupedGather) {
      const int64_t t0 = (st_begin + sc) * SK;
      const char* xg = reinterpret_cast<const char*>(p.x);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int lt = (int)t0 + drow[j];
        const bool rok = lt < n;
        const char* xr = xg + (int64_t)ridx[rok ? lt : 0] * p.ldx * 2 + (int64_t)dchunk[j] * 16;
        const bool aok = rok && fa0 + 8 * dchunk[j] < p.d;
        const bool bok = rok && fb0 + 8 * dchunk[j] < p.d;
        ad[2 * j] = aok ? (const void*)(xr + fa0 * 2) : (const void*)kZeroChunk;
        ad[2 * j + 1] = bok ? (const void*)(xr + fb0 * 2) : (const void*)kZeroChunk;
      }
    } else {
      const char* xs;
      int64_t avail;
      stage_rows(sc, xs, avail);
      const char* xa = xs + fa0 * 2;
      const char* xb = xs + fb0 * 2;
      if (fast_ok && avail >= SK) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          ad[2 * j] = xa + doff[j];
          ad[2 * j + 1] = xb + doff[j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const bool rok = drow[j] < avail;
          const bool aok = rok && fa0 + 8 * dchunk[j] < p.d;
          const bool bok = rok && fb0 + 8 * dchunk[j] < p.d;
          ad[2 * j] = aok ? (const void*)(xa + doff[j]) : (const void*)kZeroChunk;
          ad[2 * j + 1] = bok ? (const void*)(xb + doff[j]) : (const void*)kZeroChunk;
        }
      }
    }
  };
  auto issue = [&](int64_t stage, int slot) __attribute__((always_inline)) {
    const int64_t sc = stage < nst ? stage : nst - 1;
    const char* xs = nullptr;
    int64_t avail = 0;
    if constexpr (MODE != kGroupedGather) stage_rows(sc, xs, avail);
    if (fast_ok && avail >= SK) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        dma_s(doff[j], xs + fa0 * 2, sa[slot] + 1024u * j);
        dma_s(doff[j], xs + fb0 * 2, sb[slot] + 1024u * j);
      }
    } else {
      const void* ad[NDMA];
      dma_addrs(stage, ad);
#pragma unroll
      for (int i = 0; i < NDMA; ++i) dma_v(ad[i], ((i & 1) ? sb[slot] : sa[slot]) + 1024u * (i >> 1));
    }
  };

  // transposed-read lane offsets: lane 16 g + 4 e + q supplies row
  // 8 (g >> 1) + e (+ 16 kk + 4 h) and features 16 (g & 1) + 4 q of the
  // 32-feature block; with the swizzle the 16-byte position of 32-feature
  // block B of the row is 4 (B ^ e) + 2 (g & 1) + (q >> 1)
  const int g = lane >> 4, e = (lane >> 2) & 3, q = lane & 3;
  const int rbase = (8 * (g >> 1) + e) * SROW + 8 * (q & 1);
  int ra[MB], rb[NBN];
#pragma unroll
  for (int b = 0; b < MB; ++b) ra[b] = rbase + 16 * (4 * ((MB * wm + b) ^ e) + 2 * (g & 1) + (q >> 1));
#pragma unroll
  for (int b = 0; b < NBN; ++b) rb[b] = rbase + 16 * (4 * ((NBN * wn + b) ^ e) + 2 * (g & 1) + (q >> 1));

  f32x16_t acc[MB][NBN];
#pragma unroll
  for (int x = 0; x < MB; ++x)
#pragma unroll
    for (int y = 0; y < NBN; ++y)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[x][y][r] = 0.f;

  // Software pipeline over half-stages (16-token steps): the MFMAs of one
  // step run while the operands of the next step are read, including across
  // the stage boundary, so the barrier that publishes stage st + 1 sits in
  // the middle of stage st (between its two steps) and the MFMA pipe does not
  // drain at stage boundaries.  F0 / F1 hold the operands of step 0 / step 1.
  bf16x8_t fa0r[MB], fb0r[NBN], fa1r[MB], fb1r[NBN];
  auto read_op = [&](const char* la, const char* lb, int kk, int i, bf16x8_t* fa, bf16x8_t* fb)
      __attribute__((always_inline)) {
    // operand i of a step: A fragments 0..MB-1, then B fragments
    if (i < MB)
      fa[i] = tr_pair(la, ra[i] + kk * 16 * SROW, ra[i] + (kk * 16 + 4) * SROW);
    else
      fb[i - MB] = tr_pair(lb, rb[i - MB] + kk * 16 * SROW, rb[i - MB] + (kk * 16 + 4) * SROW);
  };
  // MFMAs of one step (operands fa, fb) interleaved with the 2 NB fragment
  // reads of the next step: two tr reads per MFMA for the first NB MFMAs
  auto half = [&](const bf16x8_t* fa, const bf16x8_t* fb, const char* la, const char* lb, int kk, bf16x8_t* na,
                  bf16x8_t* nb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < MB + NBN; ++i) read_op(la, lb, kk, i, na, nb);
#pragma unroll
    for (int x = 0; x < MB; ++x)
#pragma unroll
      for (int y = 0; y < NBN; ++y)
        acc[x][y] = mfma16<F16>(fa[x], fb[y], acc[x][y]);
#pragma unroll
    for (int i = 0; i < MB + NBN; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, MB * NBN - (MB + NBN), 0);
  };
  // Step MFMAs with the next step's reads and one DMA after every two MFMAs.
  // A burst of DMAs right after the barrier stalls the issuing wave until the
  // load path drains them (and its MFMAs with it); one DMA per 64 MFMA cycles
  // keeps the path under half load.  A scheduling barrier after each group
  // keeps the interleave in source order.
  auto half_dma = [&](const bf16x8_t* fa, const bf16x8_t* fb, const char* la, const char* lb, int kk, bf16x8_t* na,
                      bf16x8_t* nb, const void* const* ad, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < MB * NBN; ++i) {
      const int x = i / NBN, y = i % NBN;
      acc[x][y] = mfma16<F16>(fa[x], fb[y], acc[x][y]);
      if (i < MB + NBN) read_op(la, lb, kk, i, na, nb);
      if constexpr (WAVES == 8) {
        if (i < 4) dma_v(ad[i], ((i & 1) ? sb[slot] : sa[slot]) + 1024u * (i >> 1));
      } else if ((i & 1) == 0) {
        const int k = i >> 1;
        dma_v(ad[k], ((k & 1) ? sb[slot] : sa[slot]) + 1024u * (k >> 1));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // stage st (slot st % 4 = cur): step-0 MFMAs with the step-1 reads of stage
  // st; barrier publishing stage st + 1 (this wave's DMA of stage st + 1 done:
  // only stage st + 2 may be in flight) and freeing slot st - 1, which takes
  // stage st + 3; step-1 MFMAs with the step-0 reads of stage st + 1 and the
  // DMA of stage st + 3.  (A bare s_barrier: __syncthreads would also wait
  // for the DMA of stage st + 2.)
  auto stage = [&](int64_t st, int cur, const char* la, const char* lb, const char* lan, const char* lbn)
      __attribute__((always_inline)) {
    const void* ad[NDMA];
    dma_addrs(st + 3, ad);
    half(fa0r, fb0r, la, lb, 1, fa1r, fb1r);
    if constexpr (NDMA == 4)
      asm volatile("s_waitcnt vmcnt(4)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
    half_dma(fa1r, fb1r, lan, lbn, 0, fa0r, fb0r, ad, (cur + 3) & 3);
  };

  if (nst > 0) {
    issue(0, 0);
    issue(1, 1);
    issue(2, 2);
    if constexpr (NDMA == 4)
      asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int i = 0; i < MB + NBN; ++i) read_op(a0, b0, 0, i, fa0r, fb0r);
    for (int64_t st = 0; st < nst; st += 4) {
      stage(st, 0, a0, b0, a1, b1);
      if (st + 1 < nst) stage(st + 1, 1, a1, b1, a2, b2);
      if (st + 2 < nst) stage(st + 2, 2, a2, b2, a3, b3);
      if (st + 3 < nst) stage(st + 3, 3, a3, b3, a0, b0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }

  if (slot < 0) {
    const bool diag = ti == tj;
    const int64_t ldh = (MODE == kDense || MODE == kDenseSeg) ? p.ldh : p.d;
    if (p.beta == 0.f) {
      // H not read: each accumulator register goes straight to its row of H
      // (a store covers 32 consecutive columns of two rows, lanes 0..31 and
      // 32..63), with no pass through LDS and no barrier.  An off-diagonal
      // tile inside H stores without a test (per-element tests put each of
      // the 128 stores per lane in a branch of its own).
      auto put = [&](auto masked) __attribute__((always_inline)) {
#pragma unroll
        for (int x = 0; x < MB; ++x)
#pragma unroll
          for (int y = 0; y < NBN; ++y)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int64_t gi = fa0 + wm * 128 + x * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
              const int64_t gj = fb0 + wn * NBN * 32 + y * 32 + (lane & 31);
              if (!decltype(masked)::value || (gi < p.d && gj < p.d && (!diag || gi <= gj)))
                mat.h[gi * ldh + gj] = p.alpha * acc[x][y][r];
            }
      };
      if (!diag && fa0 + TM <= p.d && fb0 + TM <= p.d) put(std::false_type{}); else put(std::true_type{});
      return;
    }
    if ((ldh & 3) == 0 && (p.d & 3) == 0 && (reinterpret_cast<uintptr_t>(mat.h) & 15) == 0) {
      // H = beta H + alpha acc on the upper triangle through the LDS ring,
      // one half of the tile (128 rows, the accumulators of waves wm == hh)
      // at a time: the accumulators are written row-major into LDS, then
      // wave w updates rows RR w .. RR w + RR - 1 of the half (RR = 128 /
      // WAVES), one 256-float row (1 KB, a float4 per lane) per store.  All
      // RR reads of H are issued before the first store, from clamped
      // in-range addresses so that none is conditional: a conditional read
      // makes the compiler wait for every memory operation in flight at each
      // use, the earlier rows' stores included, which serialised the stores.
      // A float4 that straddles the diagonal writes its lower elements back
      // unchanged.
      float* const tile = reinterpret_cast<float*>(ring);
      const int64_t gj = fb0 + 4 * lane;
      const int64_t gjc = gj < p.d ? gj : p.d - 4;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        __syncthreads();   // the ring (or the previous half) is no longer read
        if (wm == hh) {
#pragma unroll
          for (int x = 0; x < MB; ++x)
#pragma unroll
            for (int y = 0; y < NBN; ++y)
#pragma unroll
              for (int r = 0; r < 16; ++r)
                tile[(x * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * 256 + wn * NBN * 32 + y * 32 +
                     (lane & 31)] = acc[x][y][r];
        }
        __syncthreads();
        constexpr int RR = 128 / WAVES;   // rows per wave, in batches of 16
#pragma unroll
        for (int k0 = 0; k0 < RR; k0 += 16) {
          f32x4_t hv[16];
#pragma unroll
          for (int k = 0; k < 16; ++k) {
            const int64_t gi = fa0 + hh * 128 + wave * RR + k0 + k;
            hv[k] = *reinterpret_cast<const f32x4_t*>(mat.h + (gi < p.d ? gi : p.d - 1) * ldh + gjc);
          }
          // the reads complete here, before any store
#pragma unroll
          for (int k = 0; k < 16; ++k) asm volatile("" ::"v"(hv[k]) : "memory");
#pragma unroll
          for (int k = 0; k < 16; ++k) {
            const int lr = wave * RR + k0 + k;
            const int64_t gi = fa0 + hh * 128 + lr;
            if (gi < p.d && gj < p.d && (!diag || gi <= gj + 3)) {
              const f32x4_t v = *reinterpret_cast<const f32x4_t*>(tile + lr * 256 + 4 * lane);
              f32x4_t o;
#pragma unroll
              for (int c = 0; c < 4; ++c)
                o[c] = (!diag || gi <= gj + c) ? scaled(hv[k][c], p.beta) + p.alpha * v[c] : hv[k][c];
              *reinterpret_cast<f32x4_t*>(mat.h + gi * ldh + gj) = o;
            }
          }
        }
      }
      return;
    }
    // unaligned H: one 32 x 32 block at a time: lanes 0..31 / 32..63 of
    // register r hold columns 0..31 of rows 8 (r / 4) + r % 4 and that + 4
    // (the scheduling barrier keeps the blocks' loads from being hoisted
    // together)
#pragma unroll
    for (int x = 0; x < MB; ++x)
#pragma unroll
      for (int y = 0; y < NBN; ++y) {
        const int mb = wm * 128 + x * 32, nb = wn * NBN * 32 + y * 32;
        const int64_t gib = fa0 + mb, gjb = fb0 + nb;
        float* hb = mat.h + gib * ldh + gjb;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int mi = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3), nj = lane & 31;
          if (gib + mi < p.d && gjb + nj < p.d && (!diag || mb + mi <= nb + nj)) {
            float* hp = hb + (int64_t)mi * ldh + nj;
            *hp = scaled(*hp, p.beta) + p.alpha * acc[x][y][r];
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    return;
  }
  // partial slot.  Slot layout: 256 chunks of 64 lanes x 4 floats, chunk
  // ((wave MB + x) NBN + y) 4 + r4 holding accumulator registers
  // 4 r4 .. 4 r4 + 3 of block (x, y), so every store and every load of the
  // reduction moves 1 KB of consecutive bytes.
  float* dst = p.ws + slot * C::TILE + 4 * lane;
#pragma unroll
  for (int x = 0; x < MB; ++x)
#pragma unroll
    for (int y = 0; y < NBN; ++y)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        f32x4_t v = {acc[x][y][4 * r4], acc[x][y][4 * r4 + 1], acc[x][y][4 * r4 + 2], acc[x][y][4 * r4 + 3]};
        *reinterpret_cast<f32x4_t*>(dst + (((wave * MB + x) * NBN + y) * 4 + r4) * 256) = v;
      }
}

// Dense mode: one work item per workgroup (tile t, token split s = blockIdx
// % S, so each XCD streams its own split; dense tail tiles in tail_f parts
// per split).  Grouped modes: persistent workgroups (one per CU) take items
// i = chunk * T + t from eight queues, queue x holding items [x per, (x + 1)
// per) in chunk-major order: a workgroup first drains the queue of its XCD
// (blockIdx % 8, workgroups being dispatched round-robin over the XCDs) so
// the tiles of one chunk run on one XCD and share its rows in L2, then
// takes what is left in the others.  Chunks hold 1 .. 4096 routed rows, so
// equal item counts per XCD can mean very unequal work (routed rows per
// expert vary 85-fold in the Zipf-routed MoE layer); the queues even it out.
// Every queue ends, so every workgroup exits.
// The segment table is a kernel argument of kDenseSeg only.
template <int MODE> struct SegArg { int unused; };
template <> struct SegArg<kDenseSeg> { SegTable t; };

template <bool F16, int MODE, int WAVES>
__global__ __launch_bounds__(64 * WAVES, 1) void syrk_stream_kernel(SyrkParams p, SegArg<MODE> sa) {
  __shared__ __attribute__((aligned(1024))) char ring[8 * SOP];
  // row indices of a gathered chunk
  __shared__ int ridx[MODE == kGroupedGather ? kChunkTokens : 1];
  if constexpr (MODE == kDense || MODE == kDenseSeg) {
    const int S = p.S;
    int t, s, part = 0, nparts = 1;
    int64_t slot;
    const int64_t nfull = (int64_t)p.tail_start * S;
    if (S < 8) {
      // Fewer splits than XCDs (large d, short calls): XCD x (= blockIdx % 8)
      // takes split x % S and the (x / S)-th of 8 / S contiguous runs of its
      // tiles, so the tiles resident on one XCD at once are neighbours in
      // super-block order and share their feature slices in that XCD's L2
      // (tiles strided across XCDs shared none).
      const int G = 8 / S;
      const int x = (int)(blockIdx.x & 7u), k = (int)(blockIdx.x >> 3);
      const int per = (p.tail_start + G - 1) / G;   // tail_start = T: no tail parts below 8 splits
      s = x % S;
      t = (x / S) * per + k;
      if (k >= per || t >= p.tail_start) return;
      slot = S > 1 ? (int64_t)t * S + s : -1;
    } else if ((int64_t)blockIdx.x < nfull) {
      s = blockIdx.x % S;
      t = blockIdx.x / S;
      slot = (S > 1) ? (int64_t)t * S + s : -1;
    } else {
      const int b = (int)(blockIdx.x - nfull);
      s = b % S;
      const int j = b / S;
      t = p.tail_start + j / p.tail_f;
      part = j % p.tail_f;
      nparts = p.tail_f;
      slot = nfull + ((int64_t)(t - p.tail_start) * S + s) * p.tail_f + part;
    }
    const SegTable* sg = nullptr;
    if constexpr (MODE == kDenseSeg) sg = &sa.t;
    stream_item<F16, MODE, WAVES>(p, ring, ridx, t, s, part, nparts, S, slot, p.single, sg);
  } else {
    __shared__ int s_item;
    const int N = p.gcounts[0] * p.T;
    const int per = (N + 7) >> 3;
    const int home = (int)(blockIdx.x & 7u);
    for (;;) {
      if (threadIdx.x == 0) {
        int it = -1;
        for (int q = 0; q < 8 && it < 0; ++q) {
          const int x = (home + q) & 7;
          const int b = x * per, e = b + per < N ? b + per : N;
          if (b >= e) continue;
          const int v = __hip_atomic_fetch_add(p.queues + x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (v < e - b) it = b + v;
        }
        s_item = it;
      }
      __syncthreads();
      const int i = s_item;
      if (i < 0) break;
      const GChunk c = p.chunks[i / p.T];
      if (c.e >= 0) {
        const int t = i % p.T;
        const Matrix mat{c.tok_begin, c.count < kChunkTokens ? c.count : kChunkTokens,
                         p.h0 + (int64_t)c.e * p.h_stride};
        stream_item<F16, MODE, WAVES>(p, ring, ridx, t, 0, 0, 1, 1, c.sbase < 0 ? -1 : c.sbase + t, mat);
      }
      __syncthreads();   // the ring, the row cache and s_item are free for the next item
    }
  }
}

// Finishes the streaming kernel's tiles: for each tile the S split slots
// are summed in split order (a tail tile's split being first the sum of its
// tail_f part slots, in part order) and H is updated.  Workgroup
// (t, blockIdx.y) takes chunks 16 blockIdx.y .. + 15 of tile t, four per
// wave, one float4 per lane of each slot's chunk; all loads of a wave are
// issued before its first sum, and all H reads before its first store.
constexpr int RED_CPW = 4;  // chunks per wave of the streaming reduction

// H (upper triangle of tile (ti, tj)) = beta H + alpha tot for the RED_CPW
// slot chunks ch0 .. ch0 + RED_CPW - 1 of this lane: chunk -> wave (wm, wn)
// of the stream kernel's layout (2 x 4 waves of 4 x 2 blocks, or 2 x 2 of
// 4 x 4), block (x, y), registers 4 r4 + q
template <int WAVES>
__device__ __forceinline__ void stream_update_h(const f32x4_t* tot, int ch0, int lane, int ti, int tj, float* hm,
                                                int64_t d, int64_t ldh, float alpha, float beta) {
  constexpr int TM = 256, MB = 4, NBN = WAVES == 8 ? 2 : 4, WN = WAVES == 8 ? 4 : 2;
  constexpr int PER_W = MB * NBN * 4;   // chunks per wave
  int64_t gi[RED_CPW], gj[RED_CPW];
  float h[RED_CPW][4];
#pragma unroll
  for (int c = 0; c < RED_CPW; ++c) {
    const int ch = ch0 + c;
    const int w = ch / PER_W, x = (ch / (NBN * 4)) % MB, y = (ch >> 2) % NBN, r4 = ch & 3;
    gi[c] = (int64_t)ti * TM + (w / WN) * 128 + x * 32 + 8 * r4 + 4 * (lane >> 5);
    gj[c] = (int64_t)tj * TM + (w % WN) * (NBN * 32) + y * 32 + (lane & 31);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      h[c][q] = (gi[c] + q < d && gj[c] < d && gi[c] + q <= gj[c]) ? hm[(gi[c] + q) * ldh + gj[c]] : 0.f;
  }
#pragma unroll
  for (int c = 0; c < RED_CPW; ++c)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (gi[c] + q < d && gj[c] < d && gi[c] + q <= gj[c])
        hm[(gi[c] + q) * ldh + gj[c]] = scaled(h[c][q], beta) + alpha * tot[c][q];
}

template <int WAVES>
__global__ __launch_bounds__(NT) void syrk_stream_reduce_kernel(const float* __restrict__ ws, int S,
                                                                int tail_start, int tail_f, Matrix single,
                                                                int64_t d, int64_t ldh, int nt, float alpha,
                                                                float beta) {
  constexpr int TM = 256, TILE = TM * TM;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x;
  int ti, tj;
  tile_coords(t, nt, ti, tj);
  const int ch0 = (NT / 64) * RED_CPW * blockIdx.y + RED_CPW * wave;
  const float* src = ws + ch0 * 256 + 4 * lane;
  f32x4_t tot[RED_CPW];
#pragma unroll
  for (int c = 0; c < RED_CPW; ++c) tot[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if (t < tail_start) {
    f32x4_t v[8][RED_CPW];
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (s < S)
#pragma unroll
        for (int c = 0; c < RED_CPW; ++c)
          v[s][c] = *reinterpret_cast<const f32x4_t*>(src + ((int64_t)t * S + s) * TILE + c * 256);
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (s < S)
#pragma unroll
        for (int c = 0; c < RED_CPW; ++c)
#pragma unroll
          for (int q = 0; q < 4; ++q) tot[c][q] += v[s][c][q];
  } else {
    const int64_t base = (int64_t)tail_start * S + (int64_t)(t - tail_start) * S * tail_f;
    for (int s = 0; s < S; ++s) {
      f32x4_t v[4][RED_CPW];
#pragma unroll
      for (int pp = 0; pp < 4; ++pp)
        if (pp < tail_f)
#pragma unroll
          for (int c = 0; c < RED_CPW; ++c)
            v[pp][c] = *reinterpret_cast<const f32x4_t*>(src + (base + (int64_t)s * tail_f + pp) * TILE + c * 256);
#pragma unroll
      for (int c = 0; c < RED_CPW; ++c) {
        f32x4_t ps = v[0][c];
#pragma unroll
        for (int pp = 1; pp < 4; ++pp)
          if (pp < tail_f)
#pragma unroll
            for (int q = 0; q < 4; ++q) ps[q] += v[pp][c][q];
#pragma unroll
        for (int q = 0; q < 4; ++q) tot[c][q] += ps[q];
      }
    }
  }
  stream_update_h<WAVES>(tot, ch0, lane, ti, tj, single.h, d, ldh, alpha, beta);
}

// Grouped: adds the later chunks' slots of (expert, tile) to H in chunk
// order (workgroup x: item x / T, tile x % T; y: 16-chunk group as above).
template <int WAVES>
__global__ __launch_bounds__(NT) void syrk_group_reduce_kernel(const float* __restrict__ ws,
                                                               const GReduce* __restrict__ reds,
                                                               const int* __restrict__ gcounts, int T, int nt,
                                                               int64_t d, float* h0, int64_t h_stride, float alpha) {
  constexpr int TILE = 256 * 256;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int item = (int)blockIdx.x / T, t = (int)blockIdx.x % T;
  if (item >= gcounts[1]) return;
  const GReduce rd = reds[item];
  int ti, tj;
  tile_coords(t, nt, ti, tj);
  const int ch0 = (NT / 64) * RED_CPW * blockIdx.y + RED_CPW * wave;
  const float* src = ws + ch0 * 256 + 4 * lane;
  f32x4_t tot[RED_CPW];
#pragma unroll
  for (int c = 0; c < RED_CPW; ++c) tot[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < rd.nslots; k0 += 4) {
    f32x4_t v[4][RED_CPW];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k0 + k < rd.nslots)
#pragma unroll
        for (int c = 0; c < RED_CPW; ++c)
          v[k][c] = *reinterpret_cast<const f32x4_t*>(src + (rd.sbase + (int64_t)(k0 + k) * T + t) * TILE + c * 256);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k0 + k < rd.nslots)
#pragma unroll
        for (int c = 0; c < RED_CPW; ++c)
#pragma unroll
          for (int q = 0; q < 4; ++q) tot[c][q] += v[k][c][q];
  }
  stream_update_h<WAVES>(tot, ch0, lane, ti, tj, h0 + (int64_t)rd.e * h_stride, d, d, alpha, 1.f);
}

// Builds the grouped chunk table from the expert offsets (one workgroup of
// 1024 threads, 1024 experts per round): expert e takes
// m_e = ceil(n_e / kChunkTokens) chunks, its first adds to H directly and
// the m_e - 1 others get T partial slots each.  Offsets are clamped into
// [0, n_rows] and the table never exceeds its bounds (max_chunks, max_slot
// chunks, max_reduce), which non-decreasing offsets with offsets[E] <= n_rows
// never reach.
__global__ __launch_bounds__(1024) void grouped_plan_kernel(const int64_t* __restrict__ offsets, int E,
                                                            int64_t n_rows, int T, int max_chunks,
                                                            int max_slot_chunks, int max_reduce, int all_experts,
                                                            GChunk* chunks, GReduce* reds, int* gcounts) {
  __shared__ int sm[1024], sr[1024], ss[1024];
  const int tid = threadIdx.x;
  int base_c = 0, base_r = 0, base_s = 0;
  for (int e0 = 0; e0 < E; e0 += 1024) {
    const int e = e0 + tid;
    int64_t b = 0, n = 0;
    if (e < E) {
      b = offsets[e];
      int64_t en = offsets[e + 1];
      b = b < 0 ? 0 : (b > n_rows ? n_rows : b);
      en = en < b ? b : (en > n_rows ? n_rows : en);
      n = en - b;
    }
    int m = (int)((n + kChunkTokens - 1) / kChunkTokens);
    if (all_experts && e < E && m == 0) m = 1;   // an expert without rows still writes its H
    sm[tid] = m;
    sr[tid] = m > 1 ? 1 : 0;
    ss[tid] = m > 1 ? m - 1 : 0;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {   // inclusive scans
      const int vm = tid >= o ? sm[tid - o] : 0, vr = tid >= o ? sr[tid - o] : 0, vs = tid >= o ? ss[tid - o] : 0;
      __syncthreads();
      sm[tid] += vm;
      sr[tid] += vr;
      ss[tid] += vs;
      __syncthreads();
    }
    const int cm = base_c + sm[tid] - m;                       // this expert's first chunk
    const int cs = base_s + ss[tid] - (m > 1 ? m - 1 : 0);     // its first slotted chunk
    const int cr = base_r + sr[tid] - (m > 1 ? 1 : 0);
    for (int k = 0; k < m; ++k) {
      const int c = cm + k, sc = cs + k - 1;
      if (c >= max_chunks) break;   // past the table (gcounts[0] stops before it)
      const int64_t left = n - (int64_t)k * kChunkTokens;
      // a chunk past the slot bound is skipped (expert -1: adds nothing)
      chunks[c] = (k == 0 || sc < max_slot_chunks)
                      ? GChunk{e, (int)(left < kChunkTokens ? left : kChunkTokens), b + (int64_t)k * kChunkTokens,
                               k == 0 ? -1 : (int64_t)sc * T}
                      : GChunk{-1, 0, 0, -1};
    }
    if (m > 1 && cr < max_reduce) {
      const int room = cs < max_slot_chunks ? max_slot_chunks - cs : 0;
      reds[cr] = GReduce{e, m - 1 < room ? m - 1 : room, (int64_t)cs * T};
    }
    base_c += sm[1023];
    base_r += sr[1023];
    base_s += ss[1023];
    __syncthreads();
  }
  if (tid == 0) {
    gcounts[0] = base_c < max_chunks ? base_c : max_chunks;
    gcounts[1] = base_r < max_reduce ? base_r : max_reduce;
  }
  if (tid < 8) gcounts[2 + tid] = 0;   // the stream kernel's work-queue counters
}

// Sums the S partial slots of a tile in split order and updates H.  Each
// workgroup finishes one row of 32 x 32 blocks of its wave tiles
// (blockIdx.y = bm), so a TM = 256 tile is finished by four workgroups.
template <int TM>
__global__ __launch_bounds__(NT) void syrk_reduce_kernel(const float* __restrict__ ws, int S, Matrix mat,
                                                         int64_t d, int64_t ldh, int nt, float alpha,
                                                         float beta) {
  using C = Cfg<TM>;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int bm = blockIdx.y;
  const int t = blockIdx.x;
  const int64_t slot0 = (int64_t)t * S;
  int ti, tj;
  tile_coords(t, nt, ti, tj);
  float sum[C::NB * 16];
#pragma unroll
  for (int r = 0; r < C::NB * 16; ++r) sum[r] = 0.f;
  for (int s = 0; s < S; ++s) {
    const float* src = ws + ((slot0 + s) * NT + tid) * C::ACC + bm * C::NB * 16;
#pragma unroll
    for (int q = 0; q < C::NB * 4; ++q) {
      const f32x4_t v = *reinterpret_cast<const f32x4_t*>(src + 4 * q);
      sum[4 * q] += v[0];
      sum[4 * q + 1] += v[1];
      sum[4 * q + 2] += v[2];
      sum[4 * q + 3] += v[3];
    }
  }
  const int64_t gi0 = (int64_t)ti * TM, gj0 = (int64_t)tj * TM;
#pragma unroll
  for (int bn = 0; bn < C::NB; ++bn)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = wm * C::W + bm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      const int nn = wn * C::W + bn * 32 + (lane & 31);
      const int64_t gi = gi0 + m, gj = gj0 + nn;
      if (gi < d && gj < d && gi <= gj) {
        float* hp = mat.h + gi * ldh + gj;
        *hp = scaled(*hp, beta) + alpha * sum[bn * 16 + r];
      }
    }
}

__global__ void symmetrize_kernel(float* h, int64_t d, int64_t ldh) {
  __shared__ float tile[32][33];
  const int bi = blockIdx.y, bj = blockIdx.x;  // source tile (bi <= bj) in the upper triangle
  if (bi > bj) return;
  const int tx = threadIdx.x, ty = threadIdx.y;  // 32 x 8
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = (int64_t)bi * 32 + k, c = (int64_t)bj * 32 + tx;
    tile[k][tx] = (r < d && c < d) ? h[r * ldh + c] : 0.f;
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = (int64_t)bj * 32 + k, c = (int64_t)bi * 32 + tx;  // lower (r, c) = upper (c, r)
    if (r < d && c < d && r > c) h[r * ldh + c] = tile[tx][k];
  }
}

// Token splits of a T-tile matrix over n tokens: up to 8 (at least 2048
// tokens each), one per XCD, while the tiles alone would leave CUs idle;
// with more than two rounds of tiles per CU, at most 2 (each split slot
// costs a 256 KiB partial written and read back: at d = 14336 and 16384
// tokens, 8 splits move 6.7 GB for 3.4 TFLOP of work).
// Compute units of the current device (256 on an MI355X: 8 XCDs of 32).
int device_cus() {
  int dev = 0, ncu = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) !=
      hipSuccess || ncu <= 0)
    return 256;
  return ncu;
}

int choose_splits(int64_t n, int T, int cus) {
  const int64_t s = n / 2048;
  int S = s >= 8 ? 8 : s >= 4 ? 4 : s >= 2 ? 2 : 1;
  // Wide Hessians (over two rounds of tiles) take at most 4 splits, and 4
  // only over 131072 tokens or more, where the rounds saved outweigh the
  // larger reduction: d = 14336 over 524288 tokens 25 rounds of a quarter of
  // the tokens instead of 13 of half, 101.4 -> 99.1 ms; d = 8192 over 262144
  // tokens 9 instead of 10 half-rounds, 17.7 -> 16.5 ms (65536 tokens at
  // d = 14336: 12.3 -> 12.5 ms, so shorter calls keep two).
  if (T > 2 * cus && S > 2) S = n >= 131072 ? 4 : 2;
  if (S == 8) return S;  // the dense plan's tail parts even out its rounds
  // Below that, the fewest splits that reach the shortest time: k splits
  // take ceil(T k / cus) rounds on the CUs, each 1 / k of the tokens, and
  // every split beyond one adds a reduction (d = 4096 and 4096 tokens on
  // 256 CUs: one split, one round of 136 tiles, rather than two rounds of
  // halves).
  const auto rounds_x4 = [T, cus](int k) { return (T * k + cus - 1) / cus * (4 / k); };
  int best = 1;
  for (int k = 2; k <= S; k *= 2)
    if (rounds_x4(k) < rounds_x4(best)) best = k;
  return best;
}

inline int tile_edge(int64_t d) { return d >= 512 ? 256 : 128; }
inline int tiles_per_edge(int64_t d) {
  const int tm = tile_edge(d);
  return (int)((d + tm - 1) / tm);
}
inline int upper_tiles(int nt) { return nt * (nt + 1) / 2; }
inline size_t tile_floats(int64_t d) { return (size_t)tile_edge(d) * tile_edge(d); }

// Dense work plan.  With S = 8 token splits, split s runs on XCD s (work
// items are dispatched round-robin over the 8 XCDs), so each XCD takes T
// items of equal length on its 32 CUs (one workgroup per CU): T / 32 full
// rounds and a last round with only T % 32 items.  The last rem = T % 32
// tiles are therefore cut into f = min(4, 32 / rem) parts per split, so the
// last round takes 1 / f of a full one (d = 4096: T = 136, rem = 8, f = 4,
// 4.25 rounds instead of 5).  The reduction sums their f part slots per
// split, in part order, before adding the split.  The CU count is the
// device's (queried), so the workspace size and the launch agree on it.
constexpr int kXcds = 8;
struct DensePlan {
  int S = 1, T = 0, tail_start = 0, tail_f = 1;
  int64_t grid = 0, slots = 0;
};
DensePlan plan_dense(int64_t n, int64_t d) {
  DensePlan pl;
  const int cus = device_cus();
  const int per_xcd = cus / kXcds > 0 ? cus / kXcds : 1;
  pl.T = upper_tiles(tiles_per_edge(d));
  pl.S = choose_splits(n, pl.T, cus);
  pl.tail_start = pl.T;
  const int rem = pl.T % per_xcd;
  if (pl.S == 8 && tile_edge(d) == 256 && rem > 0 && rem <= per_xcd / 2) {
    pl.tail_f = per_xcd / rem < 4 ? per_xcd / rem : 4;
    pl.tail_start = pl.T - rem;
  }
  const int64_t nfull = (int64_t)pl.tail_start * pl.S;
  const int64_t ntail = (int64_t)(pl.T - pl.tail_start) * pl.S;
  pl.grid = nfull + ntail * pl.tail_f;
  pl.slots = pl.S > 1 ? pl.grid : 0;
  if (pl.S < kXcds && tile_edge(d) == 256) {
    // fewer splits than XCDs: each split's tiles in 8 / S contiguous runs,
    // one per XCD (the stream kernel's dense decode; the 128-tile kernel of
    // d < 512 keeps one item per workgroup in item order)
    const int G = kXcds / pl.S;
    pl.grid = (int64_t)kXcds * ((pl.T + G - 1) / G);
    pl.slots = pl.S > 1 ? (int64_t)pl.T * pl.S : 0;
  }
  return pl;
}

template <bool F16>
void launch_syrk_t(const SyrkParams& p, int64_t d, unsigned grid, hipStream_t st) {
  if (tile_edge(d) == 256) {
    hipLaunchKernelGGL((syrk_stream_kernel<F16, kDense, kStreamWaves>), dim3(grid), dim3(SNT), 0, st, p,
                       SegArg<kDense>{});
  } else {
    hipLaunchKernelGGL((syrk_bf16_kernel<128, F16>), dim3(grid), dim3(NT), 0, st, p);
  }
}

void launch_syrk(const SyrkParams& p, int64_t d, unsigned grid, hipStream_t st, bool f16) {
  if (f16) launch_syrk_t<true>(p, d, grid, st); else launch_syrk_t<false>(p, d, grid, st);
}

// reduction of syrk_bf16_kernel partials (2 x 2 fragment order)
void launch_reduce(const float* ws, int S, const Matrix& single, int64_t d, int64_t ldh, int nt, float alpha,
                   float beta, unsigned ntiles, hipStream_t st) {
  if (tile_edge(d) == 256)
    hipLaunchKernelGGL(syrk_reduce_kernel<256>, dim3(ntiles, Cfg<256>::NB), dim3(NT), 0, st, ws, S, single, d, ldh,
                       nt, alpha, beta);
  else
    hipLaunchKernelGGL(syrk_reduce_kernel<128>, dim3(ntiles, Cfg<128>::NB), dim3(NT), 0, st, ws, S, single, d, ldh,
                       nt, alpha, beta);
}

// H[i][j] *= beta on the upper triangle (a call without tokens)
__global__ void scale_upper_kernel(float* h, int64_t d, int64_t ldh, float beta) {
  const int64_t i = blockIdx.y;
  for (int64_t j = i + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < d; j += (int64_t)gridDim.x * blockDim.x)
    h[i * ldh + j] = h[i * ldh + j] * beta;
}

}  // namespace

}  // namespace mi355q

using namespace mi355q;

extern "C" size_t mi355q_hessian_workspace_size(int64_t n_tokens, int64_t d) {
  if (n_tokens <= 0 || d <= 0) return 0;
  return (size_t)plan_dense(n_tokens, d).slots * tile_floats(d) * sizeof(float);
}

namespace {
// Kernel parameters of a dense call over n_tokens rows at x.
SyrkParams dense_params(const uint16_t* x, int64_t n_tokens, int64_t d, int64_t ldx, float* h_dev, int64_t ldh,
                        float alpha, float beta, const DensePlan& pl, void* workspace_dev) {
  SyrkParams p{};
  p.x = x;
  p.ldx = ldx;
  p.d = d;
  p.ldh = ldh;
  p.nt = tiles_per_edge(d);
  p.alpha = alpha;
  p.beta = beta;
  p.single = Matrix{0, n_tokens, h_dev};
  p.S = pl.S;
  p.tail_start = pl.tail_start;
  p.tail_f = pl.tail_f;
  p.ws = static_cast<float*>(workspace_dev);
  return p;
}

// H = beta H + alpha X^T X (upper) for 16-bit X: bf16, or fp16 (f16)
int hessian16_impl(const void* x_dev, bool f16, int64_t n_tokens, int64_t d, int64_t ldx, float* h_dev,
                   int64_t ldh, float alpha, float beta, void* workspace_dev, size_t workspace_bytes, void* stream) {
  MQ_CHECK_ARG(d > 0 && d % 8 == 0, "hessian: d must be a positive multiple of 8 (got %lld)", (long long)d);
  MQ_CHECK_ARG(ldx >= d && ldx % 8 == 0, "hessian: ldx must be >= d and a multiple of 8");
  MQ_CHECK_ARG(ldx <= (int64_t(1) << 24), "hessian: ldx above 2^24 elements is not supported");
  MQ_CHECK_ARG(ldh >= d, "hessian: ldh must be >= d");
  MQ_CHECK_ARG(n_tokens >= 0, "hessian: negative token count");
  MQ_CHECK_ARG(h_dev != nullptr, "hessian: null H");
  if (n_tokens == 0) {
    if (beta != 1.f) {
      hipLaunchKernelGGL(scale_upper_kernel, dim3((unsigned)((d + 255) / 256), (unsigned)d), dim3(256), 0,
                         reinterpret_cast<hipStream_t>(stream), h_dev, d, ldh, beta);
      MQ_LAUNCH_CHECK();
    }
    return MI355Q_OK;
  }
  MQ_CHECK_ARG(x_dev != nullptr && aligned16(x_dev), "hessian: x must be non-null and 16-byte aligned");
  const int nt = tiles_per_edge(d);
  const DensePlan pl = plan_dense(n_tokens, d);
  const int T = pl.T, S = pl.S;
  const size_t need = mi355q_hessian_workspace_size(n_tokens, d);
  MQ_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace_dev != nullptr),
               "hessian: workspace too small (%zu < %zu)", workspace_bytes, need);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);

  SyrkParams p = dense_params(static_cast<const uint16_t*>(x_dev), n_tokens, d, ldx, h_dev, ldh, alpha, beta, pl,
                              workspace_dev);
  launch_syrk(p, d, (unsigned)pl.grid, st, f16);
  MQ_LAUNCH_CHECK();
  if (S > 1) {
    if (tile_edge(d) == 256)  // the streaming kernel's slots
      hipLaunchKernelGGL(syrk_stream_reduce_kernel<kStreamWaves>, dim3((unsigned)T, 256 / ((NT / 64) * RED_CPW)), dim3(NT), 0,
                         st, p.ws, S, pl.tail_start, pl.tail_f, p.single, d, ldh, nt, alpha, beta);
    else
      launch_reduce(p.ws, S, p.single, d, ldh, nt, alpha, beta, (unsigned)T, st);
    MQ_LAUNCH_CHECK();
  }
  return MI355Q_OK;
}

// Stages of a segment of `rows` rows (the last one zero-padded).
inline int64_t seg_stages(int64_t rows) { return (rows + SK - 1) / SK; }

// Workspace of a segmented call: d >= 512 runs the non-empty segments in
// groups of kMaxSegments, one launch over each group's padded rows; d < 512
// runs one dense call per segment.
size_t seg_workspace(const int64_t* rows, int nseg, int64_t d) {
  size_t need = 0;
  auto upd = [&need](size_t v) { need = v > need ? v : need; };
  if (tile_edge(d) != 256) {
    for (int k = 0; k < nseg; ++k)
      if (rows[k] > 0) upd(mi355q_hessian_workspace_size(rows[k], d));
    return need;
  }
  int in_group = 0;
  int64_t stages = 0;
  for (int k = 0; k < nseg; ++k) {
    if (rows[k] <= 0) continue;
    stages += seg_stages(rows[k]);
    if (++in_group == kMaxSegments) {
      upd(mi355q_hessian_workspace_size(stages * SK, d));
      in_group = 0;
      stages = 0;
    }
  }
  if (in_group) upd(mi355q_hessian_workspace_size(stages * SK, d));
  return need;
}

// H = beta H + alpha sum_k X_k^T X_k over row segments X_k (host arrays of
// device pointers and row counts), summed as the rows of one call would be:
// segments in order, each starting a new stage.
int hessian_seg_impl(const void* const* xs, const int64_t* rows, int nseg, mi355q_dtype dtype, int64_t d,
                     int64_t ldx, float* h_dev, int64_t ldh, float alpha, float beta, void* workspace_dev,
                     size_t workspace_bytes, void* stream) {
  MQ_CHECK_ARG(nseg >= 0 && (nseg == 0 || (xs != nullptr && rows != nullptr)),
               "hessian segments: null segment arrays");
  int nz = 0;
  for (int k = 0; k < nseg; ++k) {
    MQ_CHECK_ARG(rows[k] >= 0, "hessian segments: negative row count in segment %d", k);
    MQ_CHECK_ARG(rows[k] == 0 || xs[k] != nullptr, "hessian segments: null rows in segment %d", k);
    nz += rows[k] > 0;
  }
  const bool seg16 = (dtype == MI355Q_BF16 || dtype == MI355Q_F16) && d >= 512;
  if (!seg16 || nz <= 1) {
    // one dense call per non-empty segment, beta with the first
    float b = beta;
    for (int k = 0; k < nseg; ++k) {
      if (rows[k] == 0) continue;
      const int rc = mi355q_hessian_syrk(xs[k], dtype, rows[k], d, ldx, h_dev, ldh, alpha, b, workspace_dev,
                                         workspace_bytes, stream);
      if (rc != MI355Q_OK) return rc;
      b = 1.f;
    }
    if (nz == 0) return mi355q_hessian_syrk(nullptr, dtype, 0, d, ldx, h_dev, ldh, alpha, beta, nullptr, 0, stream);
    return MI355Q_OK;
  }
  const bool f16 = dtype == MI355Q_F16;
  MQ_CHECK_ARG(d % 8 == 0, "hessian: d must be a positive multiple of 8 (got %lld)", (long long)d);
  MQ_CHECK_ARG(ldx >= d && ldx % 8 == 0, "hessian: ldx must be >= d and a multiple of 8");
  MQ_CHECK_ARG(ldx <= (int64_t(1) << 24), "hessian: ldx above 2^24 elements is not supported");
  MQ_CHECK_ARG(ldh >= d, "hessian: ldh must be >= d");
  MQ_CHECK_ARG(h_dev != nullptr, "hessian: null H");
  for (int k = 0; k < nseg; ++k)
    MQ_CHECK_ARG(rows[k] == 0 || aligned16(xs[k]), "hessian segments: segment %d is not 16-byte aligned", k);
  const size_t need = seg_workspace(rows, nseg, d);
  MQ_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace_dev != nullptr),
               "hessian: workspace too small (%zu < %zu)", workspace_bytes, need);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int nt = tiles_per_edge(d);
  float b = beta;
  for (int k = 0; k < nseg;) {
    SegArg<kDenseSeg> sa{};
    SegTable& tb = sa.t;
    int64_t stages = 0;
    for (; k < nseg && tb.n < kMaxSegments; ++k) {
      if (rows[k] == 0) continue;
      tb.stage0[tb.n] = stages;
      tb.rows[tb.n] = rows[k];
      tb.x[tb.n] = static_cast<const uint16_t*>(xs[k]);
      stages += seg_stages(rows[k]);
      ++tb.n;
    }
    if (tb.n == 0) break;
    tb.stage0[tb.n] = stages;
    int rc = MI355Q_OK;
    if (tb.n == 1) {
      rc = hessian16_impl(tb.x[0], f16, tb.rows[0], d, ldx, h_dev, ldh, alpha, b, workspace_dev, workspace_bytes,
                          stream);
    } else {
      const int64_t n_eff = stages * SK;   // the padded stages' rows
      const DensePlan pl = plan_dense(n_eff, d);
      const SyrkParams p = dense_params(tb.x[0], n_eff, d, ldx, h_dev, ldh, alpha, b, pl, workspace_dev);
      if (f16)
        hipLaunchKernelGGL((syrk_stream_kernel<true, kDenseSeg, kStreamWaves>), dim3((unsigned)pl.grid), dim3(SNT),
                           0, st, p, sa);
      else
        hipLaunchKernelGGL((syrk_stream_kernel<false, kDenseSeg, kStreamWaves>), dim3((unsigned)pl.grid), dim3(SNT),
                           0, st, p, sa);
      MQ_LAUNCH_CHECK();
      if (pl.S > 1) {
        hipLaunchKernelGGL(syrk_stream_reduce_kernel<kStreamWaves>, dim3((unsigned)pl.T, 256 / ((NT / 64) * RED_CPW)),
                           dim3(NT), 0, st, p.ws, pl.S, pl.tail_start, pl.tail_f, p.single, d, ldh, nt, alpha, b);
        MQ_LAUNCH_CHECK();
      }
    }
    if (rc != MI355Q_OK) return rc;
    b = 1.f;
  }
  return MI355Q_OK;
}
}  // namespace

extern "C" int mi355q_hessian_syrk_scaled_bf16(const void* x_dev, int64_t n_tokens, int64_t d, int64_t ldx,
                                               float* h_dev, int64_t ldh, float alpha, float beta,
                                               void* workspace_dev, size_t workspace_bytes, void* stream) {
  return hessian16_impl(x_dev, false, n_tokens, d, ldx, h_dev, ldh, alpha, beta, workspace_dev, workspace_bytes,
                        stream);
}

extern "C" size_t mi355q_hessian_syrk_workspace_size(int64_t n_tokens, int64_t d, mi355q_dtype dtype) {
  return dtype == MI355Q_F32 ? 0 : mi355q_hessian_workspace_size(n_tokens, d);
}

extern "C" int mi355q_hessian_syrk(const void* x_dev, mi355q_dtype dtype, int64_t n_tokens, int64_t d, int64_t ldx,
                                   float* h_dev, int64_t ldh, float alpha, float beta, void* workspace_dev,
                                   size_t workspace_bytes, void* stream) {
  if (dtype == MI355Q_BF16 || dtype == MI355Q_F16)
    return hessian16_impl(x_dev, dtype == MI355Q_F16, n_tokens, d, ldx, h_dev, ldh, alpha, beta, workspace_dev,
                          workspace_bytes, stream);
  MQ_CHECK_ARG(dtype == MI355Q_F32, "hessian: dtype must be bf16, fp16 or fp32");
  MQ_CHECK_ARG(d > 0 && ldx >= d && ldh >= d && n_tokens >= 0, "hessian: bad shape");
  MQ_CHECK_ARG(h_dev != nullptr, "hessian: null H");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (n_tokens == 0) {
    if (beta != 1.f) {
      hipLaunchKernelGGL(scale_upper_kernel, dim3((unsigned)((d + 255) / 256), (unsigned)d), dim3(256), 0, st, h_dev,
                         d, ldh, beta);
      MQ_LAUNCH_CHECK();
    }
    return MI355Q_OK;
  }
  MQ_CHECK_ARG(x_dev != nullptr, "hessian: null x");
  return syrk_f32_upper(static_cast<const float*>(x_dev), n_tokens, d, ldx, h_dev, ldh, alpha, beta, st);
}

extern "C" int mi355q_hessian_syrk_bf16(const void* x_dev, int64_t n_tokens, int64_t d, int64_t ldx,
                                        float* h_dev, int64_t ldh, float alpha, void* workspace_dev,
                                        size_t workspace_bytes, void* stream) {
  return mi355q_hessian_syrk_scaled_bf16(x_dev, n_tokens, d, ldx, h_dev, ldh, alpha, 1.f, workspace_dev,
                                         workspace_bytes, stream);
}

extern "C" size_t mi355q_hessian_syrk_segments_workspace_size(const int64_t* n_tokens, int n_segments, int64_t d,
                                                              mi355q_dtype dtype) {
  if (dtype == MI355Q_F32 || n_segments <= 0 || n_tokens == nullptr || d <= 0) return 0;
  return seg_workspace(n_tokens, n_segments, d);
}

extern "C" int mi355q_hessian_syrk_segments(const void* const* x_devs, const int64_t* n_tokens, int n_segments,
                                            mi355q_dtype dtype, int64_t d, int64_t ldx, float* h_dev, int64_t ldh,
                                            float alpha, float beta, void* workspace_dev, size_t workspace_bytes,
                                            void* stream) {
  return hessian_seg_impl(x_devs, n_tokens, n_segments, dtype, d, ldx, h_dev, ldh, alpha, beta, workspace_dev,
                          workspace_bytes, stream);
}

namespace {
// Grouped workspace: [partial slots][chunk table][reduce table][2 counts],
// every part sized for the largest table the arguments allow.
struct GroupedBounds {
  int T = 0, max_chunks = 0, max_slot_chunks = 0, max_reduce = 0;
  size_t off_chunks = 0, off_reds = 0, off_counts = 0, total = 0;
};
GroupedBounds grouped_bounds(int64_t n_rows, int E, int64_t d) {
  GroupedBounds g;
  g.T = upper_tiles((int)((d + 255) / 256));
  const int64_t full = n_rows / kChunkTokens;   // chunks after an expert's first are whole
  g.max_chunks = (int)(E + full);
  g.max_slot_chunks = (int)full;
  g.max_reduce = (int)(full < E ? full : E);
  auto align = [](size_t v) { return (v + 255) & ~(size_t)255; };
  size_t off = align((size_t)g.max_slot_chunks * g.T * 256 * 256 * sizeof(float));
  g.off_chunks = off;
  off = align(off + (size_t)g.max_chunks * sizeof(GChunk));
  g.off_reds = off;
  off = align(off + (size_t)(g.max_reduce > 0 ? g.max_reduce : 1) * sizeof(GReduce));
  g.off_counts = off;
  g.total = align(off + 10 * sizeof(int));   // chunk and reduce counts, 8 work-queue counters
  return g;
}
}  // namespace

extern "C" size_t mi355q_hessian_grouped_syrk_workspace_size(int64_t n_rows, int n_experts, int64_t d) {
  if (n_rows < 0 || n_experts <= 0 || d <= 0) return 0;
  return grouped_bounds(n_rows, n_experts, d).total;
}

extern "C" int mi355q_hessian_grouped_syrk(const void* x_dev, mi355q_dtype dtype, int64_t n_x, int64_t ldx,
                                           int64_t d, const int32_t* rows_dev, int64_t n_rows,
                                           const int64_t* offsets_dev, int n_experts, float* h_dev,
                                           int64_t h_stride, float alpha, float beta, void* workspace_dev,
                                           size_t workspace_bytes, void* stream) {
  MQ_CHECK_ARG(dtype == MI355Q_BF16 || dtype == MI355Q_F16, "grouped hessian: dtype must be bf16 or fp16");
  MQ_CHECK_ARG(d > 0 && d % 8 == 0, "grouped hessian: d must be a positive multiple of 8");
  MQ_CHECK_ARG(ldx >= d && ldx % 8 == 0, "grouped hessian: ldx must be >= d and a multiple of 8");
  MQ_CHECK_ARG(ldx <= (int64_t(1) << 24), "grouped hessian: ldx above 2^24 elements is not supported");
  MQ_CHECK_ARG(n_experts > 0 && offsets_dev != nullptr, "grouped hessian: bad expert table");
  MQ_CHECK_ARG(n_x >= 0 && n_rows >= 0, "grouped hessian: negative row count");
  MQ_CHECK_ARG(rows_dev != nullptr || n_rows <= n_x, "grouped hessian: n_rows > n_x without a row index");
  MQ_CHECK_ARG(h_dev != nullptr && h_stride >= d * d, "grouped hessian: bad H / stride");
  MQ_CHECK_ARG(beta == 0.f || beta == 1.f, "grouped hessian: beta must be 0 (H is written) or 1 (H is added to)");
  const bool fresh = beta == 0.f;
  if ((n_rows == 0 || n_x == 0) && !fresh) return MI355Q_OK;
  if (n_x == 0) n_rows = 0;   // nothing to read: every H is written as zero
  MQ_CHECK_ARG(n_rows == 0 || (x_dev != nullptr && aligned16(x_dev)), "grouped hessian: null or misaligned x");
  const GroupedBounds gb = grouped_bounds(n_rows, n_experts, d);
  MQ_CHECK_ARG(workspace_dev != nullptr && workspace_bytes >= gb.total,
               "grouped hessian: workspace too small (%zu < %zu)", workspace_bytes, gb.total);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace_dev);
  GChunk* chunks = reinterpret_cast<GChunk*>(ws + gb.off_chunks);
  GReduce* reds = reinterpret_cast<GReduce*>(ws + gb.off_reds);
  int* counts = reinterpret_cast<int*>(ws + gb.off_counts);
  hipLaunchKernelGGL(grouped_plan_kernel, dim3(1), dim3(1024), 0, st, offsets_dev, n_experts, n_rows, gb.T,
                     gb.max_chunks, gb.max_slot_chunks, gb.max_reduce, fresh ? 1 : 0, chunks, reds, counts);
  MQ_LAUNCH_CHECK();

  SyrkParams p{};
  p.x = static_cast<const uint16_t*>(x_dev);
  p.ldx = ldx;
  p.d = d;
  p.ldh = d;
  p.nt = (int)((d + 255) / 256);
  p.alpha = alpha;
  p.beta = beta;
  p.S = 1;
  p.ws = reinterpret_cast<float*>(ws);
  p.rows = rows_dev;
  p.n_x = n_x;
  p.chunks = chunks;
  p.gcounts = counts;
  p.queues = counts + 2;
  p.T = gb.T;
  p.h0 = h_dev;
  p.h_stride = h_stride;
  // persistent workgroups, one per CU (no more than there are items)
  const int64_t items = (int64_t)gb.max_chunks * gb.T;
  const int cus = device_cus();
  const unsigned grid = (unsigned)(items < cus ? items : cus);
  const bool f16 = dtype == MI355Q_F16;
  if (rows_dev) {
    if (f16) hipLaunchKernelGGL((syrk_stream_kernel<true, kGroupedGather, kStreamWaves>), dim3(grid), dim3(SNT), 0, st, p,
                                  SegArg<kGroupedGather>{});
    else     hipLaunchKernelGGL((syrk_stream_kernel<false, kGroupedGather, kStreamWaves>), dim3(grid), dim3(SNT), 0, st, p,
                                  SegArg<kGroupedGather>{});
  } else {
    if (f16) hipLaunchKernelGGL((syrk_stream_kernel<true, kGrouped, kStreamWaves>), dim3(grid), dim3(SNT), 0, st, p,
                                  SegArg<kGrouped>{});
    else     hipLaunchKernelGGL((syrk_stream_kernel<false, kGrouped, kStreamWaves>), dim3(grid), dim3(SNT), 0, st, p,
                                  SegArg<kGrouped>{});
  }
  MQ_LAUNCH_CHECK();
  if (gb.max_reduce > 0) {
    hipLaunchKernelGGL(syrk_group_reduce_kernel<kStreamWaves>, dim3((unsigned)(gb.max_reduce * gb.T), 256 / ((NT / 64) * RED_CPW)),
                       dim3(NT), 0, st, p.ws, reds, counts, gb.T, p.nt, d, h_dev, h_stride, alpha);
    MQ_LAUNCH_CHECK();
  }
  return MI355Q_OK;
}

extern "C" int mi355q_symmetrize_upper(float* h_dev, int64_t d, int64_t ldh, void* stream) {
  MQ_CHECK_ARG(h_dev != nullptr && d > 0 && ldh >= d, "symmetrize: bad arguments");
  const unsigned nb = (unsigned)((d + 31) / 32);
  hipLaunchKernelGGL(symmetrize_kernel, dim3(nb, nb), dim3(32, 8), 0,
                     reinterpret_cast<hipStream_t>(stream), h_dev, d, ldh);
  MQ_LAUNCH_CHECK();
  return MI355Q_OK;
}
