// 16-lane GPTQ sweeps on the float grids (fp8 e4m3, fp4 e2m1).
#include "gptq_sweep.h"

namespace mi355q {
namespace gsw {

namespace {
template <class K>
void go(K kernel, dim3 grid, hipStream_t st, const SweepLaunch& a) {
  hipLaunchKernelGGL(kernel, grid, dim3(SW_NT), 0, st, a.W, a.rows, a.cols, a.hinv, a.i1, a.count, a.scale, a.zp,
                     a.ld_scale, a.g_idx, a.strategy, a.block_h, a.qmin, a.qmax, a.gscale, a.codes, a.losses, a.err,
                     a.lde, a.err_col, a.npre, a.pre_k0, a.pre_err_col, a.sb);
}
}  // namespace

void launch_sweep_float(int qk, bool full, bool bf16, dim3 grid, hipStream_t st, const SweepLaunch& a) {
  if (qk == QK_FP8) {
    if (full) bf16 ? go(sweep_block_kernel<true, true, false, QK_FP8>, grid, st, a)
              : go(sweep_block_kernel<true, false, false, QK_FP8>, grid, st, a);
    else      bf16 ? go(sweep_block_kernel<false, true, false, QK_FP8>, grid, st, a)
              : go(sweep_block_kernel<false, false, false, QK_FP8>, grid, st, a);
  } else {
    if (full) bf16 ? go(sweep_block_kernel<true, true, false, QK_FP4>, grid, st, a)
              : go(sweep_block_kernel<true, false, false, QK_FP4>, grid, st, a);
    else      bf16 ? go(sweep_block_kernel<false, true, false, QK_FP4>, grid, st, a)
              : go(sweep_block_kernel<false, false, false, QK_FP4>, grid, st, a);
  }
}

}  // namespace gsw
}  // namespace mi355q
