// 4-lane GPTQ sweeps (whole integer blocks, symmetric scales, large grids).
#include "gptq_sweep.h"

namespace mi355q {
namespace gsw {

namespace {
template <class K>
void go(K kernel, dim3 grid, hipStream_t st, const SweepLaunch& a) {
  hipLaunchKernelGGL(kernel, grid, dim3(SW_NT), 0, st, a.W, a.rows, a.cols, a.hinv, a.i1, a.scale, a.ld_scale,
                     a.g_idx, a.strategy, a.block_h, a.qmin, a.qmax, a.gscale, a.codes, a.losses, a.err, a.lde,
                     a.err_col, a.sb);
}
}  // namespace

void launch_sweep4(bool bf16, dim3 grid, hipStream_t st, const SweepLaunch& a) {
  bf16 ? go(sweep4_block_kernel<true>, grid, st, a) : go(sweep4_block_kernel<false>, grid, st, a);
}

}  // namespace gsw
}  // namespace mi355q
