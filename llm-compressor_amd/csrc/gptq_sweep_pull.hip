// 16-lane GPTQ sweeps of whole integer blocks that first apply the K = 128
// updates of the earlier blocks of their mid-block.
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

void launch_sweep_pull(bool bf16, bool zp, dim3 grid, hipStream_t st, const SweepLaunch& a) {
  if (bf16) zp ? go(sweep_block_kernel<true, true, true, QK_INT, true>, grid, st, a)
            : go(sweep_block_kernel<true, true, false, QK_INT, true>, grid, st, a);
  else      zp ? go(sweep_block_kernel<true, false, true, QK_INT, true>, grid, st, a)
            : go(sweep_block_kernel<true, false, false, QK_INT, true>, grid, st, a);
}

}  // namespace gsw
}  // namespace mi355q
