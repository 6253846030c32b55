// Launch of the residual / combine kernel (block_attn_kernel) for one configuration.  The build compiles
// this unit once per padded key width DP (16, 32, 64, 128, 256), value-column tile count DVT (1, 2, 4,
// 8, 16) and element size ES (4: fp32, 2: bf16 / fp16), given as -DSTA_BLOCK_DP=, -DSTA_BLOCK_DVT= and
// -DSTA_BLOCK_ES=, so the fifty configurations compile in parallel; each object holds the fp32-product
// kernel (and its degree 5 .. 8 form) and the split-bf16-product kernel of its configuration (16-bit
// objects also the split kernel for bf16 key / value rows, which leaves out their zero lo planes).
#include "api_common.hpp"
#include "block_attn.hip"

#if !defined(STA_BLOCK_DP) || !defined(STA_BLOCK_DVT) || !defined(STA_BLOCK_ES)
#error "launch_block.hip is compiled with -DSTA_BLOCK_DP= -DSTA_BLOCK_DVT= -DSTA_BLOCK_ES="
#endif

namespace sta_api {

template <int DP, int DVT, int ES>
int launch_block(const sta::BlockArgs& a, int64_t bh, hipStream_t s) {
  const int64_t grid = bh * a.n_tiles;
  if (grid <= 0 || grid > 0x7fffffff) return STA_ERR_SHAPE;
  if (a.split && ES == 2 && a.dtype == sta::BF16 && a.rep_k == nullptr)  // key / value rows exact in bf16
    hipLaunchKernelGGL((sta::block_attn_kernel<DP, DVT, 2, ES, true, ES == 2>), dim3(static_cast<unsigned>(grid)),
                       dim3(256), 0, s, a);
  else if (a.split)
    hipLaunchKernelGGL((sta::block_attn_kernel<DP, DVT, 2, ES, true>), dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                       s, a);
  else if (a.degree > 4)
    hipLaunchKernelGGL((sta::block_attn_kernel<DP, DVT, 2, ES, false, false, true>), dim3(static_cast<unsigned>(grid)),
                       dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((sta::block_attn_kernel<DP, DVT, 2, ES, false>), dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                       s, a);
  return check_launch();
}

template int launch_block<STA_BLOCK_DP, STA_BLOCK_DVT, STA_BLOCK_ES>(const sta::BlockArgs&, int64_t, hipStream_t);

}  // namespace sta_api
