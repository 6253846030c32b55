// Launch of the exact causal softmax attention (flash_attn_kernel) for one configuration.  The build
// compiles this unit once per padded key width DP (16, 32, 64, 128), value-column tile count DVT (1, 2,
// 4, 8, 16) and element size ES (4: fp32, 2: bf16 / fp16), given as -DSTA_FLASH_DP=, -DSTA_FLASH_DVT= and
// -DSTA_FLASH_ES=, so the forty instantiations compile in parallel.
#include "api_common.hpp"
#include "flash_attn.hip"

#if !defined(STA_FLASH_DP) || !defined(STA_FLASH_DVT) || !defined(STA_FLASH_ES)
#error "launch_flash.hip is compiled with -DSTA_FLASH_DP= -DSTA_FLASH_DVT= -DSTA_FLASH_ES="
#endif

namespace sta_api {

template <int DP, int DVT, int ES>
int launch_flash(const sta::FlashArgs& a, int64_t bh, hipStream_t s) {
  const int64_t grid = bh * a.n_tiles;
  if (grid <= 0 || grid > 0x7fffffff) return STA_ERR_SHAPE;
  if constexpr (ES == 4) {
    hipLaunchKernelGGL((sta::flash_attn_kernel<DP, DVT, 2, 4>), dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, a);
  } else if (a.dtype == STA_F16) {
    hipLaunchKernelGGL((sta::flash_attn16_kernel<DP, DVT, 2, true>), dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                       s, a);
  } else {
    hipLaunchKernelGGL((sta::flash_attn16_kernel<DP, DVT, 2, false>), dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                       s, a);
  }
  return check_launch();
}

template int launch_flash<STA_FLASH_DP, STA_FLASH_DVT, STA_FLASH_ES>(const sta::FlashArgs&, int64_t, hipStream_t);

}  // namespace sta_api
