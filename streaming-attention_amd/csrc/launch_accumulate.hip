// Launches of the in-place moment accumulation into a decode state (moment_accumulate_kernel), one
// instantiation per wave-tile count, extra-factor count (NX), d > 64 flag and element size.
#include "api_common.hpp"
#include "moments.hip"

namespace sta_api {
namespace {

template <int NT, int NX, bool DBIG, int ES, bool SPLIT>
int launch(const sta::MomArgs& a, int64_t bh, hipStream_t s) {
  const size_t smem = static_cast<size_t>(sta::mom_acc_smem_floats(DBIG, NT)) * sizeof(float);
  auto fn = sta::moment_accumulate_kernel<NT, NX, DBIG, ES, SPLIT>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
  if (e != hipSuccess) return hip_status(e);
  const int64_t grid = bh * a.fsplit * a.csplit;
  if (grid <= 0 || grid > 0x7fffffff) return STA_ERR_SHAPE;
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(grid)), dim3(sta::MOM_THREADS), smem, s, a);
  return check_launch();
}

template <int NT, int NX, int ES, int CT>
int launch_block(const sta::MomArgs& a, int64_t bh, hipStream_t s) {
  const size_t smem = static_cast<size_t>(sta::momb_smem_floats(NT, CT)) * sizeof(float);
  auto fn = sta::moment_block_kernel<NT, NX, ES, CT>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
  if (e != hipSuccess) return hip_status(e);
  const int64_t grid = bh * (a.csplit * 32 / (16 * CT));
  if (grid <= 0 || grid > 0x7fffffff) return STA_ERR_SHAPE;
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(grid)), dim3(sta::MOMB_THREADS), smem, s, a);
  return check_launch();
}

}  // namespace

int dispatch_accumulate_block(const sta::MomArgs& a, int64_t bh, hipStream_t s, int nt, int nx, int ct) {
#define STA_CASE(NT, NX, CT)                                                                        \
  if (nt == NT && nx == NX && ct == CT)                                                           \
    return a.esize == 4 ? launch_block<NT, NX, 4, CT>(a, bh, s) : launch_block<NT, NX, 2, CT>(a, bh, s);
  STA_MOMENT_BLOCK_CONFIGS(STA_CASE)
#undef STA_CASE
  return STA_ERR_UNSUPPORTED;
}

int dispatch_accumulate(const sta::MomArgs& a, int64_t bh, hipStream_t s, int nt, int nx, bool split) {
  const bool big = a.d > 64;
#define STA_CASE(NT, D3, BIG)                                                                       \
  if (nt == NT && nx == D3 && big == BIG) {                                                       \
    if (split) return a.esize == 4 ? launch<NT, D3, BIG, 4, true>(a, bh, s) : launch<NT, D3, BIG, 2, true>(a, bh, s); \
    return a.esize == 4 ? launch<NT, D3, BIG, 4, false>(a, bh, s) : launch<NT, D3, BIG, 2, false>(a, bh, s); \
  }
  STA_MOMENT_CONFIGS(STA_CASE)
#undef STA_CASE
#define STA_CASE(NT, NX, BIG)                                                                       \
  if (nt == NT && nx == NX && big == BIG && !split)                                               \
    return a.esize == 4 ? launch<NT, NX, BIG, 4, false>(a, bh, s) : launch<NT, NX, BIG, 2, false>(a, bh, s);
  STA_MOMENT_CONFIGS_HI(STA_CASE)
#undef STA_CASE
  return STA_ERR_UNSUPPORTED;
}

}  // namespace sta_api
