// Launches of the prefill moment scan (moments_kernel), one instantiation per wave-tile count, degree-3
// flag, d > 64 flag and element size (4: fp32, 2: bf16 / fp16, so the chunk staging is straight-line).
// The build compiles this unit three times: -DSTA_MOM_SPLIT=0 (fp32 matrix-core products),
// -DSTA_MOM_SPLIT=1 (split-bf16 products) and -DSTA_MOM_SPLIT=1 -DSTA_MOM_CG=64 (split-bf16 products,
// 64 value columns per workgroup, for the configurations in STA_MOMENT_CONFIGS_64).
#include "api_common.hpp"
#include "moments.hip"

#if !defined(STA_MOM_SPLIT)
#error "launch_moments.hip is compiled with -DSTA_MOM_SPLIT=<0|1>"
#endif
#if !defined(STA_MOM_CG)
#define STA_MOM_CG 32
#endif

namespace sta_api {
namespace {

template <int NT, int NX, bool DBIG, int ES, bool SPLIT, int CG, bool FULL>
int launch_full(const sta::MomArgs& a, int64_t bh, hipStream_t s) {
  const size_t smem = static_cast<size_t>(sta::mom_smem_floats(DBIG, NT, CG)) * sizeof(float);
  auto fn = sta::moments_kernel<NT, NX, DBIG, ES, SPLIT, CG, FULL>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
  if (e != hipSuccess) return hip_status(e);
  const int64_t grid = bh * a.fsplit * a.csplit;
  if (grid <= 0 || grid > 0x7fffffff) return STA_ERR_SHAPE;
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(grid)), dim3(sta::MOM_THREADS), smem, s, a);
  return check_launch();
}

// fp32 rows of exactly the kernel's row width take the instantiation without dummy staging slots
template <int NT, int NX, bool DBIG, int ES, bool SPLIT, int CG>
int launch(const sta::MomArgs& a, int64_t bh, hipStream_t s) {
  if constexpr (ES == 4) {
    if (sta::mom_full_slots(DBIG, ES, a.d)) return launch_full<NT, NX, DBIG, ES, SPLIT, CG, true>(a, bh, s);
  }
  return launch_full<NT, NX, DBIG, ES, SPLIT, CG, false>(a, bh, s);
}

}  // namespace

template <bool SPLIT, int CG>
int dispatch_moments(const sta::MomArgs& a, int64_t bh, hipStream_t s, int nt, int nx) {
  const bool big = a.d > 64;
#define STA_CASE(NT, D3, BIG)                                                                       \
  if (nt == NT && nx == D3 && big == BIG)                                                         \
    return a.esize == 4 ? launch<NT, D3, BIG, 4, SPLIT, CG>(a, bh, s) : launch<NT, D3, BIG, 2, SPLIT, CG>(a, bh, s);
#if STA_MOM_CG == 64
  STA_MOMENT_CONFIGS_64(STA_CASE)
#else
  STA_MOMENT_CONFIGS(STA_CASE)
#if !STA_MOM_SPLIT
  STA_MOMENT_CONFIGS_HI(STA_CASE)
#endif
#endif
#undef STA_CASE
  return STA_ERR_UNSUPPORTED;
}

template int dispatch_moments<STA_MOM_SPLIT != 0, STA_MOM_CG>(const sta::MomArgs&, int64_t, hipStream_t, int, int);

}  // namespace sta_api
