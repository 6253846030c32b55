// Launches of the wave-specialised prefill moment scan (moments_ws_kernel, split-bf16 products).  The
// build compiles this unit once per element size and column-tile count (-DSTA_WS_ES=4|2,
// -DSTA_WS_CT=4|2); each object holds the configurations of STA_MOMENT_WS_CONFIGS.
#include <type_traits>

#include "api_common.hpp"
#include "moments_ws.hip"

#if !defined(STA_WS_ES) || !defined(STA_WS_CT)
#error "launch_moments_ws.hip is compiled with -DSTA_WS_ES= -DSTA_WS_CT="
#endif

namespace sta_api {
namespace {

template <int NTS, int NX, bool DBIG, int ES, int CT>
int launch_ws(const sta::WsArgs& a, int64_t bh, hipStream_t s) {
  const size_t smem = static_cast<size_t>(sta::ws_smem_floats(DBIG, 16 * CT, NTS)) * sizeof(float);
  // phase 1 of a segmented scan (segment totals, TOT 1) and phase 3 (accumulation into a persistent
  // state, TOT 2) are update-only instantiations: no query work at all; bf16 values (exact in bf16) take
  // the instantiation without the products of their zero lo plane
  const bool vx = ES == 2 && a.m.dtype == sta::BF16;
  auto pick = [&](auto tot) {
    constexpr int T = decltype(tot)::value;
    return vx ? sta::moments_ws_kernel<NTS, NX, DBIG, ES, CT, T, ES == 2> : sta::moments_ws_kernel<NTS, NX, DBIG, ES, CT, T, false>;
  };
  auto fn = a.phase == 1 ? pick(std::integral_constant<int, 1>{})
                         : a.phase == 3 ? pick(std::integral_constant<int, 2>{}) : pick(std::integral_constant<int, 0>{});
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
  if (e != hipSuccess) return hip_status(e);
  const int64_t grid = bh * a.m.fsplit * a.m.csplit * a.nseg;
  if (grid <= 0 || grid > 0x7fffffff) return STA_ERR_SHAPE;
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(grid)), dim3(sta::WS_THREADS), smem, s, a);
  return check_launch();
}

}  // namespace

template <int ES, int CT>
int dispatch_moments_ws(const sta::WsArgs& a, int64_t bh, hipStream_t s, int nts, int nx) {
  const bool big = a.m.d > 64;
#define STA_CASE(NTS, NX, BIG) \
  if (nts == NTS && nx == NX && big == BIG) return launch_ws<NTS, NX, BIG, ES, CT>(a, bh, s);
  STA_MOMENT_WS_CONFIGS(STA_CASE)
#undef STA_CASE
  return STA_ERR_UNSUPPORTED;
}

template int dispatch_moments_ws<STA_WS_ES, STA_WS_CT>(const sta::WsArgs&, int64_t, hipStream_t, int, int);

}  // namespace sta_api
