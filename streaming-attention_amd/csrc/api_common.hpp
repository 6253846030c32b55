// Shared by the translation units of libstreamattn.so: status helpers, argument limits, the moment
// kernel configurations and the dispatch functions one unit provides to another.  The kernels are
// compiled in separate units (moments, moment accumulation, block attention per configuration, the
// rest) so the build runs them in parallel.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/streamattn.h"

namespace sta {
struct MomArgs;
struct WsArgs;
struct BlockArgs;
struct FlashArgs;
}  // namespace sta

namespace sta_api {

extern thread_local int g_last_hip_error;  // defined in api.hip

inline int hip_status(hipError_t e) {
  if (e == hipSuccess) return STA_OK;
  g_last_hip_error = static_cast<int>(e);
  return STA_ERR_HIP;
}

inline int check_launch() { return hip_status(hipGetLastError()); }

inline bool dtype_ok(int dt) { return dt == STA_F32 || dt == STA_BF16 || dt == STA_F16; }

// Key width: rows up to 128 dimensions are staged whole; wider keys (up to kMaxD) through dimension
// windows (MomArgs::win): every feature split stages the 4 blocks of 32 dimensions its monomials use.
constexpr int kMaxD = 256;
constexpr int kMaxStagedD = 128;
constexpr int kMaxDv = 256;
constexpr int kMaxDegree = 8;
constexpr int kMaxDegreeWindows = 4;  // a monomial of degree <= 4 touches at most the 4 blocks of a window
constexpr int kMaxDHighDegree = 64;   // degree >= 5 (NX >= 3): rows of at most 64 dimensions
constexpr int kTileRows = 128;
constexpr int kMaxFlashD = 128;  // the exact flash baseline (the reference's Triton bound)

// Per-wave tile counts the moment kernels are instantiated for, per (extra factors, d > 64).  Every
// entry must appear in STA_MOMENT_CONFIGS (or STA_MOMENT_CONFIGS_HI).
constexpr int kNtD2[] = {2, 4, 5, 9, 16};
constexpr int kNtD3[] = {4, 8, 16};
constexpr int kNtBigD2[] = {5, 16};
constexpr int kNtBigD3[] = {4, 16};
constexpr int kNtD4[] = {4, 8, 16};
constexpr int kNtBigD4[] = {4, 16};
constexpr int kNtHi[] = {4};  // degree 5 .. 8: d <= 64, fp32 products

// X(NT, NX, DBIG) for every instantiated moment configuration; NX = extra factors per feature quad
// (0: degree <= 2, 1: degree 3, 2: degree 4).
#define STA_MOMENT_CONFIGS(X)                                                                       \
  X(2, 0, false) X(4, 0, false) X(5, 0, false) X(9, 0, false) X(16, 0, false)                       \
  X(4, 1, false) X(8, 1, false) X(16, 1, false) X(5, 0, true) X(16, 0, true)                        \
  X(4, 1, true) X(16, 1, true) X(4, 2, false) X(8, 2, false) X(16, 2, false)                        \
  X(4, 2, true) X(16, 2, true)

// Degrees 5 .. 8 (NX = 3 .. 6): fp32 products only (the fp32-product scan and accumulation).
#define STA_MOMENT_CONFIGS_HI(X) X(4, 3, false) X(4, 4, false) X(4, 5, false) X(4, 6, false)

// X(NTS, NX, DBIG) of the wave-specialised moment kernels (moments_ws_kernel; split-bf16 products,
// degree <= 3): tiles per slot, extra factors per quad, d > 64.
#define STA_MOMENT_WS_CONFIGS(X)                                                                    \
  X(2, 0, false) X(3, 0, false) X(4, 0, false) X(5, 0, false)                                      \
  X(2, 1, false) X(3, 1, false) X(4, 1, false) X(5, 1, false)                                      \
  X(3, 0, true) X(5, 0, true)
constexpr int kWsNts[] = {2, 3, 4, 5};

// X(NT, NX, CT) of the block accumulation (moment_block_kernel: split-bf16 products, d <= 64; degree
// <= 2: more tiles, column tiles or extra factors spill its registers next to the prefetched slice).
#define STA_MOMENT_BLOCK_CONFIGS(X) X(2, 0, 2) X(4, 0, 2) X(2, 0, 4)

// X(NT, NX, DBIG) of the 64-column (split-product) moment kernels.
#define STA_MOMENT_CONFIGS_64(X) X(5, 0, false)

template <size_t L>
int next_nt(const int (&tab)[L], int want) {
  for (size_t i = 0; i < L; ++i)
    if (tab[i] >= want) return tab[i];
  return -1;
}

// 64 value columns per workgroup: split products, a configuration in STA_MOMENT_CONFIGS_64, and
// 32 < dv <= 64 (so the workgroup's columns are the whole row of the partials).
inline bool moment_columns64_ok(int d, int degree, int dv, int wave_tiles, int products) {
  return products == STA_PRODUCTS_SPLIT_BF16 && d <= 64 && degree <= 2 && dv > 32 && dv <= 64 && wave_tiles == 5;
}

// extra factors per feature quad of a degree (the NX of the moment kernels)
inline int moment_extra_factors(int degree) { return degree <= 2 ? 0 : degree - 2; }

// d: the staged (virtual) key width, at most kMaxStagedD.
inline int moment_wave_tiles(int d, int degree, int want) {
  if (want < 1) want = 1;
  const int nx = moment_extra_factors(degree);
  const bool big = d > 64;
  if (d > kMaxStagedD) return -1;
  if (nx >= 3) return big ? -1 : next_nt(kNtHi, want);
  if (nx == 2) return big ? next_nt(kNtBigD4, want) : next_nt(kNtD4, want);
  if (!big) return nx ? next_nt(kNtD3, want) : next_nt(kNtD2, want);
  return nx ? next_nt(kNtBigD3, want) : next_nt(kNtBigD2, want);
}

// launch_moments.hip, one object per (SPLIT, CG): the prefill moment scan (moments_kernel) for wave-tile
// count nt, with fp32 (SPLIT false) or split-bf16 (SPLIT true) matrix-core products and CG value columns
// per workgroup (64: split products, STA_MOMENT_CONFIGS_64 only).
template <bool SPLIT, int CG>
int dispatch_moments(const sta::MomArgs& a, int64_t bh, hipStream_t s, int nt, int nx);
// launch_moments_ws.hip, one object per (ES, CT): the wave-specialised moment scan for nts tiles per
// slot (moments_ws_kernel, 16 CT value columns per workgroup).
template <int ES, int CT>
int dispatch_moments_ws(const sta::WsArgs& a, int64_t bh, hipStream_t s, int nts, int nx);
// launch_accumulate.hip: in-place accumulation into a decode state (moment_accumulate_kernel).
int dispatch_accumulate(const sta::MomArgs& a, int64_t bh, hipStream_t s, int nt, int nx, bool split);
int dispatch_accumulate_block(const sta::MomArgs& a, int64_t bh, hipStream_t s, int nt, int nx, int ct);
// 1 when moment_block_kernel is built for (wave tiles, extra factors, column tiles).
inline bool accumulate_block_ok(int nt, int nx, int ct) {
#define STA_CASE(NT, NX, CT) if (nt == NT && nx == NX && ct == CT) return true;
  STA_MOMENT_BLOCK_CONFIGS(STA_CASE)
#undef STA_CASE
  return false;
}
// launch_block.hip, one object per (DP, DVT, ES): the residual / combine kernel (block_attn_kernel) for
// padded key width DP, value-column tile count DVT and element size ES.
template <int DP, int DVT, int ES>
int launch_block(const sta::BlockArgs& a, int64_t bh, hipStream_t s);
// launch_flash.hip, one object per (DP, DVT, ES): exact causal softmax attention (flash_attn_kernel).
template <int DP, int DVT, int ES>
int launch_flash(const sta::FlashArgs& a, int64_t bh, hipStream_t s);

}  // namespace sta_api
