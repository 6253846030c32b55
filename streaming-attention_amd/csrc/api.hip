// extern "C" entry points of libstreamattn.so (declared in include/streamattn.h): argument checks and
// kernel launches.  The moment and block-attention kernels are instantiated and launched from their own
// units (launch_moments.hip, launch_accumulate.hip, launch_block.hip); this unit includes their sources
// for the argument structs only.  The library allocates nothing; every buffer is the caller's, except
// the fixed static scratch of sta_decode_step_static (below).
#include <algorithm>
#include <mutex>

#include "api_common.hpp"
#include "block_attn.hip"
#include "compress.hip"
#include "decode.hip"
#include "flash_attn.hip"
#include "moments_ws.hip"

namespace sta_api {
thread_local int g_last_hip_error = 0;
}  // namespace sta_api

using namespace sta_api;

// Device memory of sta_decode_step_static, the entry point for callers that cannot allocate: the
// decode query's moment partials, part_num [S][splits][ldv] and then part_den [S][splits] from the next
// 64-float (256-byte) boundary.  Each device the library runs on holds its own copy from module load
// to process end.  In host code the name is not a device address: kernels get the per-device pointer
// from static_scratch_ptr().
static __device__ __align__(256) float scratch[STA_STATIC_SCRATCH_BYTES / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// Address of `scratch` on `device`, looked up once per device with that device current.
int static_scratch_ptr(int device, float** out) {
  if (device < 0 || device >= kMaxDevices) return STA_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    int cur = -1;
    int st = hip_status(hipGetDevice(&cur));
    if (st != STA_OK) return st;
    if (cur != device && (st = hip_status(hipSetDevice(device))) != STA_OK) return st;
    void* p = nullptr;
    st = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (cur != device) {
      const int back = hip_status(hipSetDevice(cur));
      if (st == STA_OK) st = back;
    }
    if (st != STA_OK) return st;
    if (!p) return STA_ERR_HIP;
    g_scratch_ptr[device] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[device];
  return STA_OK;
}

// Dynamic LDS above the default 64 KiB needs the kernel's limit raised first (gfx950: 160 KiB per
// workgroup).
int lds_limit(const void* kernel, size_t bytes) {
  if (bytes <= 65536) return STA_OK;
  return hip_status(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)));
}

__global__ void zero_fill_kernel(float* p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = 0.f;
}

}  // namespace

namespace {

__global__ void selftest_mfma_kernel(const float* a, const float* b, float* d) {
  const int l = threadIdx.x;
  sta::floatx4 c = sta::floatx4{0.f, 0.f, 0.f, 0.f};
  c = sta::mfma4(a[l], b[l], c);
  const int i = l & 15, g = l >> 4;
  for (int r = 0; r < 4; ++r) d[(4 * g + r) * 16 + i] = c[r];
}

// Residual and flash kernel configurations by value width (value-column tiles of 16).
template <int DP, int ES>
int dispatch_dvt(const sta::BlockArgs& a, int64_t bh, hipStream_t s) {
  if (a.dv <= 16) return launch_block<DP, 1, ES>(a, bh, s);
  if (a.dv <= 32) return launch_block<DP, 2, ES>(a, bh, s);
  if (a.dv <= 64) return launch_block<DP, 4, ES>(a, bh, s);
  if (a.dv <= 128) return launch_block<DP, 8, ES>(a, bh, s);
  if (a.dv <= 256) return launch_block<DP, 16, ES>(a, bh, s);
  return STA_ERR_UNSUPPORTED;
}

template <int DP, int ES>
int dispatch_flash_dvt(const sta::FlashArgs& a, int64_t bh, hipStream_t s) {
  if (a.dv <= 16) return launch_flash<DP, 1, ES>(a, bh, s);
  if (a.dv <= 32) return launch_flash<DP, 2, ES>(a, bh, s);
  if (a.dv <= 64) return launch_flash<DP, 4, ES>(a, bh, s);
  if (a.dv <= 128) return launch_flash<DP, 8, ES>(a, bh, s);
  if (a.dv <= 256) return launch_flash<DP, 16, ES>(a, bh, s);
  return STA_ERR_UNSUPPORTED;
}

// Exclusive scan over the segments of each (head, feature split, column group): seg_state[p] <- sum of
// the totals of segments 0 .. p - 1, in segment order (deterministic).  One thread per float of a unit.
__global__ __launch_bounds__(256) void ws_seg_scan_kernel(float* seg_state, int64_t groups, int nseg, int unit) {
  const int64_t total = groups * unit;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t g = e / unit;
    const int64_t off = e - g * unit;
    float* base = seg_state + g * nseg * static_cast<int64_t>(unit) + off;
    float acc = 0.f;
    for (int p = 0; p < nseg; ++p) {
      const float t = base[static_cast<int64_t>(p) * unit];
      base[static_cast<int64_t>(p) * unit] = acc;
      acc += t;
    }
  }
}

}  // namespace

extern "C" {

int sta_version(void) { return 100; }

const char* sta_status_string(int status) {
  switch (status) {
    case STA_OK: return "ok";
    case STA_ERR_SHAPE: return "inconsistent shape or count";
    case STA_ERR_UNSUPPORTED: return "unsupported size or degree for the HIP kernels";
    case STA_ERR_DTYPE: return "unknown dtype code";
    case STA_ERR_HIP: return "HIP runtime error";
    case STA_ERR_ARG: return "invalid argument";
    case STA_ERR_SCRATCH: return "working set exceeds the static scratch (sta_static_scratch_bytes per device)";
    default: return "unknown status";
  }
}

int sta_last_hip_error(void) { return g_last_hip_error; }

int sta_limits(int* max_d, int* max_dv, int* max_degree, int* max_compress_in) {
  if (max_d) *max_d = kMaxD;
  if (max_dv) *max_dv = kMaxDv;
  if (max_degree) *max_degree = kMaxDegree;
  if (max_compress_in) *max_compress_in = sta::CMP_MAX_IN;
  return STA_OK;
}

int sta_flash_attention(const void* q, const void* k, const void* v, int dtype, int64_t bh, int64_t n, int d,
                        int dv, int ld_qk, int ld_v, float scale, void* out, int out_dtype, void* stream) {
  if (!q || !k || !v || !out) return STA_ERR_ARG;
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype)) return STA_ERR_DTYPE;
  if (bh <= 0 || n <= 0 || d <= 0 || dv <= 0) return STA_ERR_SHAPE;
  if (d > kMaxFlashD || dv > kMaxDv) return STA_ERR_UNSUPPORTED;
  if (ld_qk < d || ld_qk % 4 != 0 || ld_v < dv || ld_v % 4 != 0) return STA_ERR_ARG;
  if (((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15u) != 0)
    return STA_ERR_ARG;
  if (n >= (int64_t(1) << 31) - 128) return STA_ERR_UNSUPPORTED;
  constexpr int kFlashRows = 128;  // 64 RS query rows per workgroup, RS = 2
  sta::FlashArgs a;
  a.q = q; a.k = k; a.v = v; a.dtype = dtype; a.n = n; a.d = d; a.dv = dv; a.ldqk = ld_qk; a.ldv = ld_v;
  a.scale2 = scale * 1.4426950408889634f;
  a.n_tiles = static_cast<int>((n + kFlashRows - 1) / kFlashRows);
  a.out = out; a.out_dtype = out_dtype;
  a.vec_out = (out_dtype == STA_F32 && dv % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0) ? 1 : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool f32 = dtype == STA_F32;
  if (d <= 16) return f32 ? dispatch_flash_dvt<16, 4>(a, bh, s) : dispatch_flash_dvt<16, 2>(a, bh, s);
  if (d <= 32) return f32 ? dispatch_flash_dvt<32, 4>(a, bh, s) : dispatch_flash_dvt<32, 2>(a, bh, s);
  if (d <= 64) return f32 ? dispatch_flash_dvt<64, 4>(a, bh, s) : dispatch_flash_dvt<64, 2>(a, bh, s);
  return f32 ? dispatch_flash_dvt<128, 4>(a, bh, s) : dispatch_flash_dvt<128, 2>(a, bh, s);
}

int sta_tile_rows(void) { return kTileRows; }

int sta_moment_chunk(int d) { return d > 0 ? sta::MOM_C : 0; }

int sta_moment_wave_tiles(int d, int degree, int want) {
  if (d <= 0 || d > kMaxD || degree < 0 || degree > kMaxDegree) return -1;
  return moment_wave_tiles(d, degree, want);
}

int sta_moment_partials_layout(int64_t n, int dv, int64_t* rows, int* ld, int* row_offset) {
  if (n <= 0 || dv <= 0 || !rows || !ld || !row_offset) return STA_ERR_ARG;
  *rows = n + 2 * sta::MOM_GUARD;
  *ld = 32 * ((dv + 31) / 32);
  *row_offset = sta::MOM_GUARD;
  return STA_OK;
}

int sta_moment_mixed_ok(int d, int degree, int wave_tiles) {
  return (d > 0 && d <= 64 && degree >= 0 && degree <= 4 && (wave_tiles == 4 || wave_tiles == 5) &&
          moment_wave_tiles(d, degree, wave_tiles) == wave_tiles)
             ? 1
             : 0;
}

int sta_moment_columns_ok(int d, int degree, int dv, int wave_tiles, int products) {
  return moment_columns64_ok(d, degree, dv, wave_tiles, products) ? 1 : 0;
}

int sta_moment_occupancy(int d, int wave_tiles) {
  return (wave_tiles > 0 && d > 0) ? sta::mom_wg_per_cu(wave_tiles, d > 64) : 0;
}

int sta_moment_occupancy_degree(int d, int degree, int wave_tiles) {
  return (wave_tiles > 0 && d > 0 && degree >= 0)
             ? sta::mom_wg_per_cu(wave_tiles, d > 64, 32, moment_extra_factors(degree))
             : 0;
}

// Row stride and window checks shared by sta_moments and sta_moment_accumulate: without windows the
// rows are d long (ld_qk == d); with windows d is the staged width kMaxStagedD, ld_qk a multiple of 32
// of at least 128 and at most kMaxD, degree <= kMaxDegreeWindows.
static int window_check(int d, int ld_qk, int degree, const int32_t* windows) {
  if (!windows) return ld_qk == d ? STA_OK : STA_ERR_ARG;
  if (d != kMaxStagedD || ld_qk < kMaxStagedD || ld_qk > kMaxD || ld_qk % 32 != 0) return STA_ERR_ARG;
  if (degree > kMaxDegreeWindows) return STA_ERR_UNSUPPORTED;
  return STA_OK;
}

int sta_moments(const void* q, const void* k, const void* v, int dtype, int64_t bh, int64_t n, int d, int ld_qk,
                int dv, int ldv, int degree, float scale, int chunk, int shift, int fsplit, int wave_tiles, int mixed,
                int products, int columns, const uint32_t* feat_quads, const float* feat_coef,
                const int32_t* windows, float* low_num, float* low_den, void* stream) {
  if (!q || !k || !v || !feat_quads || !feat_coef || !low_num || !low_den) return STA_ERR_ARG;
  if (!dtype_ok(dtype)) return STA_ERR_DTYPE;
  if (bh <= 0 || n <= 0 || d <= 0 || dv <= 0 || fsplit <= 0 || wave_tiles <= 0) return STA_ERR_SHAPE;
  if (d > kMaxStagedD || dv > kMaxDv || degree < 0 || degree > kMaxDegree) return STA_ERR_UNSUPPORTED;
  if (moment_wave_tiles(d, degree, wave_tiles) != wave_tiles) return STA_ERR_UNSUPPORTED;
  if (const int wst = window_check(d, ld_qk, degree, windows); wst != STA_OK) return wst;
  // degree >= 5 runs fp32 products on 32 columns only
  if (moment_extra_factors(degree) >= 3 && (products != STA_PRODUCTS_FP32 || columns != 32)) return STA_ERR_UNSUPPORTED;
  if (chunk != sta_moment_chunk(d) || shift < 0 || shift >= chunk) return STA_ERR_ARG;
  if (mixed != 0 && (mixed != 1 || fsplit % 2 != 0 || !sta_moment_mixed_ok(d, degree, wave_tiles))) return STA_ERR_ARG;
  if (products != STA_PRODUCTS_FP32 && products != STA_PRODUCTS_SPLIT_BF16) return STA_ERR_ARG;
  if (columns != 32 && (columns != 64 || mixed != 0 || !moment_columns64_ok(d, degree, dv, wave_tiles, products)))
    return STA_ERR_ARG;
  // rows are read in 16-byte units: d must be a whole number of units, v rows whole 32-column groups,
  // every base 16-byte aligned, and a head's rows addressable with 32-bit byte offsets
  const int esize = dtype == STA_F32 ? 4 : 2;
  if ((d * esize) % 16 != 0 || ldv < dv || ldv % 32 != 0) return STA_ERR_ARG;
  if (((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15u) != 0)
    return STA_ERR_ARG;
  if (n * static_cast<int64_t>(ldv > ld_qk ? ldv : ld_qk) * esize >= (int64_t(1) << 32) || n >= (int64_t(1) << 30))
    return STA_ERR_UNSUPPORTED;
  sta::MomArgs a;
  a.q = q; a.k = k; a.v = v; a.dtype = dtype; a.n = n; a.d = d; a.dv = dv; a.scale = scale; a.shift = shift;
  a.fsplit = fsplit; a.mixed = mixed; a.csplit = (dv + columns - 1) / columns; a.quads = feat_quads;
  a.fcoef = feat_coef; a.low_num = low_num; a.low_den = low_den; a.ldv = ldv; a.esize = esize;
  a.ldo = 32 * ((dv + 31) / 32); a.ldk = ld_qk; a.win = windows;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (columns == 64) return dispatch_moments<true, 64>(a, bh, s, wave_tiles, moment_extra_factors(degree));
  return products == STA_PRODUCTS_SPLIT_BF16 ? dispatch_moments<true, 32>(a, bh, s, wave_tiles, moment_extra_factors(degree))
                                             : dispatch_moments<false, 32>(a, bh, s, wave_tiles, moment_extra_factors(degree));
}

int sta_moments_ws_ok(int d, int degree, int slot_tiles, int column_tiles, int dv) {
  if (d <= 0 || d > kMaxStagedD || degree < 0 || degree > 3 || dv <= 0 || dv > kMaxDv) return 0;
  if (column_tiles != 4 && column_tiles != 2) return 0;
  if (column_tiles == 4 && ((dv + 31) / 32) % 2 != 0) return 0;
  const int nx = moment_extra_factors(degree);
  const bool big = d > 64;
#define STA_CASE(NTS, NX, BIG) \
  if (slot_tiles == NTS && nx == NX && big == BIG) return 1;
  STA_MOMENT_WS_CONFIGS(STA_CASE)
#undef STA_CASE
  return 0;
}

int64_t sta_moments_ws_handoff_bytes(int64_t bh, int fsplit, int slot_tiles, int column_tiles, int dv) {
  if (bh <= 0 || fsplit <= 0 || slot_tiles <= 0 || (column_tiles != 2 && column_tiles != 4) || dv <= 0) return -1;
  const int64_t csplit = (dv + 16 * column_tiles - 1) / (16 * column_tiles);
  const int64_t pairs = (slot_tiles + 1) / 2;
  // [grid][2 parities][4 slots][pairs][column tiles][hi, lo][64 lanes] of 16 bytes
  return bh * fsplit * csplit * 2 * 4 * pairs * column_tiles * 2 * 64 * 16;
}

int64_t sta_moments_ws_seg_bytes(int64_t bh, int fsplit, int slot_tiles, int column_tiles, int dv, int nseg) {
  if (bh <= 0 || fsplit <= 0 || slot_tiles <= 0 || (column_tiles != 2 && column_tiles != 4) || dv <= 0 || nseg <= 0)
    return -1;
  const int64_t csplit = (dv + 16 * column_tiles - 1) / (16 * column_tiles);
  return bh * fsplit * csplit * nseg * sta::ws_seg_floats(slot_tiles, column_tiles) * int64_t(sizeof(float));
}

int sta_moments_ws_seg(const void* q, const void* k, const void* v, int dtype, int64_t bh, int64_t n, int d, int dv,
                       int ldv, int degree, float scale, int query_block, int shift, int fsplit, int slot_tiles,
                       int mixed, int column_tiles, const uint32_t* feat_quads, const float* feat_coef, void* handoff,
                       float* low_num, float* low_den, int nseg, int seg_blocks, float* seg_state, void* stream) {
  if (!q || !k || !v || !feat_quads || !feat_coef || !handoff || !low_num || !low_den) return STA_ERR_ARG;
  if (!dtype_ok(dtype)) return STA_ERR_DTYPE;
  if (bh <= 0 || n <= 0 || d <= 0 || dv <= 0 || fsplit <= 0 || slot_tiles <= 0) return STA_ERR_SHAPE;
  if (!sta_moments_ws_ok(d, degree, slot_tiles, column_tiles, dv)) return STA_ERR_UNSUPPORTED;
  if (query_block < 2 * sta::MOM_C || query_block % sta::MOM_C != 0 || shift < 0 || shift >= sta::MOM_C)
    return STA_ERR_ARG;
  if (mixed != 0 && (mixed != 1 || slot_tiles < 2)) return STA_ERR_ARG;
  const int esize = dtype == STA_F32 ? 4 : 2;
  if ((d * esize) % 16 != 0 || ldv < dv || ldv % 32 != 0 || ldv % (16 * column_tiles) != 0) return STA_ERR_ARG;
  if (((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
        reinterpret_cast<uintptr_t>(handoff)) & 15u) != 0)
    return STA_ERR_ARG;
  if (n * static_cast<int64_t>(ldv > d ? ldv : d) * esize >= (int64_t(1) << 32) || n >= (int64_t(1) << 30))
    return STA_ERR_UNSUPPORTED;
  // segments of seg_blocks query blocks, every one non-empty
  const int cpb = query_block / sta::MOM_C;
  const int64_t nch = (n + shift + sta::MOM_C - 1) / sta::MOM_C;
  if (nseg <= 0 || (nseg > 1 && (seg_blocks <= 0 || !seg_state))) return STA_ERR_ARG;
  const int64_t seg_chunks = nseg > 1 ? static_cast<int64_t>(seg_blocks) * cpb : nch;
  if (nseg > 1 && ((nseg - 1) * seg_chunks >= nch || nseg * seg_chunks < nch)) return STA_ERR_SHAPE;
  if (nseg > 1 && (reinterpret_cast<uintptr_t>(seg_state) & 15u) != 0) return STA_ERR_ARG;
  sta::WsArgs w;
  sta::MomArgs& a = w.m;
  a.q = q; a.k = k; a.v = v; a.dtype = dtype; a.n = n; a.d = d; a.dv = dv; a.scale = scale; a.shift = shift;
  a.fsplit = fsplit; a.mixed = mixed; a.csplit = (dv + 16 * column_tiles - 1) / (16 * column_tiles);
  a.quads = feat_quads; a.fcoef = feat_coef; a.low_num = low_num; a.low_den = low_den; a.ldv = ldv; a.esize = esize;
  a.ldo = 32 * ((dv + 31) / 32); a.ldk = d; a.win = nullptr;
  a.head_rows = n; a.rowmap = nullptr; a.state_num = nullptr; a.state_den = nullptr; a.n_feat = 0;
  w.cpb = cpb;
  w.mixed = mixed;
  w.hand = static_cast<uint4*>(handoff);
  w.nseg = nseg;
  w.seg_chunks = static_cast<int>(seg_chunks);
  w.phase = nseg > 1 ? 1 : 0;
  w.seg_state = nseg > 1 ? seg_state : nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nx = moment_extra_factors(degree);
  auto run = [&]() {
    if (column_tiles == 4)
      return esize == 4 ? dispatch_moments_ws<4, 4>(w, bh, s, slot_tiles, nx)
                        : dispatch_moments_ws<2, 4>(w, bh, s, slot_tiles, nx);
    return esize == 4 ? dispatch_moments_ws<4, 2>(w, bh, s, slot_tiles, nx)
                      : dispatch_moments_ws<2, 2>(w, bh, s, slot_tiles, nx);
  };
  int st = run();
  if (st != STA_OK || nseg == 1) return st;
  // segment totals -> the state before each segment, then every segment's scan from it
  const int unit = sta::ws_seg_floats(slot_tiles, column_tiles);
  const int64_t groups = bh * a.fsplit * a.csplit;
  const int64_t blocks = std::min<int64_t>((groups * unit + 255) / 256, 4096);
  hipLaunchKernelGGL(ws_seg_scan_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, seg_state, groups,
                     nseg, unit);
  if ((st = check_launch()) != STA_OK) return st;
  w.phase = 2;
  return run();
}

int sta_moments_ws(const void* q, const void* k, const void* v, int dtype, int64_t bh, int64_t n, int d, int dv,
                   int ldv, int degree, float scale, int query_block, int shift, int fsplit, int slot_tiles, int mixed,
                   int column_tiles, const uint32_t* feat_quads, const float* feat_coef, void* handoff,
                   float* low_num, float* low_den, void* stream) {
  return sta_moments_ws_seg(q, k, v, dtype, bh, n, d, dv, ldv, degree, scale, query_block, shift, fsplit, slot_tiles,
                            mixed, column_tiles, feat_quads, feat_coef, handoff, low_num, low_den, 1, 0, nullptr,
                            stream);
}

int sta_moment_accumulate(const void* k, const void* v, int dtype, int64_t bh, int64_t n, int64_t head_rows, int d,
                          int ld_k, int dv, int ldv, int degree, int fsplit, int wave_tiles,
                          const uint32_t* feat_quads, const float* feat_coef, const int32_t* feat_rows,
                          const int32_t* windows, int n_feat, int products, float* state_num, float* state_den,
                          void* stream) {
  if (!k || !v || !feat_quads || !feat_coef || !feat_rows || !state_num || !state_den) return STA_ERR_ARG;
  if (!dtype_ok(dtype)) return STA_ERR_DTYPE;
  if (bh <= 0 || n < 0 || head_rows < n || d <= 0 || dv <= 0 || fsplit <= 0 || wave_tiles <= 0 || n_feat <= 0)
    return STA_ERR_SHAPE;
  if (d > kMaxStagedD || dv > kMaxDv || degree < 0 || degree > kMaxDegree) return STA_ERR_UNSUPPORTED;
  if (moment_wave_tiles(d, degree, wave_tiles) != wave_tiles) return STA_ERR_UNSUPPORTED;
  if (products != STA_PRODUCTS_FP32 && products != STA_PRODUCTS_SPLIT_BF16) return STA_ERR_ARG;
  if (const int wst = window_check(d, ld_k, degree, windows); wst != STA_OK) return wst;
  if (moment_extra_factors(degree) >= 3 && products != STA_PRODUCTS_FP32) return STA_ERR_UNSUPPORTED;
  if (n == 0) return STA_OK;
  const int esize = dtype == STA_F32 ? 4 : 2;
  if ((d * esize) % 16 != 0 || ldv < dv || ldv % 32 != 0) return STA_ERR_ARG;
  if (((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15u) != 0) return STA_ERR_ARG;
  if (head_rows * static_cast<int64_t>(ldv > ld_k ? ldv : ld_k) * esize >= (int64_t(1) << 32) ||
      n >= (int64_t(1) << 30))
    return STA_ERR_UNSUPPORTED;
  sta::MomArgs a;
  a.q = k; a.k = k; a.v = v; a.dtype = dtype; a.n = n; a.d = d; a.dv = dv; a.scale = 1.0f; a.shift = 0;
  a.fsplit = fsplit; a.mixed = 0; a.csplit = (dv + 31) / 32; a.quads = feat_quads; a.fcoef = feat_coef;
  a.low_num = nullptr; a.low_den = nullptr; a.ldv = ldv; a.esize = esize; a.ldo = 32 * a.csplit;
  a.ldk = ld_k; a.win = windows;
  a.head_rows = head_rows; a.rowmap = feat_rows; a.state_num = state_num; a.state_den = state_den; a.n_feat = n_feat;
  return dispatch_accumulate(a, bh, static_cast<hipStream_t>(stream), wave_tiles, moment_extra_factors(degree),
                             products == STA_PRODUCTS_SPLIT_BF16);
}

int sta_moment_accumulate_block(const void* k, const void* v, int dtype, int64_t bh, int64_t n, int64_t head_rows,
                                int d, int dv, int ldv, int degree, int fsplit, int wave_tiles, int column_tiles,
                                const uint32_t* feat_quads, const float* feat_coef, const int32_t* feat_rows,
                                int n_feat, float* state_num, float* state_den, void* stream) {
  if (!k || !v || !feat_quads || !feat_coef || !feat_rows || !state_num || !state_den) return STA_ERR_ARG;
  if (!dtype_ok(dtype)) return STA_ERR_DTYPE;
  if (bh <= 0 || n < 0 || head_rows < n || d <= 0 || dv <= 0 || fsplit <= 0 || wave_tiles <= 0 || n_feat <= 0)
    return STA_ERR_SHAPE;
  if (d > 64 || dv > kMaxDv || degree < 0 || degree > 2) return STA_ERR_UNSUPPORTED;
  if (moment_wave_tiles(d, degree, wave_tiles) != wave_tiles ||
      !accumulate_block_ok(wave_tiles, moment_extra_factors(degree), column_tiles))
    return STA_ERR_UNSUPPORTED;
  if (n == 0) return STA_OK;
  const int esize = dtype == STA_F32 ? 4 : 2;
  // the state's rows are 32 ceil(dv / 32) floats, whole column groups of 16 column_tiles
  if ((d * esize) % 16 != 0 || ldv < dv || ldv % 32 != 0 || (32 * ((dv + 31) / 32)) % (16 * column_tiles) != 0)
    return STA_ERR_ARG;
  if (((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15u) != 0) return STA_ERR_ARG;
  if (head_rows * static_cast<int64_t>(ldv > d ? ldv : d) * esize >= (int64_t(1) << 32) || n >= (int64_t(1) << 30))
    return STA_ERR_UNSUPPORTED;
  sta::MomArgs a;
  a.q = k; a.k = k; a.v = v; a.dtype = dtype; a.n = n; a.d = d; a.dv = dv; a.scale = 1.0f; a.shift = 0;
  a.fsplit = fsplit; a.mixed = 0; a.csplit = (dv + 31) / 32; a.quads = feat_quads; a.fcoef = feat_coef;
  a.low_num = nullptr; a.low_den = nullptr; a.ldv = ldv; a.esize = esize; a.ldo = 32 * a.csplit;
  a.ldk = d; a.win = nullptr;
  a.head_rows = head_rows; a.rowmap = feat_rows; a.state_num = state_num; a.state_den = state_den; a.n_feat = n_feat;
  return dispatch_accumulate_block(a, bh, static_cast<hipStream_t>(stream), wave_tiles, moment_extra_factors(degree),
                                   column_tiles);
}

int sta_moment_accumulate_ws(const void* k, const void* v, int dtype, int64_t bh, int64_t n, int64_t head_rows, int d,
                             int ld_k, int dv, int ldv, int degree, int fsplit, int slot_tiles, int mixed,
                             int column_tiles, const uint32_t* feat_quads, const float* feat_coef,
                             const int32_t* feat_rows, int n_feat, float* state_num, float* state_den, void* stream) {
  if (!k || !v || !feat_quads || !feat_coef || !feat_rows || !state_num || !state_den) return STA_ERR_ARG;
  if (!dtype_ok(dtype)) return STA_ERR_DTYPE;
  if (bh <= 0 || n < 0 || head_rows < n || d <= 0 || dv <= 0 || fsplit <= 0 || slot_tiles <= 0 || n_feat <= 0)
    return STA_ERR_SHAPE;
  if (!sta_moments_ws_ok(d, degree, slot_tiles, column_tiles, dv)) return STA_ERR_UNSUPPORTED;
  if (mixed != 0 && (mixed != 1 || slot_tiles < 2)) return STA_ERR_ARG;
  const int esize = dtype == STA_F32 ? 4 : 2;
  const int ldo = 32 * ((dv + 31) / 32);  // the state's row stride
  if ((d * esize) % 16 != 0 || ld_k < d || (ld_k * esize) % 16 != 0 || ldv < dv || ldv % 32 != 0 ||
      ldv % (16 * column_tiles) != 0 || ldo % (16 * column_tiles) != 0)
    return STA_ERR_ARG;
  if (((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15u) != 0) return STA_ERR_ARG;
  if (head_rows * static_cast<int64_t>(ldv > ld_k ? ldv : ld_k) * esize >= (int64_t(1) << 32) ||
      n >= (int64_t(1) << 30))
    return STA_ERR_UNSUPPORTED;
  if (n == 0) return STA_OK;
  sta::WsArgs w;
  sta::MomArgs& a = w.m;
  a.q = k; a.k = k; a.v = v; a.dtype = dtype; a.n = n; a.d = d; a.dv = dv; a.scale = 1.0f; a.shift = 0;
  a.fsplit = fsplit; a.mixed = mixed; a.csplit = (dv + 16 * column_tiles - 1) / (16 * column_tiles);
  a.quads = feat_quads; a.fcoef = feat_coef; a.low_num = nullptr; a.low_den = nullptr; a.ldv = ldv;
  a.esize = esize; a.ldo = ldo; a.ldk = ld_k; a.win = nullptr;
  a.head_rows = head_rows; a.rowmap = feat_rows; a.state_num = state_num; a.state_den = state_den;
  a.n_feat = n_feat;
  w.cpb = 2;  // no query blocks in the update-only pass
  w.mixed = mixed;
  w.hand = nullptr;
  w.nseg = 1;
  w.seg_chunks = static_cast<int>((n + sta::MOM_C - 1) / sta::MOM_C);
  w.phase = 3;
  w.seg_state = nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nx = moment_extra_factors(degree);
  if (column_tiles == 4)
    return esize == 4 ? dispatch_moments_ws<4, 4>(w, bh, s, slot_tiles, nx) : dispatch_moments_ws<2, 4>(w, bh, s, slot_tiles, nx);
  return esize == 4 ? dispatch_moments_ws<4, 2>(w, bh, s, slot_tiles, nx) : dispatch_moments_ws<2, 2>(w, bh, s, slot_tiles, nx);
}

int sta_decode_layout(int d, int dv, int* dk, int* ldv) {
  if (d <= 0 || dv <= 0 || !dk || !ldv) return STA_ERR_ARG;
  if (d > kMaxD || dv > kMaxDv) return STA_ERR_UNSUPPORTED;
  // keys wider than the staged 128 dimensions in whole 32-dimension blocks (the accumulation's windows)
  *dk = d > kMaxStagedD ? 32 * ((d + 31) / 32) : 4 * ((d + 3) / 4);
  *ldv = 32 * ((dv + 31) / 32);
  return STA_OK;
}

int sta_decode_moments(const void* q, int dtype, int64_t streams, int d, int dv, float scale, const float* state_num,
                       const float* state_den, int n_feat, const void* feat_index, int index_width, int splits,
                       float* part_num,
                       float* part_den, void* stream) {
  if (!q || !state_num || !state_den || !feat_index || !part_num || !part_den) return STA_ERR_ARG;
  if (index_width != 4 && index_width != 8) return STA_ERR_ARG;
  if (!dtype_ok(dtype)) return STA_ERR_DTYPE;
  if (streams <= 0 || d <= 0 || dv <= 0 || n_feat <= 0 || splits <= 0 || splits > n_feat) return STA_ERR_SHAPE;
  if (d > kMaxD || dv > kMaxDv) return STA_ERR_UNSUPPORTED;
  if (((reinterpret_cast<uintptr_t>(state_num) | reinterpret_cast<uintptr_t>(part_num)) & 15u) != 0) return STA_ERR_ARG;
  const int64_t grid = streams * splits;
  if (grid > 0x7fffffff) return STA_ERR_UNSUPPORTED;
  sta::DecMomArgs a;
  a.q = q; a.dtype = dtype; a.d = d; a.scale = scale; a.state_num = state_num; a.state_den = state_den;
  a.n_feat = n_feat; a.ldm = 32 * ((dv + 31) / 32); a.rowfeat = feat_index; a.splits = splits;
  a.rows_per_split = (n_feat + splits - 1) / splits; a.part_num = part_num; a.part_den = part_den;
  if (index_width == 8)
    hipLaunchKernelGGL(sta::decode_moments_kernel<true>, dim3(static_cast<unsigned>(grid)), dim3(sta::DEC_THREADS), 0,
                       static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL(sta::decode_moments_kernel<false>, dim3(static_cast<unsigned>(grid)), dim3(sta::DEC_THREADS), 0,
                       static_cast<hipStream_t>(stream), a);
  return check_launch();
}

int sta_decode_tail(const void* q, const void* k, const void* v, int dtype, int64_t streams, int d, int dv,
                    int degree, float scale, float eps, int flags, float* buf_k, float* buf_v, int block, int buf_len,
                    const float* lev_k, const float* lev_v, const float* lev_w, int n_levels, int level_size,
                    uint64_t level_mask, const float* part_num, const float* part_den, int splits, void* out,
                    int out_dtype, float* stats, void* stream) {
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype)) return STA_ERR_DTYPE;
  if (streams <= 0 || d <= 0 || dv <= 0 || block <= 0 || buf_len < 0 || n_levels < 0 || level_size < 0)
    return STA_ERR_SHAPE;
  if (d > kMaxD || dv > kMaxDv || degree < 0 || degree > kMaxDegree) return STA_ERR_UNSUPPORTED;
  if (flags & ~(sta::DEC_APPEND | sta::DEC_CURRENT | sta::DEC_QUERY)) return STA_ERR_ARG;
  if ((flags & sta::DEC_CURRENT) && !(flags & sta::DEC_APPEND)) return STA_ERR_ARG;
  if (!buf_k || !buf_v) return STA_ERR_ARG;
  if ((flags & sta::DEC_APPEND) && (!k || !v || buf_len >= block)) return STA_ERR_ARG;
  if (buf_len > block) return STA_ERR_SHAPE;
  if (flags & sta::DEC_QUERY) {
    if (!q || !out || !part_num || !part_den || splits <= 0) return STA_ERR_ARG;
    if (n_levels > 64 || (n_levels < 64 && (level_mask >> n_levels) != 0)) return STA_ERR_SHAPE;
    if (level_mask && (!lev_k || !lev_v || !lev_w || level_size <= 0)) return STA_ERR_ARG;
  }
  if (streams > 0x7fffffff) return STA_ERR_UNSUPPORTED;
  int dk = 0, ldv = 0;
  sta_decode_layout(d, dv, &dk, &ldv);
  if (((reinterpret_cast<uintptr_t>(buf_k) | reinterpret_cast<uintptr_t>(buf_v) | reinterpret_cast<uintptr_t>(lev_k) |
        reinterpret_cast<uintptr_t>(lev_v)) & 15u) != 0)
    return STA_ERR_ARG;
  sta::DecTailArgs a;
  a.q = q; a.k = k; a.v = v; a.dtype = dtype; a.d = d; a.dv = dv; a.degree = degree; a.scale = scale; a.eps = eps;
  a.buf_k = buf_k; a.buf_v = buf_v; a.B = block; a.dk = dk; a.ldv = ldv; a.buf_len = buf_len;
  a.lev_k = lev_k; a.lev_v = lev_v; a.lev_w = lev_w; a.L = n_levels; a.m = level_size; a.level_mask = level_mask;
  a.flags = flags; a.part_num = part_num; a.part_den = part_den; a.splits = splits; a.out = out;
  a.out_dtype = out_dtype; a.stats = stats;
  const dim3 grid(static_cast<unsigned>(streams));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int kc = d <= 64 ? 1 : (d <= 128 ? 2 : 4);
  const int vc = dv <= 64 ? 1 : (dv <= 128 ? 2 : 4);
  const dim3 blk(sta::DEC_THREADS);
  if (kc == 1 && vc == 1) hipLaunchKernelGGL((sta::decode_tail_kernel<1, 1>), grid, blk, 0, s, a);
  else if (kc == 1 && vc == 2) hipLaunchKernelGGL((sta::decode_tail_kernel<1, 2>), grid, blk, 0, s, a);
  else if (kc == 1) hipLaunchKernelGGL((sta::decode_tail_kernel<1, 4>), grid, blk, 0, s, a);
  else if (kc == 2 && vc == 1) hipLaunchKernelGGL((sta::decode_tail_kernel<2, 1>), grid, blk, 0, s, a);
  else if (kc == 2 && vc == 2) hipLaunchKernelGGL((sta::decode_tail_kernel<2, 2>), grid, blk, 0, s, a);
  else if (kc == 2) hipLaunchKernelGGL((sta::decode_tail_kernel<2, 4>), grid, blk, 0, s, a);
  else if (vc == 1) hipLaunchKernelGGL((sta::decode_tail_kernel<4, 1>), grid, blk, 0, s, a);
  else if (vc == 2) hipLaunchKernelGGL((sta::decode_tail_kernel<4, 2>), grid, blk, 0, s, a);
  else hipLaunchKernelGGL((sta::decode_tail_kernel<4, 4>), grid, blk, 0, s, a);
  return check_launch();
}

int64_t sta_static_scratch_bytes(void) { return STA_STATIC_SCRATCH_BYTES; }

int sta_decode_step_static(const void* q, const void* k, const void* v, int dtype, int64_t streams, int d, int dv,
                           int degree, float scale, float eps, int flags, const float* state_num,
                           const float* state_den, int n_feat, const void* feat_index, int index_width, int splits,
                           float* buf_k,
                           float* buf_v, int block, int buf_len, const float* lev_k, const float* lev_v,
                           const float* lev_w, int n_levels, int level_size, uint64_t level_mask, void* out,
                           int out_dtype, float* stats, void* stream) {
  if (!(flags & sta::DEC_QUERY)) return STA_ERR_ARG;
  if (streams <= 0 || splits <= 0 || dv <= 0) return STA_ERR_SHAPE;
  if (dv > kMaxDv || d > kMaxD) return STA_ERR_UNSUPPORTED;
  if ((state_num == nullptr) != (state_den == nullptr)) return STA_ERR_ARG;
  const int64_t ldv = 32 * ((dv + 31) / 32);
  // part_num, then part_den from the next 64-float boundary, within the static scratch
  const int64_t num_floats = streams * splits * ldv;
  const int64_t den_off = (num_floats + 63) / 64 * 64;
  const int64_t used = den_off + streams * splits;
  if (streams > (int64_t(1) << 31) || splits > (1 << 20) || used * int64_t(sizeof(float)) > STA_STATIC_SCRATCH_BYTES)
    return STA_ERR_SCRATCH;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int device = -1;
  int st = hip_status(s ? hipStreamGetDevice(s, &device) : hipGetDevice(&device));
  if (st != STA_OK) return st;
  float* base = nullptr;
  if ((st = static_scratch_ptr(device, &base)) != STA_OK) return st;
  float* part_num = base;
  float* part_den = base + den_off;
  if (state_num) {
    st = sta_decode_moments(q, dtype, streams, d, dv, scale, state_num, state_den, n_feat, feat_index, index_width,
                            splits,
                            part_num, part_den, stream);
  } else {
    // no moment state (every token answered from the buffer): zero partials, cleared by a kernel so
    // that the call can sit in a captured graph
    const int64_t blocks = (used + 255) / 256 < 1024 ? (used + 255) / 256 : 1024;
    hipLaunchKernelGGL(zero_fill_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, base, used);
    st = check_launch();
  }
  if (st != STA_OK) return st;
  return sta_decode_tail(q, k, v, dtype, streams, d, dv, degree, scale, eps, flags, buf_k, buf_v, block, buf_len,
                         lev_k, lev_v, lev_w, n_levels, level_size, level_mask, part_num, part_den, splits, out,
                         out_dtype, stats, stream);
}

int sta_decode_compress(int64_t streams, int d, int dv, const float* buf_k, const float* buf_v, int block, int pos0,
                        float* lev_k, float* lev_v, float* lev_w, int32_t* lev_pos, int n_levels, int level_size,
                        int n_calls, const int32_t* methods, const void* dirs, const void* unif,
                        const int32_t* perms, int max_in, int score_f64, const double* buf_k64, double* lev_k64,
                        void* stream) {
  if (!buf_k || !buf_v || !lev_k || !lev_v || !lev_w || !lev_pos || !methods || !dirs || !unif || !perms)
    return STA_ERR_ARG;
  if (score_f64 != 0 && score_f64 != 1) return STA_ERR_ARG;
  if (score_f64 && (!buf_k64 || !lev_k64)) return STA_ERR_ARG;
  if (streams <= 0 || d <= 0 || dv <= 0 || block < 2 || pos0 < 0 || n_levels <= 0 || level_size <= 0)
    return STA_ERR_SHAPE;
  if (d > kMaxD || dv > kMaxDv) return STA_ERR_UNSUPPORTED;
  if (n_calls <= 0 || n_calls > n_levels) return STA_ERR_SHAPE;
  // every level holds ceil(block / 2) items and every call's input fits the LDS lists
  if (level_size != (block + 1) / 2) return STA_ERR_SHAPE;
  if (block > sta::CMP_MAX_IN || 2 * level_size > sta::CMP_MAX_IN) return STA_ERR_UNSUPPORTED;
  if (max_in < block || max_in < 2 * level_size) return STA_ERR_ARG;
  if (max_in > sta::CMP_MAX_IN) return STA_ERR_UNSUPPORTED;
  if (streams > 0x7fffffff) return STA_ERR_UNSUPPORTED;
  int dk = 0, ldv = 0;
  sta_decode_layout(d, dv, &dk, &ldv);
  sta::DecCmpArgs a;
  a.buf_k = buf_k; a.buf_v = buf_v; a.B = block; a.d = d; a.dk = dk; a.ldv = ldv; a.pos0 = pos0;
  a.lev_k = lev_k; a.lev_v = lev_v; a.lev_w = lev_w; a.lev_pos = lev_pos; a.L = n_levels; a.m = level_size;
  a.n_calls = n_calls; a.methods = methods; a.dirs = dirs; a.unif = unif; a.perms = perms; a.max_in = max_in;
  a.f64 = score_f64; a.buf_k64 = buf_k64; a.lev_k64 = lev_k64;
  const size_t smem = sizeof(float) * static_cast<size_t>(sta::dec_cmp_smem_floats(max_in, score_f64 != 0));
  const int st = lds_limit(reinterpret_cast<const void*>(sta::decode_compress_kernel), smem);
  if (st != STA_OK) return st;
  hipLaunchKernelGGL(sta::decode_compress_kernel, dim3(static_cast<unsigned>(streams)), dim3(sta::CMP_THREADS), smem,
                     static_cast<hipStream_t>(stream), a);
  return check_launch();
}

namespace {
// Checks and argument block shared by sta_compress_nodes and sta_compress_tree (status in *st).
sta::CompressArgs compress_args(const void* k, int dtype, int64_t bh, int64_t n, int d, const int32_t* batch_nodes,
                                int n_batch, const int32_t* node_desc, int n_nodes, int cap, const void* dirs,
                                const void* unif, const int32_t* perms, int n_draws, int max_in, int32_t* node_src,
                                float* node_w, const int32_t* node_level, const int32_t* anc, int anc_levels,
                                float* level_scores, size_t* smem, int* st) {
  sta::CompressArgs a{};
  *st = STA_OK;
  const bool f64 = dtype == STA_F64;
  if (!k || !batch_nodes || !node_desc || !node_src || !node_w) *st = STA_ERR_ARG;
  else if (anc_levels < 0 || anc_levels > sta::CMP_MAX_ANC) *st = STA_ERR_ARG;
  else if (anc_levels > 0 && (f64 || !level_scores)) *st = STA_ERR_ARG;
  else if (anc && anc_levels <= 0) *st = STA_ERR_ARG;
  else if (!dtype_ok(dtype) && !f64) *st = STA_ERR_DTYPE;
  else if (bh <= 0 || n <= 0 || d <= 0 || n_nodes <= 0 || cap <= 0 || max_in <= 0) *st = STA_ERR_SHAPE;
  else if (d > kMaxD || max_in > sta::CMP_MAX_IN) *st = STA_ERR_UNSUPPORTED;
  else if (n_batch > 0 && bh > 65535) *st = STA_ERR_UNSUPPORTED;
  else if (n_batch > 0 && n_draws > 0 && (!dirs || !unif || !perms)) *st = STA_ERR_ARG;
  a.k = k; a.dtype = dtype; a.n = n; a.d = d; a.batch = batch_nodes; a.desc = node_desc; a.n_nodes = n_nodes;
  a.cap = cap; a.dirs = dirs; a.unif = unif; a.perms = perms; a.n_draws = n_draws; a.max_in = max_in;
  a.node_src = node_src; a.node_w = node_w; a.f64 = f64 ? 1 : 0;
  a.anc = anc; a.node_level = node_level; a.anc_levels = anc_levels; a.lscore = level_scores;
  *smem = sizeof(float) * static_cast<size_t>(sta::cmp_smem_floats(max_in, f64, anc ? 2 * (1 + anc_levels) * d : 0));
  return a;
}
}  // namespace

int sta_compress_nodes(const void* k, int dtype, int64_t bh, int64_t n, int d, const int32_t* batch_nodes,
                       int n_batch, const int32_t* node_desc, int n_nodes, int cap, const void* dirs,
                       const void* unif, const int32_t* perms, int n_draws, int max_in, int32_t* node_src,
                       float* node_w, const int32_t* node_level, const int32_t* anc, int anc_levels,
                       float* level_scores, void* stream) {
  size_t smem = 0;
  int st = STA_OK;
  const sta::CompressArgs a = compress_args(k, dtype, bh, n, d, batch_nodes, n_batch, node_desc, n_nodes, cap, dirs,
                                            unif, perms, n_draws, max_in, node_src, node_w, node_level, anc,
                                            anc_levels, level_scores, &smem, &st);
  if (st == STA_OK && anc_levels > 0 && !node_level) st = STA_ERR_ARG;  // merges read their levels
  if (st != STA_OK || n_batch <= 0) return st;
  // the ancestor-scoring instantiation for a launch that passes the ancestor table (its raw nodes)
  const void* fn = anc ? reinterpret_cast<const void*>(sta::compress_kernel<true>)
                       : reinterpret_cast<const void*>(sta::compress_kernel<false>);
  st = lds_limit(fn, smem);
  if (st != STA_OK) return st;
  const dim3 grid(static_cast<unsigned>(n_batch), static_cast<unsigned>(bh));
  if (anc)
    hipLaunchKernelGGL(sta::compress_kernel<true>, grid, dim3(sta::CMP_THREADS), smem, static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL(sta::compress_kernel<false>, grid, dim3(sta::CMP_THREADS), smem, static_cast<hipStream_t>(stream), a);
  return check_launch();
}

int sta_compress_merges(const void* k, int dtype, int64_t bh, int64_t n, int d, const int32_t* node_table,
                        int n_groups, int steps, int groups, int group_threads, const int32_t* node_desc,
                        int n_nodes, int cap, const void* dirs, const void* unif, const int32_t* perms, int n_draws,
                        int max_in, int32_t* node_src, float* node_w, const int32_t* node_level, int anc_levels,
                        float* level_scores, void* stream) {
  size_t smem = 0;
  int st = STA_OK;
  const sta::CompressArgs a = compress_args(k, dtype, bh, n, d, node_table, n_groups, node_desc, n_nodes, cap, dirs,
                                            unif, perms, n_draws, max_in, node_src, node_w, node_level, nullptr,
                                            anc_levels, level_scores, &smem, &st);
  if (st == STA_OK && anc_levels > 0 && !node_level) st = STA_ERR_ARG;
  if (st != STA_OK) return st;
  if (group_threads != 64 && group_threads != sta::CMP_THREADS) return STA_ERR_ARG;
  if (steps <= 0 || groups <= 0 || groups * group_threads > 1024) return STA_ERR_ARG;
  if (n_groups <= 0) return STA_OK;
  const int region = sta::cmp_smem_floats(max_in, dtype == STA_F64);
  smem = sizeof(float) * static_cast<size_t>(region) * static_cast<size_t>(groups);
  if (smem > 160 * 1024) return STA_ERR_UNSUPPORTED;
  const void* fn = group_threads == 64 ? reinterpret_cast<const void*>(sta::compress_merge_kernel<64>)
                                       : reinterpret_cast<const void*>(sta::compress_merge_kernel<sta::CMP_THREADS>);
  st = lds_limit(fn, smem);
  if (st != STA_OK) return st;
  const dim3 grid(static_cast<unsigned>(n_groups), static_cast<unsigned>(bh));
  const dim3 block(static_cast<unsigned>(group_threads * groups));
  if (group_threads == 64)
    hipLaunchKernelGGL(sta::compress_merge_kernel<64>, grid, block, smem, static_cast<hipStream_t>(stream), a,
                       node_table, steps, groups, region);
  else
    hipLaunchKernelGGL(sta::compress_merge_kernel<sta::CMP_THREADS>, grid, block, smem,
                       static_cast<hipStream_t>(stream), a, node_table, steps, groups, region);
  return check_launch();
}

int sta_segment_mean(const void* k, const void* v, int dtype, int64_t bh, int64_t n, int d, int dv, int block,
                     int stride, int64_t n_rep, float* rep_k, float* rep_v, void* stream) {
  if (!k || !v || !rep_k || !rep_v) return STA_ERR_ARG;
  if (!dtype_ok(dtype)) return STA_ERR_DTYPE;
  if (bh <= 0 || n <= 0 || d <= 0 || dv <= 0 || block <= 0 || stride <= 0 || block % stride != 0)
    return STA_ERR_SHAPE;
  if (n_rep != ((n - 1) / block) * (block / stride)) return STA_ERR_SHAPE;
  if (n_rep == 0) return STA_OK;
  if (bh > 65535) return STA_ERR_UNSUPPORTED;
  sta::SegMeanArgs a;
  a.k = k; a.v = v; a.dtype = dtype; a.n = n; a.d = d; a.dv = dv; a.stride = stride; a.n_rep = n_rep;
  a.rep_k = rep_k; a.rep_v = rep_v;
  const int64_t work = n_rep * (d + dv);
  int64_t blocks = (work + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(sta::segment_mean_kernel, dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(bh)),
                     dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return check_launch();
}

int sta_block_attention(const void* q, const void* k, const void* v, int dtype, int64_t bh, int64_t n, int d,
                        int dv, int ld_qk, int ld_v, int degree, float scale, float eps, int mode, int block, int chunk,
                        int shift, int exp_clamp, int products, const float* low_num, const float* low_den, int fsplit,
                        const int32_t* tile_ptr, const int32_t* tile_nodes, int n_tiles, const int32_t* node_meta,
                        int n_nodes, int cap, const int32_t* node_src, const float* node_w, const float* rep_k,
                        const float* rep_v, int ld_rep_k, int ld_rep_v, int64_t n_rep, void* out, int out_dtype,
                        float* out_den, void* stream) {
  if (!q || !k || !v || !low_num || !low_den || !tile_ptr || !out) return STA_ERR_ARG;
  if (out_den && out_dtype != STA_F32) return STA_ERR_DTYPE;
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype)) return STA_ERR_DTYPE;
  if (bh <= 0 || n <= 0 || d <= 0 || dv <= 0 || block <= 0 || fsplit <= 0) return STA_ERR_SHAPE;
  if (d > kMaxD || dv > kMaxDv || degree < 0 || degree > kMaxDegree) return STA_ERR_UNSUPPORTED;
  if (mode < 0 || mode > 3 || chunk <= 0 || chunk % sta_moment_chunk(d) != 0 || shift < 0 || shift >= sta_moment_chunk(d))
    return STA_ERR_ARG;
  if (products != STA_PRODUCTS_FP32 && products != STA_PRODUCTS_SPLIT_BF16) return STA_ERR_ARG;
  if (n_tiles != static_cast<int>((n + shift + kTileRows - 1) / kTileRows)) return STA_ERR_SHAPE;
  if (n_nodes > 0 && (!node_meta || !node_src || !node_w || !tile_nodes || cap <= 0)) return STA_ERR_ARG;
  // rows are read in units of 4 elements: strides multiples of 4, bases 16-byte aligned; materialized
  // representatives (segment means) are fp32 and only combine with fp32 inputs
  if (ld_qk < d || ld_qk % 4 != 0 || ld_v < dv || ld_v % 4 != 0) return STA_ERR_ARG;
  if (((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15u) != 0)
    return STA_ERR_ARG;
  if (rep_k || rep_v) {
    if (!rep_k || !rep_v || n_rep <= 0 || ld_rep_k < d || ld_rep_k % 4 != 0 || ld_rep_v < dv || ld_rep_v % 4 != 0)
      return STA_ERR_ARG;
    if (((reinterpret_cast<uintptr_t>(rep_k) | reinterpret_cast<uintptr_t>(rep_v)) & 15u) != 0) return STA_ERR_ARG;
    if (dtype != STA_F32) return STA_ERR_DTYPE;
  }
  sta::BlockArgs a;
  a.q = q; a.k = k; a.v = v; a.dtype = dtype; a.n = n; a.d = d; a.dv = dv; a.degree = degree; a.scale = scale;
  a.eps = eps; a.mode = mode; a.block = block; a.chunk = chunk; a.shift = shift; a.exp_clamp = exp_clamp;
  a.low_num = low_num; a.low_den = low_den; a.fsplit = fsplit; a.tile_ptr = tile_ptr; a.tile_nodes = tile_nodes;
  a.low_rows = n + 2 * sta::MOM_GUARD; a.low_ld = 32 * ((dv + 31) / 32); a.low_off = sta::MOM_GUARD;
  a.n_tiles = n_tiles; a.node_meta = node_meta; a.n_nodes = n_nodes; a.cap = cap; a.node_src = node_src;
  a.node_w = node_w; a.rep_k = rep_k; a.rep_v = rep_v; a.n_rep = n_rep; a.out = out; a.out_dtype = out_dtype; a.out_den = out_den;
  a.ldqk = ld_qk; a.ldvr = ld_v; a.ldrk = ld_rep_k; a.ldrv = ld_rep_v;
  a.split = products == STA_PRODUCTS_SPLIT_BF16 ? 1 : 0;
  if (a.split && degree > 3) return STA_ERR_UNSUPPORTED;  // the split-product kernel's Taylor stops at 3
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool f32 = dtype == STA_F32;
  if (d <= 16) return f32 ? dispatch_dvt<16, 4>(a, bh, s) : dispatch_dvt<16, 2>(a, bh, s);
  if (d <= 32) return f32 ? dispatch_dvt<32, 4>(a, bh, s) : dispatch_dvt<32, 2>(a, bh, s);
  if (d <= 64) return f32 ? dispatch_dvt<64, 4>(a, bh, s) : dispatch_dvt<64, 2>(a, bh, s);
  if (d <= 128) return f32 ? dispatch_dvt<128, 4>(a, bh, s) : dispatch_dvt<128, 2>(a, bh, s);
  return f32 ? dispatch_dvt<256, 4>(a, bh, s) : dispatch_dvt<256, 2>(a, bh, s);
}

int sta_selftest_mfma(const float* a, const float* b, float* d_out) {
  if (!a || !b || !d_out) return STA_ERR_ARG;
  hipLaunchKernelGGL(selftest_mfma_kernel, dim3(1), dim3(64), 0, nullptr, a, b, d_out);
  int st = check_launch();
  if (st != STA_OK) return st;
  return hip_status(hipDeviceSynchronize());
}

}  // extern "C"
