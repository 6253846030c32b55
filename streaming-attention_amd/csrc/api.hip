// extern "C" entry points of libstreamattn.so (declared in include/streamattn.h): argument checks,
// template dispatch and kernel launches.  The library allocates nothing; every buffer is the caller's.
#include "../../include/streamattn.h"
#include "block_attn.hip"
#include "compress.hip"
#include "moments.hip"

namespace {

thread_local int g_last_hip_error = 0;

int hip_status(hipError_t e) {
  if (e == hipSuccess) return STA_OK;
  g_last_hip_error = static_cast<int>(e);
  return STA_ERR_HIP;
}

int check_launch() { return hip_status(hipGetLastError()); }

bool dtype_ok(int dt) { return dt == STA_F32 || dt == STA_BF16 || dt == STA_F16; }

constexpr int kMaxD = 128;
constexpr int kMaxDv = 256;
constexpr int kMaxDegree = 3;
constexpr int kNW = 8;       // waves per moment workgroup
constexpr int kTileRows = 128;

// ---------------------------------------------------------------- moments dispatch
template <bool DEG3, int NT, int CH>
int launch_moments(const sta::MomArgs& a, int64_t bh, hipStream_t s) {
  const size_t smem = sta::moments_smem_bytes(CH, kNW, a.d, a.feat_per_split);
  auto fn = sta::moments_kernel<DEG3, NT, kNW, CH>;
  if (smem > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
    if (e != hipSuccess) return hip_status(e);
  }
  const int64_t grid = bh * a.ngroups * a.fsplit;
  if (grid <= 0 || grid > 0x7fffffff) return STA_ERR_SHAPE;
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(grid)), dim3(kNW * 64), smem, s, a);
  return check_launch();
}

template <bool DEG3, int CH>
int dispatch_nt(const sta::MomArgs& a, int64_t bh, hipStream_t s, int nt) {
  if (nt <= 1) return launch_moments<DEG3, 1, CH>(a, bh, s);
  if (nt <= 2) return launch_moments<DEG3, 2, CH>(a, bh, s);
  if (nt <= 3) return launch_moments<DEG3, 3, CH>(a, bh, s);
  if (nt <= 5) return launch_moments<DEG3, 5, CH>(a, bh, s);
  if (nt <= 9) return launch_moments<DEG3, 9, CH>(a, bh, s);
  if (nt <= 13) return launch_moments<DEG3, 13, CH>(a, bh, s);
  if (nt <= 17) return launch_moments<DEG3, 17, CH>(a, bh, s);
  return STA_ERR_UNSUPPORTED;
}

// ---------------------------------------------------------------- block-attention dispatch
template <int DP, int DVT>
int launch_block(const sta::BlockArgs& a, int64_t bh, hipStream_t s) {
  const int64_t grid = bh * a.n_tiles;
  if (grid <= 0 || grid > 0x7fffffff) return STA_ERR_SHAPE;
  hipLaunchKernelGGL((sta::block_attn_kernel<DP, DVT, 2>), dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, a);
  return check_launch();
}

template <int DP>
int dispatch_dvt(const sta::BlockArgs& a, int64_t bh, hipStream_t s) {
  if (a.dv <= 16) return launch_block<DP, 1>(a, bh, s);
  if (a.dv <= 32) return launch_block<DP, 2>(a, bh, s);
  if (a.dv <= 64) return launch_block<DP, 4>(a, bh, s);
  if (a.dv <= 128) return launch_block<DP, 8>(a, bh, s);
  if (a.dv <= 256) return launch_block<DP, 16>(a, bh, s);
  return STA_ERR_UNSUPPORTED;
}

__global__ void selftest_mfma_kernel(const float* a, const float* b, float* d) {
  const int l = threadIdx.x;
  sta::floatx4 c = sta::floatx4{0.f, 0.f, 0.f, 0.f};
  c = sta::mfma4(a[l], b[l], c);
  const int i = l & 15, g = l >> 4;
  for (int r = 0; r < 4; ++r) d[(4 * g + r) * 16 + i] = c[r];
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

int sta_tile_rows(void) { return kTileRows; }

int sta_moment_chunk(int d) { return d <= 64 ? 64 : 32; }

int sta_moments(const void* q, const void* k, const void* v, int dtype, int64_t bh, int64_t n, int d, int dv,
                int degree, float scale, int chunk, int shift, int fsplit, int feat_per_split,
                const uint32_t* feat_idx, const float* feat_coef, float* low_num, float* low_den, void* stream) {
  if (!q || !k || !v || !feat_idx || !feat_coef || !low_num || !low_den) return STA_ERR_ARG;
  if (!dtype_ok(dtype)) return STA_ERR_DTYPE;
  if (bh <= 0 || n <= 0 || d <= 0 || dv <= 0 || fsplit <= 0 || feat_per_split <= 0) return STA_ERR_SHAPE;
  if (feat_per_split % 16 != 0) return STA_ERR_SHAPE;
  if (d > kMaxD || dv > kMaxDv || degree < 0 || degree > kMaxDegree) return STA_ERR_UNSUPPORTED;
  if (chunk != sta_moment_chunk(d) || shift < 0 || shift >= chunk) return STA_ERR_ARG;
  sta::MomArgs a;
  a.q = q; a.k = k; a.v = v; a.dtype = dtype; a.n = n; a.d = d; a.dv = dv; a.scale = scale; a.shift = shift;
  a.ngroups = (dv + 15) / 16; a.fsplit = fsplit; a.feat_per_split = feat_per_split;
  a.fidx = feat_idx; a.fcoef = feat_coef; a.low_num = low_num; a.low_den = low_den;
  const int nt = (feat_per_split / 16 + kNW - 1) / kNW;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool deg3 = degree >= 3;
  if (chunk == 64) return deg3 ? dispatch_nt<true, 64>(a, bh, s, nt) : dispatch_nt<false, 64>(a, bh, s, nt);
  return deg3 ? dispatch_nt<true, 32>(a, bh, s, nt) : dispatch_nt<false, 32>(a, bh, s, nt);
}

int sta_compress_nodes(const void* k, int dtype, int64_t bh, int64_t n, int d, const int32_t* batch_nodes,
                       int n_batch, const int32_t* node_desc, int n_nodes, int cap, const float* dirs,
                       const float* unif, const int32_t* perms, int n_draws, int max_in, int32_t* node_src,
                       float* node_w, void* stream) {
  if (!k || !batch_nodes || !node_desc || !node_src || !node_w) return STA_ERR_ARG;
  if (!dtype_ok(dtype)) return STA_ERR_DTYPE;
  if (bh <= 0 || n <= 0 || d <= 0 || n_nodes <= 0 || cap <= 0 || max_in <= 0) return STA_ERR_SHAPE;
  if (d > kMaxD || max_in > sta::CMP_MAX_IN) return STA_ERR_UNSUPPORTED;
  if (n_batch <= 0) return STA_OK;
  if (bh > 65535) return STA_ERR_UNSUPPORTED;
  if (n_draws > 0 && (!dirs || !unif || !perms)) return STA_ERR_ARG;
  sta::CompressArgs a;
  a.k = k; a.dtype = dtype; a.n = n; a.d = d; a.batch = batch_nodes; a.desc = node_desc; a.n_nodes = n_nodes;
  a.cap = cap; a.dirs = dirs; a.unif = unif; a.perms = perms; a.n_draws = n_draws; a.max_in = max_in;
  a.node_src = node_src; a.node_w = node_w;
  hipLaunchKernelGGL(sta::compress_kernel, dim3(static_cast<unsigned>(n_batch), static_cast<unsigned>(bh)),
                     dim3(sta::CMP_THREADS), 0, static_cast<hipStream_t>(stream), a);
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
                        int dv, int degree, float scale, float eps, int mode, int block, int chunk, int shift,
                        int exp_clamp, const float* low_num, const float* low_den, int fsplit,
                        const int32_t* tile_ptr, const int32_t* tile_nodes, int n_tiles, const int32_t* node_meta,
                        int n_nodes, int cap, const int32_t* node_src, const float* node_w, const float* rep_k,
                        const float* rep_v, int64_t n_rep, void* out, int out_dtype, float* out_den,
                        void* stream) {
  if (!q || !k || !v || !low_num || !low_den || !tile_ptr || !out) return STA_ERR_ARG;
  if (out_den && out_dtype != STA_F32) return STA_ERR_DTYPE;
  if (!dtype_ok(dtype) || !dtype_ok(out_dtype)) return STA_ERR_DTYPE;
  if (bh <= 0 || n <= 0 || d <= 0 || dv <= 0 || block <= 0 || fsplit <= 0) return STA_ERR_SHAPE;
  if (d > kMaxD || dv > kMaxDv || degree < 0 || degree > kMaxDegree) return STA_ERR_UNSUPPORTED;
  if (mode < 0 || mode > 3 || chunk != sta_moment_chunk(d) || shift < 0 || shift >= chunk) return STA_ERR_ARG;
  if (kTileRows % chunk != 0) return STA_ERR_ARG;
  if (n_tiles != static_cast<int>((n + shift + kTileRows - 1) / kTileRows)) return STA_ERR_SHAPE;
  if (n_nodes > 0 && (!node_meta || !node_src || !node_w || !tile_nodes || cap <= 0)) return STA_ERR_ARG;
  sta::BlockArgs a;
  a.q = q; a.k = k; a.v = v; a.dtype = dtype; a.n = n; a.d = d; a.dv = dv; a.degree = degree; a.scale = scale;
  a.eps = eps; a.mode = mode; a.block = block; a.chunk = chunk; a.shift = shift; a.exp_clamp = exp_clamp;
  a.low_num = low_num; a.low_den = low_den; a.fsplit = fsplit; a.tile_ptr = tile_ptr; a.tile_nodes = tile_nodes;
  a.n_tiles = n_tiles; a.node_meta = node_meta; a.n_nodes = n_nodes; a.cap = cap; a.node_src = node_src;
  a.node_w = node_w; a.rep_k = rep_k; a.rep_v = rep_v; a.n_rep = n_rep; a.out = out; a.out_dtype = out_dtype; a.out_den = out_den;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (d <= 16) return dispatch_dvt<16>(a, bh, s);
  if (d <= 32) return dispatch_dvt<32>(a, bh, s);
  if (d <= 64) return dispatch_dvt<64>(a, bh, s);
  return dispatch_dvt<128>(a, bh, s);
}

int sta_selftest_mfma(const float* a, const float* b, float* d_out) {
  if (!a || !b || !d_out) return STA_ERR_ARG;
  hipLaunchKernelGGL(selftest_mfma_kernel, dim3(1), dim3(64), 0, nullptr, a, b, d_out);
  int st = check_launch();
  if (st != STA_OK) return st;
  return hip_status(hipDeviceSynchronize());
}

}  // extern "C"
