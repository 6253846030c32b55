// K5: batched streaming decode (ArticleStreamingAttention.update / query,
// streaming_taylor_coreset_attention.py:576-609) for S independent streams advancing in lockstep.
//
// Decode state of stream s (all fp32, caller-owned):
//   state_num [S][F][ldm], state_den [S][F]  moments sum phi_k(k_j) [v_j, 1] over the tokens of the
//       completed blocks only, features in the reference's order (degree 0, 1, ..., each in
//       combinations_with_replacement order, streaming_taylor_coreset_attention.py:180-216);
//   buf_k [S][B][dk], buf_v [S][B][ldv]  the uncompressed buffer: the tokens of the current block;
//   lev_k [S][L][m][dk], lev_v [S][L][m][ldv], lev_w [S][L][m], lev_pos [S][L][m]  the level coresets
//       (level l occupied iff bit l of the completed-block counter is set; every level holds m items).
// Padding columns of dk / ldv are zero.  A query is answered as
//   low (phi_q . state: keys of completed blocks, exactly the reference's Taylor part for them)
//   + sum over buffered tokens of exp(s q.k) [v, 1]          (their Taylor part plus their exp_{>t}
//                                                             tail: together the exact exponential)
//   + sum over level items of w (exp(s q.k) - exp_{<=t}(s q.k)) [v, 1]
// which is, term by term, the reference's low + tail (:583-597) regrouped: the reference's sketch holds
// the buffered tokens too, and its coreset items() lists them with weight 1.  Keeping the buffered
// tokens out of the state makes a decode step read the state once and write nothing; the block's
// rank-B state update is applied when the block completes (moment_accumulate_kernel over the buffer).
//
// Kernels per step: decode_moments_kernel (state read, HBM-bound) and decode_tail_kernel (buffer and
// level items, HBM-bound; also appends the token).  On a block completion the host adds
// moment_accumulate_kernel (buffer -> state) and decode_compress_kernel (buffer -> level 0, then the
// cascade of merges cat(old level, new) while levels are occupied, :387-411).
#include "common.hpp"

namespace sta {

constexpr int DEC_THREADS = 256;
constexpr int DEC_GROUPS = DEC_THREADS / 16;  // items in flight per workgroup pass (16 lanes per item)
constexpr int DEC_MAX_X = 260;                // staged query features x[0..d] (d <= 256) plus zeros

enum DecFlags : int { DEC_APPEND = 1, DEC_CURRENT = 2, DEC_QUERY = 4 };

// ------------------------------------------------------------------------------------------------
// decode_moments_kernel: part_num[s][split][col] = sum_{f in split} phi_q(s q)[f] state_num[s][f][col],
// part_den[s][split] likewise with state_den.  Thread (row slot rp, column quad c4) walks the rows
// f = f0 + rp + j * rpp, 4 rows per trip with unconditional (clamped), non-temporal 16-byte loads.
struct DecMomArgs {
  const void* q;  // [S][d] current queries (dtype)
  int dtype;
  int d;
  float scale;
  const float* state_num;  // [S][n_feat][ldm]
  const float* state_den;  // [S][n_feat]
  int n_feat;
  int ldm;                  // a multiple of 32
  // the factors of every feature in x = [s q, 1] (index d = 1): WIDE = false: [n_feat] uint32 i0 | i1 << 8 |
  // i2 << 16 | i3 << 24 (d < 255, degree <= 4); WIDE = true: [n_feat][8] uint16 (any d, degree <= 8)
  const void* rowfeat;
  int splits;
  int rows_per_split;
  float* part_num;  // [S][splits][ldm]
  float* part_den;  // [S][splits]
};

template <bool WIDE>
__device__ __forceinline__ float dec_feature(const DecMomArgs& a, const float* xs, int row) {
  if constexpr (WIDE) {
    const uint4 w = static_cast<const uint4*>(a.rowfeat)[row];
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float ph = 1.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ph *= xs[(ws[j >> 1] >> (16 * (j & 1))) & 0xffffu];
    return ph;
  } else {
    const uint32_t pf = static_cast<const uint32_t*>(a.rowfeat)[row];
    return xs[pf & 255u] * xs[(pf >> 8) & 255u] * xs[(pf >> 16) & 255u] * xs[pf >> 24];
  }
}

template <bool WIDE>
__global__ __launch_bounds__(DEC_THREADS) void decode_moments_kernel(const DecMomArgs a) {
  __shared__ float xs[DEC_MAX_X];
  __shared__ floatx4 red[DEC_THREADS];
  __shared__ float dred[DEC_THREADS];
  const int wg = blockIdx.x;
  const int64_t s = wg / a.splits;
  const int sp = wg - static_cast<int>(s) * a.splits;
  const int tid = threadIdx.x;
  for (int j = tid; j < DEC_MAX_X; j += DEC_THREADS)
    xs[j] = j < a.d ? a.scale * load_elem(a.q, s * a.d + j, a.dtype) : (j == a.d ? 1.f : 0.f);
  __syncthreads();

  const int c4n = a.ldm >> 2;
  const int rpp = DEC_THREADS / c4n;
  const int rp = tid / c4n, c4 = tid - rp * c4n;
  const int f0 = sp * a.rows_per_split;
  const int f1 = min(a.n_feat, f0 + a.rows_per_split);
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  float dacc = 0.f;
  if (rp < rpp && f0 < f1) {
    const float* sn = a.state_num + s * a.n_feat * a.ldm + 4 * c4;
    const float* sd = a.state_den + s * a.n_feat;
    constexpr int U = 4;
    for (int r = f0 + rp; r < f1; r += U * rpp) {
      floatx4 S[U];
      float D[U], phi[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int row = r + u * rpp;
        const int rr = min(row, f1 - 1);
        // the state is streamed once per step: non-temporal loads keep it from displacing cached data
        S[u] = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(sn + static_cast<int64_t>(rr) * a.ldm));
        D[u] = __builtin_nontemporal_load(sd + rr);
        const float ph = dec_feature<WIDE>(a, xs, rr);
        phi[u] = row < f1 ? ph : 0.f;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        acc += phi[u] * S[u];
        dacc = fmaf(phi[u], D[u], dacc);
      }
    }
  }
  red[tid] = acc;
  dred[tid] = dacc;
  __syncthreads();
  const int64_t ob = s * a.splits + sp;
  if (tid < c4n) {
    floatx4 t = red[tid];
    for (int j = 1; j < rpp; ++j) t += red[j * c4n + tid];
    *reinterpret_cast<floatx4*>(a.part_num + ob * a.ldm + 4 * tid) = t;
  }
  if (tid == 0) {
    float t = dred[0];
    for (int j = 1; j < rpp; ++j) t += dred[j * c4n];
    a.part_den[ob] = t;
  }
}

// ------------------------------------------------------------------------------------------------
// decode_tail_kernel: one workgroup per stream.  APPEND writes the current (k, v) into buffer slot
// buf_len; QUERY answers the current query from the moment partials, the buf_len buffered tokens (plus
// the current token when CURRENT: the append of this same launch) and the occupied levels, and writes
// out = num / max(den, eps).  Items are spread over 16-lane groups: lane c of a group holds 16-byte
// column units c, c + 16, ... of the key and the value, the score is a 16-lane xor reduction.
struct DecTailArgs {
  const void* q;  // [S][d]
  const void* k;  // [S][d]
  const void* v;  // [S][dv]
  int dtype;
  int d, dv, degree;
  float scale, eps;
  float* buf_k;  // [S][B][dk]
  float* buf_v;  // [S][B][ldv]
  int B, dk, ldv;
  int buf_len;
  const float* lev_k;  // [S][L][m][dk]
  const float* lev_v;  // [S][L][m][ldv]
  const float* lev_w;  // [S][L][m]
  int L, m;
  uint64_t level_mask;
  int flags;
  const float* part_num;  // [S][splits][ldv]
  const float* part_den;  // [S][splits]
  int splits;
  void* out;  // [S][dv]
  int out_dtype;
  float* stats;  // [S][4] or null: denominator, reference low / tail denominators, items
};

template <int KC, int VC>
struct DecItem {
  floatx4 k[KC];
  floatx4 v[VC];
};

// Loads are unconditional (units past the row clamped to its last one, zeroed by a select afterwards):
// a load under a branch makes the compiler wait for it at the join, serialising the items in flight.
template <int KC, int VC>
__device__ __forceinline__ void dec_load_item(DecItem<KC, VC>& it, const float* krow, const float* vrow, int c, int dk4,
                                              int dv4) {
#pragma unroll
  for (int j = 0; j < KC; ++j) {
    const int u = c + 16 * j;
    it.k[j] = *reinterpret_cast<const floatx4*>(krow + 4 * min(u, dk4 - 1));
  }
#pragma unroll
  for (int j = 0; j < VC; ++j) {
    const int u = c + 16 * j;
    it.v[j] = *reinterpret_cast<const floatx4*>(vrow + 4 * min(u, dv4 - 1));
  }
#pragma unroll
  for (int j = 0; j < KC; ++j)
    if (c + 16 * j >= dk4) it.k[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < VC; ++j)
    if (c + 16 * j >= dv4) it.v[j] = floatx4{0.f, 0.f, 0.f, 0.f};
}

template <int KC>
__device__ __forceinline__ float dec_dot(const floatx4 (&x)[KC], const floatx4 (&k)[KC]) {
  float t = 0.f;
#pragma unroll
  for (int j = 0; j < KC; ++j) t += x[j][0] * k[j][0] + x[j][1] * k[j][1] + x[j][2] * k[j][2] + x[j][3] * k[j][3];
  t += __shfl_xor(t, 8, 16);
  t += __shfl_xor(t, 4, 16);
  t += __shfl_xor(t, 2, 16);
  t += __shfl_xor(t, 1, 16);
  return t;
}

// exp(z) on the hardware exp2 (about 1 ulp) and the Taylor truncation sum_{r<=deg} z^r / r! by Horner
// (c_r = [deg >= r] / r!, r <= 8): the residual exp - exp_{<=t} and the buffered tokens' exp need 1e-5
// relative, not the reference's term-by-term rounding.
struct DecTaylor {
  float c[9];
};
__device__ __forceinline__ DecTaylor dec_taylor(int deg) {
  DecTaylor t;
  float f = 1.f;
#pragma unroll
  for (int r = 0; r <= 8; ++r) {
    if (r > 0) f /= static_cast<float>(r);
    t.c[r] = r <= deg ? f : 0.f;
  }
  return t;
}
__device__ __forceinline__ float dec_tp(float z, const DecTaylor& t) {
  float p = t.c[8];
#pragma unroll
  for (int r = 7; r >= 0; --r) p = fmaf(z, p, t.c[r]);
  return p;
}
__device__ __forceinline__ float dec_exp(float z) { return __builtin_amdgcn_exp2f(z * 1.44269504f); }

// Items per 16-lane group in flight: NB rows are loaded before any of them is used.
constexpr int DEC_NB = 4;

template <int KC, int VC>
__global__ __launch_bounds__(DEC_THREADS) void decode_tail_kernel(const DecTailArgs a) {
  __shared__ float xs[DEC_MAX_X];
  __shared__ float cur_k[DEC_MAX_X];
  __shared__ float cur_v[4 * 16 * VC];
  __shared__ float redv[DEC_GROUPS][4 * 16 * VC];
  __shared__ float redd[DEC_GROUPS][2];
  const int64_t s = blockIdx.x;
  const int tid = threadIdx.x;
  const int dk4 = a.dk >> 2, dv4 = a.ldv >> 2;

  if (a.flags & (DEC_APPEND | DEC_CURRENT)) {
    for (int j = tid; j < a.dk + a.ldv; j += DEC_THREADS) {
      if (j < a.dk) {
        const float x = j < a.d ? load_elem(a.k, s * a.d + j, a.dtype) : 0.f;
        cur_k[j] = x;
        if (a.flags & DEC_APPEND) a.buf_k[(s * a.B + a.buf_len) * a.dk + j] = x;
      } else {
        const int c = j - a.dk;
        const float x = c < a.dv ? load_elem(a.v, s * a.dv + c, a.dtype) : 0.f;
        if (c < 4 * 16 * VC) cur_v[c] = x;
        if (a.flags & DEC_APPEND) a.buf_v[(s * a.B + a.buf_len) * a.ldv + c] = x;
      }
    }
  }
  if (!(a.flags & DEC_QUERY)) return;
  for (int j = tid; j < DEC_MAX_X; j += DEC_THREADS)
    xs[j] = j < a.d ? a.scale * load_elem(a.q, s * a.d + j, a.dtype) : 0.f;
  __syncthreads();

  const int c = tid & 15, g = tid >> 4;
  floatx4 x[KC];
#pragma unroll
  for (int j = 0; j < KC; ++j) {
    const int u = c + 16 * j;
    x[j] = u < dk4 ? *reinterpret_cast<const floatx4*>(xs + 4 * u) : floatx4{0.f, 0.f, 0.f, 0.f};
  }
  floatx4 acc[VC];
#pragma unroll
  for (int j = 0; j < VC; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
  float den = 0.f, tay = 0.f;  // tay: Taylor part of the buffered tokens (reference low denominator)

  const DecTaylor tc = dec_taylor(a.degree);
  // buffered tokens: exact exponential, weight 1 (DEC_NB items per group in flight)
  const float* bk = a.buf_k + s * a.B * a.dk;
  const float* bv = a.buf_v + s * a.B * a.ldv;
  for (int j0 = g; j0 < a.buf_len; j0 += DEC_NB * DEC_GROUPS) {
    DecItem<KC, VC> it[DEC_NB];
#pragma unroll
    for (int b = 0; b < DEC_NB; ++b) {
      const int jb = min(j0 + b * DEC_GROUPS, a.buf_len - 1);
      dec_load_item<KC, VC>(it[b], bk + jb * a.dk, bv + jb * a.ldv, c, dk4, dv4);
    }
#pragma unroll
    for (int b = 0; b < DEC_NB; ++b) {
      const float z = dec_dot<KC>(x, it[b].k);
      const bool on = j0 + b * DEC_GROUPS < a.buf_len;
      const float p = on ? dec_exp(z) : 0.f;
      den += p;
      tay += on ? dec_tp(z, tc) : 0.f;
#pragma unroll
      for (int j = 0; j < VC; ++j) acc[j] += p * it[b].v[j];
    }
  }
  // the current token of this launch (group 0)
  if ((a.flags & DEC_CURRENT) && g == 0) {
    DecItem<KC, VC> it;
    dec_load_item<KC, VC>(it, cur_k, cur_v, c, dk4, dv4);
    const float z = dec_dot<KC>(x, it.k);
    const float p = dec_exp(z);
    den += p;
    tay += dec_tp(z, tc);
#pragma unroll
    for (int j = 0; j < VC; ++j) acc[j] += p * it.v[j];
  }
  // level items: weighted exp_{>t} residual
  int n_items = a.buf_len + ((a.flags & DEC_CURRENT) ? 1 : 0);
  for (int l = 0; l < a.L; ++l) {
    if (!((a.level_mask >> l) & 1u)) continue;
    n_items += a.m;
    const int64_t base = (s * a.L + l) * a.m;
    const float* lk = a.lev_k + base * a.dk;
    const float* lv = a.lev_v + base * a.ldv;
    const float* lw = a.lev_w + base;
    for (int j0 = g; j0 < a.m; j0 += DEC_NB * DEC_GROUPS) {
      DecItem<KC, VC> it[DEC_NB];
      float w[DEC_NB];
#pragma unroll
      for (int b = 0; b < DEC_NB; ++b) {
        const int jb = min(j0 + b * DEC_GROUPS, a.m - 1);
        dec_load_item<KC, VC>(it[b], lk + jb * a.dk, lv + jb * a.ldv, c, dk4, dv4);
        w[b] = lw[jb];
      }
#pragma unroll
      for (int b = 0; b < DEC_NB; ++b) {
        const float z = dec_dot<KC>(x, it[b].k);
        const bool on = j0 + b * DEC_GROUPS < a.m;
        const float r = on ? w[b] * (dec_exp(z) - dec_tp(z, tc)) : 0.f;
        den += r;
#pragma unroll
        for (int j = 0; j < VC; ++j) acc[j] += r * it[b].v[j];
      }
    }
  }

  // ---- fixed-order combination: groups, then moment partials ----
#pragma unroll
  for (int j = 0; j < VC; ++j) *reinterpret_cast<floatx4*>(&redv[g][4 * (c + 16 * j)]) = acc[j];
  if (c == 0) {
    redd[g][0] = den;
    redd[g][1] = tay;
  }
  __syncthreads();
  float tail_den = 0.f, buf_tay = 0.f;
  for (int j = 0; j < DEC_GROUPS; ++j) {
    tail_den += redd[j][0];
    buf_tay += redd[j][1];
  }
  float low_den = 0.f;
  for (int j = 0; j < a.splits; ++j) low_den += a.part_den[s * a.splits + j];
  const float total = low_den + tail_den;
  const float safe = fmaxf(total, a.eps);
  for (int col = tid; col < a.dv; col += DEC_THREADS) {
    float num = 0.f;
    for (int j = 0; j < a.splits; ++j) num += a.part_num[(s * a.splits + j) * a.ldv + col];
    for (int j = 0; j < DEC_GROUPS; ++j) num += redv[j][col];
    store_elem(a.out, s * a.dv + col, a.out_dtype, __fdiv_rn(num, safe));
  }
  if (a.stats && tid == 0) {
    a.stats[s * 4 + 0] = total;
    a.stats[s * 4 + 1] = low_den + buf_tay;
    a.stats[s * 4 + 2] = total - (low_den + buf_tay);
    a.stats[s * 4 + 3] = static_cast<float>(n_items);
  }
}

// ------------------------------------------------------------------------------------------------
// decode_compress_kernel: one workgroup per stream, run when the buffer is full.  Call 0 compresses the
// B buffered tokens (weight 1); call i >= 1 merges cat(level i-1, output of call i-1) (old then new,
// streaming_taylor_coreset_attention.py:404-408); the output of the last call becomes level
// n_calls - 1, which is free (the counter's lowest zero bit).  An item is a handle: buffer row h < B or
// level row h - B; only handles, weights and positions move between calls, and the selected rows are
// copied once at the end, so nothing the kernel reads is written by it.
struct DecCmpArgs {
  const float* buf_k;  // [S][B][dk]
  const float* buf_v;  // [S][B][ldv]
  int B, d, dk, ldv;
  int pos0;  // sequence position of buffer row 0
  float* lev_k;
  float* lev_v;
  float* lev_w;
  int32_t* lev_pos;
  int L, m;
  int n_calls;
  const int32_t* methods;  // [n_calls] M_SORTED_PAIR or M_PERM
  const void* dirs;        // [S][n_calls][d] float (double with f64)
  const void* unif;        // [S][n_calls][max_in / 2] float (double with f64)
  const int32_t* perms;    // [S][n_calls][max_in]
  int max_in;
  // float64 scoring (f64 = 1): the key rows' float64 values, [S][B][dk] and [S][L][m][dk], scored in
  // fp64 against the float64 direction; lev_k64 rows follow lev_k's
  int f64;
  const double* buf_k64;
  double* lev_k64;
};

__global__ __launch_bounds__(CMP_THREADS) void decode_compress_kernel(const DecCmpArgs a) {
  extern __shared__ __align__(16) float dcmp_smem[];
  const bool f64 = a.f64 != 0;
  const int M = cmp_round4(a.max_in), H = cmp_round4(a.max_in / 2 + 1);
  const int KA = cmp_key_floats(a.max_in, f64);
  float* key_s = dcmp_smem;
  int* in_h = reinterpret_cast<int*>(dcmp_smem + KA);
  float* in_w = dcmp_smem + KA + M;
  int* in_p = reinterpret_cast<int*>(dcmp_smem + KA + 2 * M);
  int* pos_s = reinterpret_cast<int*>(dcmp_smem + KA + 3 * M);
  int* cur_h = reinterpret_cast<int*>(dcmp_smem + KA + 4 * M);
  float* cur_w = dcmp_smem + KA + 4 * M + H;
  int* cur_p = reinterpret_cast<int*>(dcmp_smem + KA + 4 * M + 2 * H);
  float* dir_s = dcmp_smem + KA + 4 * M + 3 * H;  // 8-byte aligned: KA, M, H are multiples of 4
  double* dir64_s = reinterpret_cast<double*>(dir_s);
  const int64_t s = blockIdx.x;
  const int tid = threadIdx.x;
  auto key_row = [&](int h) -> const float* {
    return h < a.B ? a.buf_k + (s * a.B + h) * a.dk : a.lev_k + (s * a.L * a.m + (h - a.B)) * a.dk;
  };
  auto key_row64 = [&](int h) -> const double* {
    return h < a.B ? a.buf_k64 + (s * a.B + h) * a.dk : a.lev_k64 + (s * a.L * a.m + (h - a.B)) * a.dk;
  };
  auto val_row = [&](int h) -> const float* {
    return h < a.B ? a.buf_v + (s * a.B + h) * a.ldv : a.lev_v + (s * a.L * a.m + (h - a.B)) * a.ldv;
  };

  int m_cur = 0;
  for (int call = 0; call < a.n_calls; ++call) {
    // ---- input list ----
    int n;
    if (call == 0) {
      n = a.B;
      for (int j = tid; j < n; j += CMP_THREADS) {
        in_h[j] = j;
        in_w[j] = 1.0f;
        in_p[j] = a.pos0 + j;
      }
    } else {
      n = a.m + m_cur;
      const int64_t lb = (s * a.L + (call - 1)) * a.m;
      for (int j = tid; j < n; j += CMP_THREADS) {
        if (j < a.m) {
          in_h[j] = a.B + (call - 1) * a.m + j;
          in_w[j] = a.lev_w[lb + j];
          in_p[j] = a.lev_pos[lb + j];
        } else {
          in_h[j] = cur_h[j - a.m];
          in_w[j] = cur_w[j - a.m];
          in_p[j] = cur_p[j - a.m];
        }
      }
    }
    __syncthreads();
    const int method = a.methods[call];
    const int64_t slot = s * a.n_calls + call;
    if (method == M_PERM) {
      const int mo = (n + 1) / 2;
      const int32_t* perm = a.perms + slot * a.max_in;
      const float factor = static_cast<float>(static_cast<double>(n) / static_cast<double>(mo));
      for (int j = tid; j < mo; j += CMP_THREADS) {
        const int p = perm[j];
        cur_h[j] = in_h[p];
        cur_w[j] = in_w[p] * factor;
        cur_p[j] = in_p[p];
      }
      m_cur = mo;
    } else {
      // sorted_pair: fp64 projection scores of the input rows, stable ascending sort, pair selection
      if (f64) {
        for (int e = tid; e < a.d; e += CMP_THREADS) dir64_s[e] = static_cast<const double*>(a.dirs)[slot * a.d + e];
        __syncthreads();
        uint64_t* uk = reinterpret_cast<uint64_t*>(key_s);
        for (int j = tid; j < n; j += CMP_THREADS)
          uk[j] = sort_key64(projection_score64(key_row64(in_h[j]), a.d, (a.dk & 1) == 0, dir64_s));
        rank_sort64(uk, pos_s, n, tid, CMP_THREADS);
      } else {
        for (int e = tid; e < a.d; e += CMP_THREADS) dir_s[e] = static_cast<const float*>(a.dirs)[slot * a.d + e];
        __syncthreads();
        for (int j = tid; j < n; j += 2 * CMP_THREADS) {  // rows j and j + CMP_THREADS together
          const int j1 = j + CMP_THREADS;
          const bool two = j1 < n;
          float s0, s1;
          projection_scores2(key_row(in_h[j]), 0, key_row(in_h[two ? j1 : j]), 0, two, a.d, F32, (a.d & 3) == 0,
                             dir_s, s0, s1);
          key_s[j] = s0;
          if (two) key_s[j1] = s1;
        }
        rank_sort(key_s, pos_s, n, tid, CMP_THREADS);
      }
      const float* u = static_cast<const float*>(a.unif) + slot * (a.max_in / 2);
      const double* u64 = static_cast<const double*>(a.unif) + slot * (a.max_in / 2);
      const int pc = n / 2;
      for (int p = tid; p < pc; p += CMP_THREADS) {
        const int ia = pos_s[2 * p], ib = pos_s[2 * p + 1];
        const float wa = in_w[ia], wb = in_w[ib];
        const bool first = f64 ? pair_keeps_first64(u64[p], wa, wb) : pair_keeps_first(u[p], wa, wb);
        const int keep = first ? ia : ib;
        cur_h[p] = in_h[keep];
        cur_w[p] = wa + wb;
        cur_p[p] = in_p[keep];
      }
      if ((n & 1) && tid == 0) {
        const int il = pos_s[n - 1];
        cur_h[pc] = in_h[il];
        cur_w[pc] = in_w[il];
        cur_p[pc] = in_p[il];
      }
      m_cur = pc + (n & 1);
    }
    __syncthreads();
  }

  // ---- the result becomes level n_calls - 1 ----
  const int dest = a.n_calls - 1;
  const int64_t ob = (s * a.L + dest) * a.m;
  for (int e = tid; e < m_cur * a.dk; e += CMP_THREADS) {
    const int j = e / a.dk, col = e - j * a.dk;
    a.lev_k[(ob + j) * a.dk + col] = key_row(cur_h[j])[col];
    if (f64) a.lev_k64[(ob + j) * a.dk + col] = key_row64(cur_h[j])[col];
  }
  for (int e = tid; e < m_cur * a.ldv; e += CMP_THREADS) {
    const int j = e / a.ldv, col = e - j * a.ldv;
    a.lev_v[(ob + j) * a.ldv + col] = val_row(cur_h[j])[col];
  }
  for (int j = tid; j < m_cur; j += CMP_THREADS) {
    a.lev_w[ob + j] = cur_w[j];
    a.lev_pos[ob + j] = cur_p[j];
  }
}

}  // namespace sta
