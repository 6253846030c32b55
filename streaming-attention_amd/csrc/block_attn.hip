// K2 + K4: per tile of query rows, everything except the inter-chunk moments, fused with the final
// normalisation:
//   * keys of the row's own moment chunk: Taylor polynomial exp_{<=t}(x) (closed form);
//   * keys of the row's current article block ("buffer"): residual exp(x) - exp_{<=t}(x), exact;
//     where both apply the sum is exp(x);
//   * coreset items of the tile's node list: w * (exp(x) - exp_{<=t}(x)), active for a row interval;
//   * out = (low_num + num) / max(low_den + den, eps)  (fast_article_attention.py:596-598).
//
// Row-dependent sets (reference file:line):
//   flat   : residual start rs(i) = floor(i/B)*B (fast_article_attention.py:503-512); block b's reps are
//            active for i >= (b+1)*B (fast_article_attention.py:419, :495).
//   levels : rs(i) = floor((i+1)/B)*B (the buffer after update(k_i)); the last token of a block is served
//            by the compressed block (streaming_taylor_coreset_attention.py:387-394, :576-599).
//   exact  : rs(i) = 0, no nodes (compressor == "none", fast_article_attention.py:437-464).
//   taylor : no residual at all; with raw output this yields the low-degree sums themselves
//            (low_degree_taylor_causal_sums, fast_article_attention.py:262-285).
//
// Matrix-core layout: X^T = K Q^T with A = key rows (LDS), B = q rows (registers, per wave); the P^T
// tile in the accumulator is fed straight back as the B operand of num^T += V^T P^T.
#include "common.hpp"

namespace sta {

enum BlockMode : int { MODE_FLAT = 0, MODE_LEVELS = 1, MODE_EXACT = 2, MODE_TAYLOR = 3 };
constexpr int NODE_META = 4;  // size, lo, hi, materialized (0: items index k/v, 1: items index rep_k/rep_v)

struct BlockArgs {
  const void* q;
  const void* k;
  const void* v;
  int dtype;
  int64_t n;
  int d;
  int dv;
  int degree;
  float scale;
  float eps;
  int mode;
  int block;
  int chunk;
  int shift;
  int exp_clamp;
  const float* low_num;  // [BH][fsplit][low_rows][low_ld], row i at low_off + i (sta_moments layout)
  const float* low_den;  // [BH][fsplit][low_rows]
  int fsplit;
  int64_t low_rows;
  int low_ld;
  int low_off;
  const int32_t* tile_ptr;    // [n_tiles + 1]
  const int32_t* tile_nodes;  // node ids
  int n_tiles;
  const int32_t* node_meta;  // [n_nodes][NODE_META]
  int n_nodes;
  int cap;
  const int32_t* node_src;  // [BH][n_nodes][cap]
  const float* node_w;      // [BH][n_nodes][cap]
  const float* rep_k;       // [BH][n_rep][d]   (materialized items)
  const float* rep_v;       // [BH][n_rep][dv]
  int64_t n_rep;
  void* out;  // [BH][n][dv]
  int out_dtype;
  float* out_den;  // optional [BH][n]: when set, out (fp32) receives num and out_den receives den, unnormalised
};

__device__ __forceinline__ int64_t floordiv(int64_t a, int64_t b) {
  const int64_t q = a / b;
  return (a % b != 0 && ((a < 0) != (b < 0))) ? q - 1 : q;
}

__device__ __forceinline__ int64_t chunk_start(int64_t i, int chunk, int shift) {
  return floordiv(i + shift, chunk) * chunk - shift;
}

__device__ __forceinline__ int64_t residual_start(int64_t i, int mode, int block) {
  if (mode == MODE_FLAT) return floordiv(i, block) * block;
  if (mode == MODE_LEVELS) return floordiv(i + 1, block) * block;
  if (mode == MODE_TAYLOR) return INT64_MAX;
  return 0;
}

// Taylor truncation sum_{r<=deg} x^r / r!, deg <= 3, without branches or selects: c1..c3 are 1 for the
// terms the degree includes, else 0 (uniform).  Degrees <= 2 reproduce the reference's term order and
// rounding exactly (1 + x, then + x*x/2 with exact division by 2; a zero coefficient adds exactly 0);
// the cubic term multiplies by 1/3 instead of dividing (within 1 ulp of the division).
struct TaylorCoef {
  float c1, c2, c3;
};
__host__ __device__ inline TaylorCoef taylor_coef(int deg) {
  return TaylorCoef{deg >= 1 ? 1.f : 0.f, deg >= 2 ? 1.f : 0.f, deg >= 3 ? 1.f : 0.f};
}
__device__ __forceinline__ float taylor_fast(float x, const TaylorCoef& c) {
  const float t2 = (x * x) * 0.5f;
  const float t3 = (t2 * x) * 0.333333343f;
  return fmaf(t3, c.c3, fmaf(t2, c.c2, fmaf(x, c.c1, 1.0f)));
}

// exp(x) as 2^(x log2 e) on the hardware exp2 (about 1 ulp; the fused residual needs the difference
// exp(x) - exp_{<=t}(x) to the 1e-4 relative tolerance of the outputs, not correct rounding).
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504f); }

// 4 consecutive row elements [col, col+4) as fp32 (zero beyond `width`); vector load when possible.
__device__ __forceinline__ floatx4 load4_row(const void* base, int64_t row_off, int col, int width, int dtype,
                                             bool vec) {
  if (vec && col + 3 < width) {
    if (dtype == F32) return *reinterpret_cast<const floatx4*>(static_cast<const float*>(base) + row_off + col);
    const uint2 raw = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + row_off + col);
    if (dtype == BF16)
      return floatx4{__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u), __uint_as_float(raw.y << 16),
                     __uint_as_float(raw.y & 0xffff0000u)};
    const _Float16* h = reinterpret_cast<const _Float16*>(&raw);
    return floatx4{static_cast<float>(h[0]), static_cast<float>(h[1]), static_cast<float>(h[2]), static_cast<float>(h[3])};
  }
  floatx4 r = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < 4; ++m)
    if (col + m < width) r[m] = load_elem(base, row_off + col + m, dtype);
  return r;
}

// Work layout: one workgroup per (head, tile of 64*RS query rows); wave w owns RS strips of 16 rows.
// Keys are staged in LDS 64 (or 32) at a time: K row-major, V transposed ([column][key]).  For a staged
// batch each wave computes X = K Q^T for all its (strip, 16-key subtile) pairs with interleaved MFMA
// chains (k-step kk of lane group lg covers dimension (D/4) lg + kk, so a lane's key operands are
// 16-byte LDS reads), evaluates the weights elementwise, and accumulates num^T += V^T P^T with the P^T
// tile fed straight from the accumulator as the B operand.
// Two waves per SIMD when the per-wave register arrays (queries, numerators, X and P tiles) leave room.
__host__ __device__ constexpr int block_occupancy(int dp, int dvt, int rs) {
  return (rs * dp / 4 + rs * dvt * 4 + 2 * rs * ((dp + dvt * 16 > 192) ? 2 : 4) * 4) <= 160 ? 2 : 1;
}

template <int DP, int DVT, int RS>
__global__ __launch_bounds__(256, block_occupancy(DP, DVT, RS)) void block_attn_kernel(const BlockArgs a) {
  constexpr int KB = (DP + DVT * 16 > 192) ? 32 : 64;  // keys per LDS stage
  constexpr int NSUB = KB / 16;                         // 16-key subtiles per stage
  constexpr int LDK = DP + 4;                           // = 4 (mod 64) for the 16-byte key reads
  constexpr int DV = DVT * 16;
  constexpr int LDVT = KB + 4;
  constexpr int DQ = DP / 4;  // k-steps of X = K Q^T, dimensions per lane group
  constexpr int TM = 64 * RS;
  __shared__ float Kst[KB * LDK];
  __shared__ float Vt[DV * LDVT];
  __shared__ float Wst[KB];
  __shared__ int Jst[KB];

  const int wg = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t bh = wg / a.n_tiles;
  const int t = wg % a.n_tiles;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int n = static_cast<int>(a.n);
  const int r0 = t * TM - a.shift;

  const int64_t qkbase = bh * a.n * a.d;
  const int64_t vbase = bh * a.n * a.dv;
  const bool vec = (a.d % 4 == 0) && (a.dv % 4 == 0);

  int rbase[RS], myrow[RS], csr[RS], rsr[RS];
  bool rvalid[RS];
  float qB[RS][DQ];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    rbase[rs] = r0 + (wave * RS + rs) * 16;
    myrow[rs] = rbase[rs] + li;
    rvalid[rs] = myrow[rs] >= 0 && myrow[rs] < n;
    csr[rs] = static_cast<int>(chunk_start(myrow[rs], a.chunk, a.shift));
    const int64_t rsv = residual_start(myrow[rs], a.mode, a.block);
    rsr[rs] = rsv > INT32_MAX ? INT32_MAX : static_cast<int>(rsv);
    const int64_t qoff = qkbase + static_cast<int64_t>(rvalid[rs] ? myrow[rs] : 0) * a.d;
    const float qs = rvalid[rs] ? a.scale : 0.f;  // the logits come out scaled
#pragma unroll
    for (int m = 0; m < DQ / 4; ++m) {
      const floatx4 v4 = load4_row(a.q, qoff, DQ * lg + 4 * m, a.d, a.dtype, vec);
#pragma unroll
      for (int e = 0; e < 4; ++e) qB[rs][4 * m + e] = v4[e] * qs;
    }
  }
  const int wrow_lo = r0 + wave * RS * 16, wrow_hi = wrow_lo + RS * 16 - 1;  // this wave's rows

  floatx4 num[RS][DVT];
  float den[RS];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    den[rs] = 0.f;
#pragma unroll
    for (int ct = 0; ct < DVT; ++ct) num[rs][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  const TaylorCoef tc = taylor_coef(a.degree);
  const float xmax = a.exp_clamp ? 80.f : __builtin_huge_valf();  // exp(min(x, 80)) in the Triton mode
  const int row_lo = r0 > 0 ? r0 : 0;
  const int row_hi = (r0 + TM < n ? r0 + TM : n) - 1;  // inclusive
  if (row_lo > row_hi) return;  // whole tile outside the sequence (uniform)

  // One staged batch: in-tile keys (is_node false) or the items of a node active on rows [lo, hi].
  auto process = [&](bool is_node, int lo, int hi) {
    floatx4 x[RS][NSUB];
#pragma unroll
    for (int rs = 0; rs < RS; ++rs)
#pragma unroll
      for (int kt = 0; kt < NSUB; ++kt) x[rs][kt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < DQ / 4; ++m) {
      floatx4 kv[NSUB];
#pragma unroll
      for (int kt = 0; kt < NSUB; ++kt)
        kv[kt] = *reinterpret_cast<const floatx4*>(Kst + (16 * kt + li) * LDK + DQ * lg + 4 * m);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int kt = 0; kt < NSUB; ++kt)
#pragma unroll
          for (int rs = 0; rs < RS; ++rs) x[rs][kt] = mfma4(kv[kt][e], qB[rs][4 * m + e], x[rs][kt]);
    }
    // weights, elementwise (key 16 kt + 4 lg + r, row myrow[rs])
    floatx4 P[RS][NSUB];
#pragma unroll
    for (int kt = 0; kt < NSUB; ++kt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kidx = 16 * kt + 4 * lg + r;
        const int j = Jst[kidx];
        const float w = Wst[kidx];
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) {
          const int i = myrow[rs];
          const float xv = x[rs][kt][r];
          const float ex = exp_fast(fminf(xv, xmax));
          const float tp = taylor_fast(xv, tc);
          float p;
          if (is_node) {
            const bool on = rvalid[rs] && i >= lo && i <= hi;
            p = on ? (ex - tp) * w : 0.f;
          } else {
            // own chunk (j >= cs): Taylor part; article block (j >= rs): residual; both: exp
            const bool on = rvalid[rs] && j >= 0 && j <= i;
            const float pr = (j >= rsr[rs] ? ex - tp : 0.f) + (j >= csr[rs] ? tp : 0.f);
            p = on ? pr : 0.f;
          }
          P[rs][kt][r] = p;
          den[rs] += p;
        }
      }
    }
    // num^T += V^T P^T
#pragma unroll
    for (int kt = 0; kt < NSUB; ++kt) {
#pragma unroll
      for (int ct = 0; ct < DVT; ++ct) {
        const floatx4 va = *reinterpret_cast<const floatx4*>(Vt + (16 * ct + li) * LDVT + 16 * kt + 4 * lg);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int rs = 0; rs < RS; ++rs) num[rs][ct] = mfma4(va[s], P[rs][kt][s], num[rs][ct]);
      }
    }
  };

  // Stage keys [first key j0 .. ) of the batch: k rows row-major, v rows transposed.  src(r) gives the
  // source row of batch slot r (-1: empty slot, zero-filled).
  auto stage = [&](auto src_of, bool mat) {
    constexpr int KU = DP / 4, VU = DV / 4;
    for (int e = tid; e < KB * KU; e += 256) {
      const int r = e / KU, u = e - r * KU;
      const int src = src_of(r);
      floatx4 v4 = floatx4{0.f, 0.f, 0.f, 0.f};
      if (src >= 0) {
        v4 = mat ? load4_row(a.rep_k, (bh * a.n_rep + src) * a.d, 4 * u, a.d, F32, vec)
                 : load4_row(a.k, qkbase + static_cast<int64_t>(src) * a.d, 4 * u, a.d, a.dtype, vec);
      }
      *reinterpret_cast<floatx4*>(Kst + r * LDK + 4 * u) = v4;
    }
    for (int e = tid; e < KB * VU; e += 256) {
      const int r = e % KB, u = e / KB;  // key-fast: conflict-light transposed writes
      const int src = src_of(r);
      floatx4 v4 = floatx4{0.f, 0.f, 0.f, 0.f};
      if (src >= 0) {
        v4 = mat ? load4_row(a.rep_v, (bh * a.n_rep + src) * a.dv, 4 * u, a.dv, F32, vec)
                 : load4_row(a.v, vbase + static_cast<int64_t>(src) * a.dv, 4 * u, a.dv, a.dtype, vec);
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) Vt[(4 * u + m) * LDVT + r] = v4[m];
    }
  };

  // ---- phase A: keys of the tile's own chunk / article block ----
  int kstart = static_cast<int>(chunk_start(row_lo, a.chunk, a.shift));
  const int64_t rs_lo = residual_start(row_lo, a.mode, a.block);
  if (rs_lo < kstart) kstart = static_cast<int>(rs_lo);
  if (kstart < 0) kstart = 0;
  const int kend = row_hi + 1;
  for (int kb0 = kstart; kb0 < kend; kb0 += KB) {
    __syncthreads();
    if (tid < KB) {
      const int j = kb0 + tid;
      Jst[tid] = j < kend ? j : -1;
      Wst[tid] = 1.f;
    }
    stage([&](int r) { return kb0 + r < kend ? kb0 + r : -1; }, false);
    __syncthreads();
    if (kb0 <= wrow_hi) process(false, 0, 0);  // some key of the batch precedes some row of this wave
  }

  // ---- phase B: coreset nodes visible to some row of the tile ----
  const int p_end = a.tile_ptr[t + 1];
  for (int p = a.tile_ptr[t]; p < p_end; ++p) {
    const int node = a.tile_nodes[p];
    const int32_t* meta = a.node_meta + static_cast<int64_t>(node) * NODE_META;
    const int size = meta[0];
    const int lo = meta[1], hi = meta[2];
    const bool mat = meta[3] != 0;
    const int64_t ibase = (bh * a.n_nodes + node) * a.cap;
    for (int i0 = 0; i0 < size; i0 += KB) {
      __syncthreads();
      if (tid < KB) {
        const int it = i0 + tid;
        Jst[tid] = it < size ? a.node_src[ibase + it] : -1;
        Wst[tid] = it < size ? a.node_w[ibase + it] : 0.f;
      }
      __syncthreads();
      stage([&](int r) { return Jst[r]; }, mat);
      __syncthreads();
      if (hi >= wrow_lo && lo <= wrow_hi) process(true, lo, hi);
    }
  }

  // ---- epilogue: add the moment partials, normalise, store ----
  const bool raw = a.out_den != nullptr;
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    float dsum = den[rs];
    dsum += __shfl_xor(dsum, 16);
    dsum += __shfl_xor(dsum, 32);
    if (!rvalid[rs]) continue;
    const int64_t i = myrow[rs];
    float lowd = 0.f;
    for (int f = 0; f < a.fsplit; ++f) lowd += a.low_den[(bh * a.fsplit + f) * a.low_rows + a.low_off + i];
    if (raw && lg == 0) a.out_den[bh * a.n + i] = lowd + dsum;
    const float dn = fmaxf(lowd + dsum, a.eps);
#pragma unroll
    for (int ct = 0; ct < DVT; ++ct) {
      const int c0 = 16 * ct + 4 * lg;
      if (c0 >= a.dv) continue;
      floatx4 lown = floatx4{0.f, 0.f, 0.f, 0.f};
      for (int f = 0; f < a.fsplit; ++f)
        lown += *reinterpret_cast<const floatx4*>(
            a.low_num + ((bh * a.fsplit + f) * a.low_rows + a.low_off + i) * a.low_ld + c0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int col = c0 + r;
        if (col < a.dv) {
          const float numv = num[rs][ct][r] + lown[r];
          if (raw)
            static_cast<float*>(a.out)[(bh * a.n + i) * a.dv + col] = numv;
          else
            store_elem(a.out, (bh * a.n + i) * a.dv + col, a.out_dtype, numv / dn);
        }
      }
    }
  }
}

}  // namespace sta
