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
#include <type_traits>

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
  int ldqk;  // row stride (elements) of q and k: a multiple of 4, >= d
  int ldvr;  // row stride of v: a multiple of 4, >= dv
  int ldrk;  // row stride of rep_k / rep_v (fp32; multiples of 4)
  int ldrv;
  void* out;  // [BH][n][dv]
  int out_dtype;
  float* out_den;  // optional [BH][n]: when set, out (fp32) receives num and out_den receives den, unnormalised
  int split;       // 1: split-bf16 matrix-core products (block_attn_kernel<..., true>)
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

// The logits come out in base 2: the staged queries carry scale * log2(e), so y = x log2(e) for the
// natural logit x, exp(x) = exp2(y) on the hardware exp2 (about 1 ulp; the fused residual needs the
// difference exp(x) - exp_{<=t}(x) to the 1e-4 relative tolerance of the outputs, not correct rounding)
// and the Taylor truncation sum_{r<=deg} x^r / r! (deg <= 8) is the Horner form in y,
// 1 + y (k1 + y (k2 + y (k3 + ...))) with k_r = (ln 2)^r / r! for r <= deg and 0 above, within a few
// ulp of the reference's term-by-term sum.  D4: the fp32-product kernel, which serves degree 4, takes
// the fourth fused multiply-add; HD: its high-degree instantiation (degree 5 .. 8) the eighth; the
// split-product kernel stops at degree 3 (three for every degree; sta_block_attention rejects split
// products with degree 4 or more).
struct TaylorCoef2 {
  float k1, k2, k3, k4, k5, k6, k7, k8;
};
__host__ __device__ inline TaylorCoef2 taylor_coef2(int deg) {
  return TaylorCoef2{deg >= 1 ? 0.693147180560f : 0.f, deg >= 2 ? 0.240226506959f : 0.f,
                     deg >= 3 ? 0.0555041086648f : 0.f, deg >= 4 ? 0.00961812910763f : 0.f,
                     deg >= 5 ? 1.33335581464e-3f : 0.f, deg >= 6 ? 1.54035303934e-4f : 0.f,
                     deg >= 7 ? 1.52527338041e-5f : 0.f, deg >= 8 ? 1.32154867902e-6f : 0.f};
}
template <bool D4, bool HD = false>
__device__ __forceinline__ float taylor2(float y, const TaylorCoef2& c) {
  float t4 = c.k4;
  if constexpr (HD) t4 = fmaf(y, fmaf(y, fmaf(y, fmaf(y, c.k8, c.k7), c.k6), c.k5), c.k4);
  const float t3 = (D4 || HD) ? fmaf(y, t4, c.k3) : c.k3;
  return fmaf(y, fmaf(y, fmaf(y, t3, c.k2), c.k1), 1.0f);
}
constexpr float LOG2E = 1.44269504f;

// Work layout: one workgroup per (head, tile of 64*RS query rows); wave w owns RS strips of 16 rows.
// Keys are staged in LDS 64 (or 32) at a time: K row-major, V transposed ([column][key]).  For a staged
// batch each wave computes X = K Q^T for all its (strip, 16-key subtile) pairs with interleaved MFMA
// chains (k-step kk of lane group lg covers dimension (D/4) lg + kk, so a lane's key operands are
// 16-byte LDS reads), evaluates the weights elementwise, and accumulates num^T += V^T P^T with the P^T
// tile fed straight from the accumulator as the B operand.
//
// Batches: first the keys of the tile's own chunk / article block (contiguous rows), then the coreset
// items of the tile's nodes, flattened into an LDS list (token, weight, first and last active row per
// item) filled up to BA_LIST items at a time, so a batch may span two nodes.  The rows of batch b+1 are
// loaded into registers while batch b computes (one batch of software pipelining), so the global
// latency of the gathers is hidden behind the matrix-core work.
// Two waves per SIMD when the per-wave register arrays (queries, numerators, X and P tiles, prefetched
// rows) leave room.
constexpr int BA_LIST = 1024;
__host__ __device__ constexpr int block_kb(int dp, int dvt) { return (dp + dvt * 16 > 192) ? 32 : 64; }
__host__ __device__ constexpr int block_kpt(int dp, int dvt) { return (block_kb(dp, dvt) * dp / 4 + 255) / 256; }
__host__ __device__ constexpr int block_vpt(int dp, int dvt) { return (block_kb(dp, dvt) * dvt * 4 + 255) / 256; }
__host__ __device__ constexpr int block_occupancy(int dp, int dvt, int rs) {
  return (rs * dp / 4 + rs * dvt * 4 + 2 * rs * (block_kb(dp, dvt) / 16) * 4 +
          4 * (block_kpt(dp, dvt) + block_vpt(dp, dvt))) <= 160
             ? 2
             : 1;
}

// SPLIT: split-bf16 matrix-core products (the fp32 operands as bf16 hi + lo, three 16x16x32 bf16 products
// per product; common.hpp).  The staged key and value rows are split once per workgroup when written
// to LDS (bf16 hi and lo planes), the wave's query rows once per kernel, the probabilities per pair of
// 16-key subtiles.  X = K Q^T: k-step m of lane group lg covers dimensions 32 m + 8 lg + j, j = 0..7
// (16-byte LDS reads of 8 bf16).  num^T += V^T P^T over a subtile pair (2 s, 2 s + 1): contraction
// index 8 lg + j is key 16 (2 s) + 4 lg + j (j < 4) or 16 (2 s + 1) + 4 lg + j - 4, i.e. element j & 3 of
// the lane's own P tile of that subtile; the value planes store each pair's 32 keys in that order
// (split_key_pos), so the A operand is again one 16-byte read.
__host__ __device__ constexpr int split_key_pos(int r) {
  return 32 * (r >> 5) + 8 * ((r >> 2) & 3) + 4 * ((r >> 4) & 1) + (r & 3);
}

// KVX (split products, bf16 inputs): the key and value rows are exact in bf16, so their lo planes are
// zero: the products with them (kl·qh in X, vl·ph in num) and the lo planes themselves are left out
// (X and num are those of the three-product form, bit for bit).
// HD (fp32 products only): the Taylor polynomial through degree 8 (degree 5 .. 8).
template <int DP, int DVT, int RS, int ES, bool SPLIT, bool KVX = false, bool HD = false>
__global__ __launch_bounds__(256, block_occupancy(DP, DVT, RS)) void block_attn_kernel(const BlockArgs a) {
  constexpr int KB = block_kb(DP, DVT);  // keys per LDS stage
  constexpr int NSUB = KB / 16;                         // 16-key subtiles per stage
  constexpr int LDK = DP + 4;                           // = 4 (mod 64) for the 16-byte key reads
  constexpr int DV = DVT * 16;
  constexpr int LDVT = KB + 4;
  constexpr int DQ = DP / 4;  // k-steps of X = K Q^T, dimensions per lane group
  constexpr int TM = 64 * RS;
  // split layout: dimensions padded to whole 32-dimension steps; bf16 row strides of 16 (2m + 1) bytes,
  // so the 16 rows of a 16-byte read fall on distinct bank groups
  constexpr int DPS = DP < 32 ? 32 : DP;
  constexpr int MS = DPS / 32;
  constexpr int LDKB = DPS + 8;
  constexpr int LDVB = KB + 8;
  static_assert(!SPLIT || NSUB % 2 == 0, "split products pair the 16-key subtiles");
  constexpr int F32_WORDS = KB * LDK + DV * LDVT;
  constexpr int SPLIT_WORDS = KB * LDKB + DV * LDVB;  // two bf16 planes each
  constexpr int STAGE_WORDS = SPLIT ? SPLIT_WORDS : F32_WORDS;
  __shared__ floatx4 stage4[(STAGE_WORDS + 3) / 4];
  float* const Kst = reinterpret_cast<float*>(stage4);
  float* const Vt = Kst + KB * LDK;
  __bf16* const Kh = reinterpret_cast<__bf16*>(stage4);
  __bf16* const Kl = Kh + KB * LDKB;
  __bf16* const Vh = Kl + KB * LDKB;
  __bf16* const Vl = Vh + DV * LDVB;
  __shared__ float Wst[KB];
  __shared__ int Jst[KB];
  __shared__ int Lost[KB], Hist[KB];  // active rows of the staged items (node batches)
  __shared__ int Lj[BA_LIST], Llo[BA_LIST], Lhi[BA_LIST];
  __shared__ float Lw[BA_LIST];

  const int wg = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t bh = wg / a.n_tiles;
  const int t = wg % a.n_tiles;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int n = static_cast<int>(a.n);
  const int r0 = t * TM - a.shift;

  const int64_t qkbase = bh * a.n * a.ldqk;
  const int64_t vbase = bh * a.n * a.ldvr;

  int rbase[RS], myrow[RS], csr[RS], rsr[RS];
  bool rvalid[RS];
  float qB[RS][SPLIT ? 1 : DQ];
  bf16x8 qh[RS][SPLIT ? MS : 1], ql[RS][SPLIT ? MS : 1];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    rbase[rs] = r0 + (wave * RS + rs) * 16;
    myrow[rs] = rbase[rs] + li;
    rvalid[rs] = myrow[rs] >= 0 && myrow[rs] < n;
    csr[rs] = static_cast<int>(chunk_start(myrow[rs], a.chunk, a.shift));
    const int64_t rsv = residual_start(myrow[rs], a.mode, a.block);
    rsr[rs] = rsv > INT32_MAX ? INT32_MAX : static_cast<int>(rsv);
    const int64_t qoff = qkbase + static_cast<int64_t>(rvalid[rs] ? myrow[rs] : 0) * a.ldqk;
    const float qs = rvalid[rs] ? a.scale * LOG2E : 0.f;  // the logits come out scaled, in base 2
    if constexpr (SPLIT) {
#pragma unroll
      for (int m = 0; m < MS; ++m) {
        float x[8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int col = 32 * m + 8 * lg + 4 * h;  // columns beyond the row (DPS > ldqk) are zero
          const floatx4 v4 = unit_to_f4<ES>(load_unit<ES>(a.q, qoff + min(col, a.ldqk - 4)), a.dtype,
                                             col < a.ldqk ? qs : 0.f);
#pragma unroll
          for (int e = 0; e < 4; ++e) x[4 * h + e] = v4[e];
        }
        split_bf16(x, qh[rs][m], ql[rs][m]);
      }
    } else {
#pragma unroll
      for (int m = 0; m < DQ / 4; ++m) {
        const int col = DQ * lg + 4 * m;  // columns beyond the row (DP > ldqk) are zero
        const floatx4 v4 = unit_to_f4<ES>(load_unit<ES>(a.q, qoff + min(col, a.ldqk - 4)), a.dtype,
                                           col < a.ldqk ? qs : 0.f);
#pragma unroll
        for (int e = 0; e < 4; ++e) qB[rs][SPLIT ? 0 : 4 * m + e] = v4[e];
      }
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

  const TaylorCoef2 tc = taylor_coef2(a.degree);
  const float ymax = a.exp_clamp ? 80.f * LOG2E : __builtin_huge_valf();  // exp(min(x, 80)) in the Triton mode
  const int row_lo = r0 > 0 ? r0 : 0;
  const int row_hi = (r0 + TM < n ? r0 + TM : n) - 1;  // inclusive
  if (row_lo > row_hi) return;  // whole tile outside the sequence (uniform)

  // One staged batch: in-tile keys (is_node false) or the items of a node active on rows [lo, hi].
  // One staged batch, pipelined by 16-key subtile: the X = K Q^T products of subtile kt+1 are issued
  // while the weights of subtile kt are evaluated (VALU in the matrix cores' shadow), then subtile kt's
  // num^T += V^T P^T.  X is accumulated in two halves of the dimensions (4 independent chains).
  // NODE: coreset items (weight, active rows) instead of the tile's own keys.
  // node_tag: 0 the tile's own keys, 1 coreset items with their active-row test, 2 coreset items active
  // on every row of the tile (the test is skipped), 3 as 2 for degree <= 2 without the exp clamp: the
  // Horner form stops at y^2 and the logit is not clamped (the same values for every finite logit:
  // with k3 = 0 the third fused multiply-add returns k2 exactly, and min(y, inf) = y), two VALU
  // instructions fewer per (row, item) pair on the most frequent batch kind
  auto process = [&](auto node_tag) {
    constexpr bool NODE = decltype(node_tag)::value != 0;
    constexpr bool FULL = decltype(node_tag)::value >= 2;
    constexpr bool FAST = decltype(node_tag)::value == 3;
    // weights of subtile kt from its logits X (key 16 kt + 4 lg + r, row myrow[rs]), elementwise
    auto weights = [&](int kt, const floatx4 (&X)[RS], floatx4 (&P)[RS]) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kidx = 16 * kt + 4 * lg + r;
        const int j = Jst[kidx];
        const float w = Wst[kidx];
        const int lo = NODE ? Lost[kidx] : 0, hi = NODE ? Hist[kidx] : 0;
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) {
          const int i = myrow[rs];
          const float yv = X[rs][r];
          const float ex = __builtin_amdgcn_exp2f(FAST ? yv : fminf(yv, ymax));
          const float tp = FAST ? fmaf(yv, fmaf(yv, tc.k2, tc.k1), 1.0f) : taylor2<!SPLIT, HD>(yv, tc);
          float p;
          if constexpr (FULL) {
            p = (ex - tp) * w;  // rows outside the sequence have zero queries and are never stored
          } else if constexpr (NODE) {
            const bool on = rvalid[rs] && i >= lo && i <= hi;
            p = on ? (ex - tp) * w : 0.f;
          } else {
            // own chunk (j >= cs): Taylor part; article block (j >= rs): residual; both: exp
            const bool on = rvalid[rs] && j >= 0 && j <= i;
            const float pr = (j >= rsr[rs] ? ex - tp : 0.f) + (j >= csr[rs] ? tp : 0.f);
            p = on ? pr : 0.f;
          }
          P[rs][r] = p;
          den[rs] += p;
        }
      }
    };
    if constexpr (SPLIT) {
      // X of subtiles 2 s and 2 s + 1 (2 RS independent chains of 3 MS products)
      auto qk2 = [&](int sp, floatx4 (&xq)[2][RS]) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int rs = 0; rs < RS; ++rs) xq[h][rs] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < MS; ++m) {
          bf16x8 kh[2], kl[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int off = (16 * (2 * sp + h) + li) * LDKB + 32 * m + 8 * lg;
            kh[h] = *reinterpret_cast<const bf16x8*>(Kh + off);
            if constexpr (!KVX) kl[h] = *reinterpret_cast<const bf16x8*>(Kl + off);
          }
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int rs = 0; rs < RS; ++rs) xq[h][rs] = mfma_bf16(kh[h], ql[rs][m], xq[h][rs]);
          if constexpr (!KVX) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
              for (int rs = 0; rs < RS; ++rs) xq[h][rs] = mfma_bf16(kl[h], qh[rs][m], xq[h][rs]);
          }
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int rs = 0; rs < RS; ++rs) xq[h][rs] = mfma_bf16(kh[h], qh[rs][m], xq[h][rs]);
        }
      };
      // num^T += V^T P^T over subtiles 2 s, 2 s + 1
      auto pv2 = [&](int sp, const floatx4 (&P)[2][RS]) {
        bf16x8 ph[RS], pl[RS];
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) {
          const float x[8] = {P[0][rs][0], P[0][rs][1], P[0][rs][2], P[0][rs][3],
                              P[1][rs][0], P[1][rs][1], P[1][rs][2], P[1][rs][3]};
          split_bf16(x, ph[rs], pl[rs]);
        }
#pragma unroll
        for (int ct = 0; ct < DVT; ++ct) {
          const int off = (16 * ct + li) * LDVB + 32 * sp + 8 * lg;
          const bf16x8 vh = *reinterpret_cast<const bf16x8*>(Vh + off);
#pragma unroll
          for (int rs = 0; rs < RS; ++rs) num[rs][ct] = mfma_bf16(vh, pl[rs], num[rs][ct]);
          if constexpr (!KVX) {
            const bf16x8 vl = *reinterpret_cast<const bf16x8*>(Vl + off);
#pragma unroll
            for (int rs = 0; rs < RS; ++rs) num[rs][ct] = mfma_bf16(vl, ph[rs], num[rs][ct]);
          }
#pragma unroll
          for (int rs = 0; rs < RS; ++rs) num[rs][ct] = mfma_bf16(vh, ph[rs], num[rs][ct]);
        }
      };
      floatx4 xa[2][RS], xb[2][RS];
      qk2(0, xa);
#pragma unroll
      for (int sp = 0; sp < NSUB / 2; ++sp) {
        floatx4(&xc)[2][RS] = (sp & 1) ? xb : xa;
        floatx4(&xn)[2][RS] = (sp & 1) ? xa : xb;
        if (sp + 1 < NSUB / 2) qk2(sp + 1, xn);
        floatx4 P[2][RS];
        weights(2 * sp, xc[0], P[0]);
        weights(2 * sp + 1, xc[1], P[1]);
        if (sp + 1 < NSUB / 2) {
          // the 6 RS MS products of X(sp + 1) spread over the weights' VALU of subtiles 2 sp, 2 sp + 1
#pragma unroll
          for (int g = 0; g < 6 * RS * MS; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
          }
        }
        pv2(sp, P);
      }
    } else {
      constexpr int QKM = DQ * RS;  // matrix-core ops of one subtile's X
      auto qk = [&](int kt, floatx4 (&xq)[2][RS]) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int rs = 0; rs < RS; ++rs) xq[h][rs] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < DQ / 4; ++m) {
          const floatx4 kv = *reinterpret_cast<const floatx4*>(Kst + (16 * kt + li) * LDK + DQ * lg + 4 * m);
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int rs = 0; rs < RS; ++rs)
              xq[m & 1][rs] = mfma4(kv[e], qB[rs][SPLIT ? 0 : 4 * m + e], xq[m & 1][rs]);
        }
      };
      auto pv = [&](int kt, const floatx4 (&P)[RS]) {
#pragma unroll
        for (int ct = 0; ct < DVT; ++ct) {
          const floatx4 va = *reinterpret_cast<const floatx4*>(Vt + (16 * ct + li) * LDVT + 16 * kt + 4 * lg);
#pragma unroll
          for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int rs = 0; rs < RS; ++rs) num[rs][ct] = mfma4(va[s], P[rs][s], num[rs][ct]);
        }
      };
      floatx4 xa[2][RS], xb[2][RS];
      qk(0, xa);
#pragma unroll
      for (int kt = 0; kt < NSUB; ++kt) {
        floatx4(&xc)[2][RS] = (kt & 1) ? xb : xa;
        floatx4(&xn)[2][RS] = (kt & 1) ? xa : xb;
        if (kt + 1 < NSUB) qk(kt + 1, xn);
        floatx4 X[RS], P[RS];
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) X[rs] = xc[0][rs] + xc[1][rs];
        weights(kt, X, P);
        if (kt + 1 < NSUB) {
#pragma unroll
          for (int g = 0; g < QKM; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one matrix-core op of X(kt+1)
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // then VALU of the weights of kt
          }
        }
        pv(kt, P);
      }
    }
  };
  using block_batch = std::integral_constant<int, 0>;
  using node_batch = std::integral_constant<int, 1>;
  using node_batch_full = std::integral_constant<int, 2>;
  using node_batch_full_fast = std::integral_constant<int, 3>;
  const bool fast = !a.exp_clamp && a.degree <= 2;

  // ---- batch sequence: phase A = contiguous keys [kstart, kend), phase B = the node item list ----
  int kstart = static_cast<int>(chunk_start(row_lo, a.chunk, a.shift));
  const int64_t rs_lo = residual_start(row_lo, a.mode, a.block);
  if (rs_lo < kstart) kstart = static_cast<int>(rs_lo);
  if (kstart < 0) kstart = 0;
  const int kend = row_hi + 1;
  const int n_a = kend > kstart ? (kend - kstart + KB - 1) / KB : 0;
  const bool mat = a.rep_k != nullptr;  // segment-mean items index rep_k / rep_v (every node or none)

  // node item list, filled BA_LIST items at a time in tile-list order (uniform control flow)
  int p_cur = a.tile_ptr[t], i_cur = 0;
  const int p_end = a.tile_ptr[t + 1];
  int llen = 0;
  auto fill = [&]() {
    llen = 0;
    while (p_cur < p_end && llen < BA_LIST) {
      const int node = a.tile_nodes[p_cur];
      const int32_t* meta = a.node_meta + static_cast<int64_t>(node) * NODE_META;
      const int size = meta[0], lo = meta[1], hi = meta[2];
      const int take = min(size - i_cur, BA_LIST - llen);
      const int64_t ibase = (bh * a.n_nodes + node) * a.cap + i_cur;
      for (int e = tid; e < take; e += 256) {
        Lj[llen + e] = a.node_src[ibase + e];
        Lw[llen + e] = a.node_w[ibase + e];
        Llo[llen + e] = lo;
        Lhi[llen + e] = hi;
      }
      llen += take > 0 ? take : 0;
      i_cur += take > 0 ? take : 0;
      if (i_cur >= size) {
        ++p_cur;
        i_cur = 0;
      }
    }
  };

  // prefetch registers: this thread's 4-element units of the next batch's key and value rows, raw (they
  // are converted when written to LDS, so no instruction waits on the loads before the next commit),
  // and which of them are real (row of the batch, column inside the row)
  constexpr int KU = DP / 4, VU = DV / 4;
  constexpr int KPT = block_kpt(DP, DVT), VPT = block_vpt(DP, DVT);
  // value units in key pairs (split products, an even count of units per thread covering the batch
  // exactly): units 2 k and 2 k + 1 of a thread are keys 2 rp and 2 rp + 1 of one column unit, which sit
  // next to each other in the value planes (split_key_pos), so the commit splits them as packed pairs
  // and writes 32-bit words; otherwise key-fast single units
  constexpr bool VPAIR = SPLIT && VPT % 2 == 0 && KB * VU == 256 * VPT;
  auto vunit = [&](int i, int& r, int& u) -> bool {
    if constexpr (VPAIR) {
      const int pe = tid + 256 * (i >> 1);
      r = 2 * (pe % (KB / 2)) + (i & 1);
      u = pe / (KB / 2);
      return true;
    } else {
      const int e = tid + 256 * i;
      r = e % KB;  // key-fast: conflict-light transposed writes
      u = e / KB;
      return e < KB * VU;
    }
  };
  uint4 pk[KPT], pv[VPT];
  uint32_t pk_ok = 0, pv_ok = 0;
  int pj = -1, plo = 0, phi = -1;
  float pw = 0.f;
  auto src_of = [&](bool node, int off, int r) -> int {
    if (!node) return off + r < kend ? off + r : -1;
    return off + r < llen ? Lj[off + r] : -1;
  };
  auto prefetch = [&](bool node, int off) {
    // in-block keys come from k / v; node items from rep_k / rep_v in segment mode (fp32, ES == 4 there)
    const bool from_rep = mat && node;
    const void* kb = a.k;
    const void* vb = a.v;
    int64_t kbase = qkbase, vbase2 = vbase;
    int ldk = a.ldqk, ldv = a.ldvr;
    if constexpr (ES == 4) {
      if (from_rep) {
        kb = a.rep_k;
        vb = a.rep_v;
        kbase = bh * a.n_rep * a.ldrk;
        vbase2 = bh * a.n_rep * a.ldrv;
        ldk = a.ldrk;
        ldv = a.ldrv;
      }
    }
    pk_ok = pv_ok = 0;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int e = tid + 256 * i;
      const int r = e / KU, u = e - r * KU;
      const int src = (e < KB * KU) ? src_of(node, off, r) : -1;
      const bool ok = src >= 0 && 4 * u < ldk;
      pk_ok |= ok ? (1u << i) : 0u;
      pk[i] = load_unit<ES>(kb, kbase + static_cast<int64_t>(src >= 0 ? src : 0) * ldk + min(4 * u, ldk - 4));
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      int r, u;
      const bool in = vunit(i, r, u);
      const int src = in ? src_of(node, off, r) : -1;
      const bool ok = src >= 0 && 4 * u < ldv;
      pv_ok |= ok ? (1u << i) : 0u;
      pv[i] = load_unit<ES>(vb, vbase2 + static_cast<int64_t>(src >= 0 ? src : 0) * ldv + min(4 * u, ldv - 4));
    }
    if (tid < KB) {
      pj = src_of(node, off, tid);
      const bool in = node && off + tid < llen;
      pw = in ? Lw[off + tid] : (node ? 0.f : 1.f);
      plo = in ? Llo[off + tid] : 0;
      phi = in ? Lhi[off + tid] : -1;
    }
  };
  bool item_full = true;
  auto commit = [&]() {
    if constexpr (SPLIT) {
      // bf16 hi / lo planes; keys row-major (dimension 4 u..4 u+3 of key r: 8 bytes per plane), values
      // transposed with each subtile pair's keys in contraction order (split_key_pos)
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        const int e = tid + 256 * i;
        if (e < KB * KU) {
          const int r = e / KU, u = e - r * KU;
          const floatx4 f = unit_to_f4<ES>(pk[i], a.dtype, ((pk_ok >> i) & 1u) ? 1.f : 0.f);
          uint32_t h0, h1, l0, l1;
          split_pair(f[0], f[1], h0, l0);
          split_pair(f[2], f[3], h1, l1);
          *reinterpret_cast<uint2*>(Kh + r * LDKB + 4 * u) = uint2{h0, h1};
          if constexpr (!KVX) *reinterpret_cast<uint2*>(Kl + r * LDKB + 4 * u) = uint2{l0, l1};
        }
      }
      if constexpr (VPAIR) {
#pragma unroll
        for (int k = 0; k < VPT / 2; ++k) {
          int r, u;
          vunit(2 * k, r, u);
          const floatx4 f0 = unit_to_f4<ES>(pv[2 * k], a.dtype, ((pv_ok >> (2 * k)) & 1u) ? 1.f : 0.f);
          const floatx4 f1 = unit_to_f4<ES>(pv[2 * k + 1], a.dtype, ((pv_ok >> (2 * k + 1)) & 1u) ? 1.f : 0.f);
          const int pos = split_key_pos(r);  // even: key r + 1 at pos + 1
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            uint32_t h, l;
            if constexpr (KVX) {
              h = pk_bf16(f0[m], f1[m]);  // exact bf16 values: the lo plane is zero and not kept
            } else {
              split_pair(f0[m], f1[m], h, l);
              *reinterpret_cast<uint32_t*>(Vl + (4 * u + m) * LDVB + pos) = l;
            }
            *reinterpret_cast<uint32_t*>(Vh + (4 * u + m) * LDVB + pos) = h;
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
          int r, u;
          if (vunit(i, r, u)) {
            const floatx4 f = unit_to_f4<ES>(pv[i], a.dtype, ((pv_ok >> i) & 1u) ? 1.f : 0.f);
            const int pos = split_key_pos(r);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
              const __bf16 h = static_cast<__bf16>(f[m]);
              Vh[(4 * u + m) * LDVB + pos] = h;
              if constexpr (!KVX) Vl[(4 * u + m) * LDVB + pos] = static_cast<__bf16>(f[m] - static_cast<float>(h));
            }
          }
        }
      }
    } else {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int e = tid + 256 * i;
      if (e < KB * KU) {
        const int r = e / KU, u = e - r * KU;
        *reinterpret_cast<floatx4*>(Kst + r * LDK + 4 * u) =
            unit_to_f4<ES>(pk[i], a.dtype, ((pk_ok >> i) & 1u) ? 1.f : 0.f);
      }
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int e = tid + 256 * i;
      if (e < KB * VU) {
        const int r = e % KB, u = e / KB;
        const floatx4 f = unit_to_f4<ES>(pv[i], a.dtype, ((pv_ok >> i) & 1u) ? 1.f : 0.f);
#pragma unroll
        for (int m = 0; m < 4; ++m) Vt[(4 * u + m) * LDVT + r] = f[m];
      }
    }
    }
    if (tid < KB) {
      Jst[tid] = pj;
      Wst[tid] = pw;
      Lost[tid] = plo;
      Hist[tid] = phi;
    }
    // this thread's staged item is padding or active on every row of the tile
    item_full = tid >= KB || pj < 0 || (plo <= row_lo && phi >= row_hi);
  };

  // batch b: phase A for b < n_a (offset kstart + b KB), then phase B (offset into the list chunk).  The
  // list is read only by prefetch(); once a batch is committed its items live in Jst/Wst/Lost/Hist, so
  // the list can be refilled right after the commit of its last batch.
  if constexpr (SPLIT && DPS != DP) {  // dimensions [DP, DPS) of the key planes are never written: zero
    for (int e = tid; e < KB * LDKB; e += 256) Kh[e] = Kl[e] = static_cast<__bf16>(0.f);
  }
  // Moment partials: a.fsplit partial sums per row (the feature splits of the moment scan), RS * fsplit
  // (strip, split) pairs per lane.  Pair p = RS f + rs is loaded during batch p (issued after the next
  // batch's row prefetch, so it has the batch's products to land) and added into the strip's value
  // accumulators and denominator right after the batch; the pairs beyond the tile's batch count are
  // added in the epilogue.  The accumulator layout is the partials' (lane (li, lg): row li, columns
  // 16 ct + 4 lg + r), so no exchange is needed.  Rows outside the sequence read a clamped row and are
  // never stored.  The fp32-product kernels (no register room for the in-flight pair: they would spill)
  // add every pair in the epilogue.
  constexpr bool PAIR_OVERLAP = SPLIT;
  const int fs = a.fsplit;
  const int64_t pden_stride = a.low_rows, pnum_stride = a.low_rows * a.low_ld;
  const float* pden[RS];
  const float* pnum[RS];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    const int64_t i = min(max(myrow[rs], 0), n - 1);
    pden[rs] = a.low_den + bh * fs * pden_stride + a.low_off + i;
    pnum[rs] = a.low_num + (bh * fs * a.low_rows + a.low_off + i) * a.low_ld;
  }
  const int n_pairs = RS * fs;
  float pair_d = 0.f;
  floatx4 pair_n[DVT];
  auto pair_load = [&](int p) {
    const int f = p / RS, rs = p - f * RS;
    const float* pd = pden[0];
    const float* pn = pnum[0];
#pragma unroll
    for (int r2 = 1; r2 < RS; ++r2) {
      if (rs == r2) {
        pd = pden[r2];
        pn = pnum[r2];
      }
    }
    pair_d = __builtin_nontemporal_load(pd + f * pden_stride);
#pragma unroll
    for (int ct = 0; ct < DVT; ++ct) {
      const int c0 = 16 * ct + 4 * lg;
      pair_n[ct] = __builtin_nontemporal_load(
          reinterpret_cast<const floatx4*>(pn + f * pnum_stride + (c0 < a.dv ? c0 : 0)));
    }
  };
  auto pair_add = [&](int p) {
    const int rs = p % RS;
#pragma unroll
    for (int r2 = 0; r2 < RS; ++r2) {
      if (r2 == rs) {
        if (lg == 0) den[r2] += pair_d;  // the lane-group sum below counts it once per row
#pragma unroll
        for (int ct = 0; ct < DVT; ++ct) num[r2][ct] += pair_n[ct];
      }
    }
  };

  bool cur_node = n_a == 0;
  int cur_off = cur_node ? 0 : kstart;
  // the first batch of the tile's own keys needs no list: its rows are in flight while the list's
  // chain of loads (tile list, node metadata, item indices) runs
  if (!cur_node) prefetch(false, cur_off);
  if (p_cur < p_end) fill();  // the first list chunk
  __syncthreads();
  bool have = n_a > 0 || llen > 0;
  if (have && cur_node) prefetch(true, cur_off);
  int pairs_done = 0;
  for (int b = 0; have; ++b) {
    __syncthreads();  // every wave is done with the staging buffers of the previous batch
    commit();
    bool nxt_node = true;
    int nxt_off = cur_node ? cur_off + KB : 0;
    if (!cur_node && b + 1 < n_a) {
      nxt_node = false;
      nxt_off = cur_off + KB;
    } else if (nxt_off >= llen) {  // the list chunk is used up: refill it (uniform)
      nxt_off = 0;
      if (cur_node && p_cur < p_end)
        fill();
      else if (cur_node)
        llen = 0;
    }
    const bool nxt_have = !nxt_node || nxt_off < llen;
    // staged batch and list visible; whether every staged item is active on all rows of the tile
    const bool full = __syncthreads_and(item_full ? 1 : 0) != 0;
    if (nxt_have) prefetch(nxt_node, nxt_off);
    const bool pair = PAIR_OVERLAP && pairs_done < n_pairs;
    if (pair) pair_load(pairs_done);
    if (cur_node && full && fast)
      process(node_batch_full_fast{});
    else if (cur_node && full)
      process(node_batch_full{});
    else if (cur_node)
      process(node_batch{});
    else if (cur_off <= wrow_hi)
      process(block_batch{});  // some key of the batch precedes some row of this wave
    if (pair) pair_add(pairs_done++);
    cur_node = nxt_node;
    cur_off = nxt_off;
    have = nxt_have;
  }

  // ---- epilogue: the remaining moment partials, two pairs in flight (the batch loop's registers are
  //      free; each pair still added in order: pair p's values are parked while p + 1's load is issued),
  //      normalise, store ----
  for (; pairs_done + 1 < n_pairs; pairs_done += 2) {
    pair_load(pairs_done);
    const float d0 = pair_d;
    floatx4 n0[DVT];
#pragma unroll
    for (int ct = 0; ct < DVT; ++ct) n0[ct] = pair_n[ct];
    pair_load(pairs_done + 1);
    const float d1 = pair_d;
    pair_d = d0;
#pragma unroll
    for (int ct = 0; ct < DVT; ++ct) {
      const floatx4 t = pair_n[ct];
      pair_n[ct] = n0[ct];
      n0[ct] = t;
    }
    pair_add(pairs_done);
    pair_d = d1;
#pragma unroll
    for (int ct = 0; ct < DVT; ++ct) pair_n[ct] = n0[ct];
    pair_add(pairs_done + 1);
  }
  for (; pairs_done < n_pairs; ++pairs_done) {
    pair_load(pairs_done);
    pair_add(pairs_done);
  }
  const bool raw = a.out_den != nullptr;
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    float dsum = den[rs];
    dsum += __shfl_xor(dsum, 16);
    dsum += __shfl_xor(dsum, 32);
    if (!rvalid[rs]) continue;
    const int64_t i = myrow[rs];
    if (raw && lg == 0) a.out_den[bh * a.n + i] = dsum;
    const float dn = fmaxf(dsum, a.eps);
#pragma unroll
    for (int ct = 0; ct < DVT; ++ct) {
      const int c0 = 16 * ct + 4 * lg;
      if (c0 >= a.dv) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int col = c0 + r;
        if (col < a.dv) {
          const float numv = num[rs][ct][r];
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
