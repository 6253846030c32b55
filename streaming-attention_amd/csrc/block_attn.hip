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

template <int DP, int DVT, int RS>
__global__ __launch_bounds__(256) void block_attn_kernel(const BlockArgs a) {
  constexpr int KB = (DP + DVT * 16 > 192) ? 32 : 64;  // keys per LDS stage
  constexpr int LDK = DP + 4;
  constexpr int LDV = DVT * 16 + 4;
  constexpr int TM = 64 * RS;
  __shared__ float Kst[KB * LDK];
  __shared__ float Vst[KB * LDV];
  __shared__ float Wst[KB];
  __shared__ int64_t Jst[KB];

  const int wg = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t bh = wg / a.n_tiles;
  const int t = wg % a.n_tiles;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int64_t r0 = static_cast<int64_t>(t) * TM - a.shift;

  const int64_t qkbase = bh * a.n * a.d;
  const int64_t vbase = bh * a.n * a.dv;

  int64_t rbase[RS], myrow[RS], cs[RS], rsv[RS];
  bool rvalid[RS];
  float qB[RS][DP / 4];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    rbase[rs] = r0 + (wave * RS + rs) * 16;
    myrow[rs] = rbase[rs] + li;
    rvalid[rs] = myrow[rs] >= 0 && myrow[rs] < a.n;
    cs[rs] = chunk_start(myrow[rs], a.chunk, a.shift);
    rsv[rs] = residual_start(myrow[rs], a.mode, a.block);
#pragma unroll
    for (int kk = 0; kk < DP / 4; ++kk) {
      const int dim = 4 * kk + lg;
      qB[rs][kk] = (rvalid[rs] && dim < a.d) ? load_elem(a.q, qkbase + myrow[rs] * a.d + dim, a.dtype) : 0.f;
    }
  }

  floatx4 num[RS][DVT];
  float den[RS];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    den[rs] = 0.f;
#pragma unroll
    for (int ct = 0; ct < DVT; ++ct) num[rs][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  const int64_t row_lo = r0 > 0 ? r0 : 0;
  const int64_t row_hi = (r0 + TM < a.n ? r0 + TM : a.n) - 1;  // inclusive
  if (row_lo > row_hi) return;  // whole tile outside the sequence (uniform)

  // One staged batch of keys: in-tile keys (is_node == false) or node items.
  auto process = [&](bool is_node, int64_t lo, int64_t hi) {
#pragma unroll
    for (int kt = 0; kt < KB / 16; ++kt) {
      bool act[RS];
      const int64_t j0 = Jst[16 * kt];  // first key of the sub-tile (in-tile phase)
#pragma unroll
      for (int rs = 0; rs < RS; ++rs) {
        const int64_t s_lo = rbase[rs], s_hi = rbase[rs] + 15;
        bool on = s_hi >= 0 && s_lo < a.n;
        if (is_node) {
          on = on && s_hi >= lo && s_lo <= hi;
        } else {
          on = on && j0 >= 0 && j0 <= s_hi;
        }
        act[rs] = on;
      }
      bool any = false;
#pragma unroll
      for (int rs = 0; rs < RS; ++rs) any = any || act[rs];
      if (!any) continue;

      float ka[DP / 4];
#pragma unroll
      for (int kk = 0; kk < DP / 4; ++kk) ka[kk] = Kst[(16 * kt + li) * LDK + 4 * kk + lg];

      float P[RS][4];
#pragma unroll
      for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
        for (int r = 0; r < 4; ++r) P[rs][r] = 0.f;
        if (!act[rs]) continue;
        floatx4 x = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < DP / 4; ++kk) x = mfma4(ka[kk], qB[rs][kk], x);
        const int64_t i = myrow[rs];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int kidx = 16 * kt + 4 * lg + r;
          const float xv = x[r] * a.scale;
          float p = 0.f;
          if (rvalid[rs]) {
            if (is_node) {
              const float w = Wst[kidx];
              if (i >= lo && i <= hi && w != 0.f) {
                const float e = expf(a.exp_clamp ? fminf(xv, 80.f) : xv);
                p = (e - taylor_poly(xv, a.degree)) * w;
              }
            } else {
              const int64_t j = Jst[kidx];
              if (j >= 0 && j <= i) {
                const bool inT = j >= cs[rs];
                const bool inR = j >= rsv[rs];
                if (inT || inR) {
                  const float tp = taylor_poly(xv, a.degree);
                  if (inR) {
                    const float e = expf(a.exp_clamp ? fminf(xv, 80.f) : xv);
                    p = inT ? e : e - tp;
                  } else {
                    p = tp;
                  }
                }
              }
            }
          }
          P[rs][r] = p;
          den[rs] += p;
        }
      }
#pragma unroll
      for (int ct = 0; ct < DVT; ++ct) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const float va = Vst[(16 * kt + 4 * lg + s) * LDV + 16 * ct + li];
#pragma unroll
          for (int rs = 0; rs < RS; ++rs)
            if (act[rs]) num[rs][ct] = mfma4(va, P[rs][s], num[rs][ct]);
        }
      }
    }
  };

  // ---- phase A: keys of the tile's own chunk / article block ----
  int64_t kstart = chunk_start(row_lo, a.chunk, a.shift);
  const int64_t rs_lo = residual_start(row_lo, a.mode, a.block);
  if (rs_lo < kstart) kstart = rs_lo;
  if (kstart < 0) kstart = 0;
  const int64_t kend = row_hi + 1;
  for (int64_t kb0 = kstart; kb0 < kend; kb0 += KB) {
    __syncthreads();
    for (int e = tid; e < KB * DP; e += 256) {
      const int r = e / DP, col = e % DP;
      const int64_t j = kb0 + r;
      Kst[r * LDK + col] = (j < kend && col < a.d) ? load_elem(a.k, qkbase + j * a.d + col, a.dtype) : 0.f;
    }
    for (int e = tid; e < KB * DVT * 16; e += 256) {
      const int r = e / (DVT * 16), col = e % (DVT * 16);
      const int64_t j = kb0 + r;
      Vst[r * LDV + col] = (j < kend && col < a.dv) ? load_elem(a.v, vbase + j * a.dv + col, a.dtype) : 0.f;
    }
    if (tid < KB) {
      const int64_t j = kb0 + tid;
      Jst[tid] = j < kend ? j : -1;
      Wst[tid] = 1.f;
    }
    __syncthreads();
    process(false, 0, 0);
  }

  // ---- phase B: coreset nodes visible to some row of the tile ----
  const int p_end = a.tile_ptr[t + 1];
  for (int p = a.tile_ptr[t]; p < p_end; ++p) {
    const int node = a.tile_nodes[p];
    const int32_t* meta = a.node_meta + static_cast<int64_t>(node) * NODE_META;
    const int size = meta[0];
    const int64_t lo = meta[1], hi = meta[2];
    const bool mat = meta[3] != 0;
    const int64_t ibase = (bh * a.n_nodes + node) * a.cap;
    for (int i0 = 0; i0 < size; i0 += KB) {
      __syncthreads();
      if (tid < KB) {
        const int it = i0 + tid;
        Jst[tid] = it < size ? static_cast<int64_t>(a.node_src[ibase + it]) : -1;
        Wst[tid] = it < size ? a.node_w[ibase + it] : 0.f;
      }
      __syncthreads();
      for (int e = tid; e < KB * DP; e += 256) {
        const int r = e / DP, col = e % DP;
        const int64_t src = Jst[r];
        float val = 0.f;
        if (src >= 0 && col < a.d)
          val = mat ? a.rep_k[(bh * a.n_rep + src) * a.d + col] : load_elem(a.k, qkbase + src * a.d + col, a.dtype);
        Kst[r * LDK + col] = val;
      }
      for (int e = tid; e < KB * DVT * 16; e += 256) {
        const int r = e / (DVT * 16), col = e % (DVT * 16);
        const int64_t src = Jst[r];
        float val = 0.f;
        if (src >= 0 && col < a.dv)
          val = mat ? a.rep_v[(bh * a.n_rep + src) * a.dv + col] : load_elem(a.v, vbase + src * a.dv + col, a.dtype);
        Vst[r * LDV + col] = val;
      }
      __syncthreads();
      process(true, lo, hi);
    }
  }

  // ---- epilogue: add the moment partials, normalise, store ----
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    float dsum = den[rs];
    dsum += __shfl_xor(dsum, 16);
    dsum += __shfl_xor(dsum, 32);
    if (!rvalid[rs]) continue;
    const int64_t i = myrow[rs];
    float lowd = 0.f;
    for (int f = 0; f < a.fsplit; ++f) lowd += a.low_den[(bh * a.fsplit + f) * a.low_rows + a.low_off + i];
    const bool raw = a.out_den != nullptr;
    if (raw && lg == 0) a.out_den[bh * a.n + i] = lowd + dsum;
    const float dn = fmaxf(lowd + dsum, a.eps);
#pragma unroll
    for (int ct = 0; ct < DVT; ++ct) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int col = 16 * ct + 4 * lg + r;
        if (col < a.dv) {
          float lown = 0.f;
          for (int f = 0; f < a.fsplit; ++f)
            lown += a.low_num[((bh * a.fsplit + f) * a.low_rows + a.low_off + i) * a.low_ld + col];
          const float numv = num[rs][ct][r] + lown;
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
