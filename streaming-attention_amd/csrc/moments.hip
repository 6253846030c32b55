// K1: exact low-degree Taylor moments  low_num[i] = phi_q(s*q_i) . S_{<c(i)}[:, :dv],
//                                       low_den[i] = phi_q(s*q_i) . S_{<c(i)}[:, dv]
// where S_{<c} = sum over keys before the chunk c(i) containing row i of phi_k(k_j) [v_j, 1].
//
// Reference semantics: low_degree_taylor_causal_sums_stream (fast_article_attention.py:217-259) and
// TaylorMomentSketch.update/query (streaming_taylor_coreset_attention.py:265-296).  The keys of row i's
// own chunk are added by the block kernel (closed-form Taylor polynomial), so the two kernels together
// give sum_{j<=i} exp_{<=t}(s q_i.k_j) [v_j, 1] exactly (in exact arithmetic).
//
// Decomposition: one workgroup per (head, 16-wide value-column group g, feature split fs).  It walks the
// sequence chunk by chunk, keeping its [features-in-split x 16] slice of S in MFMA accumulators for the
// whole sequence (no state ever goes to HBM).  Per chunk:
//   query : out[tok][col] += phi_q(tok)[f] * S[f][col]   (A = generated features, B = accumulators)
//   update: S[f][col]     += phi_k(tok)[f] * V[tok][col] (A = generated features, B = V from LDS)
// The denominator column (the "1" appended to v) is kept by VALU in LDS.  Partial outputs of the 8
// waves are summed in LDS in a fixed order (deterministic), and the feature-split partials are summed
// by the block kernel.
#include "common.hpp"

namespace sta {

struct MomArgs {
  const void* q;
  const void* k;
  const void* v;
  int dtype;
  int64_t n;
  int d;
  int dv;
  float scale;
  int shift;           // chunk c covers rows [c*CH - shift, (c+1)*CH - shift)
  int ngroups;         // ceil(dv / 16)
  int fsplit;          // feature splits
  int feat_per_split;  // multiple of 16
  const uint32_t* fidx;  // [fsplit * feat_per_split] packed (i0 | i1 << 8 | i2 << 16), slot d == 1.0
  const float* fcoef;    // key-side coefficient 1/prod(alpha!), 0 for padding features
  float* low_num;        // [BH][fsplit][n][dv]
  float* low_den;        // [BH][fsplit][n]
};

template <bool DEG3, int NT, int NW, int CH>
__global__ __launch_bounds__(NW * 64) void moments_kernel(const MomArgs a) {
  extern __shared__ float smem[];
  const int LD = a.d + 1;
  const int FP = a.feat_per_split;
  // Layout: [ftab | fcoef | den] persistent, then the chunk region, aliased by the reduction buffer.
  uint32_t* ftab = reinterpret_cast<uint32_t*>(smem);
  float* fcoef = smem + FP;
  float* den_s = smem + 2 * FP;
  float* region = smem + 3 * FP;
  float* Qs = region;              // [CH][LD]
  float* Ks = Qs + CH * LD;        // [CH][LD]
  float* Vs = Ks + CH * LD;        // [CH][16]
  float* red = region;             // [NW][CH][17]  (used after Qs/Ks/Vs are dead)

  const int per_head = a.ngroups * a.fsplit;
  const int wg = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t bh = wg / per_head;
  const int rem = wg % per_head;
  const int g = rem / a.fsplit;
  const int fs = rem % a.fsplit;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int ntile = FP / 16;

  for (int e = tid; e < FP; e += NW * 64) {
    ftab[e] = a.fidx[(int64_t)fs * FP + e];
    fcoef[e] = a.fcoef[(int64_t)fs * FP + e];
    den_s[e] = 0.0f;
  }

  floatx4 st[NT];
#pragma unroll
  for (int kt = 0; kt < NT; ++kt) st[kt] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int64_t qkbase = bh * a.n * a.d;
  const int64_t vbase = bh * a.n * a.dv;
  const int nchunks = static_cast<int>((a.n + a.shift + CH - 1) / CH);
  const int col0 = 16 * g;

  for (int c = 0; c < nchunks; ++c) {
    const int64_t row0 = static_cast<int64_t>(c) * CH - a.shift;
    __syncthreads();  // previous chunk's reduction buffer reads are done
    for (int e = tid; e < CH * LD; e += NW * 64) {
      const int t = e / LD, col = e - t * LD;
      const int64_t row = row0 + t;
      const bool valid = row >= 0 && row < a.n;
      float qv = 0.f, kv = 0.f;
      if (col < a.d) {
        if (valid) {
          qv = load_elem(a.q, qkbase + row * a.d + col, a.dtype) * a.scale;
          kv = load_elem(a.k, qkbase + row * a.d + col, a.dtype);
        }
      } else {
        // slot d carries the constant 1 of the monomial basis; 0 on invalid rows zeroes every feature
        qv = valid ? 1.f : 0.f;
        kv = valid ? 1.f : 0.f;
      }
      Qs[e] = qv;
      Ks[e] = kv;
    }
    for (int e = tid; e < CH * 16; e += NW * 64) {
      const int t = e >> 4, j = e & 15;
      const int64_t row = row0 + t;
      const int col = col0 + j;
      Vs[e] = (row >= 0 && row < a.n && col < a.dv) ? load_elem(a.v, vbase + row * a.dv + col, a.dtype) : 0.f;
    }
    __syncthreads();

    // ---- query with the exclusive state ----
    floatx4 o[CH / 16];
    float dq[CH / 16];
#pragma unroll
    for (int tt = 0; tt < CH / 16; ++tt) {
      o[tt] = floatx4{0.f, 0.f, 0.f, 0.f};
      dq[tt] = 0.f;
    }
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
      const int tile = wave + kt * NW;
      if (tile < ntile) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int f = 16 * tile + 4 * lg + s;
          const uint32_t idx = ftab[f];
          const int i0 = idx & 255, i1 = (idx >> 8) & 255, i2 = (idx >> 16) & 255;
          const float dnf = den_s[f];
#pragma unroll
          for (int tt = 0; tt < CH / 16; ++tt) {
            const float* qr = Qs + (16 * tt + li) * LD;
            float x = qr[i0] * qr[i1];
            if (DEG3) x = x * qr[i2];
            o[tt] = mfma4(x, st[kt][s], o[tt]);
            dq[tt] += x * dnf;
          }
        }
      }
    }

    // ---- update the state with this chunk ----
    float dacc[NT];
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) dacc[kt] = 0.f;
    for (int ks = 0; ks < CH / 4; ++ks) {
      const int tok = 4 * ks + lg;
      const float b = Vs[tok * 16 + li];
      const float* kr = Ks + tok * LD;
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
        const int tile = wave + kt * NW;
        if (tile < ntile) {
          const int f = 16 * tile + li;
          const uint32_t idx = ftab[f];
          const int i0 = idx & 255, i1 = (idx >> 8) & 255, i2 = (idx >> 16) & 255;
          float x = kr[i0] * kr[i1];
          if (DEG3) x = x * kr[i2];
          x = x * fcoef[f];
          st[kt] = mfma4(x, b, st[kt]);
          dacc[kt] += x;
        }
      }
    }
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
      const int tile = wave + kt * NW;
      float dsum = dacc[kt];
      dsum += __shfl_xor(dsum, 16);
      dsum += __shfl_xor(dsum, 32);
      if (tile < ntile && lg == 0) den_s[16 * tile + li] += dsum;
    }
    __syncthreads();  // Qs/Ks/Vs dead; den_s updated

    // ---- deterministic cross-wave reduction of the query partials ----
#pragma unroll
    for (int tt = 0; tt < CH / 16; ++tt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) red[(wave * CH + 16 * tt + 4 * lg + r) * 17 + li] = o[tt][r];
      float dsum = dq[tt];
      dsum += __shfl_xor(dsum, 16);
      dsum += __shfl_xor(dsum, 32);
      if (lg == 0) red[(wave * CH + 16 * tt + li) * 17 + 16] = dsum;
    }
    __syncthreads();
    for (int e = tid; e < CH * 17; e += NW * 64) {
      const int t = e / 17, j = e - t * 17;
      const int64_t row = row0 + t;
      if (row < 0 || row >= a.n) continue;
      float acc = 0.f;
      for (int w = 0; w < NW; ++w) acc += red[(w * CH + t) * 17 + j];
      const int64_t obase = (bh * a.fsplit + fs) * a.n + row;
      if (j < 16) {
        const int col = col0 + j;
        if (col < a.dv) a.low_num[obase * a.dv + col] = acc;
      } else if (g == 0) {
        a.low_den[obase] = acc;
      }
    }
  }
}

// Shared-memory bytes for a launch (must match the carve-up above).
inline size_t moments_smem_bytes(int CH, int NW, int d, int feat_per_split) {
  const size_t region_a = static_cast<size_t>(CH) * (d + 1) * 2 + static_cast<size_t>(CH) * 16;
  const size_t region_b = static_cast<size_t>(NW) * CH * 17;
  const size_t region = region_a > region_b ? region_a : region_b;
  return (3 * static_cast<size_t>(feat_per_split) + region) * sizeof(float);
}

}  // namespace sta
