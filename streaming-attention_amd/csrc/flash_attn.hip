// Exact causal softmax attention, the FlashAttention-style baseline of the reference's GPU module
// (_flash_causal_kernel, triton_article_attention.py:372-435; triton_flash_causal_attention :580-637):
//   out_i = sum_{j<=i} exp(s q_i.k_j - m_i) v_j / max(sum_{j<=i} exp(s q_i.k_j - m_i), 1e-20)
// with m_i the running row maximum (online softmax) and fp32 accumulation; no N x N score matrix.
//
// Matrix-core layout (as in block_attn_kernel): X^T = K Q^T with A = key rows staged in LDS and B = the
// wave's query rows in registers, pre-multiplied by s log2(e) so the logits come out in base 2; the
// probabilities P^T stay in the accumulator layout and are the B operand of num^T += V^T P^T.  A lane
// holds one query row (li) and, per 16-key subtile, four keys 4 lg + r; its accumulators hold value
// columns 16 ct + 4 lg + r of the same row.  So the batch maximum of a row needs two cross-lane steps
// (lanes li, li + 16, li + 32, li + 48) and the rescale exp2(m_old - m_new) applies to the lane's own
// accumulators.
//
// Products for fp32 inputs are fp32 matrix-core ops: exact products of the inputs (the reference's tf32
// dots round fp32 operands to 10 mantissa bits); 16-bit inputs use the 16-bit matrix cores
// (flash_attn16_kernel below).
#include <type_traits>

#include "common.hpp"

namespace sta {

struct FlashArgs {
  const void* q;
  const void* k;
  const void* v;
  int dtype;
  int64_t n;
  int d;
  int dv;
  int ldqk;      // row stride (elements) of q and k: a multiple of 4, >= d (columns >= d are ignored)
  int ldv;       // row stride of v: a multiple of 4, >= dv
  float scale2;  // softmax scale times log2(e)
  int n_tiles;   // ceil(n / (64 RS))
  void* out;     // [BH][n][dv], dense
  int out_dtype;
  int vec_out;  // fp32 output, dv % 4 == 0 and 16-byte aligned: 16-byte stores
};

// keys per LDS stage, per-thread staging units of keys and values, and waves per SIMD (the per-wave
// register arrays: queries RS DP/4, accumulators RS DVT 4, logits RS KB/16 4, staging 4 (KPT + VPT))
__host__ __device__ constexpr int flash_kb(int dp, int dvt) { return (dp + dvt * 16 > 192) ? 32 : 64; }
__host__ __device__ constexpr int flash_kpt(int dp, int dvt) { return (flash_kb(dp, dvt) * dp / 4 + 255) / 256; }
__host__ __device__ constexpr int flash_vpt(int dp, int dvt) { return (flash_kb(dp, dvt) * dvt * 4 + 255) / 256; }
__host__ __device__ constexpr int flash_occupancy(int dp, int dvt, int rs) {
  return (rs * dp / 4 + rs * dvt * 4 + rs * (flash_kb(dp, dvt) / 16) * 4 +
          4 * (flash_kpt(dp, dvt) + flash_vpt(dp, dvt))) <= 160
             ? 2
             : 1;
}

// Elements of a 4-element unit starting at column c that lie in [0, width), the rest zero (a select,
// so padding that holds non-finite bits cannot leak in).
__device__ __forceinline__ floatx4 unit_mask(floatx4 f, bool ok, int c, int width) {
  floatx4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = (ok && c + e < width) ? f[e] : 0.f;
  return r;
}

// One workgroup per (head, tile of 64 RS query rows), longest tiles (highest rows) first; wave w owns
// RS strips of 16 rows.  Keys [0, last row of the tile] are staged KB at a time (K row-major, V
// transposed), the next batch's rows loaded into registers while the current one computes.  A wave
// skips batches that lie wholly after its rows and applies the causal mask only on batches that
// straddle them.
template <int DP, int DVT, int RS, int ES>
__global__ __launch_bounds__(256, flash_occupancy(DP, DVT, RS)) void flash_attn_kernel(const FlashArgs a) {
  constexpr int KB = flash_kb(DP, DVT);
  constexpr int NSUB = KB / 16;
  constexpr int LDK = DP + 4;  // = 4 (mod 64) for the 16-byte key reads
  constexpr int DV = DVT * 16;
  constexpr int LDVT = KB + 4;
  constexpr int DQ = DP / 4;  // k-steps of X = K Q^T, dimensions per lane group
  constexpr int TM = 64 * RS;
  __shared__ float Kst[KB * LDK];
  __shared__ float Vt[DV * LDVT];

  const int wg = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t bh = wg / a.n_tiles;
  const int t = a.n_tiles - 1 - (wg - static_cast<int>(bh) * a.n_tiles);
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int n = static_cast<int>(a.n);
  const int r0 = t * TM;
  const int64_t qkbase = bh * a.n * a.ldqk;
  const int64_t vbase = bh * a.n * a.ldv;

  int myrow[RS];
  bool rvalid[RS];
  float qB[RS][DQ];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    myrow[rs] = r0 + (wave * RS + rs) * 16 + li;
    rvalid[rs] = myrow[rs] < n;
    const int64_t qoff = qkbase + static_cast<int64_t>(rvalid[rs] ? myrow[rs] : 0) * a.ldqk;
#pragma unroll
    for (int m = 0; m < DQ / 4; ++m) {
      const int col = DQ * lg + 4 * m;
      const floatx4 raw = unit_to_f4<ES>(load_unit<ES>(a.q, qoff + min(col, a.ldqk - 4)), a.dtype, a.scale2);
      const floatx4 v4 = unit_mask(raw, rvalid[rs], col, a.d);
#pragma unroll
      for (int e = 0; e < 4; ++e) qB[rs][4 * m + e] = v4[e];
    }
  }
  const int wrow_lo = r0 + wave * RS * 16, wrow_hi = wrow_lo + RS * 16 - 1;  // this wave's rows

  floatx4 num[RS][DVT];
  float den[RS], mrow[RS];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    den[rs] = 0.f;
    mrow[rs] = -1e30f;  // finite: exp2(m_old - m_new) is then 0 or 1, never a NaN
#pragma unroll
    for (int ct = 0; ct < DVT; ++ct) num[rs][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  // one staged batch of keys [off, off + KB); DIAG: some key of it follows some row of this wave
  auto process = [&](auto diag_tag, int off) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    floatx4 X[NSUB][RS];
#pragma unroll
    for (int kt = 0; kt < NSUB; ++kt)
#pragma unroll
      for (int rs = 0; rs < RS; ++rs) X[kt][rs] = floatx4{0.f, 0.f, 0.f, 0.f};
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
          for (int rs = 0; rs < RS; ++rs) X[kt][rs] = mfma4(kv[kt][e], qB[rs][4 * m + e], X[kt][rs]);
    }
#pragma unroll
    for (int rs = 0; rs < RS; ++rs) {
      float mx = -__builtin_huge_valf();
#pragma unroll
      for (int kt = 0; kt < NSUB; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if constexpr (DIAG) {
            if (off + 16 * kt + 4 * lg + r > myrow[rs]) X[kt][rs][r] = -__builtin_huge_valf();
          }
          mx = fmaxf(mx, X[kt][rs][r]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mnew = fmaxf(mrow[rs], mx);
      const float alpha = __builtin_amdgcn_exp2f(mrow[rs] - mnew);
      mrow[rs] = mnew;
      den[rs] *= alpha;
#pragma unroll
      for (int ct = 0; ct < DVT; ++ct) num[rs][ct] *= alpha;
#pragma unroll
      for (int kt = 0; kt < NSUB; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(X[kt][rs][r] - mnew);
          X[kt][rs][r] = p;
          den[rs] += p;
        }
    }
#pragma unroll
    for (int kt = 0; kt < NSUB; ++kt)
#pragma unroll
      for (int ct = 0; ct < DVT; ++ct) {
        const floatx4 va = *reinterpret_cast<const floatx4*>(Vt + (16 * ct + li) * LDVT + 16 * kt + 4 * lg);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int rs = 0; rs < RS; ++rs) num[rs][ct] = mfma4(va[s], X[kt][rs][s], num[rs][ct]);
      }
  };

  const int row_hi = (r0 + TM < n ? r0 + TM : n) - 1;  // r0 < n: t < ceil(n / TM)
  const int kend = row_hi + 1;
  const int nb = (kend + KB - 1) / KB;

  // staging registers: this thread's 4-element units of the next batch's key and value rows, raw
  constexpr int KU = DP / 4, VU = DV / 4;
  constexpr int KPT = flash_kpt(DP, DVT), VPT = flash_vpt(DP, DVT);
  uint4 pk[KPT], pv[VPT];
  uint32_t pk_ok = 0, pv_ok = 0;
  auto prefetch = [&](int off) {
    pk_ok = pv_ok = 0;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int e = tid + 256 * i;
      const int r = e / KU, u = e - r * KU;
      const bool ok = e < KB * KU && off + r < kend && 4 * u < a.d;
      pk_ok |= ok ? (1u << i) : 0u;
      const int src = ok ? off + r : 0;
      pk[i] = load_unit<ES>(a.k, qkbase + static_cast<int64_t>(src) * a.ldqk + min(4 * u, a.ldqk - 4));
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int e = tid + 256 * i;
      const int r = e % KB, u = e / KB;  // key-fast: conflict-light transposed writes
      const bool ok = e < KB * VU && off + r < kend && 4 * u < a.dv;
      pv_ok |= ok ? (1u << i) : 0u;
      const int src = ok ? off + r : 0;
      pv[i] = load_unit<ES>(a.v, vbase + static_cast<int64_t>(src) * a.ldv + min(4 * u, a.ldv - 4));
    }
  };
  auto commit = [&]() {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int e = tid + 256 * i;
      if (e < KB * KU) {
        const int r = e / KU, u = e - r * KU;
        *reinterpret_cast<floatx4*>(Kst + r * LDK + 4 * u) =
            unit_mask(unit_to_f4<ES>(pk[i], a.dtype, 1.f), (pk_ok >> i) & 1u, 4 * u, a.d);
      }
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int e = tid + 256 * i;
      if (e < KB * VU) {
        const int r = e % KB, u = e / KB;
        const floatx4 f = unit_mask(unit_to_f4<ES>(pv[i], a.dtype, 1.f), (pv_ok >> i) & 1u, 4 * u, a.dv);
#pragma unroll
        for (int m = 0; m < 4; ++m) Vt[(4 * u + m) * LDVT + r] = f[m];
      }
    }
  };

  prefetch(0);
  for (int b = 0; b < nb; ++b) {
    __syncthreads();  // every wave is done with the staging buffers of the previous batch
    commit();
    __syncthreads();  // staged batch visible
    if (b + 1 < nb) prefetch((b + 1) * KB);
    const int off = b * KB;
    if (off <= wrow_hi) {
      if (off + KB - 1 > wrow_lo)
        process(std::true_type{}, off);
      else
        process(std::false_type{}, off);
    }
  }

  // ---- epilogue: row sums over the four lane groups, normalise, store ----
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    float dsum = den[rs];
    dsum += __shfl_xor(dsum, 16);
    dsum += __shfl_xor(dsum, 32);
    if (!rvalid[rs]) continue;
    const float dn = fmaxf(dsum, 1e-20f);
    const int64_t obase = (bh * a.n + myrow[rs]) * a.dv;
#pragma unroll
    for (int ct = 0; ct < DVT; ++ct) {
      const int c0 = 16 * ct + 4 * lg;
      if (c0 >= a.dv) continue;
      floatx4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = num[rs][ct][r] / dn;
      if (a.vec_out) {
        *reinterpret_cast<floatx4*>(static_cast<float*>(a.out) + obase + c0) = o;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (c0 + r < a.dv) store_elem(a.out, obase + c0 + r, a.out_dtype, o[r]);
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------
// 16-bit inputs (bf16 / fp16): the matrix cores take the inputs as they are.  X^T = K Q^T with
// v_mfma_f32_16x16x32_{bf16,f16} is exact (16-bit products, fp32 sums) and scaled to base-2 logits
// afterwards; num^T += V^T P^T takes the fp32 probabilities as 16-bit hi + lo (P = hi + lo + e,
// |e| <= 2^-17 P for bf16, 2^-21 P for fp16) against the exact values: two products.  Lane layout as
// in the split-product residual kernel: k-step m of lane group lg covers dimensions 32 m + 8 lg + j;
// the V^T rows hold each pair of 16-key subtiles in contraction order (flash_key_pos), so every
// operand is one 16-byte LDS read.
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));

__host__ __device__ constexpr int flash_key_pos(int r) {
  return 32 * (r >> 5) + 8 * ((r >> 2) & 3) + 4 * ((r >> 4) & 1) + (r & 3);
}

template <bool F16>
__device__ __forceinline__ floatx4 mfma16(const uint4& a, const uint4& b, floatx4 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(halfx8, a), __builtin_bit_cast(halfx8, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// two fp32 values as packed 16-bit (bf16: round to nearest even; fp16: round toward zero, so the low
// part x - hi keeps the sign of x) and back
template <bool F16>
__device__ __forceinline__ uint32_t pack16(float a, float b) {
  if constexpr (F16)
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
  else
    return pk_bf16(a, b);
}
template <bool F16>
__device__ __forceinline__ float lo16(uint32_t p) {
  if constexpr (F16)
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(p & 0xffffu)));
  else
    return __uint_as_float(p << 16);
}
template <bool F16>
__device__ __forceinline__ float hi16(uint32_t p) {
  if constexpr (F16)
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(p >> 16)));
  else
    return __uint_as_float(p & 0xffff0000u);
}

// the first `valid` of the 4 16-bit elements of a raw unit (x: elements 0, 1; y: 2, 3), the rest zero
__device__ __forceinline__ uint2 mask16(uint2 u, int valid) {
  const uint32_t m0 = valid >= 2 ? 0xffffffffu : (valid == 1 ? 0x0000ffffu : 0u);
  const uint32_t m1 = valid >= 4 ? 0xffffffffu : (valid == 3 ? 0x0000ffffu : 0u);
  return uint2{u.x & m0, u.y & m1};
}

// two workgroups per compute unit while the accumulators and staging registers fit in 256 VGPRs
__host__ __device__ constexpr int flash16_occupancy(int dp, int dvt) { return dp + 16 * dvt <= 128 ? 2 : 1; }

template <int DP, int DVT, int RS, bool F16>
__global__ __launch_bounds__(256, flash16_occupancy(DP, DVT)) void flash_attn16_kernel(const FlashArgs a) {
  constexpr int KB = 64;  // keys per LDS stage
  constexpr int NSUB = KB / 16;
  constexpr int DPS = DP < 32 ? 32 : DP;  // dimensions in whole 32-element steps
  constexpr int MS = DPS / 32;
  constexpr int LDK = DPS + 8;  // 16-bit elements per key row: 16 (2 j + 1) bytes
  constexpr int DV = DVT * 16;
  constexpr int LDV = KB + 8;
  constexpr int TM = 64 * RS;
  constexpr int KU = DP / 4, VU = DV / 4;
  constexpr int KPT = (KB * KU + 255) / 256, VPT = (KB * VU + 255) / 256;
  __shared__ uint4 kst4[(KB * LDK + 7) / 8];
  __shared__ uint4 vst4[(DV * LDV + 7) / 8];
  uint16_t* const Kst = reinterpret_cast<uint16_t*>(kst4);
  uint16_t* const Vst = reinterpret_cast<uint16_t*>(vst4);

  const int wg = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t bh = wg / a.n_tiles;
  const int t = a.n_tiles - 1 - (wg - static_cast<int>(bh) * a.n_tiles);
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int n = static_cast<int>(a.n);
  const int r0 = t * TM;
  const int64_t qkbase = bh * a.n * a.ldqk;
  const int64_t vbase = bh * a.n * a.ldv;

  // the wave's query rows as B operands (8 dimensions per lane and k-step), columns >= d zero
  int myrow[RS];
  bool rvalid[RS];
  uint4 qB[RS][MS];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    myrow[rs] = r0 + (wave * RS + rs) * 16 + li;
    rvalid[rs] = myrow[rs] < n;
    const int64_t qoff = qkbase + static_cast<int64_t>(rvalid[rs] ? myrow[rs] : 0) * a.ldqk;
#pragma unroll
    for (int m = 0; m < MS; ++m) {
      uint2 h[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int col = 32 * m + 8 * lg + 4 * hh;
        const uint4 raw = load_unit<2>(a.q, qoff + min(col, a.ldqk - 4));
        h[hh] = mask16(uint2{raw.x, raw.y}, rvalid[rs] ? a.d - col : 0);
      }
      qB[rs][m] = uint4{h[0].x, h[0].y, h[1].x, h[1].y};
    }
  }
  const int wrow_lo = r0 + wave * RS * 16, wrow_hi = wrow_lo + RS * 16 - 1;

  floatx4 num[RS][DVT];
  float den[RS], mrow[RS];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    den[rs] = 0.f;
    mrow[rs] = -1e30f;
#pragma unroll
    for (int ct = 0; ct < DVT; ++ct) num[rs][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  auto process = [&](auto diag_tag, int off) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    floatx4 X[NSUB][RS];
#pragma unroll
    for (int kt = 0; kt < NSUB; ++kt)
#pragma unroll
      for (int rs = 0; rs < RS; ++rs) X[kt][rs] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < MS; ++m)
#pragma unroll
      for (int kt = 0; kt < NSUB; ++kt) {
        const uint4 kv = *reinterpret_cast<const uint4*>(Kst + (16 * kt + li) * LDK + 32 * m + 8 * lg);
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) X[kt][rs] = mfma16<F16>(kv, qB[rs][m], X[kt][rs]);
      }
#pragma unroll
    for (int rs = 0; rs < RS; ++rs) {
      float mx = -__builtin_huge_valf();
#pragma unroll
      for (int kt = 0; kt < NSUB; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float y = X[kt][rs][r] * a.scale2;
          if constexpr (DIAG) {
            if (off + 16 * kt + 4 * lg + r > myrow[rs]) y = -__builtin_huge_valf();
          }
          X[kt][rs][r] = y;
          mx = fmaxf(mx, y);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mnew = fmaxf(mrow[rs], mx);
      const float alpha = __builtin_amdgcn_exp2f(mrow[rs] - mnew);
      mrow[rs] = mnew;
      den[rs] *= alpha;
#pragma unroll
      for (int ct = 0; ct < DVT; ++ct) num[rs][ct] *= alpha;
#pragma unroll
      for (int kt = 0; kt < NSUB; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(X[kt][rs][r] - mnew);
          X[kt][rs][r] = p;
          den[rs] += p;
        }
    }
#pragma unroll
    for (int sp = 0; sp < NSUB / 2; ++sp) {
      uint4 ph[RS], pl[RS];
#pragma unroll
      for (int rs = 0; rs < RS; ++rs) {
        uint32_t h[4], l[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const floatx4& P = X[2 * sp + (e >> 1)][rs];
          const float p0 = P[2 * (e & 1)], p1 = P[2 * (e & 1) + 1];
          h[e] = pack16<F16>(p0, p1);
          l[e] = pack16<F16>(p0 - lo16<F16>(h[e]), p1 - hi16<F16>(h[e]));
        }
        ph[rs] = uint4{h[0], h[1], h[2], h[3]};
        pl[rs] = uint4{l[0], l[1], l[2], l[3]};
      }
#pragma unroll
      for (int ct = 0; ct < DVT; ++ct) {
        const uint4 vv = *reinterpret_cast<const uint4*>(Vst + (16 * ct + li) * LDV + 32 * sp + 8 * lg);
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) num[rs][ct] = mfma16<F16>(vv, pl[rs], num[rs][ct]);
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) num[rs][ct] = mfma16<F16>(vv, ph[rs], num[rs][ct]);
      }
    }
  };

  const int row_hi = (r0 + TM < n ? r0 + TM : n) - 1;
  const int kend = row_hi + 1;
  const int nb = (kend + KB - 1) / KB;

  uint2 pk[KPT], pv[VPT];
  uint32_t pk_ok = 0, pv_ok = 0;
  auto prefetch = [&](int off) {
    pk_ok = pv_ok = 0;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int e = tid + 256 * i;
      const int r = e / KU, u = e - r * KU;
      const bool ok = e < KB * KU && off + r < kend && 4 * u < a.d;
      pk_ok |= ok ? (1u << i) : 0u;
      const int src = ok ? off + r : 0;
      const uint4 raw = load_unit<2>(a.k, qkbase + static_cast<int64_t>(src) * a.ldqk + min(4 * u, a.ldqk - 4));
      pk[i] = uint2{raw.x, raw.y};
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int e = tid + 256 * i;
      const int r = e % KB, u = e / KB;
      const bool ok = e < KB * VU && off + r < kend && 4 * u < a.dv;
      pv_ok |= ok ? (1u << i) : 0u;
      const int src = ok ? off + r : 0;
      const uint4 raw = load_unit<2>(a.v, vbase + static_cast<int64_t>(src) * a.ldv + min(4 * u, a.ldv - 4));
      pv[i] = uint2{raw.x, raw.y};
    }
  };
  auto commit = [&]() {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int e = tid + 256 * i;
      if (e < KB * KU) {
        const int r = e / KU, u = e - r * KU;
        const int valid = ((pk_ok >> i) & 1u) ? a.d - 4 * u : 0;
        *reinterpret_cast<uint2*>(Kst + r * LDK + 4 * u) = mask16(pk[i], valid);
      }
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int e = tid + 256 * i;
      if (e < KB * VU) {
        const int r = e % KB, u = e / KB;
        const uint2 w = mask16(pv[i], ((pv_ok >> i) & 1u) ? a.dv - 4 * u : 0);
        const int pos = flash_key_pos(r);
        Vst[(4 * u + 0) * LDV + pos] = static_cast<uint16_t>(w.x & 0xffffu);
        Vst[(4 * u + 1) * LDV + pos] = static_cast<uint16_t>(w.x >> 16);
        Vst[(4 * u + 2) * LDV + pos] = static_cast<uint16_t>(w.y & 0xffffu);
        Vst[(4 * u + 3) * LDV + pos] = static_cast<uint16_t>(w.y >> 16);
      }
    }
  };

  if constexpr (DPS != DP) {  // dimensions [DP, DPS) of the key rows are never written: zero them
    for (int e = tid; e < KB * LDK; e += 256) Kst[e] = 0;
  }
  prefetch(0);
  for (int b = 0; b < nb; ++b) {
    __syncthreads();
    commit();
    __syncthreads();
    if (b + 1 < nb) prefetch((b + 1) * KB);
    const int off = b * KB;
    if (off <= wrow_hi) {
      if (off + KB - 1 > wrow_lo)
        process(std::true_type{}, off);
      else
        process(std::false_type{}, off);
    }
  }

#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    float dsum = den[rs];
    dsum += __shfl_xor(dsum, 16);
    dsum += __shfl_xor(dsum, 32);
    if (!rvalid[rs]) continue;
    const float dn = fmaxf(dsum, 1e-20f);
    const int64_t obase = (bh * a.n + myrow[rs]) * a.dv;
#pragma unroll
    for (int ct = 0; ct < DVT; ++ct) {
      const int c0 = 16 * ct + 4 * lg;
      if (c0 >= a.dv) continue;
      floatx4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = num[rs][ct][r] / dn;
      if (a.vec_out) {
        *reinterpret_cast<floatx4*>(static_cast<float*>(a.out) + obase + c0) = o;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (c0 + r < a.dv) store_elem(a.out, obase + c0 + r, a.out_dtype, o[r]);
      }
    }
  }
}

}  // namespace sta
