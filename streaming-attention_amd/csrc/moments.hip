// K1: exact low-degree Taylor moments  low_num[i] = phi_q(s*q_i) . S_{<c(i)}[:, :dv],
//                                       low_den[i] = phi_q(s*q_i) . S_{<c(i)}[:, dv]
// where S_{<c} = sum over keys before the chunk c(i) containing row i of phi_k(k_j) [v_j, 1].
//
// Reference semantics: low_degree_taylor_causal_sums_stream (fast_article_attention.py:217-259) and
// TaylorMomentSketch.update/query (streaming_taylor_coreset_attention.py:265-296).  The keys of row i's
// own chunk are added by the block kernel (closed-form Taylor polynomial), so the two kernels together
// give sum_{j<=i} exp_{<=t}(s q_i.k_j) [v_j, 1] exactly (in exact arithmetic).
//
// Feature layout.  The monomials are grouped in quads x[i0] x[b+s] x[i2] x[i3], s = 0..3, b a multiple of
// 4 (x[d] = 1 lowers the degree; see feature_tiles in _plan.py), 4 quads per tile of 16 features.  NX:
// the number of factors besides x[i0] and x[b+s] the instantiation multiplies in (0: degree <= 2,
// 1: degree 3, ..., 6: degree 8; a quad is one 32-bit word of 8-bit indices i0 | b | i2 | i3, and a
// second word i4 | i5 | i6 | i7 when NX >= 3).  The
// tiles are split over `fsplit` workgroups and over the 4 waves of a workgroup, every wave holding
// exactly NT tiles (the host pads with zero tiles, so the loops are branch-free and fully unrolled).
// A workgroup also owns one 32-wide group of value columns (csplit = ceil(dv/32) per feature split).
// Each wave keeps its [NT x 16 features] x [32 columns] slice of S in MFMA accumulators for the whole
// sequence (no state ever goes to HBM) and walks the sequence in chunks of 32 tokens:
//   query : out[tok][col] += phi_q(tok)[f] S[f][col]. A (16 tok x 4 f): lane (li, lg) holds token li,
//           features of quad lg -- one 16-byte LDS read of the row-major queries gives all four
//           x[b+s], one more read x[i0].  B = the accumulator itself (see common.hpp).
//   update: S[f][col] += phi_k(tok)[f] V[tok][col].   A (16 f x 4 tok): lane (li, lg) holds feature li
//           and, at step ks, token tok(lg, ks) = 4 lg + (ks & 3) + 16 (ks >> 2); B: V[tok(lg, ks)][col]
//           with the same token mapping.  With keys and values stored token-contiguous, two 16-byte
//           reads (token blocks lg and lg + 4) give a lane its 8 steps.  A tile's quads share b and take
//           4 consecutive i0 (feature_tiles), so the 16 lanes of a key read touch 4 rows x 4 token
//           blocks; with blocks lg and lg + 4 (rather than 2 lg and 2 lg + 1) these reads and the
//           transposed staging writes run without LDS bank conflicts (measured).
// Every generated feature value feeds two MFMAs (two 16-column tiles).  The denominator column (the
// "1" appended to v) is kept by VALU per feature, in registers.  The 4 waves' query partials are
// summed in LDS in a fixed order (deterministic) and stored per feature split; the block kernel adds
// the splits.
//
// Pipeline.  Two chunk buffers and two partial buffers in LDS, one barrier per chunk.  Iteration c:
// query chunk c from buffer c&1; write c's partials; stage chunk c+1 (in registers since iteration
// c-1) into the other buffer; issue the (unconditional, clamped) 16-byte loads of chunk c+2 into the
// same registers, so they have a whole iteration to land; reduce and store chunk c-1's partials;
// update the state with chunk c; barrier.  A dependent MFMA waits ~3 issue slots for its accumulator, so both
// phases keep >= 8 independent accumulator chains in flight: the query alternates two accumulator sets
// by tile, the update walks token steps outermost over all NT tiles.  Operands of the next step are
// read while the current step's MFMAs issue.  For NT <= 5 two workgroups share a compute unit (two
// waves per SIMD), so one wave's VALU/LDS work runs under the other's matrix-core work.
//
// LDS layouts (fp32) per chunk buffer:
//   Qs [32][LDQ]   row-major scaled queries; column d = 1 (0 on rows outside the sequence), columns
//                  d+1..d+3 = 0; LDQ = 68 (d <= 64) or 132, = 4 (mod 64): the 16 rows of a 16-byte
//                  read land in distinct bank quads.
//   Kt [KR][36]    transposed keys (row = dimension), row d = constant, rows d+1..d+3 = 0.
//   Vt [32][36]    transposed values of the workgroup's 32 columns.
// Partials: red [4 waves][33][32]: column-major [column][token], column 32 = denominator, token groups
//           of 4 permuted per column (red_off).
// Running denominators: den [4 waves][NT tiles x 16 features].
#pragma once
#include "common.hpp"

namespace sta {

constexpr int MOM_C = 32;    // tokens per chunk
constexpr int MOM_LDT = 36;  // token stride of the transposed Kt / Vt rows
constexpr int MOM_LDR = 32;  // token stride of a partial column
static_assert(MOM_C <= MOM_LDT, "the bf16 value planes [2][CG][MOM_C] fit in the fp32 rows [CG][MOM_LDT]");

// bf16 offset of (column c, token t) in a value plane of the split-product update (see mom_store).
__host__ __device__ constexpr int vps_off(int c, int t) {
  return c * MOM_C + 8 * (((t >> 2) & 3) ^ ((c >> 1) & 3)) + (t & 3) + 4 * (t >> 4);
}

// Offset of token t of partial column col.  The 4-token groups of a column are permuted by
// (col / 2) mod 8, so the 16 columns a 16-byte access touches at one token group fall on 16 distinct
// bank quads (with the plain stride of 32 floats they would fall on two).
__device__ __forceinline__ int red_off(int col, int t) {
  return col * MOM_LDR + 4 * ((t >> 2) ^ ((col >> 1) & 7)) + (t & 3);
}
constexpr int MOM_WAVES = 4;
constexpr int MOM_THREADS = 64 * MOM_WAVES;
// Guard rows before and after the sequence in the partial outputs: every chunk's rows have a valid
// address, so the partial stores are unconditional (conditional stores would make the compiler's
// vmcnt accounting wait for them before the next chunk's prefetched loads).
constexpr int MOM_GUARD = 32;

struct MomArgs {
  const void* q;
  const void* k;
  const void* v;
  int dtype;
  int64_t n;
  int d;
  int dv;
  float scale;
  int shift;              // chunk c covers rows [c*32 - shift, (c+1)*32 - shift)
  int fsplit;             // feature splits (workgroups per head and column group)
  int mixed;              // 1: feature splits fs >= fsplit / 2 hold one tile less per wave (see moments_kernel)
  int csplit;             // 32-column groups
  const uint32_t* quads;  // [fsplit][4 waves][NT tiles][4][mom_quad_words(NX)] packed (i0 | b << 8 | i2 << 16 | i3 << 24,
                          // then i4 | i5 << 8 | i6 << 16 | i7 << 24)
  const float* fcoef;     // [fsplit][4 waves][NT tiles][16] key-side coefficient, 0 for padding
  float* low_num;         // [BH][fsplit][n + 2*MOM_GUARD][ldo], row r at r + MOM_GUARD
  float* low_den;         // [BH][fsplit][n + 2*MOM_GUARD]
  int ldo;                // low_num row stride: 32 * csplit
  int ldv;                // row stride of v (elements): a multiple of 32, >= dv
  int esize;              // bytes per input element (4 or 2)
  int ldk;                // row stride of q and k (elements): d, or the padded key width with windows
  // Dimension windows (keys wider than the staged rows): feature split fs stages the d = 128 "virtual"
  // dimensions 32 b + j (b < 4, j < 32) from the row's dimension win[4 fs + b] + j, and its feature
  // table indexes those virtual dimensions.  nullptr: virtual dimension = row dimension.
  const int32_t* win;
  // moment_accumulate_kernel only: persistent state in the reference's feature order
  int64_t head_rows;      // rows between consecutive heads of k / v (>= n)
  const int32_t* rowmap;  // [fsplit][4 waves][NT tiles][16] state row of each feature slot, -1 for padding
  float* state_num;       // [BH][n_feat][ldo]
  float* state_den;       // [BH][n_feat]
  int n_feat;
};

// 32-bit words per feature quad: i0, b and two extra factors in the first, four more in the second
__host__ __device__ constexpr int mom_quad_words(int nx) { return nx >= 3 ? 2 : 1; }
// Extra factor e (0 .. 5) of a quad from its words.
__device__ __forceinline__ int quad_factor(uint32_t w0, uint32_t w1, int e) {
  return static_cast<int>(((e < 2 ? w0 : w1) >> (e < 2 ? 16 + 8 * e : 8 * (e - 2))) & 255u);
}

__host__ __device__ constexpr int mom_ldq(bool dbig) { return dbig ? 132 : 68; }
__host__ __device__ constexpr int mom_krows(bool dbig) { return dbig ? 132 : 68; }
// cg: value columns per workgroup (32, or 64 for the 64-column kernels)
__host__ __device__ constexpr int mom_buf_floats(bool dbig, int cg = 32) {
  return MOM_C * mom_ldq(dbig) + mom_krows(dbig) * MOM_LDT + cg * MOM_LDT;
}
__host__ __device__ constexpr int mom_red_floats(int cg = 32) { return MOM_WAVES * (cg + 1) * MOM_LDR; }
// Shared-memory floats of a launch (must match the carve-up in moments_kernel).
__host__ __device__ constexpr int mom_smem_floats(bool dbig, int nt, int cg = 32) {
  return 2 * mom_buf_floats(dbig, cg) + 2 * mom_red_floats(cg) + MOM_WAVES * nt * 16 + 8;
}
// Workgroups per compute unit an instantiation is built for (registers <= 256 and LDS <= 80 KiB for 2;
// the 64-column kernels need 124 KiB of LDS; degree >= 5 needs the registers of one).
__host__ __device__ constexpr int mom_wg_per_cu(int nt, bool dbig, int cg = 32, int nx = 0) {
  return (nt <= 5 && !dbig && cg == 32 && nx <= 2) ? 2 : 1;
}

// Chunk staging in registers: 16-byte units (4 fp32 or 8 bf16/fp16 elements).  The host guarantees
// ldq == d with d a multiple of the unit and ldv a multiple of 32, so units never straddle the constant
// column.  Every thread's slot geometry is fixed for the whole sequence (MomSlots); per chunk only the
// row changes.  Loads are unconditional (rows clamped into the sequence), so none of them waits on
// another; rows outside the sequence are zeroed when the units are written to LDS, and unused slots
// write to a dummy LDS slot, so the staging has no branches.
template <bool DBIG, int CG>
struct MomStage {
  static constexpr int QV = MOM_C * (DBIG ? 128 : 64) * 4 / 16 / MOM_THREADS;  // 2 or 4 (fp32 rows)
  static constexpr int VV = MOM_C * CG * 4 / 16 / MOM_THREADS;                 // 1 or 2 (fp32 rows)
  uint4 q[QV];
  uint4 k[QV];
  uint4 v[VV];
};

template <bool DBIG, int CG>
struct MomSlots {
  static constexpr int QV = MomStage<DBIG, CG>::QV;
  static constexpr int VV = MomStage<DBIG, CG>::VV;
  int q_tok[QV];    // token of q slot j (row-major slots; clamped to the chunk)
  uint32_t q_off[QV];  // byte offset of the unit within its row
  int q_lds[QV];    // float offset of the unit in Qs, or the dummy slot
  bool q_use[QV];
  uint32_t k_off[QV];  // token = tid & 31 (token-fast slots)
  int k_dim[QV];    // first dimension of the unit, or -1 when unused
  uint32_t v_off[VV];  // byte offset of the unit within its v row
  int v_col[VV];       // first column (within the workgroup's CG) of the unit, or -1 when unused
};

// Byte offset within a q / k row of the 16-byte unit that holds virtual dimensions [u epu, (u + 1) epu):
// the identity without windows, else dimension win[b] + j for virtual dimension 32 b + j.
// Window entries are clamped to [0, ldk - 32], so every staged unit lies in the row whatever the table
// holds.
template <int ES>
__device__ __forceinline__ uint32_t unit_offset(int u, const int32_t* win, int ldk) {
  constexpr int epu = 16 / ES;
  if (!win) return static_cast<uint32_t>(u * 16);
  const int vd = u * epu;
  const int first = min(max(win[vd >> 5], 0), ldk - 32);
  return static_cast<uint32_t>((first + (vd & 31)) * ES);
}

// win: this workgroup's 4 window entries (MomArgs::win + 4 fs), or nullptr.
template <bool DBIG, int ES, int CG>
__device__ __forceinline__ MomSlots<DBIG, CG> mom_slots(const MomArgs& a, int col0, int dummy,
                                                       const int32_t* win = nullptr) {
  constexpr int LDQ = mom_ldq(DBIG);
  MomSlots<DBIG, CG> sl;
  const int tid = threadIdx.x;
  constexpr int epu = 16 / ES;
  const int uq = a.d / epu;  // units per staged q/k row
#pragma unroll
  for (int j = 0; j < MomStage<DBIG, CG>::QV; ++j) {
    const int e = tid + MOM_THREADS * j;
    const int t = e / uq, u = e - t * uq;
    sl.q_use[j] = t < MOM_C;
    sl.q_tok[j] = min(t, MOM_C - 1);
    sl.q_off[j] = unit_offset<ES>(u, win, a.ldk);
    sl.q_lds[j] = t < MOM_C ? t * LDQ + u * epu : dummy;
    const int uk = e >> 5;
    sl.k_off[j] = unit_offset<ES>(min(uk, uq - 1), win, a.ldk);
    sl.k_dim[j] = uk < uq ? uk * epu : -1;
  }
#pragma unroll
  for (int j = 0; j < MomStage<DBIG, CG>::VV; ++j) {
    const int uv = (tid >> 5) + (MOM_THREADS / 32) * j;  // unit of the workgroup's CG columns
    sl.v_off[j] = static_cast<uint32_t>((col0 + min(uv * epu, CG - epu)) * ES);
    sl.v_col[j] = uv * epu < CG ? uv * epu : -1;
  }
  return sl;
}

__device__ __forceinline__ int clamp_row(int row, int n) { return min(max(row, 0), n - 1); }

// Whether every staging slot of every thread is in use (mom_slots): fp32 rows of exactly 64 (or 128)
// elements; the value units always fill the CG columns for fp32.
__host__ __device__ constexpr bool mom_full_slots(bool dbig, int es, int d) { return es == 4 && d == (dbig ? 128 : 64); }

// MASK = false: the caller guarantees every row of the chunk lies in the sequence (no clamping).
template <bool DBIG, int ES, int CG, bool MASK = true>
__device__ __forceinline__ void mom_load(MomStage<DBIG, CG>& st, const MomSlots<DBIG, CG>& sl, const MomArgs& a,
                                         const char* qh, const char* kh, const char* vh, int row0) {
  const uint32_t qrow = static_cast<uint32_t>(a.ldk * ES), vrow = static_cast<uint32_t>(a.ldv * ES);
  const int ktok = row0 + (threadIdx.x & (MOM_C - 1));
  const uint32_t krow = static_cast<uint32_t>(MASK ? clamp_row(ktok, a.n) : ktok);
#pragma unroll
  for (int j = 0; j < MomStage<DBIG, CG>::QV; ++j) {
    const uint32_t r = static_cast<uint32_t>(MASK ? clamp_row(row0 + sl.q_tok[j], a.n) : row0 + sl.q_tok[j]);
    st.q[j] = *reinterpret_cast<const uint4*>(qh + r * qrow + sl.q_off[j]);
    st.k[j] = *reinterpret_cast<const uint4*>(kh + krow * qrow + sl.k_off[j]);
  }
#pragma unroll
  for (int j = 0; j < MomStage<DBIG, CG>::VV; ++j)
    st.v[j] = *reinterpret_cast<const uint4*>(vh + krow * vrow + sl.v_off[j]);
}

// The 16-byte unit u as 4 (fp32, ES = 4) or 8 (bf16 / fp16, ES = 2) floats; only f[0..16/ES) are
// meaningful.
template <int ES>
__device__ __forceinline__ void unit_floats(const uint4& u, int dtype, float (&f)[8]) {
  if constexpr (ES == 4) {
    f[0] = __uint_as_float(u.x);
    f[1] = __uint_as_float(u.y);
    f[2] = __uint_as_float(u.z);
    f[3] = __uint_as_float(u.w);
    f[4] = f[5] = f[6] = f[7] = 0.f;
  } else if (dtype == BF16) {
    f[0] = __uint_as_float(u.x << 16);
    f[1] = __uint_as_float(u.x & 0xffff0000u);
    f[2] = __uint_as_float(u.y << 16);
    f[3] = __uint_as_float(u.y & 0xffff0000u);
    f[4] = __uint_as_float(u.z << 16);
    f[5] = __uint_as_float(u.z & 0xffff0000u);
    f[6] = __uint_as_float(u.w << 16);
    f[7] = __uint_as_float(u.w & 0xffff0000u);
  } else {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int m = 0; m < 8; ++m)
      f[m] = static_cast<float>(
          __builtin_bit_cast(_Float16, static_cast<uint16_t>((m & 1) ? (w[m >> 1] >> 16) : (w[m >> 1] & 0xffffu))));
  }
}

// SPLIT: the values go to LDS as bf16 hi / lo planes (split once per workgroup for the split-product
// update) in place of the fp32 Vt rows; they fit in Vt's space.  Plane layout (vps_off): column c is a
// row of 32 bf16 in 4 blocks of 8; block g ^ ((c >> 1) & 3) holds the tokens 4 g + (j & 3) + 16 (j >> 2),
// j = 0..7, in the token order of the update's contraction, so a lane's 8 tokens are one 16-byte read.
// The XOR spreads the update's reads (16 columns x 4 blocks) over all banks, and the staging writes
// (32 tokens of one column per half-wave) stay within one row: both measured free of bank conflicts.
// FULL: every staging slot of the thread is in use (mom_full_slots), so no slot is routed to the dummy.
// MASK = false: every row of the chunk lies in the sequence (no zeroing of outside rows).
template <bool DBIG, int ES, int CG, bool SPLIT = false, bool FULL = false, bool MASK = true>
__device__ __forceinline__ void mom_store(const MomStage<DBIG, CG>& st, const MomSlots<DBIG, CG>& sl, const MomArgs& a,
                                          float* buf, int dummy_rel, int row0) {
  constexpr int LDQ = mom_ldq(DBIG);
  float* Qs = buf;
  float* Kt = Qs + MOM_C * LDQ;
  float* Vt = Kt + mom_krows(DBIG) * MOM_LDT;
  float* dmy = buf + dummy_rel;  // 8 floats nobody reads
  const int tid = threadIdx.x;
  const int tok = tid & (MOM_C - 1);
  const bool tok_ok = !MASK || (row0 + tok >= 0 && row0 + tok < a.n);
  const float kok = tok_ok ? 1.f : 0.f;
  constexpr bool wide = ES == 2;  // 8 elements per unit
#pragma unroll
  for (int j = 0; j < MomStage<DBIG, CG>::QV; ++j) {
    const int row = row0 + sl.q_tok[j];
    const float sc = ((FULL || sl.q_use[j]) && (!MASK || (row >= 0 && row < a.n))) ? a.scale : 0.f;
    float f[8];
    unit_floats<ES>(st.q[j], a.dtype, f);
    float* qd = (FULL || sl.q_use[j]) ? Qs + sl.q_lds[j] : dmy;
    *reinterpret_cast<floatx4*>(qd) = floatx4{f[0], f[1], f[2], f[3]} * sc;
    if constexpr (wide) *reinterpret_cast<floatx4*>(qd + 4) = floatx4{f[4], f[5], f[6], f[7]} * sc;
    unit_floats<ES>(st.k[j], a.dtype, f);
    const int kd = sl.k_dim[j];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      if (m < 4 || wide) {
        float* p = (FULL || kd >= 0) ? Kt + (kd + m) * MOM_LDT + tok : dmy + m;
        *p = f[m] * kok;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < MomStage<DBIG, CG>::VV; ++j) {
    float f[8];
    unit_floats<ES>(st.v[j], a.dtype, f);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      if (m < 4 || wide) {
        if constexpr (SPLIT) {
          __bf16* vh = reinterpret_cast<__bf16*>(Vt);
          const float x = f[m] * kok;
          const __bf16 h = static_cast<__bf16>(x);
          const __bf16 l = static_cast<__bf16>(x - static_cast<float>(h));
          if (FULL || sl.v_col[j] >= 0) {
            vh[vps_off(sl.v_col[j] + m, tok)] = h;
            vh[CG * MOM_C + vps_off(sl.v_col[j] + m, tok)] = l;
          } else {
            reinterpret_cast<__bf16*>(dmy + m)[0] = h;
            reinterpret_cast<__bf16*>(dmy + m)[1] = l;
          }
        } else {
          float* p = (FULL || sl.v_col[j] >= 0) ? Vt + (sl.v_col[j] + m) * MOM_LDT + tok : dmy + m;
          *p = f[m] * kok;
        }
      }
    }
  }
  // the constant factor: 1 on rows inside the sequence, 0 outside (zeroes every feature of the row)
  if (tid < MOM_C) {
    Qs[tid * LDQ + a.d] = kok;
    Kt[a.d * MOM_LDT + tid] = kok;
  }
}

// Fixed-order sum of the 4 waves' partials of the chunk starting at row0, stored unconditionally:
// low_num rows of the workgroup's CG columns and, for the workgroup that keeps the denominator column
// (DEN), the low_den rows.  A wave's partials are CG + 1 columns of MOM_LDR tokens (column CG: the
// denominator).
template <bool DEN, int CG>
__device__ __forceinline__ void mom_reduce_store(const MomArgs& a, const float* red, int64_t obase, int64_t row0,
                                                 int col0) {
  constexpr int WS = (CG + 1) * MOM_LDR;  // one wave's partials
  const int tid = threadIdx.x;
  const int t4 = 4 * (tid >> 5);  // 8 groups of 4 tokens
#pragma unroll
  for (int h = 0; h < CG / 32; ++h) {
    const int col = (tid & 31) + 32 * h;
    floatx4 acc = *reinterpret_cast<const floatx4*>(red + red_off(col, t4));
#pragma unroll
    for (int ww = 1; ww < MOM_WAVES; ++ww) acc += *reinterpret_cast<const floatx4*>(red + ww * WS + red_off(col, t4));
    float* dst = a.low_num + (obase + row0 + t4) * a.ldo + col0 + col;
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[r * a.ldo] = acc[r];
  }
  if constexpr (DEN) {
    const int tok = tid & (MOM_C - 1);
    float den = red[red_off(CG, tok)];
#pragma unroll
    for (int ww = 1; ww < MOM_WAVES; ++ww) den += red[ww * WS + red_off(CG, tok)];
    a.low_den[obase + row0 + tok] = den;
  }
}

// Per-lane feature offsets of a wave's NT tiles (constant over the sequence).  Query side: columns of
// x[i0], x[b..b+3] and the NX extra factors of quad lg in the row-major queries.  Update side: Kt rows of
// feature li plus the token offset 4 lg (token blocks lg and lg + 4), and the key-side coefficient of
// feature li.
template <int NT, int NX>
struct MomLane {
  static constexpr int NXA = NX > 0 ? NX : 1;
  int qa[NT], qb[NT], qx[NXA][NT];
  int ka[NT], kb[NT], kx[NXA][NT];
  float kcoef[NT];
};

template <int NT, int NX>
__device__ __forceinline__ MomLane<NT, NX> mom_lane(const MomArgs& a, int64_t tile0, int li, int lg) {
  constexpr int QW = mom_quad_words(NX);
  MomLane<NT, NX> m;
#pragma unroll
  for (int kt = 0; kt < NT; ++kt) {
    const uint32_t* qq = a.quads + ((tile0 + kt) * 4 + lg) * QW;
    const uint32_t pq = qq[0], pq1 = QW > 1 ? qq[QW > 1 ? 1 : 0] : 0u;
    m.qa[kt] = static_cast<int>(pq & 255u);
    m.qb[kt] = static_cast<int>((pq >> 8) & 255u);
#pragma unroll
    for (int e = 0; e < NX; ++e) m.qx[e][kt] = quad_factor(pq, pq1, e);
    const uint32_t* kq = a.quads + ((tile0 + kt) * 4 + (li >> 2)) * QW;
    const uint32_t pk = kq[0], pk1 = QW > 1 ? kq[QW > 1 ? 1 : 0] : 0u;
    m.ka[kt] = static_cast<int>(pk & 255u) * MOM_LDT + 4 * lg;
    m.kb[kt] = (static_cast<int>((pk >> 8) & 255u) + (li & 3)) * MOM_LDT + 4 * lg;
#pragma unroll
    for (int e = 0; e < NX; ++e) m.kx[e][kt] = quad_factor(pk, pk1, e) * MOM_LDT + 4 * lg;
    m.kcoef[kt] = a.fcoef[(tile0 + kt) * 16 + li];
  }
  return m;
}

// State update with one staged chunk: S[f][col] += phi_k(tok)[f] V[tok][col] for the wave's NT tiles and
// its 32 columns, den_s[f] += phi_k(tok)[f].  Token steps outermost over all tiles (2 NT independent
// chains), in two halves of 4 steps; the keys of the second half are read while the first half's
// MFMAs issue.  `mid()` runs after the first key reads are issued (work to hide under them).
template <int NT, int CT, int NX, bool DEN, class Mid>
__device__ __forceinline__ void mom_update(floatx4 (&st)[NT][CT], float* den_s, const float* Kt, const float* Vt,
                                           const MomLane<NT, NX>& m, int li, int lg, Mid mid) {
  floatx4 vv[2][CT];  // values of tokens 4 lg + 0..3 and 16 + 4 lg + 0..3
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    vv[0][ct] = *reinterpret_cast<const floatx4*>(Vt + (16 * ct + li) * MOM_LDT + 4 * lg);
    vv[1][ct] = *reinterpret_cast<const floatx4*>(Vt + (16 * ct + li) * MOM_LDT + 4 * lg + 16);
  }
  constexpr int NXA = MomLane<NT, NX>::NXA;
  floatx4 fa[2][NT], fb[2][NT], fx[2][NXA][NT];
  auto uload = [&](int h) {
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
      fa[h][kt] = *reinterpret_cast<const floatx4*>(Kt + m.ka[kt] + 16 * h);
      fb[h][kt] = *reinterpret_cast<const floatx4*>(Kt + m.kb[kt] + 16 * h);
#pragma unroll
      for (int x = 0; x < NX; ++x) fx[h][x][kt] = *reinterpret_cast<const floatx4*>(Kt + m.kx[x][kt] + 16 * h);
    }
  };
  uload(0);
  mid();
  __builtin_amdgcn_sched_barrier(0);
  float dacc[NT];
#pragma unroll
  for (int kt = 0; kt < NT; ++kt) dacc[kt] = 0.f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (h == 0) uload(1);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
        float x = fa[h][kt][e] * fb[h][kt][e];
#pragma unroll
        for (int f = 0; f < NX; ++f) x *= fx[h][f][kt][e];
        x *= m.kcoef[kt];
        if constexpr (DEN) dacc[kt] += x;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) st[kt][ct] = mfma4(x, vv[h][ct][e], st[kt][ct]);
      }
      if constexpr (DEN) {
#pragma unroll
        for (int kt = 0; kt < NT; ++kt) pin(dacc[kt]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if constexpr (DEN) {
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
      float s = dacc[kt];
      s += __shfl_xor(s, 16);
      s += __shfl_xor(s, 32);
      if (lg == 0) den_s[16 * kt + li] += s;
    }
  }
}

// Split-bf16 form of mom_update: one 16x16x32 bf16 product covers the 32 tokens of the chunk.  A (16 f x
// 32 tok): lane (li, lg) holds feature li of the tile for tokens tok(lg, j), j = 0..7 (the fp32 update's
// A values of its 8 steps); B: V[tok(lg, j)][col].  The feature values and the values are split into
// bf16 hi + lo, and S += A_hi B_lo + A_lo B_hi + A_hi B_hi (terms outermost, so the 2 NT accumulators
// are independent chains).  The denominator sums the fp32 feature values as before.
// NX = 0 (degree <= 2): the state holds the plain monomial sums and the coefficient table holds one
// coefficient per tile (repeated over its 16 slots), which mom_query_split applies to the query
// side's first factor: 1 multiply per tile and token instead of one per feature and token.  The
// planner makes every degree <= 2 tile uniform (tile_coefficients in _plan.py): the diagonal tiles
// x[4k + r] x[4k + s] take 1/2 on all 16 slots (the slot pairs (r, s), (s, r) add up to the
// off-diagonal monomial), padding slots are zero-valued monomials.
// KCOEF: apply the key-side coefficient at every degree (the decode state keeps the reference's
// coefficient-weighted moments; the prefill scan applies degree <= 2 coefficients on the query side).
template <int NT, int CT, int NX, bool DEN, class Mid, bool KCOEF = false>
__device__ __forceinline__ void mom_update_split(floatx4 (&st)[NT][CT], float* den_s, const float* Kt,
                                                 const float* Vt, const MomLane<NT, NX>& m, int li, int lg,
                                                 Mid mid) {
  constexpr int NXA = MomLane<NT, NX>::NXA;
  floatx4 fa[2][NT], fb[2][NT], fx[2][NXA][NT];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
      fa[h][kt] = *reinterpret_cast<const floatx4*>(Kt + m.ka[kt] + 16 * h);
      fb[h][kt] = *reinterpret_cast<const floatx4*>(Kt + m.kb[kt] + 16 * h);
#pragma unroll
      for (int x = 0; x < NX; ++x) fx[h][x][kt] = *reinterpret_cast<const floatx4*>(Kt + m.kx[x][kt] + 16 * h);
    }
  // the staged bf16 planes (mom_store<..., true>, vps_off): column 16 ct + li, tokens tok(lg, 0..7)
  constexpr int CG = 16 * CT;
  const __bf16* vplane = reinterpret_cast<const __bf16*>(Vt);
  bf16x8 vh[CT], vl[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    vh[ct] = *reinterpret_cast<const bf16x8*>(vplane + vps_off(16 * ct + li, 4 * lg));
    vl[ct] = *reinterpret_cast<const bf16x8*>(vplane + CG * MOM_C + vps_off(16 * ct + li, 4 * lg));
  }
  mid();  // not fenced: the scheduler interleaves the reduction with the first tiles (~1 % of K1 on 32 x 64K)
  // tile kt's products are issued as soon as its operands are split, so the next tile's VALU work runs
  // while the matrix cores work through them
#pragma unroll
  for (int kt = 0; kt < NT; ++kt) {
    float x[8];
    float dacc = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float y = fa[j >> 2][kt][j & 3] * fb[j >> 2][kt][j & 3];
#pragma unroll
      for (int f = 0; f < NX; ++f) y *= fx[j >> 2][f][kt][j & 3];
      if (NX >= 1 || KCOEF) y *= m.kcoef[kt];  // NX = 0: the tile's coefficient is applied by the query
      x[j] = y;
      if constexpr (DEN) dacc += y;
    }
    bf16x8 ah, al;
    split_bf16(x, ah, al);
    if constexpr (DEN) {
      dacc += __shfl_xor(dacc, 16);
      dacc += __shfl_xor(dacc, 32);
      if (lg == 0) den_s[16 * kt + li] += dacc;
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) st[kt][ct] = mfma_bf16(ah, vl[ct], st[kt][ct]);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) st[kt][ct] = mfma_bf16(al, vh[ct], st[kt][ct]);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) st[kt][ct] = mfma_bf16(ah, vh[ct], st[kt][ct]);
  }
}

// Split-bf16 form of the query: out[tok][col] += sum_f phi_q(tok)[f] S[f][col] over the wave's tiles,
// two tiles per 16x16x32 bf16 product.  For tile pair (t0, t1) the contraction index 8 lg + j is
// feature 4 lg + j of t0 (j < 4) or 4 lg + j - 4 of t1: lane (li, lg) supplies phi_q of token li for
// quad lg of both tiles (A) and its own accumulator elements S[t0|t1][4 lg + r][col li] (B), so the
// state is used in place, split into bf16 hi + lo once per chunk.  An odd last tile pairs with zeros.
// o[tt][ct] accumulates rows 16 tt + 4 lg + r, column 16 ct + li; dq the denominator (fp32 VALU, the
// fp32 path's order).
template <int NT, int CT, int NX, bool DEN, int LDQ>
__device__ __forceinline__ void mom_query_split(floatx4 (&o)[2][2][CT], float (&dq)[2], const floatx4 (&st)[NT][CT],
                                                const float* Qs, const float* den_s, const MomLane<NT, NX>& m,
                                                int li, int lg) {
  constexpr int TT = 2;
  constexpr int NP = (NT + 1) / 2;
  const float* qrow = Qs + li * LDQ;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int t0 = 2 * p, t1 = 2 * p + 1;
    const bool has1 = t1 < NT;
    bf16x8 sh[CT], sl[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      float t[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        t[r] = st[t0][ct][r];
        t[4 + r] = has1 ? st[has1 ? t1 : t0][ct][r] : 0.f;
      }
      split_bf16(t, sh[ct], sl[ct]);
    }
    floatx4 dn0, dn1;
    if constexpr (DEN) {
      dn0 = *reinterpret_cast<const floatx4*>(den_s + 16 * t0 + 4 * lg);
      dn1 = has1 ? *reinterpret_cast<const floatx4*>(den_s + 16 * (has1 ? t1 : t0) + 4 * lg) : floatx4{0.f, 0.f, 0.f, 0.f};
    }
    bf16x8 ah[TT], al[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      float x[8];
      {
        const float a0 = (NX == 0) ? qrow[16 * tt * LDQ + m.qa[t0]] * m.kcoef[t0] : qrow[16 * tt * LDQ + m.qa[t0]];
        const floatx4 b0 = *reinterpret_cast<const floatx4*>(qrow + 16 * tt * LDQ + m.qb[t0]);
        float c0[MomLane<NT, NX>::NXA];
#pragma unroll
        for (int f = 0; f < NX; ++f) c0[f] = qrow[16 * tt * LDQ + m.qx[f][t0]];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float y = a0 * b0[s];
#pragma unroll
          for (int f = 0; f < NX; ++f) y *= c0[f];
          x[s] = y;
          if constexpr (DEN) dq[tt] = fmaf(y, dn0[s], dq[tt]);
        }
      }
      if (has1) {
        const int u = has1 ? t1 : t0;
        const float a1 = (NX == 0) ? qrow[16 * tt * LDQ + m.qa[u]] * m.kcoef[u] : qrow[16 * tt * LDQ + m.qa[u]];
        const floatx4 b1 = *reinterpret_cast<const floatx4*>(qrow + 16 * tt * LDQ + m.qb[u]);
        float c1[MomLane<NT, NX>::NXA];
#pragma unroll
        for (int f = 0; f < NX; ++f) c1[f] = qrow[16 * tt * LDQ + m.qx[f][u]];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float y = a1 * b1[s];
#pragma unroll
          for (int f = 0; f < NX; ++f) y *= c1[f];
          x[4 + s] = y;
          if constexpr (DEN) dq[tt] = fmaf(y, dn1[s], dq[tt]);
        }
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) x[4 + s] = 0.f;
      }
      if constexpr (DEN) pin(dq[tt]);
      split_bf16(x, ah[tt], al[tt]);
    }
    floatx4(&oc)[TT][CT] = o[p & 1];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) oc[tt][ct] = mfma_bf16(ah[tt], sl[ct], oc[tt][ct]);
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) oc[tt][ct] = mfma_bf16(al[tt], sh[ct], oc[tt][ct]);
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) oc[tt][ct] = mfma_bf16(ah[tt], sh[ct], oc[tt][ct]);
  }
}

// The kernel body for one workgroup (head bh, feature split fs, column group cs) with NT tiles per wave
// out of the NTS the split table holds per wave.  DEN: this workgroup also keeps the denominator column
// (only column group 0 does; the others would compute bit-identical values).
template <int NT, int NTS, int NX, bool DBIG, int ES, bool DEN, bool SPLIT, int CG, bool FULL>
__device__ __forceinline__ void moments_body(const MomArgs& a, int64_t bh, int fs, int cs) {
  constexpr int LDQ = mom_ldq(DBIG);
  constexpr int BUF = mom_buf_floats(DBIG, CG);
  constexpr int RED = mom_red_floats(CG);
  constexpr int CT = CG / 16;     // 16-column tiles per wave
  constexpr int TT = MOM_C / 16;  // 16-token tiles per chunk (query)
  constexpr int KS = MOM_C / 4;   // update steps per chunk (token tok(lg, ks))
  static_assert(KS == 8, "update token mapping assumes 32-token chunks");
  extern __shared__ float smem[];
  float* red_all = smem + 2 * BUF;
  float* den_all = red_all + 2 * RED;  // [4 waves][NT * 16]
  const int dummy_abs = 2 * BUF + 2 * RED + MOM_WAVES * NT * 16;  // 8 floats, write-only

  const int col0 = CG * cs;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  float* den_s = den_all + w * NT * 16;  // running denominator of every feature of this wave's tiles

  const int64_t tile0 = (static_cast<int64_t>(fs) * MOM_WAVES + w) * NTS;  // NTS: table tiles per wave
  const MomLane<NT, NX> m = mom_lane<NT, NX>(a, tile0, li, lg);

  floatx4 st[NT][CT];
#pragma unroll
  for (int kt = 0; kt < NT; ++kt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) st[kt][ct] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int n = static_cast<int>(a.n);
  const int nchunks = (n + a.shift + MOM_C - 1) / MOM_C;
  const int64_t obase = (bh * a.fsplit + fs) * (a.n + 2 * MOM_GUARD) + MOM_GUARD;
  const int first = -a.shift;
  const char* qh = static_cast<const char*>(a.q) + bh * a.n * a.ldk * ES;
  const char* kh = static_cast<const char*>(a.k) + bh * a.n * a.ldk * ES;
  const char* vh = static_cast<const char*>(a.v) + bh * a.n * a.ldv * ES;
  const MomSlots<DBIG, CG> sl = mom_slots<DBIG, ES, CG>(a, col0, dummy_abs, a.win ? a.win + 4 * fs : nullptr);

  // zero both chunk buffers (their padding rows / columns are never written again) and the denominators
  for (int e = tid; e < 2 * BUF; e += MOM_THREADS) smem[e] = 0.f;
  for (int e = tid; e < MOM_WAVES * NT * 16; e += MOM_THREADS) den_all[e] = 0.f;
  __syncthreads();
  MomStage<DBIG, CG> pre;
  mom_load<DBIG, ES, CG>(pre, sl, a, qh, kh, vh, first);
  mom_store<DBIG, ES, CG, SPLIT, FULL>(pre, sl, a, smem, dummy_abs, first);
  __syncthreads();
  mom_load<DBIG, ES, CG>(pre, sl, a, qh, kh, vh, first + MOM_C);

  for (int c = 0; c < nchunks; ++c) {
    const int cur = c & 1;
    const int row0 = first + c * MOM_C;
    const float* Qs = smem + cur * BUF;
    const float* Kt = Qs + MOM_C * LDQ;
    const float* Vt = Kt + mom_krows(DBIG) * MOM_LDT;

    // ---- query with the state of all previous chunks: two accumulator sets (tile parity), so 8
    //      independent MFMA chains; tile kt+1's operands are read during tile kt ----
    floatx4 o[2][TT][CT];
    float dq[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      dq[tt] = 0.f;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) o[0][tt][ct] = o[1][tt][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    if constexpr (SPLIT) {
      mom_query_split<NT, CT, NX, DEN, LDQ>(o, dq, st, Qs, den_s, m, li, lg);
    } else {
      float x0[2][TT], xe[2][MomLane<NT, NX>::NXA][TT];
      floatx4 x1[2][TT], dn[2];
      const float* qrow = Qs + li * LDQ;
      auto qload = [&](int kt, int buf) {
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
          x0[buf][tt] = qrow[16 * tt * LDQ + m.qa[kt]];
          x1[buf][tt] = *reinterpret_cast<const floatx4*>(qrow + 16 * tt * LDQ + m.qb[kt]);
#pragma unroll
          for (int f = 0; f < NX; ++f) xe[buf][f][tt] = qrow[16 * tt * LDQ + m.qx[f][kt]];
        }
        if constexpr (DEN) dn[buf] = *reinterpret_cast<const floatx4*>(den_s + 16 * kt + 4 * lg);
      };
      qload(0, 0);
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
        const int cb = kt & 1;
        if (kt + 1 < NT) qload(kt + 1, cb ^ 1);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
          for (int tt = 0; tt < TT; ++tt) {
            float x = x0[cb][tt] * x1[cb][tt][s];
#pragma unroll
            for (int f = 0; f < NX; ++f) x *= xe[cb][f][tt];
            if constexpr (DEN) dq[tt] = fmaf(x, dn[cb][s], dq[tt]);
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) o[cb][tt][ct] = mfma4(x, st[kt][ct][s], o[cb][tt][ct]);
          }
        }
        if constexpr (DEN) {
#pragma unroll
          for (int tt = 0; tt < TT; ++tt) pin(dq[tt]);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the one-tile-ahead pipeline shape
      }
    }

    // ---- this wave's query partials -> red[cur] (column-major, 4 tokens per 16-byte write) ----
    {
      float* rw = red_all + cur * RED + w * (CG + 1) * MOM_LDR;
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
          *reinterpret_cast<floatx4*>(rw + red_off(16 * ct + li, 16 * tt + 4 * lg)) = o[0][tt][ct] + o[1][tt][ct];
        if constexpr (DEN) {
          float s = dq[tt];
          s += __shfl_xor(s, 16);
          s += __shfl_xor(s, 32);
          if (lg == 0) rw[red_off(CG, 16 * tt + li)] = s;
        }
      }
    }
    // ---- stage chunk c+1 into the other buffer (loaded a whole iteration earlier), then prefetch chunk
    //      c+2 into the same registers (unconditional, clamped rows) ----
    // (interior chunks, every row inside the sequence, skip the clamping and zeroing: a uniform branch)
    if (c + 1 < nchunks) {
      float* nb = smem + (cur ^ 1) * BUF;
      const int nd = dummy_abs - (cur ^ 1) * BUF;
      if (row0 + MOM_C >= 0 && row0 + 2 * MOM_C <= n)
        mom_store<DBIG, ES, CG, SPLIT, FULL, false>(pre, sl, a, nb, nd, row0 + MOM_C);
      else
        mom_store<DBIG, ES, CG, SPLIT, FULL, true>(pre, sl, a, nb, nd, row0 + MOM_C);
    }
    if (row0 + 2 * MOM_C >= 0 && row0 + 3 * MOM_C <= n)
      mom_load<DBIG, ES, CG, false>(pre, sl, a, qh, kh, vh, row0 + 2 * MOM_C);
    else
      mom_load<DBIG, ES, CG, true>(pre, sl, a, qh, kh, vh, row0 + 2 * MOM_C);
    if constexpr (!SPLIT) __builtin_amdgcn_sched_barrier(0);  // the split update schedules better unfenced

    // ---- update with chunk c; the previous chunk's partials are reduced and stored under the first
    //      key reads ----
    auto mid = [&]() {
      if (c > 0) mom_reduce_store<DEN, CG>(a, red_all + (cur ^ 1) * RED, obase, row0 - MOM_C, col0);
    };
    if constexpr (SPLIT)
      mom_update_split<NT, CT, NX, DEN>(st, den_s, Kt, Vt, m, li, lg, mid);
    else
      mom_update<NT, CT, NX, DEN>(st, den_s, Kt, Vt, m, li, lg, mid);
    __syncthreads();
  }
  mom_reduce_store<DEN, CG>(a, red_all + ((nchunks - 1) & 1) * RED, obase, first + (nchunks - 1) * MOM_C, col0);
}

// Workgroup -> (head, feature split, column group).  Workgroups are dispatched round-robin over the 8
// XCDs and, within an XCD, one per compute unit before a compute unit gets its second one.  When the
// grid divides evenly, the first wave of an XCD's workgroups takes column group 0 and the next column
// group 1, ..., over the (head, feature split) pairs of that XCD: every compute unit then holds one
// workgroup that keeps the denominator column and one that does not, and a head's workgroups share
// one L2.  Otherwise the plain XCD-contiguous order.
__device__ __forceinline__ void mom_workgroup(const MomArgs& a, int64_t& bh, int& fs, int& cs) {
  const int total = gridDim.x;
  const int nper = total >> 3;
  if ((total & 7) == 0 && nper % a.csplit == 0) {
    const int per_cs = nper / a.csplit;
    const int x = blockIdx.x & 7, p = blockIdx.x >> 3;
    cs = p / per_cs;
    const int hf = x * per_cs + (p - cs * per_cs);
    bh = hf / a.fsplit;
    fs = hf - static_cast<int>(bh) * a.fsplit;
    // mixed tile counts: the partner of a full split is a short one (fs + fsplit / 2)
    if (a.mixed && cs == 1) fs = (fs + a.fsplit / 2) % a.fsplit;
    return;
  }
  const int per_head = a.fsplit * a.csplit;
  const int wg = xcd_remap(blockIdx.x, total);
  bh = wg / per_head;
  const int rem = wg - static_cast<int>(bh) * per_head;
  fs = rem / a.csplit;
  cs = rem - fs * a.csplit;
}

// Mixed tile counts (a.mixed, instantiated for NT = 4 and 5): the feature splits fs >= fsplit / 2 run
// NT - 1 tiles per wave (their table slot NT is padding), so the tiles need fsplit * 4 * (NT - 1/2)
// slots instead of fsplit * 4 * NT, and every compute unit holds one full and one short workgroup.
// SPLIT: split-bf16 matrix-core products (mom_query_split / mom_update_split) instead of fp32 ones.
// CG: value columns per workgroup, 32 or 64.  With 64 the feature values of a token are generated and
// split once for 4 column tiles instead of twice for 2 (the 32-column workgroups of a head each do
// their own), at one workgroup per compute unit (124 KiB of LDS).
// FULL: mom_full_slots(DBIG, ES, a.d) (the host picks the instantiation).
template <int NT, int NX, bool DBIG, int ES, bool SPLIT, int CG, bool FULL>
__global__ __launch_bounds__(MOM_THREADS, mom_wg_per_cu(NT, DBIG, CG, NX)) void moments_kernel(const MomArgs a) {
  int64_t bh;
  int fs, cs;
  mom_workgroup(a, bh, fs, cs);
  constexpr bool MIX = (NT == 4 || NT == 5) && !DBIG && CG == 32 && NX <= 2;
  if (MIX && a.mixed && fs >= a.fsplit / 2) {
    constexpr int NTL = MIX ? NT - 1 : NT;
    if (cs == 0)
      moments_body<NTL, NT, NX, DBIG, ES, true, SPLIT, CG, FULL>(a, bh, fs, cs);
    else
      moments_body<NTL, NT, NX, DBIG, ES, false, SPLIT, CG, FULL>(a, bh, fs, cs);
  } else {
    if (cs == 0)
      moments_body<NT, NT, NX, DBIG, ES, true, SPLIT, CG, FULL>(a, bh, fs, cs);
    else
      moments_body<NT, NT, NX, DBIG, ES, false, SPLIT, CG, FULL>(a, bh, fs, cs);
  }
}

// Shared-memory floats of moment_accumulate_kernel: one chunk buffer, the running denominators, a dummy.
__host__ __device__ constexpr int mom_acc_smem_floats(bool dbig, int nt) {
  return mom_buf_floats(dbig) + MOM_WAVES * nt * 16 + 8;
}

// Persistent-state form of the moment update (the decode state of a stream):
//   state_num[f][col] += sum_{j < n} phi_k(k_j)[f] v_j[col],  state_den[f] += sum_{j < n} phi_k(k_j)[f]
// over the n rows of each head, the state kept in the reference's feature order
// (streaming_taylor_coreset_attention.py:180-216, TaylorMomentSketch.update :265-280).  Same feature
// tiles, chunk staging and MFMA update as moments_kernel; the wave's slice of the state is loaded into
// the accumulators at the start and written back at the end (each (head, feature, column) belongs to
// exactly one wave of the grid, so the read-modify-write has no race).  Rows [0, n) of every head are
// read at k + bh * head_rows * d (v: ldv).
// SPLIT: split-bf16 matrix-core products (the staged values as bf16 hi / lo planes, mom_update_split with
// key-side coefficients) instead of fp32 ones.
template <int NT, int NX, bool DBIG, int ES, bool SPLIT>
__global__ __launch_bounds__(MOM_THREADS, 1) void moment_accumulate_kernel(const MomArgs a) {
  constexpr int BUF = mom_buf_floats(DBIG);
  constexpr int CT = 2;
  extern __shared__ float smem[];
  float* den_all = smem + BUF;
  const int dummy_abs = BUF + MOM_WAVES * NT * 16;

  const int per_head = a.fsplit * a.csplit;
  const int wg = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t bh = wg / per_head;
  const int rem = wg - static_cast<int>(bh) * per_head;
  const int fs = rem / a.csplit;
  const int cs = rem - fs * a.csplit;
  const int col0 = 32 * cs;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  float* den_s = den_all + w * NT * 16;
  const int64_t tile0 = (static_cast<int64_t>(fs) * MOM_WAVES + w) * NT;
  const MomLane<NT, NX> m = mom_lane<NT, NX>(a, tile0, li, lg);

  // ---- the wave's slice of the state -> accumulators and running denominators ----
  float* snum = a.state_num + bh * a.n_feat * a.ldo;
  float* sden = a.state_den + bh * a.n_feat;
  floatx4 st[NT][CT];
#pragma unroll
  for (int kt = 0; kt < NT; ++kt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = a.rowmap[(tile0 + kt) * 16 + 4 * lg + r];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        st[kt][ct][r] = row >= 0 ? snum[static_cast<int64_t>(row) * a.ldo + col0 + 16 * ct + li] : 0.f;
    }
    if (lg == 0) {
      const int row = a.rowmap[(tile0 + kt) * 16 + li];
      den_s[16 * kt + li] = row >= 0 ? sden[row] : 0.f;
    }
  }

  const char* kh = static_cast<const char*>(a.k) + bh * a.head_rows * a.ldk * ES;
  const char* vh = static_cast<const char*>(a.v) + bh * a.head_rows * a.ldv * ES;
  const MomSlots<DBIG, 32> sl = mom_slots<DBIG, ES, 32>(a, col0, dummy_abs, a.win ? a.win + 4 * fs : nullptr);
  const int nchunks = static_cast<int>((a.n + MOM_C - 1) / MOM_C);
  for (int e = tid; e < BUF; e += MOM_THREADS) smem[e] = 0.f;  // padding rows / columns stay 0
  for (int c = 0; c < nchunks; ++c) {
    MomStage<DBIG, 32> stg;
    mom_load<DBIG, ES, 32>(stg, sl, a, kh, kh, vh, c * MOM_C);  // the query slots are staged but not used
    __syncthreads();  // the previous chunk's update is done with the buffer
    mom_store<DBIG, ES, 32, SPLIT>(stg, sl, a, smem, dummy_abs, c * MOM_C);
    __syncthreads();
    const float* Kt = smem + MOM_C * mom_ldq(DBIG);
    const float* Vt = Kt + mom_krows(DBIG) * MOM_LDT;
    auto none = []() {};
    if constexpr (SPLIT)
      mom_update_split<NT, CT, NX, true, decltype(none), true>(st, den_s, Kt, Vt, m, li, lg, none);
    else
      mom_update<NT, CT, NX, true>(st, den_s, Kt, Vt, m, li, lg, none);
  }

  // ---- write the slice back (the denominators once per feature split) ----
#pragma unroll
  for (int kt = 0; kt < NT; ++kt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = a.rowmap[(tile0 + kt) * 16 + 4 * lg + r];
      if (row >= 0) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) snum[static_cast<int64_t>(row) * a.ldo + col0 + 16 * ct + li] = st[kt][ct][r];
      }
    }
    if (lg == 0 && cs == 0) {
      const int row = a.rowmap[(tile0 + kt) * 16 + li];
      if (row >= 0) sden[row] = den_s[16 * kt + li];
    }
  }
}

// Block form of moment_accumulate_kernel (split-bf16 products, d <= 64 without windows): one workgroup of
// MOMB_WAVES waves per (head, 32-column group) stages up to MOMB_CHUNKS chunks of its rows at once (keys
// transposed, values as bf16 hi / lo planes, the layouts of mom_store), then every wave takes the
// chunked kernel's wave slices j = wave, wave + MOMB_WAVES, ... (NT tiles each, tile0 = j NT) and runs
// the staged chunks through mom_update_split with no barrier, the next slice's state and feature table
// loads in flight meanwhile.  A slice's accumulators see the chunks in the same order and through the
// same products as moment_accumulate_kernel's, so the state is the same bit for bit; the rows are staged
// once per column group instead of once per feature split.  More than MOMB_CHUNKS chunks: groups of
// chunks, the state read and written back per group.
constexpr int MOMB_WAVES = 8;
constexpr int MOMB_THREADS = 64 * MOMB_WAVES;
constexpr int MOMB_CHUNKS = 8;
// LDS floats of one staged chunk: transposed keys (mom_krows(false) rows) and the value planes of the
// workgroup's 16 CT columns
__host__ __device__ constexpr int momb_chunk_floats(int ct) { return mom_krows(false) * MOM_LDT + 16 * ct * MOM_LDT; }
__host__ __device__ constexpr int momb_smem_floats(int nt, int ct) {
  return MOMB_CHUNKS * momb_chunk_floats(ct) + MOMB_WAVES * nt * 16 + 8;
}

// CT column tiles of 16 per workgroup (2: 32 columns, a.csplit groups; 4: 64 columns, every key feature
// generated once per head; the products of each 16-column tile are the same either way).
template <int NT, int NX, int ES, int CT>
__global__ __launch_bounds__(MOMB_THREADS, 1) void moment_block_kernel(const MomArgs a) {
  constexpr int CG = 16 * CT;
  constexpr int CF = momb_chunk_floats(CT);
  constexpr int KROWS = mom_krows(false);
  constexpr int EPU = 16 / ES;
  extern __shared__ float smem[];
  float* den_all = smem + MOMB_CHUNKS * CF;

  const int groups = a.csplit * 32 / CG;  // column groups per head (the host keeps a.ldo a multiple of CG)
  const int wg = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t bh = wg / groups;
  const int cs = wg - static_cast<int>(bh) * groups;
  const int col0 = CG * cs;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  float* den_s = den_all + wave * NT * 16;
  float* snum = a.state_num + bh * a.n_feat * a.ldo;
  float* sden = a.state_den + bh * a.n_feat;
  const char* kh = static_cast<const char*>(a.k) + bh * a.head_rows * a.ldk * ES;
  const char* vh = static_cast<const char*>(a.v) + bh * a.head_rows * a.ldv * ES;
  const int uq = a.d / EPU;                         // key units per row
  const int n_slices = a.fsplit * MOM_WAVES;        // the chunked kernel's wave slices
  const int n_rows = static_cast<int>(a.n);

  // state rows of slice j's accumulator elements (rowmap, -1: padding) and of its denominators
  struct Rows {
    int r[NT][4];
    int d[NT];
  };
  auto load_rows = [&](int j, Rows& R) {
    const int64_t tile0 = static_cast<int64_t>(j) * NT;
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) R.r[kt][r] = a.rowmap[(tile0 + kt) * 16 + 4 * lg + r];
      R.d[kt] = a.rowmap[(tile0 + kt) * 16 + li];
    }
  };
  // a slice's state into accumulators, its denominators into registers
  auto load_state = [&](const Rows& R, floatx4 (&st)[NT][CT], float (&dn)[NT]) {
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = R.r[kt][r];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
          st[kt][ct][r] = row >= 0 ? snum[static_cast<int64_t>(row) * a.ldo + col0 + 16 * ct + li] : 0.f;
      }
      dn[kt] = R.d[kt] >= 0 ? sden[R.d[kt]] : 0.f;
    }
  };

  for (int e = tid; e < MOMB_CHUNKS * CF; e += MOMB_THREADS) smem[e] = 0.f;  // padding rows stay 0
  for (int g0 = 0; g0 < n_rows; g0 += MOMB_CHUNKS * MOM_C) {
    const int nch = min(MOMB_CHUNKS, (n_rows - g0 + MOM_C - 1) / MOM_C);
    // ---- stage the group's chunks: unit loads first (rows clamped into the sequence), then the stores;
    //      token-fast units so that a half-wave writes one transposed row / plane row ----
    {
      constexpr int KJ = MOMB_CHUNKS * MOM_C * (64 / EPU) / MOMB_THREADS;  // key units per thread (max)
      constexpr int VJ = MOMB_CHUNKS * MOM_C * (CG / EPU) / MOMB_THREADS;  // value units per thread
      const int kunits = nch * MOM_C * uq, vunits = nch * MOM_C * (CG / EPU);
      uint4 ku[KJ], vu[VJ];
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        const int e = min(tid + MOMB_THREADS * j, kunits - 1);
        const int c = e / (MOM_C * uq), r = e - c * (MOM_C * uq);
        const int row = clamp_row(g0 + c * MOM_C + (r & (MOM_C - 1)), n_rows);
        ku[j] = *reinterpret_cast<const uint4*>(kh + (static_cast<int64_t>(row) * a.ldk + (r >> 5) * EPU) * ES);
      }
#pragma unroll
      for (int j = 0; j < VJ; ++j) {
        const int e = min(tid + MOMB_THREADS * j, vunits - 1);
        const int c = e / (MOM_C * (CG / EPU)), r = e - c * (MOM_C * (CG / EPU));
        const int row = clamp_row(g0 + c * MOM_C + (r & (MOM_C - 1)), n_rows);
        vu[j] = *reinterpret_cast<const uint4*>(vh + (static_cast<int64_t>(row) * a.ldv + col0 + (r >> 5) * EPU) * ES);
      }
      __syncthreads();  // the previous group's updates are done with the chunk buffers
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        const int e = tid + MOMB_THREADS * j;
        if (e < kunits) {
          const int c = e / (MOM_C * uq), r = e - c * (MOM_C * uq);
          const int tok = r & (MOM_C - 1), u = r >> 5;
          const float kok = g0 + c * MOM_C + tok < n_rows ? 1.f : 0.f;
          float f[8];
          unit_floats<ES>(ku[j], a.dtype, f);
          float* kt = smem + c * CF;
#pragma unroll
          for (int m = 0; m < EPU; ++m) kt[(u * EPU + m) * MOM_LDT + tok] = f[m] * kok;
        }
      }
#pragma unroll
      for (int j = 0; j < VJ; ++j) {
        const int e = tid + MOMB_THREADS * j;
        if (e < vunits) {
          const int c = e / (MOM_C * (CG / EPU)), r = e - c * (MOM_C * (CG / EPU));
          const int tok = r & (MOM_C - 1), u = r >> 5;
          const float kok = g0 + c * MOM_C + tok < n_rows ? 1.f : 0.f;
          float f[8];
          unit_floats<ES>(vu[j], a.dtype, f);
          __bf16* vp = reinterpret_cast<__bf16*>(smem + c * CF + KROWS * MOM_LDT);
#pragma unroll
          for (int m = 0; m < EPU; ++m) {
            const float x = f[m] * kok;
            const __bf16 h = static_cast<__bf16>(x);
            const __bf16 l = static_cast<__bf16>(x - static_cast<float>(h));
            vp[vps_off(u * EPU + m, tok)] = h;
            vp[CG * MOM_C + vps_off(u * EPU + m, tok)] = l;
          }
        }
      }
      // the constant factor: 1 on rows inside the sequence, 0 outside
      for (int e = tid; e < nch * MOM_C; e += MOMB_THREADS) {
        const int c = e >> 5, tok = e & (MOM_C - 1);
        smem[c * CF + a.d * MOM_LDT + tok] = g0 + c * MOM_C + tok < n_rows ? 1.f : 0.f;
      }
      __syncthreads();
    }

    // ---- the wave's slices, each through every staged chunk.  Pipelined: while slice j runs, the state
    //      and feature tables of slice j + W and the state rows of slice j + 2 W are in flight ----
    auto none = []() {};
    floatx4 st[NT][CT];
    float dn[NT];
    Rows rn;
    int j = wave;
    if (j < n_slices) {
      load_rows(j, rn);
      load_state(rn, st, dn);
    }
    if (j + MOMB_WAVES < n_slices) load_rows(j + MOMB_WAVES, rn);
    MomLane<NT, NX> m = mom_lane<NT, NX>(a, static_cast<int64_t>(min(j, n_slices - 1)) * NT, li, lg);
    while (j < n_slices) {
#pragma unroll
      for (int kt = 0; kt < NT; ++kt)
        if (lg == 0) den_s[16 * kt + li] = dn[kt];
      const int jn = j + MOMB_WAVES;
      floatx4 stn[NT][CT];
      float dnn[NT];
      Rows rc, rnn;
      load_rows(j, rc);  // this slice's rows again, for its stores (no wait before the updates)
      if (jn < n_slices) load_state(rn, stn, dnn);
      if (jn + MOMB_WAVES < n_slices) load_rows(jn + MOMB_WAVES, rnn);
      const MomLane<NT, NX> mn = mom_lane<NT, NX>(a, static_cast<int64_t>(min(jn, n_slices - 1)) * NT, li, lg);
      for (int c = 0; c < nch; ++c) {
        const float* Kt = smem + c * CF;
        mom_update_split<NT, CT, NX, true, decltype(none), true>(st, den_s, Kt, Kt + KROWS * MOM_LDT, m, li, lg, none);
      }
      // write the slice back (the denominators once per column group 0)
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = rc.r[kt][r];
          if (row >= 0) {
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) snum[static_cast<int64_t>(row) * a.ldo + col0 + 16 * ct + li] = st[kt][ct][r];
          }
        }
        if (lg == 0 && cs == 0 && rc.d[kt] >= 0) sden[rc.d[kt]] = den_s[16 * kt + li];
      }
      j = jn;
      if (j < n_slices) {
#pragma unroll
        for (int kt = 0; kt < NT; ++kt) {
          dn[kt] = dnn[kt];
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) st[kt][ct] = stn[kt][ct];
        }
        rn = rnn;
        m = mn;
      }
    }
  }
}

}  // namespace sta
