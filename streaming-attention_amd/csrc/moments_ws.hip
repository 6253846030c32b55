// K1, wave-specialised form (split-bf16 products): the exact low-degree Taylor moment scan
//   low_num[i] = phi_q(s q_i) . S_{<b(i)}[:, :dv],   low_den[i] = phi_q(s q_i) . S_{<b(i)}[:, dv]
// where b(i) is the query block of row i (blocks of QB = cpb * 32 rows, offset by `shift` like the
// chunks) and S_{<b} = sum over the keys before the block of phi_k(k_j) [v_j, 1].  The residual kernel
// adds every key of the row's own query block (the Taylor polynomial, or exp where the key is also in
// the row's article block); with QB equal to the article block the two sets coincide and the residual
// kernel's in-block keys carry exp(x) whole.  Reference semantics as moments_kernel:
// low_degree_taylor_causal_sums_stream (fast_article_attention.py:217-259).
//
// Work split.  A workgroup of 512 threads = (head, feature split, 64-column group) holds 4 slots of
// tiles (16 features each, the feature_tiles layout of moments.hip).  Waves 0-3 ("update waves") keep
// the fp32 state of slot w in MFMA accumulators for the whole sequence and add every 32-token chunk:
// S += phi_k^T [V, 1].  Waves 4-7 ("query waves") keep a frozen copy of the state of slot (w + 2) & 3
// as split bf16 hi / lo operands, refreshed once per query block, and answer the chunk's queries:
// out += phi_q S_frozen, 3 bf16 products per fp32 product.  Each wave generates one kind of feature
// value only, every value feeds 4 column tiles (64 columns), and no state is re-split per chunk.  With
// mixed tile counts slots 2 and 3 hold one tile less: a SIMD runs one update and one query wave
// (waves w and w + 4) of slots w and (w + 2) & 3, so every SIMD carries the same number of tiles.
//
// Pipeline (one barrier per chunk).  Iteration c: update waves add chunk c; query waves answer chunk
// c - 1 (one chunk behind, so the state of a new block is in flight for a whole iteration) and write
// their partials to red[(c - 1) & 1]; the staging threads (ws_stagers) stage the keys / values of chunk
// c + 1 and the queries of chunk c into the other LDS buffers and issue the global loads of the next
// slot; the update waves reduce red[(c - 2) & 1] over the 4 query waves in a fixed order
// (deterministic) into the partial outputs.  At the last chunk of a block the update waves split their
// state and write it to a per-workgroup handoff buffer in global memory (one copy; two by block parity
// when a block is 2 chunks) and the running denominators to LDS (two by block parity); the query waves
// load the state in the next iteration, right after their last use of the old copy.  The handoff stays
// within the workgroup (stores, barrier, loads on one compute unit).
//
// Sequence segments (few heads).  With nseg > 1 each (head, feature split, column group) is cut into
// nseg segments of seg_chunks chunks (whole query blocks), one workgroup each, in two passes.  Phase
// 1: the update waves sum their segment's keys from a zero state (no queries, no outputs) and write
// the total to seg_state; an exclusive scan over the segments (ws_seg_scan_kernel, api.hip) turns the
// totals into S_init(p), the state before segment p.  Phase 2: the ordinary scan of each segment,
// starting from S_init(p) (the update waves' accumulators and the query waves' operands and
// denominators are loaded from it) instead of zero.
#pragma once
#include "moments.hip"

namespace sta {

constexpr int WS_WAVES = 8;
constexpr int WS_THREADS = 64 * WS_WAVES;
// Threads that stage the chunks (STG): at degree <= 2 and d <= 64 the 256 of the update waves (the query
// waves set the pace of a chunk and the update waves have time to spare: c3 6.04 -> 5.88 ms); at degree 3
// or d > 64 all 512 (no registers for twice the staged units next to the extra factor or wider rows).
__host__ __device__ constexpr int ws_stagers(int nx, bool dbig) { return nx == 0 && !dbig ? 256 : 512; }
constexpr int WS_REDUCERS = 256;  // the update waves reduce the partials

struct WsArgs {
  MomArgs m;        // inputs, feature table [fsplit][4 slots][NTS][..], partial outputs (moments_kernel layout)
  int cpb;          // chunks per query block (>= 2)
  int mixed;        // slots 2 and 3 hold NTS - 1 tiles
  uint4* hand;      // [grid][2][4][NPS][CT][2][64]: split state as query operands (see ws_body)
  int nseg;         // sequence segments per (head, feature split, column group); 1: the whole sequence
  int seg_chunks;   // chunks per segment (a multiple of cpb)
  int phase;        // 0: whole sequence; 1: segment totals (update only); 2: segment scans from S_init
  float* seg_state; // [bh][fsplit][csplit][nseg][ws_seg_floats]: segment totals, then S_init (nseg > 1)
};

// Per (head, feature split, column group, segment): the 4 update waves' accumulators [4][NTS][CT][64
// lanes] floatx4, then the denominators [4][NTS][16].
__host__ __device__ constexpr int ws_seg_floats(int nts, int ct) { return nts * (1024 * ct + 64); }

__host__ __device__ constexpr int ws_kv_floats(bool dbig, int cg) { return mom_krows(dbig) * MOM_LDT + cg * MOM_C; }
__host__ __device__ constexpr int ws_q_floats(bool dbig) { return MOM_C * mom_ldq(dbig); }
__host__ __device__ constexpr int ws_red_floats(int cg) { return 4 * (cg + 4) * MOM_LDR; }
// frozen running denominators of the query waves: [2 block parities][4 slots][nts * 16]
__host__ __device__ constexpr int ws_den_floats(int nts) { return 2 * 4 * nts * 16; }
__host__ __device__ constexpr int ws_smem_floats(bool dbig, int cg, int nts) {
  return 2 * ws_kv_floats(dbig, cg) + 2 * ws_q_floats(dbig) + 2 * ws_red_floats(cg) + ws_den_floats(nts);
}

// Chunk staging in registers by the STG staging threads (tid < STG): unit e = tid + STG j of 16 bytes (4
// fp32 or 8 bf16 / fp16).
// q: row-major units (token e / uq); k and v: token-fast units (token tid & 31) for the transposed LDS
// rows.  Geometry per thread is fixed for the whole sequence.
template <bool DBIG, int ES, int CG, int STG>
struct WsStage {
  static constexpr int QU = MOM_C * (DBIG ? 128 : 64) * ES / 16;
  static constexpr int QV = (QU + STG - 1) / STG;
  static constexpr int VU = MOM_C * CG * ES / 16;
  static constexpr int VV = (VU + STG - 1) / STG;
  // token pairs (fp32 rows, two key and two value units per thread): units 0 and 1 are one 16-byte
  // unit of tokens 2 p and 2 p + 1, which sit next to each other in the transposed key rows and the
  // value planes, so the stores are 8-byte key pairs and packed 32-bit bf16 pairs
  static constexpr bool PAIR = !DBIG && ES == 4 && QV == 2 && VV == 2 && QU == 2 * STG && VU == 2 * STG;
  // the same for 16-bit rows (one key and one value unit per thread): 8-byte half units (4 elements) of
  // tokens 2 p and 2 p + 1 held in one register set, {token 2 p: elements 0..3, token 2 p + 1: 0..3}
  static constexpr bool PAIR16 = !DBIG && ES == 2 && QV == 1 && VV == 1 && QU == STG && VU == STG;
  uint4 q[QV];
  uint4 k[QV];
  uint4 v[VV];
};

template <bool DBIG, int ES, int CG, int STG>
struct WsSlots {
  static constexpr int QV = WsStage<DBIG, ES, CG, STG>::QV;
  static constexpr int VV = WsStage<DBIG, ES, CG, STG>::VV;
  // *_rel: byte offset of the unit from the start of the chunk's first row (the unit's token times the
  // row stride plus its offset in the row), so that a chunk inside the sequence loads from one uniform
  // row address plus these loop-invariant offsets
  int q_tok[QV];
  uint32_t q_rel[QV];
  int q_lds[QV];
  bool q_use[QV];
  uint32_t k_rel[QV];
  int k_dim[QV];  // -1: unused
  uint32_t v_rel[VV];
  int v_col[VV];  // -1: unused
  int sidx;       // this thread's index among the staging threads
};

// token of staged key / value unit j (PAIR16: unit 0's two half units, j = 0, 1)
template <bool DBIG, int ES, int CG, int STG>
__device__ __forceinline__ int ws_kv_tok(int sidx, int j) {
  constexpr bool pair = WsStage<DBIG, ES, CG, STG>::PAIR || WsStage<DBIG, ES, CG, STG>::PAIR16;
  return pair ? 2 * (sidx & 15) + j : sidx & (MOM_C - 1);
}

template <bool DBIG, int ES, int CG, int STG>
__device__ __forceinline__ WsSlots<DBIG, ES, CG, STG> ws_slots(const MomArgs& a, int col0, int sidx) {
  constexpr int LDQ = mom_ldq(DBIG);
  constexpr int epu = 16 / ES;
  WsSlots<DBIG, ES, CG, STG> sl;
  const int tid = sidx;
  sl.sidx = sidx;
  const int uq = a.d / epu;
  const uint32_t qrow = static_cast<uint32_t>(a.ldk * ES), vrow = static_cast<uint32_t>(a.ldv * ES);
  constexpr bool PAIR = WsStage<DBIG, ES, CG, STG>::PAIR;
  constexpr bool PAIR16 = WsStage<DBIG, ES, CG, STG>::PAIR16;
#pragma unroll
  for (int j = 0; j < WsStage<DBIG, ES, CG, STG>::QV; ++j) {
    const int e = tid + STG * j;
    const int t = e / uq, u = e - t * uq;
    sl.q_use[j] = t < MOM_C;
    sl.q_tok[j] = min(t, MOM_C - 1);
    sl.q_rel[j] = static_cast<uint32_t>(sl.q_tok[j]) * qrow + static_cast<uint32_t>(u * 16);
    sl.q_lds[j] = t * LDQ + u * epu;
    const uint32_t ktok = static_cast<uint32_t>(ws_kv_tok<DBIG, ES, CG, STG>(tid, j));
    if constexpr (PAIR16) {  // half unit tid >> 4: elements 4 hu .. 4 hu + 3
      const int hu = tid >> 4;
      sl.k_rel[j] = ktok * qrow + static_cast<uint32_t>(min(hu, a.d / 4 - 1) * 8);
      sl.k_dim[j] = 4 * hu < a.d ? 4 * hu : -1;
    } else {
      const int uk = PAIR ? tid >> 4 : e >> 5;
      sl.k_rel[j] = ktok * qrow + static_cast<uint32_t>(min(uk, uq - 1) * 16);
      sl.k_dim[j] = uk < uq ? uk * epu : -1;
    }
  }
#pragma unroll
  for (int j = 0; j < WsStage<DBIG, ES, CG, STG>::VV; ++j) {
    const uint32_t vtok = static_cast<uint32_t>(ws_kv_tok<DBIG, ES, CG, STG>(tid, j));
    if constexpr (PAIR16) {
      const int hu = tid >> 4;
      sl.v_rel[j] = vtok * vrow + static_cast<uint32_t>((col0 + min(4 * hu, CG - 4)) * ES);
      sl.v_col[j] = 4 * hu < CG ? 4 * hu : -1;
    } else {
      const int uv = PAIR ? tid >> 4 : (tid + STG * j) >> 5;
      sl.v_rel[j] = vtok * vrow + static_cast<uint32_t>((col0 + min(uv * epu, CG - epu)) * ES);
      sl.v_col[j] = uv * epu < CG ? uv * epu : -1;
    }
  }
  return sl;
}

// MASK = false: every row of the chunk lies in the sequence: one uniform row address plus each unit's
// loop-invariant offset.  MASK = true: rows clamped into the sequence one by one.
// The head's q / k / v rows as buffer resources (a head's rows span < 2^31 bytes, which the kernel's
// callers check).
struct WsRows {
  __amdgpu_buffer_rsrc_t q, k, v;
};

// Offsets of the staged units of the chunk at row0 in the buffers of WsRows: with every row of the
// chunk in the sequence, one uniform row offset (so) and the loop-invariant per-unit offsets; else
// so = 0 and each unit's row clamped into the sequence (its staged value is zeroed).  Only the
// offsets depend on the case, so the loads themselves are one code path.
template <int U>
struct WsOffs {
  uint32_t v[U];
  int so;
};

template <int U>
__device__ __forceinline__ WsOffs<U> ws_offs(const uint32_t (&rel)[U], const int (&tok)[U], uint32_t rowb, int row0,
                                             int n) {
  WsOffs<U> o;
  if (row0 >= 0 && row0 + MOM_C <= n) {
    o.so = static_cast<int>(static_cast<uint32_t>(row0) * rowb);
#pragma unroll
    for (int j = 0; j < U; ++j) o.v[j] = rel[j];
  } else {
    o.so = 0;
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const uint32_t r = static_cast<uint32_t>(clamp_row(row0 + tok[j], n));
      o.v[j] = r * rowb + (rel[j] - static_cast<uint32_t>(tok[j]) * rowb);
    }
  }
  return o;
}

template <bool DBIG, int ES, int CG, int STG>
__device__ __forceinline__ void ws_load_q(WsStage<DBIG, ES, CG, STG>& st, const WsSlots<DBIG, ES, CG, STG>& sl,
                                          const MomArgs& a, const WsRows& rs, int row0) {
  constexpr int QV = WsStage<DBIG, ES, CG, STG>::QV;
  const WsOffs<QV> o = ws_offs<QV>(sl.q_rel, sl.q_tok, static_cast<uint32_t>(a.ldk * ES), row0, static_cast<int>(a.n));
#pragma unroll
  for (int j = 0; j < QV; ++j)
    st.q[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.q, o.v[j], o.so, 0));
}

template <bool DBIG, int ES, int CG, int STG>
__device__ __forceinline__ void ws_load_kv(WsStage<DBIG, ES, CG, STG>& st, const WsSlots<DBIG, ES, CG, STG>& sl,
                                           const MomArgs& a, const WsRows& rs, int row0) {
  constexpr bool PAIR16 = WsStage<DBIG, ES, CG, STG>::PAIR16;
  constexpr int QV = WsStage<DBIG, ES, CG, STG>::QV, VV = WsStage<DBIG, ES, CG, STG>::VV;
  const uint32_t krow_b = static_cast<uint32_t>(a.ldk * ES), vrow_b = static_cast<uint32_t>(a.ldv * ES);
  const int n = static_cast<int>(a.n);
  if constexpr (PAIR16) {
    // half units of tokens 2 p and 2 p + 1 (k_rel / v_rel: token 2 p's)
    const int t0 = ws_kv_tok<DBIG, ES, CG, STG>(sl.sidx, 0);
    const uint32_t krel[2] = {sl.k_rel[0], sl.k_rel[0] + krow_b}, vrel[2] = {sl.v_rel[0], sl.v_rel[0] + vrow_b};
    const int tok[2] = {t0, t0 + 1};
    const WsOffs<2> ko = ws_offs<2>(krel, tok, krow_b, row0, n), vo = ws_offs<2>(vrel, tok, vrow_b, row0, n);
    const uint2 k0 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs.k, ko.v[0], ko.so, 0));
    const uint2 k1 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs.k, ko.v[1], ko.so, 0));
    const uint2 v0 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs.v, vo.v[0], vo.so, 0));
    const uint2 v1 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs.v, vo.v[1], vo.so, 0));
    st.k[0] = uint4{k0.x, k0.y, k1.x, k1.y};
    st.v[0] = uint4{v0.x, v0.y, v1.x, v1.y};
    return;
  }
  int ktok[QV], vtok[VV];
#pragma unroll
  for (int j = 0; j < QV; ++j) ktok[j] = ws_kv_tok<DBIG, ES, CG, STG>(sl.sidx, j);
#pragma unroll
  for (int j = 0; j < VV; ++j) vtok[j] = ws_kv_tok<DBIG, ES, CG, STG>(sl.sidx, j);
  const WsOffs<QV> ko = ws_offs<QV>(sl.k_rel, ktok, krow_b, row0, n);
  const WsOffs<VV> vo = ws_offs<VV>(sl.v_rel, vtok, vrow_b, row0, n);
#pragma unroll
  for (int j = 0; j < QV; ++j)
    st.k[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.k, ko.v[j], ko.so, 0));
#pragma unroll
  for (int j = 0; j < VV; ++j)
    st.v[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.v, vo.v[j], vo.so, 0));
}

// An empty use of every staged register: the compiler completes their loads before it (where the
// stores have consumed them already this costs nothing).
template <bool DBIG, int ES, int CG, int STG>
__device__ __forceinline__ void ws_settle(const WsStage<DBIG, ES, CG, STG>& st) {
#pragma unroll
  for (int j = 0; j < WsStage<DBIG, ES, CG, STG>::QV; ++j) {
    asm volatile("" ::"v"(st.q[j].x), "v"(st.q[j].y), "v"(st.q[j].z), "v"(st.q[j].w));
    asm volatile("" ::"v"(st.k[j].x), "v"(st.k[j].y), "v"(st.k[j].z), "v"(st.k[j].w));
  }
#pragma unroll
  for (int j = 0; j < WsStage<DBIG, ES, CG, STG>::VV; ++j)
    asm volatile("" ::"v"(st.v[j].x), "v"(st.v[j].y), "v"(st.v[j].z), "v"(st.v[j].w));
}

// queries of the chunk at row0 -> Qs (scaled; column d = 1, or 0 on rows outside the sequence)
template <bool DBIG, int ES, int CG, int STG, bool MASK>
__device__ __forceinline__ void ws_store_q(const WsStage<DBIG, ES, CG, STG>& st, const WsSlots<DBIG, ES, CG, STG>& sl,
                                           const MomArgs& a, float* Qs, int row0) {
  constexpr int LDQ = mom_ldq(DBIG);
  constexpr bool wide = ES == 2;
#pragma unroll
  for (int j = 0; j < WsStage<DBIG, ES, CG, STG>::QV; ++j) {
    if (!sl.q_use[j]) continue;
    const int row = row0 + sl.q_tok[j];
    const float sc = (!MASK || (row >= 0 && row < a.n)) ? a.scale : 0.f;
    float f[8];
    unit_floats<ES>(st.q[j], a.dtype, f);
    float* qd = Qs + sl.q_lds[j];
    // element by element (a vector times sc kept a splat of sc in four scalar registers)
    *reinterpret_cast<floatx4*>(qd) = floatx4{f[0] * sc, f[1] * sc, f[2] * sc, f[3] * sc};
    if constexpr (wide) *reinterpret_cast<floatx4*>(qd + 4) = floatx4{f[4] * sc, f[5] * sc, f[6] * sc, f[7] * sc};
  }
  const int tid = sl.sidx;
  if (tid < MOM_C) Qs[tid * LDQ + a.d] = (!MASK || (row0 + tid >= 0 && row0 + tid < a.n)) ? 1.f : 0.f;
}

// keys (transposed, row d = constant) and values (bf16 hi / lo planes, vps_off) of the chunk at row0;
// VX: bf16 values, whose lo plane is zero and not written (nor read)
template <bool DBIG, int ES, int CG, int STG, bool MASK, bool VX = false>
__device__ __forceinline__ void ws_store_kv(const WsStage<DBIG, ES, CG, STG>& st, const WsSlots<DBIG, ES, CG, STG>& sl,
                                            const MomArgs& a, float* Kt, __bf16* vplane, int row0) {
  constexpr bool wide = ES == 2;
  auto in_seq = [&](int t) { return (!MASK || (row0 + t >= 0 && row0 + t < a.n)) ? 1.f : 0.f; };
  if constexpr (WsStage<DBIG, ES, CG, STG>::PAIR) {
    const int t0 = 2 * (sl.sidx & 15);
    const float ok0 = in_seq(t0), ok1 = in_seq(t0 + 1);
    const int kd = sl.k_dim[0];
    if (kd >= 0) {
      const floatx4 f0 = __builtin_bit_cast(floatx4, st.k[0]), f1 = __builtin_bit_cast(floatx4, st.k[1]);
      // two 4-byte stores per dimension (one ds_write2_b32 from the loaded registers as they are; an
      // 8-byte store would need the pair copied into adjacent registers first)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        float* kp = Kt + (kd + m) * MOM_LDT + t0;
        kp[0] = f0[m] * ok0;
        kp[1] = f1[m] * ok1;
      }
    }
    const int c0 = sl.v_col[0];
    if (c0 >= 0) {
      const floatx4 f0 = __builtin_bit_cast(floatx4, st.v[0]), f1 = __builtin_bit_cast(floatx4, st.v[1]);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        uint32_t h, l;
        split_pair(f0[m] * ok0, f1[m] * ok1, h, l);
        *reinterpret_cast<uint32_t*>(vplane + vps_off(c0 + m, t0)) = h;  // t0 even: t0 + 1 is the next bf16
        if constexpr (!VX) *reinterpret_cast<uint32_t*>(vplane + CG * MOM_C + vps_off(c0 + m, t0)) = l;
      }
    }
    if (sl.sidx < MOM_C) Kt[a.d * MOM_LDT + sl.sidx] = in_seq(sl.sidx);
    return;
  }
  if constexpr (WsStage<DBIG, ES, CG, STG>::PAIR16) {
    const int t0 = 2 * (sl.sidx & 15);
    const float ok0 = in_seq(t0), ok1 = in_seq(t0 + 1);
    const int kd = sl.k_dim[0];
    if (kd >= 0) {
      float f[8];  // token t0: f[0..3], token t0 + 1: f[4..7]
      unit_floats<ES>(st.k[0], a.dtype, f);
#pragma unroll
      for (int m = 0; m < 4; ++m) *reinterpret_cast<floatx2*>(Kt + (kd + m) * MOM_LDT + t0) = floatx2{f[m] * ok0, f[4 + m] * ok1};
    }
    const int c0 = sl.v_col[0];
    if (c0 >= 0) {
      float f[8];
      unit_floats<ES>(st.v[0], a.dtype, f);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        uint32_t h, l = 0u;
        if constexpr (VX)
          h = pk_bf16(f[m] * ok0, f[4 + m] * ok1);  // exact bf16 values: no lo plane
        else
          split_pair(f[m] * ok0, f[4 + m] * ok1, h, l);
        *reinterpret_cast<uint32_t*>(vplane + vps_off(c0 + m, t0)) = h;
        if constexpr (!VX) *reinterpret_cast<uint32_t*>(vplane + CG * MOM_C + vps_off(c0 + m, t0)) = l;
      }
    }
    if (sl.sidx < MOM_C) Kt[a.d * MOM_LDT + sl.sidx] = in_seq(sl.sidx);
    return;
  }
  const int tok = sl.sidx & (MOM_C - 1);
  const float kok = in_seq(tok);
#pragma unroll
  for (int j = 0; j < WsStage<DBIG, ES, CG, STG>::QV; ++j) {
    const int kd = sl.k_dim[j];
    if (kd < 0) continue;
    float f[8];
    unit_floats<ES>(st.k[j], a.dtype, f);
#pragma unroll
    for (int m = 0; m < 8; ++m)
      if (m < 4 || wide) Kt[(kd + m) * MOM_LDT + tok] = f[m] * kok;
  }
#pragma unroll
  for (int j = 0; j < WsStage<DBIG, ES, CG, STG>::VV; ++j) {
    const int c0 = sl.v_col[j];
    if (c0 < 0) continue;
    float f[8];
    unit_floats<ES>(st.v[j], a.dtype, f);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      if (m < 4 || wide) {
        const float x = f[m] * kok;
        const __bf16 h = static_cast<__bf16>(x);
        vplane[vps_off(c0 + m, tok)] = h;
        if constexpr (!VX) vplane[CG * MOM_C + vps_off(c0 + m, tok)] = static_cast<__bf16>(x - static_cast<float>(h));
      }
    }
  }
  if (sl.sidx < MOM_C) Kt[a.d * MOM_LDT + sl.sidx] = kok;
}

// Update wave: S[f][col] += phi_k(tok)[f] V[tok][col] over the chunk for the slot's NT tiles and the
// 16 CT columns; den_p[kt] += this lane's 8 tokens of phi_k (feature li of tile kt; the lanes' partials
// are summed over lg when the state is handed to the query waves).  One 16x16x32 bf16 product covers
// the 32 tokens (the token mapping of mom_update_split).  The next tile's key reads are issued as soon
// as the current tile's feature values are formed (into the same registers), so they land while the
// current tile's operands are split and its products issue.
// KC: the key-side coefficient also at NX = 0 (a persistent state in the reference's feature order; the
// scan applies the tile coefficients on the query side instead)
template <int NT, int CT, int NX, bool VX, bool KC = false>
__device__ __forceinline__ void ws_update(floatx4 (&st)[NT][CT], float (&den_p)[NT], const float* Kt,
                                          const __bf16* vplane, const MomLane<NT, NX>& m, int li, int lg) {
  constexpr int CG = 16 * CT;
  bf16x8 vh[CT], vl[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    vh[ct] = *reinterpret_cast<const bf16x8*>(vplane + vps_off(16 * ct + li, 4 * lg));
    if constexpr (!VX) vl[ct] = *reinterpret_cast<const bf16x8*>(vplane + CG * MOM_C + vps_off(16 * ct + li, 4 * lg));
  }
  // key reads two tiles ahead: set kt & 1 holds tile kt's, reloaded with tile kt + 2's once its feature
  // values are formed
  floatx4 fa[2][2], fb[2][2], fc[2][2], fe[2][2];
  auto load = [&](int kt) {
    const int b = kt & 1;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      fa[b][h] = *reinterpret_cast<const floatx4*>(Kt + m.ka[kt] + 16 * h);
      fb[b][h] = *reinterpret_cast<const floatx4*>(Kt + m.kb[kt] + 16 * h);
      if (NX >= 1) fc[b][h] = *reinterpret_cast<const floatx4*>(Kt + m.kx[0][kt] + 16 * h);
      if (NX >= 2) fe[b][h] = *reinterpret_cast<const floatx4*>(Kt + m.kx[NX >= 2 ? 1 : 0][kt] + 16 * h);
    }
  };
  load(0);
  if (NT > 1) load(NT > 1 ? 1 : 0);
#pragma unroll
  for (int kt = 0; kt < NT; ++kt) {
    const int b = kt & 1;
    float x[8];
    float dacc = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float y = fa[b][j >> 2][j & 3] * fb[b][j >> 2][j & 3];
      if (NX >= 1) y *= fc[b][j >> 2][j & 3];
      if (NX >= 2) y *= fe[b][j >> 2][j & 3];
      if (NX >= 1 || KC) y *= m.kcoef[kt];  // NX = 0: the tile coefficient is applied by the query waves
      x[j] = y;
      dacc += y;
    }
    if (kt + 2 < NT) load(kt + 2 < NT ? kt + 2 : 0);
    den_p[kt] += dacc;
    bf16x8 ah, al;
    split_bf16(x, ah, al);
    if constexpr (!VX) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) st[kt][ct] = mfma_bf16(ah, vl[ct], st[kt][ct]);
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) st[kt][ct] = mfma_bf16(al, vh[ct], st[kt][ct]);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) st[kt][ct] = mfma_bf16(ah, vh[ct], st[kt][ct]);
  }
}

// Query-side operands of one tile for the lane's two tokens (li and 16 + li): x[i0] (times the tile
// coefficient at NX = 0), x[b .. b + 3] and the extra factors.
struct WsQOps {
  float a[2];
  floatx4 b[2];
  float c[2], e[2];
};

template <int NT, int NX, int LDQ>
__device__ __forceinline__ void ws_qload(WsQOps& o, int u, const float* Qs, const MomLane<NT, NX>& m, int li) {
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const float* qr = Qs + (li + 16 * tt) * LDQ;
    o.a[tt] = (NX == 0) ? qr[m.qa[u]] * m.kcoef[u] : qr[m.qa[u]];
    o.b[tt] = *reinterpret_cast<const floatx4*>(qr + m.qb[u]);
    if (NX >= 1) o.c[tt] = qr[m.qx[0][u]];
    if (NX >= 2) o.e[tt] = qr[m.qx[NX >= 2 ? 1 : 0][u]];
  }
}

// phi_q of token tt (4 features of the lane's quad) from loaded operands
template <int NX>
__device__ __forceinline__ void ws_qfeat(float (&x)[4], const WsQOps& o, int tt) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    float y = o.a[tt] * o.b[tt][s];
    if (NX >= 1) y *= o.c[tt];
    if (NX >= 2) y *= o.e[tt];
    x[s] = y;
  }
}

// The frozen denominators of a slot for the query waves' VALU dot phi_q . den: the fp32 values of the
// features the lane forms, in the pair layout of ws_qpair_mma (features 4 lg .. 4 lg + 3 of tiles 2 p
// and 2 p + 1: dv[p][0], dv[p][1]) and the odd tile's (od).  src: the slot's [NTS][16] denominators.
template <int NT>
__device__ __forceinline__ void ws_den_vals(floatx4 (&dv)[NT / 2 > 0 ? NT / 2 : 1][2], floatx4& od, const float* src,
                                            int lg) {
#pragma unroll
  for (int p = 0; p < NT / 2; ++p) {
    dv[p][0] = *reinterpret_cast<const floatx4*>(src + (2 * p) * 16 + 4 * lg);
    dv[p][1] = *reinterpret_cast<const floatx4*>(src + (2 * p + 1) * 16 + 4 * lg);
  }
  if constexpr ((NT & 1) != 0) od = *reinterpret_cast<const floatx4*>(src + (NT - 1) * 16 + 4 * lg);
}

typedef short shortx4 __attribute__((ext_vector_type(4)));

// Products of a tile pair: o[tt][ct] (rows 16 tt + 4 lg + r, column 16 ct + li) += phi_q . S_frozen with
// the pair's 32 features as the contraction (mom_query_split's layout), 3 bf16 products per term.
template <int CT>
__device__ __forceinline__ void ws_qpair_mma(floatx4 (&o)[2][CT], const bf16x8 (&ah)[2], const bf16x8 (&al)[2],
                                             const bf16x8 (&sh)[CT], const bf16x8 (&sl)[CT]) {
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) o[tt][ct] = mfma_bf16(ah[tt], sl[ct], o[tt][ct]);
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) o[tt][ct] = mfma_bf16(al[tt], sh[ct], o[tt][ct]);
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) o[tt][ct] = mfma_bf16(ah[tt], sh[ct], o[tt][ct]);
}

typedef short shortx4 __attribute__((ext_vector_type(4)));

// Products of a single (odd last) tile: one 16x16x16 bf16 product per term, the tile's 16 features as the
// contraction (lane (li, lg): features 4 lg + j).
template <int CT>
__device__ __forceinline__ void ws_qsingle_mma(floatx4 (&o)[2][CT], const uint2 (&ah)[2], const uint2 (&al)[2],
                                               const uint2 (&sh)[CT], const uint2 (&sl)[CT]) {
  auto mf = [](uint2 a, uint2 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(shortx4, a), __builtin_bit_cast(shortx4, b), c, 0,
                                                    0, 0);
  };
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) o[tt][ct] = mf(ah[tt], sl[ct], o[tt][ct]);
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) o[tt][ct] = mf(al[tt], sh[ct], o[tt][ct]);
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) o[tt][ct] = mf(ah[tt], sh[ct], o[tt][ct]);
}

// Fixed-order sum of the 4 query waves' partials of the chunk at row0 -> low_num rows of the CG columns
// (non-temporal stores: the partials are read only by the next kernel, and the workgroups' state
// handoff, rewritten every query block, should keep its place in L2)
// (CG * 8 threads, 4 tokens each) and, with den, low_den (column CG of a wave's partials: its
// denominator sums).
constexpr int WS_RCOLS_EXTRA = 4;
// Byte offsets of a reducing thread's output units from the chunk's first output row (4 rows of one
// column per unit): loop-invariant, so every chunk's stores take one uniform row address plus these.
template <int CG>
struct WsRedRel {
  static constexpr int IT = CG * 8 / WS_REDUCERS;
  uint32_t rel[IT];
};
template <int CG>
__device__ __forceinline__ WsRedRel<CG> ws_red_rel(const MomArgs& a, int tid) {
  WsRedRel<CG> rr;
#pragma unroll
  for (int it = 0; it < WsRedRel<CG>::IT; ++it) {
    const int e = it * WS_REDUCERS + tid;
    const int col = e % CG, t4 = 4 * (e / CG);
    rr.rel[it] = static_cast<uint32_t>(t4 * a.ldo + col) * 4u;
  }
  return rr;
}

template <int CG>
__device__ __forceinline__ void ws_reduce_store(const MomArgs& a, const float* red, int64_t obase, int64_t row0,
                                                int col0, bool den, const WsRedRel<CG>& rr) {
  constexpr int WS = (CG + WS_RCOLS_EXTRA) * MOM_LDR;
  constexpr int IT = WsRedRel<CG>::IT;
  const int tid = threadIdx.x;  // < WS_REDUCERS
  // every LDS read first (one wait for all of them instead of one per read), then the sums in the
  // fixed wave order
  floatx4 part[IT][4];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int e = it * WS_REDUCERS + tid;
    const int col = e % CG, t4 = 4 * (e / CG);
#pragma unroll
    for (int q = 0; q < 4; ++q) part[it][q] = *reinterpret_cast<const floatx4*>(red + q * WS + red_off(col, t4));
  }
  // the chunk's first output row of this column group as a buffer resource (uniform; rebuilt per chunk
  // by scalar instructions, so the offsets stay small at any sequence length)
  const __amdgpu_buffer_rsrc_t out = raw_rsrc(a.low_num + (obase + row0) * a.ldo + col0);
  const int rstep = __builtin_amdgcn_readfirstlane(a.ldo * 4);
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    floatx4 acc = part[it][0];
#pragma unroll
    for (int q = 1; q < 4; ++q) acc += part[it][q];
    // (each element through a float first: hipcc lowered __builtin_bit_cast of the vector element acc[r]
    // itself to element 0 for every r)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float x = acc[r];
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, x), out, rr.rel[it], r * rstep, BUF_NT);
    }
  }
  if (den && tid >= WS_REDUCERS - MOM_C) {
    const int tok = tid - (WS_REDUCERS - MOM_C);
    float dsum = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) dsum += red[q * WS + red_off(CG, tok)];
    __builtin_nontemporal_store(dsum, a.low_den + obase + row0 + tok);
  }
}

// Staging of iteration c by one thread (keys / values of chunk c + 1, with WQ queries of chunk c, into
// LDS from the registers, loads of slot c + 2 into them): the main loop's staging step, for the query
// waves of a segment-totals pass, which only stage (keys and values: that pass has no queries).
template <bool DBIG, int ES, int CG, int STG, bool WQ, bool VX>
__device__ __forceinline__ void ws_stage_step(WsStage<DBIG, ES, CG, STG>& pre, const WsSlots<DBIG, ES, CG, STG>& sl,
                                              const MomArgs& a, float* kvb, float* qb, int c, int nch, int first,
                                              const WsRows& rs) {
  constexpr int KVF = ws_kv_floats(DBIG, CG);
  constexpr int QF = ws_q_floats(DBIG);
  const int kv_row = first + (c + 1) * MOM_C;
  const int q_row = first + c * MOM_C;
  if (c + 1 < nch) {
    float* Kt = kvb + ((c + 1) & 1) * KVF;
    ws_store_kv<DBIG, ES, CG, STG, true, VX>(pre, sl, a, Kt, reinterpret_cast<__bf16*>(Kt + mom_krows(DBIG) * MOM_LDT),
                                             kv_row);
  }
  if (WQ && c < nch) ws_store_q<DBIG, ES, CG, STG, true>(pre, sl, a, qb + (c & 1) * QF, q_row);
  ws_load_kv<DBIG, ES, CG, STG>(pre, sl, a, rs, kv_row + MOM_C);
  if (WQ) ws_load_q<DBIG, ES, CG, STG>(pre, sl, a, rs, q_row + MOM_C);
}

// The whole scan for one wave: UPD = update wave (slot = w) or query wave (slot = (w + 2) & 3), NT tiles
// out of the NTS the table holds per slot.  Every instantiation runs the same iterations and barriers.
//
// Handoff layout (global, per workgroup and block parity): for slot s, tile pair p = kt / 2 and column
// tile ct, two uint4 per lane, the query operands hi and lo of the pair: bf16 of the 4 state values
// the lane holds for tile 2 p (.xy) and tile 2 p + 1 (.zw); an odd last tile fills .xy only.  The
// update wave writes its uint2 halves, the query wave loads whole operands.  The running denominators
// go to LDS (den_lds[parity][slot][tile * 16 + feature]).
template <bool UPD, int NT, int NTS, int NX, bool DBIG, int ES, int CT, int TOT, bool VX>
__device__ __forceinline__ void ws_body(const WsArgs& wa, int wg, int64_t bh, int fs, int cs, int seg, int slot,
                                        int qw) {
  const MomArgs& a = wa.m;
  constexpr int CG = 16 * CT;
  constexpr int LDQ = mom_ldq(DBIG);
  constexpr int KVF = ws_kv_floats(DBIG, CG);
  constexpr int QF = ws_q_floats(DBIG);
  constexpr int REDF = ws_red_floats(CG);
  // staging threads: in a segment-totals pass the query waves (indices tid - 256), else ws_stagers
  constexpr int STG = TOT != 0 ? 256 : ws_stagers(NX, DBIG);
  constexpr int NPS = (NTS + 1) / 2;  // operand pairs per slot in the handoff
  constexpr int NP = NT / 2;          // full tile pairs of this wave
  constexpr bool ODD = (NT & 1) != 0;
  extern __shared__ float smem[];
  float* const kvb = smem;              // [2][KVF]: Kt [KR][36], then the bf16 value planes
  float* const qb = smem + 2 * KVF;     // [2][QF]
  float* const redb = qb + 2 * QF;      // [2][REDF]
  float* const denb = redb + 2 * REDF;  // [2][4][NTS * 16]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int col0 = CG * cs;
  const bool den = cs == 0;
  const int n = static_cast<int>(a.n);
  const int nch_all = (n + a.shift + MOM_C - 1) / MOM_C;
  // this workgroup's chunks: [seg * seg_chunks, ...) of the sequence (the whole of it when nseg = 1)
  const int c_begin = wa.nseg > 1 ? seg * wa.seg_chunks : 0;
  const int nch = wa.nseg > 1 ? min(wa.seg_chunks, nch_all - c_begin) : nch_all;
  const int first = -a.shift + c_begin * MOM_C;
  const int cpb = wa.cpb;
  // handoff copies: the query waves load a block's state in the iteration after the update waves write
  // it and first use it one iteration later; with cpb >= 3 the next write comes after that iteration's
  // barrier, so one copy serves (half the footprint in L2), with cpb = 2 two alternate by block parity
  const int hmask = cpb >= 3 ? 0 : 1;
  constexpr bool totals = TOT != 0;       // phases 1 and 3: update only (TOT 1 and 2)
  const bool from_init = wa.phase == 2;   // start from the state before the segment
  // segment state of this (head, feature split, column group, segment): [4][NTS][CT][64] floatx4, den
  float* const sstate = wa.nseg > 1
                            ? wa.seg_state + ((((bh * a.fsplit + fs) * a.csplit + cs) * wa.nseg + seg) *
                                              static_cast<int64_t>(ws_seg_floats(NTS, CT)))
                            : nullptr;
  float* const sden = sstate ? sstate + 4 * NTS * CT * 256 : nullptr;
  const int64_t obase = (bh * a.fsplit + fs) * (a.n + 2 * MOM_GUARD) + MOM_GUARD;
  // TOT = 2 (phase 3, update only): accumulate into a persistent state in the reference's feature order
  // (a decode state), rows [0, n) of every head at head_rows rows apart; its own instantiation, so the
  // segment-totals pass (TOT = 1) keeps its registers
  constexpr bool persist = TOT == 2;
  const int64_t hstride = persist ? a.head_rows : a.n;
  const char* qh = static_cast<const char*>(a.q) + bh * hstride * a.ldk * ES;
  const char* kh = static_cast<const char*>(a.k) + bh * hstride * a.ldk * ES;
  const char* vh = static_cast<const char*>(a.v) + bh * hstride * a.ldv * ES;
  const WsRows rs{raw_rsrc(qh), raw_rsrc(kh), raw_rsrc(vh)};
  const int64_t tile0 = (static_cast<int64_t>(fs) * 4 + slot) * NTS;
  const MomLane<NT, NX> m = mom_lane<NT, NX>(a, tile0, li, lg);
  const WsSlots<DBIG, ES, CG, STG> sl = ws_slots<DBIG, ES, CG, STG>(a, col0, TOT != 0 ? tid - 256 : tid);
  const WsRedRel<CG> rrel = ws_red_rel<CG>(a, tid);
  // operand (pair p, column tile ct, hi / lo) of this slot and block parity par
  auto hand_at = [&](int par, int p, int ct, int hl) -> uint4* {
    return wa.hand + ((((static_cast<int64_t>(wg) * 2 + par) * 4 + slot) * NPS + p) * CT + ct) * 128 + hl * 64 + lane;
  };

  floatx4 st[UPD ? NT : 1][CT];
  float den_p[UPD ? NT : 1];  // per-lane partial denominators (this lane's tokens)
  bf16x8 sh[UPD || NP == 0 ? 1 : NP][CT], sv[UPD || NP == 0 ? 1 : NP][CT];
  uint2 oh[CT], ov[CT];  // the odd last tile's operands
  floatx4 dvv[UPD || NP == 0 ? 1 : NP][2];  // the frozen denominators of the lane's features (fp32)
  floatx4 odv = floatx4{0.f, 0.f, 0.f, 0.f};
  if constexpr (UPD) {
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
      den_p[kt] = 0.f;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) st[kt][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  } else {
    const bf16x8 z = __builtin_bit_cast(bf16x8, uint4{0u, 0u, 0u, 0u});
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
      for (int p = 0; p < NP; ++p) sh[p][ct] = sv[p][ct] = z;
      oh[ct] = ov[ct] = uint2{0u, 0u};
    }
#pragma unroll
    for (int p = 0; p < (NP > 0 ? NP : 1); ++p) dvv[p][0] = dvv[p][1] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  // zero every staging buffer (padding rows / columns are never written again) and the denominators of
  // block 0 (parity 0: the state before the first block is empty)
  for (int e = tid; e < 2 * (KVF + QF); e += WS_THREADS) smem[e] = 0.f;
  for (int e = tid; e < ws_den_floats(NTS); e += WS_THREADS) denb[e] = 0.f;
  __syncthreads();
  if constexpr (UPD && persist) {
    {
      // phase 3: the accumulators start at the persistent state (rowmap: the state row of every feature
      // slot, -1 for padding); its denominators ride in lane group 0's partials
      const float* snum = a.state_num + bh * a.n_feat * a.ldo;
      const float* sdn = a.state_den + bh * a.n_feat;
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = a.rowmap[(tile0 + kt) * 16 + 4 * lg + r];
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
            st[kt][ct][r] = row >= 0 ? snum[static_cast<int64_t>(row) * a.ldo + col0 + 16 * ct + li] : 0.f;
        }
        const int row = a.rowmap[(tile0 + kt) * 16 + li];
        den_p[kt] = (lg == 0 && row >= 0) ? sdn[row] : 0.f;
      }
    }
  }
  if constexpr (UPD) {
    if (from_init) {
      // phase 2: the accumulators start at S_init; its denominators ride in lane group 0's partials
      const floatx4* ss = reinterpret_cast<const floatx4*>(sstate) + (slot * NTS) * CT * 64 + lane;
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) st[kt][ct] = ss[(kt * CT + ct) * 64];
        den_p[kt] = lg == 0 ? sden[(slot * NTS + kt) * 16 + li] : 0.f;
      }
    }
  } else {
    if (from_init) {
      // phase 2: the rows of the segment's first block see S_init: split it into this wave's operands
      // and take its denominators
      const floatx4* ss = reinterpret_cast<const floatx4*>(sstate) + (slot * NTS) * CT * 64 + lane;
      auto tile = [&](int kt, int ct) { return ss[(kt * CT + ct) * 64]; };
#pragma unroll
      for (int p = 0; p < NP; ++p) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const floatx4 s0 = tile(2 * p, ct), s1 = tile(2 * p + 1, ct);
          uint4 h, l;
          split_pair(s0[0], s0[1], h.x, l.x);
          split_pair(s0[2], s0[3], h.y, l.y);
          split_pair(s1[0], s1[1], h.z, l.z);
          split_pair(s1[2], s1[3], h.w, l.w);
          sh[p][ct] = __builtin_bit_cast(bf16x8, h);
          sv[p][ct] = __builtin_bit_cast(bf16x8, l);
        }
      }
      if constexpr (ODD) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const floatx4 s0 = tile(NT - 1, ct);
          split_pair(s0[0], s0[1], oh[ct].x, ov[ct].x);
          split_pair(s0[2], s0[3], oh[ct].y, ov[ct].y);
        }
      }
      if (den) ws_den_vals<NT>(dvv, odv, sden + slot * NTS * 16, lg);
    }
  }
  // one register set of staged units: slot x (keys / values of chunk x, queries of chunk x - 1) is loaded
  // in iteration x - 2 and stored into LDS in iteration x - 1, so a load has one iteration to land.  (Two
  // sets alternating by iteration parity gave the loads two iterations, but the compiler merged the
  // sets with register copies at the loop latch, which wait for every load in flight: 6.42 against
  // 6.0 ms on c3.)
  // this wave stages chunks: in a segment-totals pass the query waves (the update waves only update)
  constexpr bool STAGE = TOT != 0 ? !UPD : (UPD || STG == WS_THREADS);
  WsStage<DBIG, ES, CG, STG> pre;
  if constexpr (STAGE) {
    ws_load_kv<DBIG, ES, CG, STG>(pre, sl, a, rs, first);
    ws_store_kv<DBIG, ES, CG, STG, true, VX>(pre, sl, a, kvb, reinterpret_cast<__bf16*>(kvb + mom_krows(DBIG) * MOM_LDT),
                                             first);
  }
  __syncthreads();
  if constexpr (STAGE) {
    ws_load_kv<DBIG, ES, CG, STG>(pre, sl, a, rs, first + MOM_C);  // slot 1
    if constexpr (TOT == 0) ws_load_q<DBIG, ES, CG, STG>(pre, sl, a, rs, first);
  }

  if constexpr (!UPD && TOT != 0) {
    // segment totals: the query waves stage the keys and values, with the same iterations and barriers
    for (int c = 0; c <= nch; ++c) {
      ws_stage_step<DBIG, ES, CG, STG, false, VX>(pre, sl, a, kvb, qb, c, nch, first, rs);
      __syncthreads();
    }
    return;
  }
  // staging of slot c + 1 (keys / values of chunk c + 1, queries of chunk c) from the registers and
  // loads of slot c + 2 into them; update waves: the reduction of chunk c - 2's partials.  The update
  // waves do it before their products (it touches only the next chunk's buffers and the partials of
  // two chunks back), so their VALU and matrix-core phases fall against the query waves' other ones;
  // the query waves after theirs (their state reload follows the last use of the old copy)
  auto stage_block = [&](int c) {
      {
        const int kv_row = first + (c + 1) * MOM_C;
        const int q_row = first + c * MOM_C;
        if (STAGE && c + 1 < nch) {
          float* Kt = kvb + ((c + 1) & 1) * KVF;
          __bf16* vp = reinterpret_cast<__bf16*>(Kt + mom_krows(DBIG) * MOM_LDT);
          if (kv_row >= 0 && kv_row + MOM_C <= n)
            ws_store_kv<DBIG, ES, CG, STG, false, VX>(pre, sl, a, Kt, vp, kv_row);
          else
            ws_store_kv<DBIG, ES, CG, STG, true, VX>(pre, sl, a, Kt, vp, kv_row);
        }
        if (STAGE && c < nch) {
          float* Qs = qb + (c & 1) * QF;
          if (q_row >= 0 && q_row + MOM_C <= n)
            ws_store_q<DBIG, ES, CG, STG, false>(pre, sl, a, Qs, q_row);
          else
            ws_store_q<DBIG, ES, CG, STG, true>(pre, sl, a, Qs, q_row);
        }
        // every path through the (conditional) stores above has the staged registers' loads complete here,
        // so the loads below into the same registers never wait for the younger handoff loads
        if constexpr (STAGE) ws_settle<DBIG, ES, CG, STG>(pre);
        if constexpr (!UPD) {
          // the state of the block chunk c starts (the query waves answer chunk c next iteration), written
          // by the update waves before the last barrier: loaded after this iteration's stores and before
          // the next slot's loads, so that waiting for the staged rows never waits for these
          if (c >= 1 && c % cpb == 0 && c < nch) {
            const int par = (c / cpb) & hmask;
  #pragma unroll
            for (int p = 0; p < NP; ++p) {
  #pragma unroll
              for (int ct = 0; ct < CT; ++ct) {
                sh[p][ct] = __builtin_bit_cast(bf16x8, *hand_at(par, p, ct, 0));
                sv[p][ct] = __builtin_bit_cast(bf16x8, *hand_at(par, p, ct, 1));
              }
            }
            if constexpr (ODD) {
  #pragma unroll
              for (int ct = 0; ct < CT; ++ct) {
                oh[ct] = *reinterpret_cast<const uint2*>(hand_at(par, NT / 2, ct, 0));
                ov[ct] = *reinterpret_cast<const uint2*>(hand_at(par, NT / 2, ct, 1));
              }
            }
            // the block's denominators (written with the state, block parity): zero in a workgroup
            // without the denominator column
            ws_den_vals<NT>(dvv, odv, denb + (((c / cpb) & 1) * 4 + slot) * NTS * 16, lg);
          }
        }
        // slot c + 2: unconditional loads with rows clamped into the sequence (past the end they are
        // never stored), one code path, so nothing waits on them before their store an iteration on
        if constexpr (STAGE) {
          ws_load_kv<DBIG, ES, CG, STG>(pre, sl, a, rs, kv_row + MOM_C);
          ws_load_q<DBIG, ES, CG, STG>(pre, sl, a, rs, q_row + MOM_C);
        }
        if constexpr (UPD) {
          if (!totals && c >= 2)
            ws_reduce_store<CG>(a, redb + (c & 1) * REDF, obase, first + (c - 2) * MOM_C, col0, den, rrel);
        }
      }
  };
  for (int c = 0; c <= nch; ++c) {
    if constexpr (UPD) stage_block(c);
    if constexpr (UPD) {
      if (c < nch) {
        const float* Kt = kvb + (c & 1) * KVF;
        if constexpr (persist)
          ws_update<NT, CT, NX, VX, true>(st, den_p, Kt, reinterpret_cast<const __bf16*>(Kt + mom_krows(DBIG) * MOM_LDT),
                                          m, li, lg);
        else
          ws_update<NT, CT, NX, VX>(st, den_p, Kt, reinterpret_cast<const __bf16*>(Kt + mom_krows(DBIG) * MOM_LDT), m, li,
                                  lg);
        if (!totals && (c + 1) % cpb == 0 && c + 1 < nch) {
          // the state the queries of block (c + 1) / cpb see -> handoff (parity of that block)
          const int par = ((c + 1) / cpb) & 1;
          const int hp = par & hmask;
#pragma unroll
          for (int kt = 0; kt < NT; ++kt) {
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
              uint32_t h0, h1, l0, l1;
              split_pair(st[kt][ct][0], st[kt][ct][1], h0, l0);
              split_pair(st[kt][ct][2], st[kt][ct][3], h1, l1);
              reinterpret_cast<uint2*>(hand_at(hp, kt >> 1, ct, 0))[kt & 1] = uint2{h0, h1};
              reinterpret_cast<uint2*>(hand_at(hp, kt >> 1, ct, 1))[kt & 1] = uint2{l0, l1};
            }
            if (den) {
              float t = den_p[kt];
              t += __shfl_xor(t, 16);
              t += __shfl_xor(t, 32);
              if (lg == 0) denb[(par * 4 + slot) * NTS * 16 + kt * 16 + li] = t;
            }
          }
        }
      }
    } else {
      if (c >= 1) {
        const float* Qs = qb + ((c - 1) & 1) * QF;
        floatx4 o[2][CT];
        float dq[2] = {0.f, 0.f};  // phi_q . den over the lane's features, row li + 16 tt (VALU, fp32)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) o[tt][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
        // operands of the first two tiles; each pair's successor is loaded once its features are formed
        WsQOps op0, op1;
        ws_qload<NT, NX, LDQ>(op0, 0, Qs, m, li);
        if (NT > 1) ws_qload<NT, NX, LDQ>(op1, NT > 1 ? 1 : 0, Qs, m, li);
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          bf16x8 ah[2], al[2];
          float x[2][8];
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            float x0[4], x1[4];
            ws_qfeat<NX>(x0, op0, tt);
            ws_qfeat<NX>(x1, op1, tt);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              x[tt][j] = x0[j];
              x[tt][4 + j] = x1[j];
            }
          }
          if (2 * p + 2 < NT) ws_qload<NT, NX, LDQ>(op0, 2 * p + 2 < NT ? 2 * p + 2 : 0, Qs, m, li);
          if (2 * p + 3 < NT) ws_qload<NT, NX, LDQ>(op1, 2 * p + 3 < NT ? 2 * p + 3 : 0, Qs, m, li);
          // the denominators' dot from the fp32 features, before the in-place split consumes them
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
            for (int j = 0; j < 4; ++j) dq[tt] = fmaf(x[tt][j], dvv[p][0][j], dq[tt]);
#pragma unroll
            for (int j = 0; j < 4; ++j) dq[tt] = fmaf(x[tt][4 + j], dvv[p][1][j], dq[tt]);
          }
          // materialised here, ahead of the split (left to the compiler, the chain sinks to its one use
          // after the products and every feature value then needs a copy next to its in-place split)
          asm volatile("" : "+v"(dq[0]), "+v"(dq[1]));
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) split_bf16(x[tt], ah[tt], al[tt]);
          ws_qpair_mma<CT>(o, ah, al, sh[p], sv[p]);
        }
        if constexpr (ODD) {
          uint2 ah[2], al[2];
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            float x0[4];
            ws_qfeat<NX>(x0, op0, tt);
#pragma unroll
            for (int j = 0; j < 4; ++j) dq[tt] = fmaf(x0[j], odv[j], dq[tt]);
            asm volatile("" : "+v"(dq[tt]));
            split_pair(x0[0], x0[1], ah[tt].x, al[tt].x);
            split_pair(x0[2], x0[3], ah[tt].y, al[tt].y);
          }
          ws_qsingle_mma<CT>(o, ah, al, oh, ov);
        }
        // this wave's partials of chunk c - 1 -> red[(c - 1) & 1], column-major (red_off); column CG:
        // the denominator sums (the lanes' dots summed over the 4 lane groups)
        float* rw = redb + ((c - 1) & 1) * REDF + qw * (CG + WS_RCOLS_EXTRA) * MOM_LDR;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
            *reinterpret_cast<floatx4*>(rw + red_off(16 * ct + li, 16 * tt + 4 * lg)) = o[tt][ct];
          if (den) {
            float t = dq[tt];
            t += __shfl_xor(t, 16);
            t += __shfl_xor(t, 32);
            if (lg == 0) rw[red_off(CG, 16 * tt + li)] = t;
          }
        }
      }
    }

    if constexpr (!UPD) stage_block(c);
    __syncthreads();
    }
  // partials of the last chunk (written by the query waves in iteration nch)
  if constexpr (UPD) {
    if (!totals) ws_reduce_store<CG>(a, redb + ((nch - 1) & 1) * REDF, obase, first + (nch - 1) * MOM_C, col0, den, rrel);
    if (totals && persist) {
      // phase 3: the slice back into the persistent state (each (head, feature, column) belongs to one
      // lane of the grid); the denominators from column group 0
      float* snum = a.state_num + bh * a.n_feat * a.ldo;
      float* sdn = a.state_den + bh * a.n_feat;
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
        float t = den_p[kt];
        t += __shfl_xor(t, 16);
        t += __shfl_xor(t, 32);
        const int row = a.rowmap[(tile0 + kt) * 16 + li];
        if (lg == 0 && cs == 0 && row >= 0) sdn[row] = t;
      }
    } else if (totals) {
      // phase 1: the segment's total (its keys only) for the scan over segments
      floatx4* ss = reinterpret_cast<floatx4*>(sstate) + (slot * NTS) * CT * 64 + lane;
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) ss[(kt * CT + ct) * 64] = st[kt][ct];
        float t = den_p[kt];
        t += __shfl_xor(t, 16);
        t += __shfl_xor(t, 32);
        if (lg == 0) sden[(slot * NTS + kt) * 16 + li] = t;
      }
    }
  }
}

// Workgroup -> (head, feature split, column group): consecutive logical ids share an XCD, so a head's
// workgroups share one L2 for its q / k / v rows.  Waves 0-3 update, 4-7 query.
// VX: bf16 values (ES = 2, dtype BF16), exact in bf16: the update leaves out the product with their zero
// lo plane (the state is that of the three-product form, bit for bit)
template <int NTS, int NX, bool DBIG, int ES, int CT, int TOT, bool VX>
__global__ __launch_bounds__(WS_THREADS, 1) void moments_ws_kernel(const WsArgs wa) {
  const MomArgs& a = wa.m;
  const int wg = xcd_remap(blockIdx.x, gridDim.x);
  // logical order (head, segment, feature split, column group): a segment's splits share an XCD
  const int per_seg = a.fsplit * a.csplit;
  const int per_head = per_seg * wa.nseg;
  const int64_t bh = wg / per_head;
  const int rem0 = wg - static_cast<int>(bh) * per_head;
  const int seg = rem0 / per_seg;
  const int rem = rem0 - seg * per_seg;
  const int fs = rem / a.csplit;
  const int cs = rem - fs * a.csplit;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int NTL = NTS > 1 ? NTS - 1 : NTS;
  if (w < 4) {
    const int slot = w;
    if (NTS > 1 && wa.mixed && slot >= 2)
      ws_body<true, NTL, NTS, NX, DBIG, ES, CT, TOT, VX>(wa, wg, bh, fs, cs, seg, slot, 0);
    else
      ws_body<true, NTS, NTS, NX, DBIG, ES, CT, TOT, VX>(wa, wg, bh, fs, cs, seg, slot, 0);
  } else {
    const int slot = (w - 4 + 2) & 3;
    if (NTS > 1 && wa.mixed && slot >= 2)
      ws_body<false, NTL, NTS, NX, DBIG, ES, CT, TOT, VX>(wa, wg, bh, fs, cs, seg, slot, w - 4);
    else
      ws_body<false, NTS, NTS, NX, DBIG, ES, CT, TOT, VX>(wa, wg, bh, fs, cs, seg, slot, w - 4);
  }
}

}  // namespace sta
