// K3: block compressor (sorted_pair / random / copy) for the flat block coreset and for the
// merge-and-reduce level tree.
//
// Reference semantics:
//   flat : _compress_one_completed_block (fast_article_attention.py:312-361)
//   levels: MergeReduceCoreset._compress / _compress_random / _compress_sorted_pair
//           (streaming_taylor_coreset_attention.py:413-467), merge input = cat(old, new) (:404-408).
// A coreset item is represented by the global token index it came from plus its weight, so a merge
// node only needs its two children's (index, weight) lists; key rows are gathered from k for the
// projection score.  Random draws (normalised projection direction, pair uniforms, permutations) are
// inputs: they are a pure function of the seed and are replayed on the host in the reference order.
//
// sorted_pair on n items: score_i = <k_i, dir> accumulated in fp64 in index order then rounded to
// fp32; stable ascending sort of (score, position); pair p = sorted positions (2p, 2p+1); keep the
// first with probability w_a / max(w_a + w_b, 1e-30) (u_p < prob); the kept item carries w_a + w_b;
// an odd last item is kept with its own weight.
//
// float64 scoring (f64 = 1): the reference runs a float64 caller's compress calls in float64
// (directions and uniforms drawn as float64, scores keys @ direction in float64,
// fast_article_attention.py:339-348, streaming_taylor_coreset_attention.py:441-457).  The kernels then
// read the float64 key rows, the float64 direction and uniforms, keep the full fp64 score (rounded fp64
// products added in index order) as a 64-bit sort key and decide u < w_a / max(w_a + w_b, 1e-30) in
// fp64.
//
// A node is latency-bound work for one workgroup: every thread scores its own items straight from
// the key rows (16-byte loads, fp64 chain in dimension order), then the sorted order comes from one
// rank computation per item (count of smaller keys plus equal keys at lower positions), so the whole
// call needs three barriers.
#include "common.hpp"

namespace sta {

enum NodeKind : int { KIND_RAW = 0, KIND_MERGE = 1 };
enum NodeMethod : int { M_COPY = 0, M_SORTED_PAIR = 1, M_PERM = 2 };
constexpr int NODE_DESC = 8;  // kind, a, b, n_in, n_out, method, draw_slot, n_out of child a (merge)
constexpr int CMP_MAX_IN = 4096;
constexpr int CMP_THREADS = 256;
constexpr int CMP_MAX_D = 256;  // key width the direction buffer holds
// Ancestor scores (levels plans): a level-0 call also projects its key rows onto the directions of its
// node's ancestors at levels 1 .. CMP_MAX_ANC, so the merges there read one score per item instead of
// gathering the item's key row (the lower levels, where the merges' gathers are largest).
constexpr int CMP_MAX_ANC = 4;

// Dynamic LDS of compress_kernel for calls of at most max_in items (M = max_in rounded up to 4):
// sort keys [M] (16-byte aligned, padded for 4-wide reads; [2M] as 64-bit keys with f64), source
// indices [M], weights [M], sorted positions [M], projection direction [CMP_MAX_D] floats (doubles
// with f64), then with ancestor scores the node's and its ancestors' directions as doubles
// [1 + anc][d] (anc_dirs = 2 (1 + anc) d floats).
__host__ __device__ constexpr int cmp_round4(int n) { return (n + 3) & ~3; }
__host__ __device__ constexpr int cmp_key_floats(int max_in, bool f64) { return (f64 ? 2 : 1) * cmp_round4(max_in); }
__host__ __device__ constexpr int cmp_smem_floats(int max_in, bool f64 = false, int anc_dirs = 0) {
  return cmp_key_floats(max_in, f64) + 3 * cmp_round4(max_in) + (f64 ? 2 : 1) * CMP_MAX_D + anc_dirs;
}
// decode_compress_kernel: sort keys (as above), input handles, weights, positions, sorted positions [M]
// each, the running output's handles, weights, positions [M/2 + 1 rounded up to 4] each, direction.
__host__ __device__ constexpr int dec_cmp_smem_floats(int max_in, bool f64 = false) {
  return cmp_key_floats(max_in, f64) + 4 * cmp_round4(max_in) + 3 * cmp_round4(max_in / 2 + 1) +
         (f64 ? 2 : 1) * CMP_MAX_D;
}

struct CompressArgs {
  const void* k;
  int dtype;
  int64_t n;
  int d;
  const int32_t* batch;  // node ids handled by this launch (one workgroup per node and head)
  const int32_t* desc;   // [n_nodes][NODE_DESC]
  int n_nodes;
  int cap;
  const void* dirs;       // [BH][n_draws][d] float (double with f64)
  const void* unif;       // [BH][n_draws][max_in / 2] float (double with f64)
  const int32_t* perms;   // [BH][n_draws][max_in]
  int n_draws;
  int max_in;
  int32_t* node_src;  // [BH][n_nodes][cap]
  float* node_w;      // [BH][n_nodes][cap]
  int f64;            // 1: k is float64 [BH][n][d], draws float64 (float64 scoring)
  // ancestor scores (fp32 / 16-bit keys): anc [n_nodes][anc_levels] the draw slots of a raw node's
  // ancestors at levels 1 .. anc_levels (-1: no sorted_pair call there), node_level [n_nodes], lscore
  // [BH][anc_levels][n] the scores of every key row for its ancestor at each level; anc_levels = 0: off
  const int32_t* anc;
  const int32_t* node_level;
  int anc_levels;
  float* lscore;
};

// A bf16 / fp16 element from its 16 bits.
__device__ __forceinline__ float half_bits_to_float(uint16_t h, int dtype) {
  return dtype == BF16 ? __uint_as_float(static_cast<uint32_t>(h) << 16)
                       : static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Projection scores <row, dir> of one or two key rows (`two`): fp64 accumulation in dimension order,
// rounded to fp32 once (every fp32 x fp32 product is exact in fp64, so a score is a fixed function of
// the inputs).  Row r starts at element offset off_r of k_r (fp32 / bf16 / fp16) and is read in
// 16-byte units when `vec` (row starts 16-byte aligned, d a whole number of units).  The units of both
// rows are loaded B at a time before their products are accumulated, so up to 2 B loads are in flight
// instead of one load per accumulation step.
template <int B = 8>
__device__ __forceinline__ void projection_scores2(const void* k0, int64_t off0, const void* k1, int64_t off1,
                                                   bool two, int d, int dtype, bool vec, const float* dir,
                                                   float& s0, float& s1) {
  double a0 = 0.0, a1 = 0.0;
  if (vec && dtype == F32) {
    const floatx4* r0 = reinterpret_cast<const floatx4*>(static_cast<const float*>(k0) + off0);
    const floatx4* r1 = reinterpret_cast<const floatx4*>(static_cast<const float*>(k1) + off1);
    const int nu = d / 4;
    for (int u0 = 0; u0 < nu; u0 += B) {
      floatx4 x0[B], x1[B];
#pragma unroll
      for (int t = 0; t < B; ++t) {
        if (u0 + t < nu) {
          x0[t] = r0[u0 + t];
          if (two) x1[t] = r1[u0 + t];
        }
      }
#pragma unroll
      for (int t = 0; t < B; ++t) {
        if (u0 + t < nu) {
          const float* dr = dir + 4 * (u0 + t);
#pragma unroll
          for (int e = 0; e < 4; ++e) a0 = fma(static_cast<double>(x0[t][e]), static_cast<double>(dr[e]), a0);
          if (two) {
#pragma unroll
            for (int e = 0; e < 4; ++e) a1 = fma(static_cast<double>(x1[t][e]), static_cast<double>(dr[e]), a1);
          }
        }
      }
    }
  } else if (vec) {
    const uint4* r0 = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(k0) + off0);
    const uint4* r1 = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(k1) + off1);
    const int nu = d / 8;
    for (int u0 = 0; u0 < nu; u0 += B) {
      uint4 x0[B], x1[B];
#pragma unroll
      for (int t = 0; t < B; ++t) {
        if (u0 + t < nu) {
          x0[t] = r0[u0 + t];
          if (two) x1[t] = r1[u0 + t];
        }
      }
#pragma unroll
      for (int t = 0; t < B; ++t) {
        if (u0 + t < nu) {
          const float* dr = dir + 8 * (u0 + t);
          const uint32_t w0[4] = {x0[t].x, x0[t].y, x0[t].z, x0[t].w};
          const uint32_t w1[4] = {x1[t].x, x1[t].y, x1[t].z, x1[t].w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const double de = static_cast<double>(dr[e]);
            const int sh = (e & 1) * 16;
            a0 = fma(static_cast<double>(half_bits_to_float(static_cast<uint16_t>(w0[e >> 1] >> sh), dtype)), de, a0);
            if (two)
              a1 = fma(static_cast<double>(half_bits_to_float(static_cast<uint16_t>(w1[e >> 1] >> sh), dtype)), de, a1);
          }
        }
      }
    }
  } else {
    for (int col = 0; col < d; ++col) {
      const double de = static_cast<double>(dir[col]);
      a0 = fma(static_cast<double>(load_elem(k0, off0 + col, dtype)), de, a0);
      if (two) a1 = fma(static_cast<double>(load_elem(k1, off1 + col, dtype)), de, a1);
    }
  }
  s0 = static_cast<float>(a0);
  s1 = static_cast<float>(a1);
}

// Projection scores of one key row onto its node's direction (dird[0 .. d)) and its ancestors'
// (dird[(1 + l) d ..) for l < na), the directions held as doubles: every chain accumulates the fp64
// products in dimension order, as projection_scores2 does, so each equals the score the call at that
// level would compute from the row.  acc[0] is the node's own score, acc[1 + l] the ancestor's at level
// 1 + l.  fp32 rows are read in 16-byte units when `vec`; each element is converted once.
// rows of the level-0 launch read 4 units (64 bytes) at a time: 74 registers, 6 workgroups per compute
// unit (8 units: 90 registers, 5 per unit, c3 level 0 0.367 -> 0.338 ms for the 3 launches; 2 units:
// 66 registers, 7 per unit, 0.392 ms)
constexpr int ANC_RB = 4;
__device__ __forceinline__ void projection_scores_anc(const void* k, int64_t off, int d, int dtype, bool vec,
                                                      const double* dird, int na, double (&acc)[1 + CMP_MAX_ANC]) {
#pragma unroll
  for (int l = 0; l <= CMP_MAX_ANC; ++l) acc[l] = 0.0;
  auto step = [&](double x, int col) {
#pragma unroll
    for (int l = 0; l <= CMP_MAX_ANC; ++l)
      if (l <= na) acc[l] = fma(x, dird[l * d + col], acc[l]);
  };
  if (vec && dtype == F32) {
    const floatx4* r = reinterpret_cast<const floatx4*>(static_cast<const float*>(k) + off);
    const int nu = d / 4;
    for (int u0 = 0; u0 < nu; u0 += ANC_RB) {
      floatx4 x[ANC_RB];
#pragma unroll
      for (int t = 0; t < ANC_RB; ++t)
        if (u0 + t < nu) x[t] = r[u0 + t];
#pragma unroll
      for (int t = 0; t < ANC_RB; ++t) {
        if (u0 + t >= nu) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) step(static_cast<double>(x[t][e]), 4 * (u0 + t) + e);
      }
    }
  } else {
    for (int col = 0; col < d; ++col) step(static_cast<double>(load_elem(k, off + col, dtype)), col);
  }
}

// Unsigned key whose order is the float order (-0 = +0; NaN above everything), so that (key, position)
// is a strict total order and the ranks below are a permutation whatever the scores are.
__device__ __forceinline__ uint32_t sort_key(float f) {
  if (f == 0.f) return 0x80000000u;
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// The threads that compute one compress call together: the whole workgroup (CMP_THREADS threads,
// workgroup barriers) or one wave (64 lanes; its LDS accesses are ordered by the wave's own
// instruction order, so a code-motion barrier stands in for the workgroup barrier).
struct BlockGroup {
  static constexpr int threads = CMP_THREADS;
  // 16-byte units of a gathered key row in flight (projection_scores2): 4 keeps compress_kernel<false> at
  // 75 registers, 6 workgroups per compute unit (8: 107 registers, 4 per unit; compressor of c4 0.241 ->
  // 0.214 ms, of c2 0.037 -> 0.034 ms; 2: 59 registers, c4 0.206 but c2 0.039 ms)
  static constexpr int row_batch = 4;
  int tid;
  __device__ __forceinline__ void sync() const { __syncthreads(); }
};
// CMP_THREADS threads of a larger workgroup computing one compress call, in lockstep with the other
// groups: sync() is the workgroup barrier, counted, so that every group can pad its step to the same
// number of barriers (CMP_NODE_SYNCS) whatever path its call took.
struct LockGroup {
  static constexpr int threads = CMP_THREADS;
  static constexpr int row_batch = 4;  // the registers of a 1024-thread workgroup
  int tid;
  int* syncs;
  __device__ __forceinline__ void sync() const {
    __syncthreads();
    ++*syncs;
  }
};
// Workgroup barriers a compress call takes on any path: none (refused descriptor), 1 (the input list
// gathered: copy / permutation calls) or 3 (and the two of rank_sort / rank_sort64: sorted_pair).
constexpr int CMP_NODE_SYNCS = 3;

struct WaveGroup {
  static constexpr int threads = 64;
  static constexpr int row_batch = 4;
  int tid;  // lane
  __device__ __forceinline__ void sync() const {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
};

// Stable ascending order of n keys (ties by position): pos_s[rank(i)] = i with rank(i) = #{j: key_j <
// key_i} + #{j < i: key_j == key_i} = #{j < i: key_j <= key_i} + #{j > i: key_j < key_i}.  A wave ranks
// 64 consecutive items i0 .. i0 + 63 at a time: keys before i0 are compared with <=, keys after the
// band with <, only the band itself needs the position test (one compare and one add per key elsewhere).
// key_s holds the scores on entry (overwritten with sort keys); n <= CMP_MAX_IN; two group barriers.
template <class G>
__device__ __forceinline__ void rank_sort(float* key_s, int* pos_s, int n, const G& g) {
  const int tid = g.tid;
  constexpr int nthreads = G::threads;
  uint32_t* uk = reinterpret_cast<uint32_t*>(key_s);
  for (int i = tid; i < n; i += nthreads) uk[i] = sort_key(key_s[i]);
  for (int i = n + tid; i < ((n + 3) & ~3); i += nthreads) uk[i] = 0xffffffffu;  // padding of the 4-wide reads
  g.sync();
  const int n4 = (n + 3) & ~3;
  const int lane = tid & 63;
  // i0 and the loop bounds are wave-uniform (scalar loops); the key reads are issued 4 at a time (16
  // keys) before they are compared, into two counters
  for (int i0 = __builtin_amdgcn_readfirstlane(tid - lane); i0 < n; i0 += nthreads) {
    const int i = i0 + lane;
    const uint32_t me = i < n ? uk[i] : 0u;
    int r0 = 0, r1 = 0;
    for (int j = 0; j < i0; j += 16) {  // i0 is a multiple of 64
      uint4 o[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) o[t] = *reinterpret_cast<const uint4*>(uk + j + 4 * t);
#pragma unroll
      for (int t = 0; t < 4; t += 2) {
        r0 += (o[t].x <= me ? 1 : 0) + (o[t].y <= me ? 1 : 0) + (o[t].z <= me ? 1 : 0) + (o[t].w <= me ? 1 : 0);
        r1 += (o[t + 1].x <= me ? 1 : 0) + (o[t + 1].y <= me ? 1 : 0) + (o[t + 1].z <= me ? 1 : 0) +
              (o[t + 1].w <= me ? 1 : 0);
      }
    }
    const int band = min(i0 + 64, n4);
    for (int j = i0; j < band; j += 4) {
      const uint4 o = *reinterpret_cast<const uint4*>(uk + j);
      r0 += (o.x < me || (o.x == me && j + 0 < i)) ? 1 : 0;
      r1 += (o.y < me || (o.y == me && j + 1 < i)) ? 1 : 0;
      r0 += (o.z < me || (o.z == me && j + 2 < i)) ? 1 : 0;
      r1 += (o.w < me || (o.w == me && j + 3 < i)) ? 1 : 0;
    }
    int j = band;
    for (; j + 16 <= n4; j += 16) {  // padding keys (0xffffffff) are never below a key
      uint4 o[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) o[t] = *reinterpret_cast<const uint4*>(uk + j + 4 * t);
#pragma unroll
      for (int t = 0; t < 4; t += 2) {
        r0 += (o[t].x < me ? 1 : 0) + (o[t].y < me ? 1 : 0) + (o[t].z < me ? 1 : 0) + (o[t].w < me ? 1 : 0);
        r1 += (o[t + 1].x < me ? 1 : 0) + (o[t + 1].y < me ? 1 : 0) + (o[t + 1].z < me ? 1 : 0) +
              (o[t + 1].w < me ? 1 : 0);
      }
    }
    for (; j < n4; j += 4) {
      const uint4 o = *reinterpret_cast<const uint4*>(uk + j);
      r0 += (o.x < me ? 1 : 0) + (o.y < me ? 1 : 0) + (o.z < me ? 1 : 0) + (o.w < me ? 1 : 0);
    }
    if (i < n) pos_s[r0 + r1] = i;
  }
  g.sync();
}
__device__ __forceinline__ void rank_sort(float* key_s, int* pos_s, int n, int tid, int nthreads) {
  rank_sort(key_s, pos_s, n, BlockGroup{tid});
  (void)nthreads;  // CMP_THREADS
}

// Keep-first decision of the weighted pair rule: u < w_a / max(w_a + w_b, 1e-30)
// (streaming_taylor_coreset_attention.py:452-457; with unit weights the flat rule rand < 0.5,
// fast_article_attention.py:348).
__device__ __forceinline__ bool pair_keeps_first(float u, float wa, float wb) {
  return u < __fdiv_rn(wa, fmaxf(wa + wb, 1e-30f));
}
// The same in fp64 (float64 scoring: float64 uniforms; the weights are integers or products of n/m
// factors held in fp32, converted exactly).
__device__ __forceinline__ bool pair_keeps_first64(double u, float wa, float wb) {
  const double a = static_cast<double>(wa), b = static_cast<double>(wb);
  return u < a / fmax(a + b, 1e-30);
}

// Projection score of one float64 row: each fp64 product rounded, then added, in dimension order (no
// fused multiply-add, so the score is a fixed function of the inputs; 16-byte loads of two elements
// when `vec`).
__device__ __forceinline__ double fp64_mul_add(double acc, double x, double y) { return __dadd_rn(acc, __dmul_rn(x, y)); }
__device__ __forceinline__ double projection_score64(const double* row, int d, bool vec, const double* dir) {
  double acc = 0.0;
  if (vec) {
    const double2* r = reinterpret_cast<const double2*>(row);
    const int nu = d / 2;
    for (int u0 = 0; u0 < nu; u0 += 8) {
      double2 x[8];
#pragma unroll
      for (int t = 0; t < 8; ++t)
        if (u0 + t < nu) x[t] = r[u0 + t];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        if (u0 + t < nu) {
          acc = fp64_mul_add(acc, x[t].x, dir[2 * (u0 + t)]);
          acc = fp64_mul_add(acc, x[t].y, dir[2 * (u0 + t) + 1]);
        }
      }
    }
  } else {
    for (int col = 0; col < d; ++col) acc = fp64_mul_add(acc, row[col], dir[col]);
  }
  return acc;
}

// 64-bit unsigned key whose order is the double order (-0 = +0; NaN above everything).
__device__ __forceinline__ uint64_t sort_key64(double f) {
  if (f == 0.0) return 0x8000000000000000ull;
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(f));
  if ((u & 0x7fffffffffffffffull) > 0x7ff0000000000000ull) return 0xffffffffffffffffull;
  return (u & 0x8000000000000000ull) ? ~u : (u | 0x8000000000000000ull);
}

// Stable ascending order of n 64-bit keys (ties by position), the rule of rank_sort without its
// banded fast path: every thread counts, for each of its items, the keys below it and the equal keys
// at lower positions (float64 scoring only).  Two barriers.
template <class G>
__device__ __forceinline__ void rank_sort64(const uint64_t* uk, int* pos_s, int n, const G& g) {
  g.sync();
  for (int i = g.tid; i < n; i += G::threads) {
    const uint64_t me = uk[i];
    int r = 0;
    for (int j = 0; j < n; ++j) {
      const uint64_t o = uk[j];
      r += (o < me || (o == me && j < i)) ? 1 : 0;
    }
    pos_s[r] = i;
  }
  g.sync();
}
__device__ __forceinline__ void rank_sort64(const uint64_t* uk, int* pos_s, int n, int tid, int nthreads) {
  rank_sort64(uk, pos_s, n, BlockGroup{tid});
  (void)nthreads;  // CMP_THREADS
}

// One compress call: node `node` of sequence bh, computed by the threads of group g in their LDS region
// smem (cmp_smem_floats floats, 16-byte aligned).  ANC: raw (level-0) nodes also write their
// ancestors' scores (a separate instantiation: its score registers would cost every other launch
// occupancy).  Ends without a barrier after its last LDS read.
template <bool ANC, class G>
__device__ __forceinline__ void compress_node(const CompressArgs& a, const int node, const int64_t bh, const G& g,
                                              float* cmp_smem) {
  constexpr int CMP_THREADS = G::threads;  // the group's threads, in every loop below
  const int M = cmp_round4(a.max_in);
  const bool f64 = a.f64 != 0;
  const int KA = cmp_key_floats(a.max_in, f64);
  float* key_s = cmp_smem;
  int* src_s = reinterpret_cast<int*>(cmp_smem + KA);
  float* w_s = cmp_smem + KA + M;
  int* pos_s = reinterpret_cast<int*>(cmp_smem + KA + 2 * M);
  float* dir_s = cmp_smem + KA + 3 * M;  // 8-byte aligned: KA and M are multiples of 4
  double* dir64_s = reinterpret_cast<double*>(dir_s);

  const int tid = g.tid;
  const int32_t* dsc = a.desc + static_cast<int64_t>(node) * NODE_DESC;
  const int kind = dsc[0], ia = dsc[1], ib = dsc[2], n_in = dsc[3], n_out = dsc[4];
  const int method = dsc[5], slot = dsc[6], na = dsc[7];
  // descriptors come from the host plan; refuse anything the LDS arrays cannot hold (uniform exit)
  if (n_in <= 0 || n_in > CMP_MAX_IN || n_in > a.max_in || n_out > a.cap) return;
  if (kind == KIND_RAW && (ia < 0 || ia + n_in > a.n)) return;
  if (kind == KIND_MERGE && (na < 0 || na > n_in)) return;

  // ---- gather the input item list; in the same round trip the projection direction and the uniforms
  //      of this thread's first two pairs ----
  const bool pairs = method == M_SORTED_PAIR;
  const int64_t uoff = (bh * a.n_draws + slot) * (a.max_in / 2);
  const float* u = static_cast<const float*>(a.unif) + uoff;
  const double* u64 = static_cast<const double*>(a.unif) + uoff;
  const int pc = n_in / 2;
  double u_first[2] = {0.0, 0.0};  // a float uniform converts exactly
  // ancestor scores: a raw node's ancestors with a sorted_pair call (their directions follow the
  // node's own in LDS; slots of -1 get a zero direction, their scores are not written)
  const int na_lev = (ANC && kind == KIND_RAW && !f64 && a.anc_levels > 0) ? a.anc_levels : 0;
  double* dird_s = reinterpret_cast<double*>(dir_s + CMP_MAX_D);  // 8-byte aligned: CMP_MAX_D is even
  const int32_t* anc = a.anc + static_cast<int64_t>(node) * (na_lev > 0 ? na_lev : 0);
  if (pairs) {
    const int64_t doff = (bh * a.n_draws + slot) * a.d;
    if (f64) {
      for (int e = tid; e < a.d; e += CMP_THREADS) dir64_s[e] = static_cast<const double*>(a.dirs)[doff + e];
    } else {
      for (int e = tid; e < a.d; e += CMP_THREADS) dir_s[e] = static_cast<const float*>(a.dirs)[doff + e];
      // with ancestor scores: the node's direction and its ancestors' as doubles after the float one
      for (int e = tid; e < (na_lev > 0 ? (1 + na_lev) * a.d : 0); e += CMP_THREADS) {
        const int l = e / a.d;
        const int s_l = l == 0 ? slot : anc[l - 1];
        dird_s[e] = s_l >= 0 ? static_cast<double>(
                                   static_cast<const float*>(a.dirs)[(bh * a.n_draws + s_l) * a.d + (e - l * a.d)])
                             : 0.0;
      }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r)
      if (tid + r * CMP_THREADS < pc) u_first[r] = f64 ? u64[tid + r * CMP_THREADS] : u[tid + r * CMP_THREADS];
  }
  if (kind == KIND_RAW) {
    for (int i = tid; i < n_in; i += CMP_THREADS) {
      src_s[i] = ia + i;
      w_s[i] = 1.0f;
    }
  } else {
    const int64_t baseA = (bh * a.n_nodes + ia) * a.cap;
    const int64_t baseB = (bh * a.n_nodes + ib) * a.cap;
    // the children's token indices index key rows and score rows below: clamped to the sequence, so a
    // child list that was never written reads rows of this sequence instead of faulting
    const int hi = static_cast<int>(a.n - 1);
    for (int i = tid; i < n_in; i += CMP_THREADS) {
      const int64_t p = i < na ? baseA + i : baseB + (i - na);
      src_s[i] = min(max(a.node_src[p], 0), hi);
      w_s[i] = a.node_w[p];
    }
  }
  g.sync();

  const int64_t obase = (bh * a.n_nodes + node) * a.cap;
  if (method == M_COPY) {
    for (int i = tid; i < n_in; i += CMP_THREADS) {
      a.node_src[obase + i] = src_s[i];
      a.node_w[obase + i] = w_s[i];
    }
    return;
  }
  if (method == M_PERM) {
    const int32_t* perm = a.perms + (bh * a.n_draws + slot) * a.max_in;
    const float factor = static_cast<float>(static_cast<double>(n_in) / static_cast<double>(n_out));
    for (int i = tid; i < n_out; i += CMP_THREADS) {
      const int p = perm[i];
      a.node_src[obase + i] = src_s[p];
      a.node_w[obase + i] = w_s[p] * factor;
    }
    return;
  }

  // ---- sorted_pair: projection scores (fp64 accumulation, fixed index order), one item per thread ----
  if (f64) {
    const double* k64 = static_cast<const double*>(a.k);
    const bool vec64 = (a.d % 2) == 0 && (reinterpret_cast<uintptr_t>(a.k) & 15u) == 0;
    uint64_t* uk = reinterpret_cast<uint64_t*>(key_s);
    for (int i = tid; i < n_in; i += CMP_THREADS)
      uk[i] = sort_key64(projection_score64(k64 + (bh * a.n + src_s[i]) * a.d, a.d, vec64, dir64_s));
    rank_sort64(uk, pos_s, n_in, g);
  } else if (na_lev > 0) {
    // level-0 call with ancestor scores: the node's own score and the scores for its ancestors' calls
    // from one pass over each row
    const bool vec = a.dtype == F32 && (a.d % 4) == 0 && (reinterpret_cast<uintptr_t>(a.k) & 15u) == 0;
    for (int i = tid; i < n_in; i += CMP_THREADS) {
      double acc[1 + CMP_MAX_ANC];
      projection_scores_anc(a.k, (bh * a.n + src_s[i]) * a.d, a.d, a.dtype, vec, dird_s, na_lev, acc);
      key_s[i] = static_cast<float>(acc[0]);
#pragma unroll
      for (int l = 0; l < CMP_MAX_ANC; ++l) {
        if (l >= na_lev) break;
        if (anc[l] >= 0) a.lscore[(bh * na_lev + l) * a.n + src_s[i]] = static_cast<float>(acc[1 + l]);
      }
    }
    rank_sort(key_s, pos_s, n_in, g);
  } else if (kind == KIND_MERGE && !f64 && a.anc_levels > 0 && a.node_level[node] >= 1 &&
             a.node_level[node] <= a.anc_levels) {
    // a merge whose items' scores for this call were written by their level-0 calls
    const float* ls = a.lscore + (bh * a.anc_levels + (a.node_level[node] - 1)) * a.n;
    for (int i = tid; i < n_in; i += CMP_THREADS) key_s[i] = ls[src_s[i]];
    rank_sort(key_s, pos_s, n_in, g);
  } else {
    const int epu = a.dtype == F32 ? 4 : 8;
    const bool vec = (a.d % epu) == 0 && (reinterpret_cast<uintptr_t>(a.k) & 15u) == 0;
    for (int i = tid; i < n_in; i += 2 * CMP_THREADS) {  // items i and i + CMP_THREADS together
      const int i1 = i + CMP_THREADS;
      const bool two = i1 < n_in;
      float s0, s1;
      // (groups of a merge launch keep 4 units of each row in flight: their registers are shared by
      // every step of the launch; the level-0 launch with ancestor scores keeps 2 on this path, which
      // its raw nodes do not take, so that it does not set the launch's register count)
      projection_scores2<ANC ? 2 : G::row_batch>(a.k, (bh * a.n + src_s[i]) * a.d, a.k,
                                       (bh * a.n + src_s[two ? i1 : i]) * a.d, two, a.d, a.dtype, vec, dir_s, s0, s1);
      key_s[i] = s0;
      if (two) key_s[i1] = s1;
    }
    // ---- stable ascending order of (score, position) ----
    rank_sort(key_s, pos_s, n_in, g);
  }

  // ---- pair selection with weight transfer ----
  for (int p = tid; p < pc; p += CMP_THREADS) {
    const int ia2 = pos_s[2 * p], ib2 = pos_s[2 * p + 1];
    const float wa = w_s[ia2], wb = w_s[ib2];
    const int r = (p - tid) / CMP_THREADS;
    const bool choose_a = f64 ? pair_keeps_first64(r < 2 ? u_first[r] : u64[p], wa, wb)
                              : pair_keeps_first(r < 2 ? static_cast<float>(u_first[r]) : u[p], wa, wb);
    a.node_src[obase + p] = choose_a ? src_s[ia2] : src_s[ib2];
    a.node_w[obase + p] = wa + wb;
  }
  if ((n_in & 1) && tid == 0) {
    const int il = pos_s[n_in - 1];
    a.node_src[obase + pc] = src_s[il];
    a.node_w[obase + pc] = w_s[il];
  }
}

// One node of a.batch per workgroup (x) and sequence (y).
template <bool ANC>
__global__ __launch_bounds__(CMP_THREADS) void compress_kernel(const CompressArgs a) {
  extern __shared__ __align__(16) float cmp_smem[];
  compress_node<ANC>(a, a.batch[blockIdx.x], blockIdx.y, BlockGroup{static_cast<int>(threadIdx.x)}, cmp_smem);
}

// Merge nodes of several tree levels in one launch: workgroup x of sequence y runs `steps` steps; in
// step r its group g (GT threads: one wave, or CMP_THREADS threads in lockstep with the other groups)
// computes node table[(x * steps + r) * groups + g] (-1: none), then the workgroup meets at a barrier,
// so a step may read what the steps before it wrote (a subtree of merges: the nodes of its lowest
// level, then their parents, ...).  Each group has its own LDS region of region_floats floats.
template <int GT>
__global__ __launch_bounds__(1024) void compress_merge_kernel(const CompressArgs a, const int32_t* table, int steps,
                                                              int groups, int region_floats) {
  extern __shared__ __align__(16) float cmp_smem[];
  const int grp = threadIdx.x / GT;
  const int gtid = threadIdx.x - grp * GT;
  float* smem = cmp_smem + grp * region_floats;
  const int32_t* t = table + static_cast<int64_t>(blockIdx.x) * steps * groups + grp;
  for (int r = 0; r < steps; ++r) {
    const int node = __builtin_amdgcn_readfirstlane(t[r * groups]);
    const bool real = node >= 0 && node < a.n_nodes;
    if constexpr (GT == 64) {
      if (real) compress_node<false>(a, node, blockIdx.y, WaveGroup{gtid}, smem);
    } else {
      // every group takes exactly CMP_NODE_SYNCS workgroup barriers per step (padding after its call)
      int syncs = 0;
      if (real) compress_node<false>(a, node, blockIdx.y, LockGroup{gtid, &syncs}, smem);
      for (int k = __builtin_amdgcn_readfirstlane(syncs); k < CMP_NODE_SYNCS; ++k) __syncthreads();
    }
    __syncthreads();  // this step's node lists (global memory) and LDS reads before the next step
  }
}

// Segment-mean representatives (triton_article_attention.py:189-245): completed blocks that have a
// later query ((n-1)//block of them) are cut into block/stride segments of `stride` consecutive tokens;
// each representative is the mean key and mean value of its segment.  Output is fp32 [BH][R][d|dv].
struct SegMeanArgs {
  const void* k;
  const void* v;
  int dtype;
  int64_t n;
  int d;
  int dv;
  int stride;
  int64_t n_rep;  // R = ((n-1)//block) * (block/stride)
  float* rep_k;
  float* rep_v;
};

__global__ __launch_bounds__(256) void segment_mean_kernel(const SegMeanArgs a) {
  const int64_t bh = blockIdx.y;
  const int width = a.d + a.dv;
  const int64_t total = a.n_rep * width;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = e / width;
    const int col = static_cast<int>(e - r * width);
    const int64_t tok0 = r * a.stride;  // segments tile the usable prefix contiguously
    float acc = 0.f;
    if (col < a.d) {
      for (int s = 0; s < a.stride; ++s) acc += load_elem(a.k, (bh * a.n + tok0 + s) * a.d + col, a.dtype);
      a.rep_k[(bh * a.n_rep + r) * a.d + col] = acc / static_cast<float>(a.stride);
    } else {
      const int cv = col - a.d;
      for (int s = 0; s < a.stride; ++s) acc += load_elem(a.v, (bh * a.n + tok0 + s) * a.dv + cv, a.dtype);
      a.rep_v[(bh * a.n_rep + r) * a.dv + cv] = acc / static_cast<float>(a.stride);
    }
  }
}

}  // namespace sta
