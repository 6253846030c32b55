// Host replay of the compressor's seed-derived randomness: for every sequence, its own CPU generator
// seeded with the sequence seed, consumed call after call exactly as the reference's compress calls
// consume it (fast_article_attention.py:326-348, streaming_taylor_coreset_attention.py:427-447):
//   * n_in <= 1 or compressor "none": nothing;
//   * compressor "random", or n_in <= 2: randperm(n_in);
//   * "sorted_pair": randn(d) normalised by clamp(norm, 1e-12), then rand(n_in / 2).
// The reference's randomness is torch's CPU generator (mt19937), so the replay issues the same ATen
// factory calls on at::CPUGeneratorImpl; what it removes is the per-call interpreter overhead, and
// independent sequences run on up to at::get_num_threads() host threads (each op is far below any
// intra-op parallel grain, so it runs on its calling thread).
//
// A plain C ABI (no torch types in the signatures).  Built with g++ against libtorch_cpu / libc10 into
// libstadraws.so, separate from the HIP library.

#include "../../include/stadraws.h"

#include <ATen/ATen.h>
#include <ATen/CPUGeneratorImpl.h>
#include <ATen/Parallel.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstring>
#include <exception>
#include <mutex>
#include <string>
#include <thread>
#include <type_traits>
#include <vector>

namespace {

enum { COMP_NONE = 0, COMP_RANDOM = 1, COMP_SORTED_PAIR = 2 };

thread_local std::string g_err;

int fail(const std::string& msg) {
  g_err = msg;
  return 1;
}

// Element types of the draws: the keys' dtype, since the reference draws the direction and the
// uniforms in it (fast_article_attention.py:339, :348; streaming_taylor_coreset_attention.py:441, :456),
// which selects torch's float, double or 16-bit sampling path.  Tables hold double for DRAW_F64 and float
// otherwise (16-bit values convert to float exactly).
enum { DRAW_F32 = 0, DRAW_F64 = 1, DRAW_BF16 = 2, DRAW_F16 = 3 };

at::ScalarType draw_scalar(int dt) {
  switch (dt) {
    case DRAW_F64: return at::kDouble;
    case DRAW_BF16: return at::kBFloat16;
    case DRAW_F16: return at::kHalf;
    default: return at::kFloat;
  }
}

// One sequence's calls; rows are zero-filled by the caller where a call draws nothing.  T is the
// table element (double for DRAW_F64, else float).
template <class T>
void replay(at::Generator& g, const int32_t* sizes, int n_calls, int d, int comp, int draw_type, T* dirs, T* unif,
            int32_t* perms, int max_in) {
  const auto opts = at::TensorOptions().dtype(draw_scalar(draw_type));
  const auto table = std::is_same<T, double>::value ? at::kDouble : at::kFloat;
  for (int c = 0; c < n_calls; ++c) {
    const int64_t n_in = sizes[c];
    if (comp == COMP_NONE || n_in <= 1) continue;
    if (comp == COMP_RANDOM || n_in <= 2) {
      at::Tensor p = at::randperm(n_in, g);  // int64, as torch.randperm
      const int64_t* src = p.data_ptr<int64_t>();
      int32_t* dst = perms + static_cast<int64_t>(c) * max_in;
      for (int64_t i = 0; i < n_in; ++i) dst[i] = static_cast<int32_t>(src[i]);
      continue;
    }
    at::Tensor dir = at::randn({d}, g, opts);
    dir = (dir / at::clamp(at::linalg_vector_norm(dir), 1e-12)).to(table);
    std::memcpy(dirs + static_cast<int64_t>(c) * d, dir.data_ptr<T>(), sizeof(T) * d);
    at::Tensor u = at::rand({n_in / 2}, g, opts).to(table);
    std::memcpy(unif + static_cast<int64_t>(c) * (max_in / 2), u.data_ptr<T>(), sizeof(T) * (n_in / 2));
  }
}

}  // namespace

namespace {

struct DrawSet {
  std::vector<at::Generator> gens;  // one per sequence / stream, in order
};

// Host threads for n_seq independent sequences: `want` (0: at::get_num_threads()), at most n_seq.
int threads_for(int64_t n_seq, int want) {
  const int base = want > 0 ? want : std::max(1, at::get_num_threads());
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(base, n_seq)));
}

// Runs fn(s) for s in [0, n_seq) on `threads` host threads (this one included); the first exception's
// message becomes the error.
template <class Fn>
int for_each_sequence(int64_t n_seq, int threads, Fn fn, const char* what) {
  std::atomic<int> bad{0};
  std::atomic<int64_t> next{0};
  std::mutex mu;
  std::string first_err;
  auto work = [&]() {
    for (int64_t s = next.fetch_add(1); s < n_seq; s = next.fetch_add(1)) {
      try {
        fn(s);
      } catch (const std::exception& e) {
        std::lock_guard<std::mutex> lock(mu);
        if (bad.fetch_add(1) == 0) first_err = e.what();
      }
    }
  };
  std::vector<std::thread> pool;
  try {
    for (int t = 1; t < threads; ++t) pool.emplace_back(work);
  } catch (const std::exception&) {
    // fewer threads than asked for: the ones running (and this one) take every sequence
  }
  work();
  for (auto& th : pool) th.join();
  if (bad.load()) return fail(what + first_err);
  return 0;
}

// Runs every sequence's calls, sequences spread over up to at::get_num_threads() threads; dirs / unif
// are double tables for DRAW_F64, float tables otherwise.
int run_calls(DrawSet& set, const int32_t* call_sizes, int n_calls, int d, int compressor, int max_in, int draw_type,
              void* dirs, void* unif, int32_t* perms) {
  const int64_t n_seq = static_cast<int64_t>(set.gens.size());
  if (n_calls < 0 || d <= 0 || max_in < 2) return fail("sta_draws: bad sizes");
  if (compressor < COMP_NONE || compressor > COMP_SORTED_PAIR) return fail("sta_draws: bad compressor");
  if (draw_type < DRAW_F32 || draw_type > DRAW_F16) return fail("sta_draws: bad draw element type");
  for (int c = 0; c < n_calls; ++c)
    if (call_sizes[c] < 0 || call_sizes[c] > max_in) return fail("sta_draws: call size above max_in");
  return for_each_sequence(n_seq, threads_for(n_seq, 0), [&](int64_t s) {
    if (draw_type == DRAW_F64)
      replay(set.gens[s], call_sizes, n_calls, d, compressor, draw_type, static_cast<double*>(dirs) + s * n_calls * d,
             static_cast<double*>(unif) + s * n_calls * (max_in / 2), perms + s * n_calls * max_in, max_in);
    else
      replay(set.gens[s], call_sizes, n_calls, d, compressor, draw_type, static_cast<float*>(dirs) + s * n_calls * d,
             static_cast<float*>(unif) + s * n_calls * (max_in / 2), perms + s * n_calls * max_in, max_in);
  }, "sta_draws: ");
}

// ---------------------------------------------------------------------------------------------------
// Reference-order selections.  The HIP compressor orders a call's items by fixed-order fp64 projection
// scores.  The reference orders them by torch's own `keys @ direction` (a BLAS gemv on the CPU, whose
// summation order belongs to the BLAS build and the host CPU) and torch.argsort
// (fast_article_attention.py:340-341, streaming_taylor_coreset_attention.py:443-444), so where two
// scores tie to within a few ulps the orders can differ.  select_sequence runs every compress call of
// one sequence's node plan on the host with those same ATen calls, in the keys' own dtype, on key
// matrices laid out as the reference's are (flat: a view of the caller's rows; levels: freshly
// stacked or concatenated rows), and applies the pair rule in that dtype; what it produces is the node
// tables the residual kernel reads.  The node plan is the one the HIP compressor runs
// (NODE_DESC ints per node: kind, a, b, n_in, n_out, method, draw slot, n_out of child a).

enum { KIND_RAW = 0, KIND_MERGE = 1 };
enum { M_COPY = 0, M_SORTED_PAIR = 1, M_PERM = 2 };
constexpr int NODE_DESC = 8;

// E: the keys' element type; Op: the type torch computes E's elementwise arithmetic in (float for
// float and the 16-bit types, double for double); T: the draw tables' element type.
template <class E>
using OpOf = typename std::conditional<std::is_same<E, double>::value, double, float>::type;

template <class E, class T>
void select_sequence(const E* keys, int64_t n, int d, at::ScalarType st, bool levels, const int32_t* desc,
                     int n_nodes, int cap, const T* dirs, const T* unif, const int32_t* perms, int max_in,
                     int32_t* node_src, float* node_w) {
  using Op = OpOf<E>;
  const auto opts = at::TensorOptions().dtype(st);
  const auto table = std::is_same<T, double>::value ? at::kDouble : at::kFloat;
  at::Tensor kall = at::from_blob(const_cast<E*>(keys), {n, d}, opts);
  std::vector<E> wts(static_cast<size_t>(n_nodes) * cap);  // node weights in E (merges read their children's)
  std::vector<int32_t> src;
  std::vector<E> w;
  for (int node = 0; node < n_nodes; ++node) {
    const int32_t* de = desc + static_cast<int64_t>(node) * NODE_DESC;
    const int kind = de[0], a = de[1], b = de[2], n_in = de[3], n_out = de[4], method = de[5], slot = de[6],
              na = de[7];
    if (n_in <= 0) continue;
    src.resize(n_in);
    w.resize(n_in);
    if (kind == KIND_RAW) {
      for (int i = 0; i < n_in; ++i) {
        src[i] = a + i;
        w[i] = E(1);
      }
    } else {
      for (int i = 0; i < n_in; ++i) {
        const int64_t at_ = i < na ? static_cast<int64_t>(a) * cap + i : static_cast<int64_t>(b) * cap + (i - na);
        src[i] = node_src[at_];
        w[i] = wts[at_];
      }
    }
    int32_t* osrc = node_src + static_cast<int64_t>(node) * cap;
    E* ow = wts.data() + static_cast<int64_t>(node) * cap;
    if (method == M_COPY) {
      for (int i = 0; i < n_in; ++i) {
        osrc[i] = src[i];
        ow[i] = w[i];
      }
    } else if (method == M_PERM) {
      // levels: weights[perm] * (n / m), in E's arithmetic (streaming_taylor_coreset_attention.py:427-437);
      // flat: a fresh full(m, n / m) (fast_article_attention.py:326-337)
      const int32_t* perm = perms + static_cast<int64_t>(slot) * max_in;
      const double factor = static_cast<double>(n_in) / static_cast<double>(n_out);
      for (int i = 0; i < n_out; ++i) {
        osrc[i] = src[perm[i]];
        ow[i] = levels ? E(static_cast<Op>(w[perm[i]]) * static_cast<Op>(factor)) : E(static_cast<Op>(factor));
      }
    } else {
      at::Tensor kk;
      if (kind == KIND_RAW) {
        kk = kall.narrow(0, a, n_in);
        if (levels) kk = kk.clone();  // the reference stacks the buffered rows into a fresh matrix
      } else {
        at::Tensor idx = at::empty({n_in}, at::TensorOptions().dtype(at::kLong));
        int64_t* ip = idx.data_ptr<int64_t>();
        for (int i = 0; i < n_in; ++i) ip[i] = src[i];
        kk = at::index_select(kall, 0, idx);  // fresh, as the reference's concatenated level rows
      }
      at::Tensor dir = at::empty({d}, opts);
      dir.copy_(at::from_blob(const_cast<T*>(dirs + static_cast<int64_t>(slot) * d), {d},
                              at::TensorOptions().dtype(table)));
      const at::Tensor order = at::argsort(at::matmul(kk, dir));
      const int64_t* ord = order.data_ptr<int64_t>();
      const T* u = unif + static_cast<int64_t>(slot) * (max_in / 2);
      const int pc = n_in / 2;
      for (int p = 0; p < pc; ++p) {
        const int64_t ia = ord[2 * p], ib = ord[2 * p + 1];
        const E wa = w[ia], wb = w[ib];
        const E ws = E(static_cast<Op>(wa) + static_cast<Op>(wb));
        const E lim = E(static_cast<Op>(1e-30));
        const E prob = E(static_cast<Op>(wa) / static_cast<Op>(static_cast<Op>(ws) < static_cast<Op>(lim) ? lim : ws));
        const bool keep_a = static_cast<Op>(E(static_cast<Op>(u[p]))) < static_cast<Op>(prob);
        osrc[p] = keep_a ? src[ia] : src[ib];
        ow[p] = ws;
      }
      if (n_in & 1) {
        const int64_t il = ord[n_in - 1];
        osrc[pc] = src[il];
        ow[pc] = w[il];
      }
    }
    float* ofw = node_w + static_cast<int64_t>(node) * cap;
    for (int i = 0; i < n_out; ++i) ofw[i] = static_cast<float>(ow[i]);
  }
}

// Checks a node plan before any node runs: kinds, methods, sizes within cap / max_in / n, children
// before their parents, draw slots within n_calls.
int check_plan(const int32_t* desc, int n_nodes, int cap, int64_t n, int n_calls, int max_in) {
  for (int node = 0; node < n_nodes; ++node) {
    const int32_t* de = desc + static_cast<int64_t>(node) * NODE_DESC;
    const int kind = de[0], a = de[1], b = de[2], n_in = de[3], n_out = de[4], method = de[5], slot = de[6],
              na = de[7];
    if (n_in <= 0) continue;
    if (n_out < 1 || n_out > cap || n_out > n_in) return fail("sta_host_select: node size out of range");
    if (method < M_COPY || method > M_PERM) return fail("sta_host_select: bad method");
    if (method == M_COPY && n_out != n_in) return fail("sta_host_select: copy node changes its size");
    if (method == M_SORTED_PAIR && (n_in < 3 || n_out != (n_in + 1) / 2))
      return fail("sta_host_select: sorted_pair node size");
    if (method == M_PERM && n_out != (n_in + 1) / 2) return fail("sta_host_select: permutation node size");
    if (method != M_COPY && (slot < 0 || slot >= n_calls || n_in > max_in))
      return fail("sta_host_select: draw slot or call size out of range");
    if (kind == KIND_RAW) {
      if (a < 0 || static_cast<int64_t>(a) + n_in > n) return fail("sta_host_select: raw node outside the sequence");
    } else if (kind == KIND_MERGE) {
      if (a < 0 || b < 0 || a >= node || b >= node) return fail("sta_host_select: merge child after its parent");
      const int nb = n_in - na;
      if (na < 0 || nb < 0 || na != desc[static_cast<int64_t>(a) * NODE_DESC + 4] ||
          nb != desc[static_cast<int64_t>(b) * NODE_DESC + 4])
        return fail("sta_host_select: merge sizes do not match the children");
    } else {
      return fail("sta_host_select: bad node kind");
    }
  }
  return 0;
}

}  // namespace

extern "C" {

// A set of n_seq CPU generators, generator s seeded seeds[s] (torch.Generator().manual_seed(seed)).
// Returns nullptr with sta_draws_error() set on failure.
void* sta_draws_open(const int64_t* seeds, int n_seq) {
  if (n_seq < 0) {
    fail("sta_draws_open: bad n_seq");
    return nullptr;
  }
  try {
    auto* set = new DrawSet;
    set->gens.reserve(n_seq);
    for (int s = 0; s < n_seq; ++s)
      set->gens.push_back(at::make_generator<at::CPUGeneratorImpl>(static_cast<uint64_t>(seeds[s])));
    return set;
  } catch (const std::exception& e) {
    fail(std::string("sta_draws_open: ") + e.what());
    return nullptr;
  }
}

void sta_draws_close(void* handle) { delete static_cast<DrawSet*>(handle); }

// Continues every generator of the set through n_calls compress calls of call_sizes[c] input items,
// in call order.  Outputs, zero-filled by the caller (a call that draws nothing leaves its rows):
//   dirs  float [n_seq, n_calls, d]          unit projection directions (sorted_pair calls)
//   unif  float [n_seq, n_calls, max_in/2]   pair uniforms (sorted_pair calls)
//   perms int32 [n_seq, n_calls, max_in]     permutations (random calls and calls on 2 items)
// compressor: 0 none, 1 random, 2 sorted_pair.  Returns 0, or 1 with sta_draws_error() set.
int sta_draws_next(void* handle, const int32_t* call_sizes, int n_calls, int d, int compressor, int max_in,
                   float* dirs, float* unif, int32_t* perms) {
  return sta_draws_next_typed(handle, call_sizes, n_calls, d, compressor, max_in, 0, dirs, unif, perms);
}

// sta_draws_next with the directions and uniforms drawn in the element type draw_type (0 float32,
// 1 float64: double tables; 2 bfloat16, 3 float16: float tables holding the 16-bit values).
int sta_draws_next_typed(void* handle, const int32_t* call_sizes, int n_calls, int d, int compressor, int max_in,
                         int draw_type, void* dirs, void* unif, int32_t* perms) {
  if (!handle) return fail("sta_draws_next: null handle");
  return run_calls(*static_cast<DrawSet*>(handle), call_sizes, n_calls, d, compressor, max_in, draw_type, dirs, unif,
                   perms);
}

// Bytes of one generator's state (the layout torch.Generator.get_state() returns for a CPU generator).
int64_t sta_draws_state_bytes(void) {
  try {
    return at::make_generator<at::CPUGeneratorImpl>(0).get_state().numel();
  } catch (const std::exception& e) {
    fail(std::string("sta_draws_state_bytes: ") + e.what());
    return -1;
  }
}

// Copies every generator's state out to / in from out[n_seq, sta_draws_state_bytes()].
int sta_draws_get_state(void* handle, uint8_t* out) {
  if (!handle) return fail("sta_draws_get_state: null handle");
  try {
    auto& gens = static_cast<DrawSet*>(handle)->gens;
    for (size_t s = 0; s < gens.size(); ++s) {
      at::Tensor st = gens[s].get_state();
      std::memcpy(out + s * st.numel(), st.data_ptr<uint8_t>(), st.numel());
    }
    return 0;
  } catch (const std::exception& e) {
    return fail(std::string("sta_draws_get_state: ") + e.what());
  }
}

int sta_draws_set_state(void* handle, const uint8_t* in) {
  if (!handle) return fail("sta_draws_set_state: null handle");
  try {
    auto& gens = static_cast<DrawSet*>(handle)->gens;
    const int64_t nb = sta_draws_state_bytes();
    if (nb <= 0) return 1;
    for (size_t s = 0; s < gens.size(); ++s) {
      at::Tensor st = at::empty({nb}, at::TensorOptions().dtype(at::kByte));
      std::memcpy(st.data_ptr<uint8_t>(), in + s * nb, nb);
      gens[s].set_state(st);
    }
    return 0;
  } catch (const std::exception& e) {
    return fail(std::string("sta_draws_set_state: ") + e.what());
  }
}

// One-shot form: fresh generators seeded seeds[s], run through the calls, then released.
int sta_host_draws(const int64_t* seeds, int n_seq, const int32_t* call_sizes, int n_calls, int d, int compressor,
                   int max_in, float* dirs, float* unif, int32_t* perms) {
  return sta_host_draws_typed(seeds, n_seq, call_sizes, n_calls, d, compressor, max_in, 0, dirs, unif, perms);
}

int sta_host_draws_typed(const int64_t* seeds, int n_seq, const int32_t* call_sizes, int n_calls, int d,
                         int compressor, int max_in, int draw_type, void* dirs, void* unif, int32_t* perms) {
  void* h = sta_draws_open(seeds, n_seq);
  if (!h) return 1;
  const int st = sta_draws_next_typed(h, call_sizes, n_calls, d, compressor, max_in, draw_type, dirs, unif, perms);
  sta_draws_close(h);
  return st;
}

int sta_host_select(const void* keys, int key_type, int64_t n_seq, int64_t n, int d, int levels,
                    const int32_t* desc, int n_nodes, int cap, const void* dirs, const void* unif,
                    const int32_t* perms, int n_calls, int max_in, int threads, int32_t* node_src, float* node_w) {
  if (!keys || !desc || !node_src || !node_w || (n_calls > 0 && (!dirs || !unif || !perms)))
    return fail("sta_host_select: null pointer");
  if (key_type < DRAW_F32 || key_type > DRAW_F16) return fail("sta_host_select: bad key element type");
  if (n_seq < 0 || n < 0 || d <= 0 || n_nodes < 0 || cap < 1 || n_calls < 0 || max_in < 2 || threads < 0)
    return fail("sta_host_select: bad sizes");
  if (check_plan(desc, n_nodes, cap, n, n_calls, max_in)) return 1;
  const at::ScalarType st = draw_scalar(key_type);
  const int64_t esz = static_cast<int64_t>(c10::elementSize(st));
  const bool lev = levels != 0;
  return for_each_sequence(n_seq, threads_for(n_seq, threads), [&](int64_t s) {
    const char* kb = static_cast<const char*>(keys) + s * n * d * esz;
    int32_t* os = node_src + s * n_nodes * cap;
    float* ow = node_w + s * n_nodes * cap;
    const int32_t* pm = perms + s * n_calls * max_in;
    const int64_t dro = s * n_calls * d, uo = s * n_calls * (max_in / 2);
    switch (key_type) {
      case DRAW_F64:
        select_sequence(reinterpret_cast<const double*>(kb), n, d, st, lev, desc, n_nodes, cap,
                        static_cast<const double*>(dirs) + dro, static_cast<const double*>(unif) + uo, pm, max_in, os, ow);
        break;
      case DRAW_BF16:
        select_sequence(reinterpret_cast<const c10::BFloat16*>(kb), n, d, st, lev, desc, n_nodes, cap,
                        static_cast<const float*>(dirs) + dro, static_cast<const float*>(unif) + uo, pm, max_in, os, ow);
        break;
      case DRAW_F16:
        select_sequence(reinterpret_cast<const c10::Half*>(kb), n, d, st, lev, desc, n_nodes, cap,
                        static_cast<const float*>(dirs) + dro, static_cast<const float*>(unif) + uo, pm, max_in, os, ow);
        break;
      default:
        select_sequence(reinterpret_cast<const float*>(kb), n, d, st, lev, desc, n_nodes, cap,
                        static_cast<const float*>(dirs) + dro, static_cast<const float*>(unif) + uo, pm, max_in, os, ow);
    }
  }, "sta_host_select: ");
}

const char* sta_draws_error(void) { return g_err.c_str(); }

}  // extern "C"
