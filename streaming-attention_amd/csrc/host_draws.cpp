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

// One sequence's calls; rows are zero-filled by the caller where a call draws nothing.  The direction
// and uniforms are drawn in the element type T (float, or double for a float64 caller: the reference
// draws them in the keys' dtype, fast_article_attention.py:339, :348; streaming_taylor_coreset_attention.py:441,
// :456), which selects torch's float or double sampling path.
template <class T>
void replay(at::Generator& g, const int32_t* sizes, int n_calls, int d, int comp, T* dirs, T* unif,
            int32_t* perms, int max_in) {
  const auto f32 = at::TensorOptions().dtype(std::is_same<T, double>::value ? at::kDouble : at::kFloat);
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
    at::Tensor dir = at::randn({d}, g, f32);
    dir = dir / at::clamp(at::linalg_vector_norm(dir), 1e-12);
    std::memcpy(dirs + static_cast<int64_t>(c) * d, dir.data_ptr<T>(), sizeof(T) * d);
    at::Tensor u = at::rand({n_in / 2}, g, f32);
    std::memcpy(unif + static_cast<int64_t>(c) * (max_in / 2), u.data_ptr<T>(), sizeof(T) * (n_in / 2));
  }
}

}  // namespace

namespace {

struct DrawSet {
  std::vector<at::Generator> gens;  // one per sequence / stream, in order
};

// Runs every sequence's calls, sequences spread over up to at::get_num_threads() threads; dirs / unif
// are float, or double when f64.
int run_calls(DrawSet& set, const int32_t* call_sizes, int n_calls, int d, int compressor, int max_in, int f64,
              void* dirs, void* unif, int32_t* perms) {
  const int64_t n_seq = static_cast<int64_t>(set.gens.size());
  if (n_calls < 0 || d <= 0 || max_in < 2) return fail("sta_draws: bad sizes");
  if (compressor < COMP_NONE || compressor > COMP_SORTED_PAIR) return fail("sta_draws: bad compressor");
  if (f64 != 0 && f64 != 1) return fail("sta_draws: bad element type flag");
  for (int c = 0; c < n_calls; ++c)
    if (call_sizes[c] < 0 || call_sizes[c] > max_in) return fail("sta_draws: call size above max_in");
  std::atomic<int> bad{0};
  std::atomic<int64_t> next{0};
  std::mutex mu;
  std::string first_err;
  auto work = [&]() {
    for (int64_t s = next.fetch_add(1); s < n_seq; s = next.fetch_add(1)) {
      try {
        if (f64)
          replay(set.gens[s], call_sizes, n_calls, d, compressor, static_cast<double*>(dirs) + s * n_calls * d,
                 static_cast<double*>(unif) + s * n_calls * (max_in / 2), perms + s * n_calls * max_in, max_in);
        else
          replay(set.gens[s], call_sizes, n_calls, d, compressor, static_cast<float*>(dirs) + s * n_calls * d,
                 static_cast<float*>(unif) + s * n_calls * (max_in / 2), perms + s * n_calls * max_in, max_in);
      } catch (const std::exception& e) {
        std::lock_guard<std::mutex> lock(mu);
        if (bad.fetch_add(1) == 0) first_err = e.what();
      }
    }
  };
  const int threads = static_cast<int>(std::min<int64_t>(std::max(1, at::get_num_threads()), n_seq));
  std::vector<std::thread> pool;
  try {
    for (int t = 1; t < threads; ++t) pool.emplace_back(work);
  } catch (const std::exception&) {
    // fewer threads than asked for: the ones running (and this one) take every sequence
  }
  work();
  for (auto& th : pool) th.join();
  if (bad.load()) return fail("sta_draws: " + first_err);
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

// sta_draws_next with the directions and uniforms drawn as float64 (f64 = 1; dirs / unif are double
// tables) or float32 (f64 = 0; float tables).
int sta_draws_next_typed(void* handle, const int32_t* call_sizes, int n_calls, int d, int compressor, int max_in,
                         int f64, void* dirs, void* unif, int32_t* perms) {
  if (!handle) return fail("sta_draws_next: null handle");
  return run_calls(*static_cast<DrawSet*>(handle), call_sizes, n_calls, d, compressor, max_in, f64, dirs, unif,
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
                         int compressor, int max_in, int f64, void* dirs, void* unif, int32_t* perms) {
  void* h = sta_draws_open(seeds, n_seq);
  if (!h) return 1;
  const int st = sta_draws_next_typed(h, call_sizes, n_calls, d, compressor, max_in, f64, dirs, unif, perms);
  sta_draws_close(h);
  return st;
}

const char* sta_draws_error(void) { return g_err.c_str(); }

}  // extern "C"
