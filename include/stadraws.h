/* libstadraws.so: host replay of the coreset compressor's seed-derived randomness.
 *
 * The reference draws the randomness of every compress call from torch's CPU generator, one
 * sequence (or stream) per generator seeded seed + b*H + h, in call order:
 *   - sorted_pair on n_in > 2 items: randn(d), normalised by clamp(norm, 1e-12), then rand(n_in / 2)
 *     (fast_article_attention.py:339-348, streaming_taylor_coreset_attention.py:439-447);
 *   - random, or n_in <= 2: randperm(n_in) (fast_article_attention.py:326-337,
 *     streaming_taylor_coreset_attention.py:427-437);
 *   - none, or n_in <= 1: nothing.
 * These entry points issue the same generator calls on at::CPUGeneratorImpl (so the draws are the
 * reference's bit for bit) for many sequences in parallel host threads.  They replace the
 * per-call Python loop a binding would otherwise run; the HIP library (streamattn.h) consumes the
 * tables they fill (dirs / unif / perms arguments of sta_compress_nodes and sta_decode_compress).
 *
 * Tables, zero-filled by the caller, row-major:
 *   dirs  float   [n_seq, n_calls, d]
 *   unif  float   [n_seq, n_calls, max_in / 2]
 *   perms int32_t [n_seq, n_calls, max_in]
 * compressor: 0 none, 1 random, 2 sorted_pair.  Functions returning int return 0 on success and 1 on
 * failure, with the message in sta_draws_error() (per calling thread).
 */
#ifndef STADRAWS_H
#define STADRAWS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Fresh generators seeded seeds[s], run through the calls, released. */
int sta_host_draws(const int64_t* seeds, int n_seq, const int32_t* call_sizes, int n_calls, int d, int compressor,
                   int max_in, float* dirs, float* unif, int32_t* perms);

/* Persistent generator sets for streaming decode (one generator per stream, continued block after
 * block, as the reference's coreset object keeps its generator, streaming_taylor_coreset_attention.py:367-368). */
void* sta_draws_open(const int64_t* seeds, int n_seq);
void sta_draws_close(void* handle);
int sta_draws_next(void* handle, const int32_t* call_sizes, int n_calls, int d, int compressor, int max_in,
                   float* dirs, float* unif, int32_t* perms);

/* The same with the directions and uniforms drawn as float64 when f64 = 1 (dirs / unif are double
 * tables): the reference draws them in the keys' dtype (fast_article_attention.py:339, :348;
 * streaming_taylor_coreset_attention.py:441, :456), so a float64 caller's draws come from torch's double
 * sampling path.  f64 = 0 is sta_host_draws / sta_draws_next (float tables). */
int sta_host_draws_typed(const int64_t* seeds, int n_seq, const int32_t* call_sizes, int n_calls, int d,
                         int compressor, int max_in, int f64, void* dirs, void* unif, int32_t* perms);
int sta_draws_next_typed(void* handle, const int32_t* call_sizes, int n_calls, int d, int compressor, int max_in,
                         int f64, void* dirs, void* unif, int32_t* perms);

/* Generator states in torch.Generator.get_state()'s CPU layout: out / in are [n_seq, state_bytes]. */
int64_t sta_draws_state_bytes(void);
int sta_draws_get_state(void* handle, uint8_t* out);
int sta_draws_set_state(void* handle, const uint8_t* in);

const char* sta_draws_error(void);

#ifdef __cplusplus
}
#endif

#endif /* STADRAWS_H */
