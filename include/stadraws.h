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

/* The same with the directions and uniforms drawn in the element type draw_type: the reference draws
 * them in the keys' dtype (fast_article_attention.py:339, :348; streaming_taylor_coreset_attention.py:441,
 * :456), which selects torch's float, double or 16-bit sampling path.  draw_type: STA_DRAW_F32 (float
 * tables; sta_host_draws / sta_draws_next), STA_DRAW_F64 (double tables), STA_DRAW_BF16 / STA_DRAW_F16
 * (float tables holding the 16-bit values exactly). */
#define STA_DRAW_F32 0
#define STA_DRAW_F64 1
#define STA_DRAW_BF16 2
#define STA_DRAW_F16 3
int sta_host_draws_typed(const int64_t* seeds, int n_seq, const int32_t* call_sizes, int n_calls, int d,
                         int compressor, int max_in, int draw_type, void* dirs, void* unif, int32_t* perms);
int sta_draws_next_typed(void* handle, const int32_t* call_sizes, int n_calls, int d, int compressor, int max_in,
                         int draw_type, void* dirs, void* unif, int32_t* perms);

/* Reference-order selections: every compress call of a prefill's node plan run on the host, with the
 * items ordered as the reference orders them, by torch's CPU `keys @ direction` and torch.argsort in the
 * keys' dtype (fast_article_attention.py:339-361; streaming_taylor_coreset_attention.py:413-467), instead
 * of the HIP compressor's fixed-order fp64 scores (sta_compress_nodes).  The reference's score order
 * belongs to the host's BLAS, so this reproduces its selections on the host it runs on.
 *   keys      [n_seq, n, d] host rows in key_type (an STA_DRAW_* code), laid out as the caller's tensor
 *   levels    1: merge-and-reduce levels (raw blocks stacked fresh, permutation weights w * n / m);
 *             0: flat block coreset (raw blocks as views of the rows, permutation weights n / m)
 *   desc      int32 [n_nodes, 8] the node plan sta_compress_nodes runs (kind, a, b, n_in, n_out, method,
 *             draw slot, n_out of child a), children before parents
 *   dirs, unif, perms  the draw tables of sta_host_draws_typed for key_type, [n_seq, n_calls, ...]
 *   threads   host threads (0: torch's intra-op thread count)
 *   node_src  int32 [n_seq, n_nodes, cap], node_w float [n_seq, n_nodes, cap]: the tables
 *             sta_block_attention reads (global token index and weight of every kept item) */
int sta_host_select(const void* keys, int key_type, int64_t n_seq, int64_t n, int d, int levels,
                    const int32_t* desc, int n_nodes, int cap, const void* dirs, const void* unif,
                    const int32_t* perms, int n_calls, int max_in, int threads, int32_t* node_src, float* node_w);

/* Generator states in torch.Generator.get_state()'s CPU layout: out / in are [n_seq, state_bytes]. */
int64_t sta_draws_state_bytes(void);
int sta_draws_get_state(void* handle, uint8_t* out);
int sta_draws_set_state(void* handle, const uint8_t* in);

const char* sta_draws_error(void);

#ifdef __cplusplus
}
#endif

#endif /* STADRAWS_H */
