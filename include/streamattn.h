/*
 * streamattn.h -- C ABI of the MI355X (gfx950) streaming Taylor+coreset causal attention library
 * (libstreamattn.so).
 *
 * The reference (PositiveLoss/streaming-attention) is pure Python/PyTorch; its only host->device
 * crossing is the Triton launch at triton_article_attention.py:535-559.  Every entry point below is a
 * kernel launch that replaces one piece of the reference's hot path; the Python modules of this
 * package bind them with ctypes behind the reference's own Python API.
 *
 * Conventions
 *   - All tensors are caller-owned device buffers passed as raw pointers; the library never
 *     allocates or frees device memory (sta_decode_step_static's fixed static scratch aside).
 *     q/k are contiguous [BH, N, D], v is [BH, N, Dv].
 *   - dtype codes: STA_F32, STA_BF16, STA_F16 (inputs are read as such, arithmetic is fp32).
 *   - `stream` is a hipStream_t (NULL = the default stream); launches are asynchronous.
 *   - Every function returns STA_OK (0) or a positive status; sta_status_string() names it.
 */
#ifndef STREAMATTN_H
#define STREAMATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STA_OK 0
#define STA_ERR_SHAPE 1       /* inconsistent sizes / counts                          */
#define STA_ERR_UNSUPPORTED 2 /* degree, D, Dv or block beyond the kernels' limits     */
#define STA_ERR_DTYPE 3       /* unknown dtype code                                    */
#define STA_ERR_HIP 4         /* a HIP runtime call failed (see sta_last_hip_error)    */
#define STA_ERR_ARG 5         /* null pointer or out-of-range scalar argument          */
#define STA_ERR_SCRATCH 6     /* working set beyond the static scratch (sta_decode_step_static) */

/* Bytes of the static device scratch of sta_decode_step_static, per device. */
#define STA_STATIC_SCRATCH_BYTES ((int64_t)16 << 20)

#define STA_F32 0
#define STA_BF16 1
#define STA_F16 2
#define STA_F64 3 /* sta_compress_nodes only: float64 keys scored in fp64 against float64 draws */

#define STA_PRODUCTS_FP32 0       /* matrix-core products in fp32                                 */
#define STA_PRODUCTS_SPLIT_BF16 1 /* fp32 operands as bf16 hi + lo, three bf16 products            */

/* Library version (major*10000 + minor*100 + patch). */
int sta_version(void);

/* Human-readable name of a status code. */
const char* sta_status_string(int status);

/* hipError_t of the last failing HIP call made by this library on this thread (0 if none). */
int sta_last_hip_error(void);

/* Kernel limits: max D, max Dv, max Taylor degree, max compressor input size.  Within them: degree
 * 5 .. 8 needs D <= 64; the exact flash baseline (sta_flash_attention) takes D <= 128. */
int sta_limits(int* max_d, int* max_dv, int* max_degree, int* max_compress_in);

/*
 * Exact low-degree Taylor moments over all keys *before* each row's chunk (K1).
 * Replaces low_degree_taylor_causal_sums / _stream / _prefix (fast_article_attention.py:184-285) and
 * TaylorMomentSketch.update/query (streaming_taylor_coreset_attention.py:265-296).
 *   chunk c covers rows [c*chunk - shift, (c+1)*chunk - shift); chunk must be sta_moment_chunk(d).
 *   feat_quads [fsplit][4][wave_tiles][4], feat_coef [fsplit][4][wave_tiles][16]: the symmetric monomial
 *     basis in tiles of 4 quads, wave_tiles tiles for each of the 4 waves of each feature split (padded
 *     with coefficient-0 tiles).  A quad packs i0 | b<<8 | i2<<16 | i3<<24 (b a multiple of 4, at most d;
 *     unused factors = d) and holds the features x[i0] x[b+s] x[i2] x[i3], s = 0..3, of
 *     [x_0..x_{D-1}, 1, 0, 0, 0] (degree 4 needs d <= 64; index d+1 selects a 0, for zero-valued
 *     padding); feat_coef is the key-side coefficient 1/prod(alpha!) of each feature (0 for padding).
 *     Exception: with STA_PRODUCTS_SPLIT_BF16 and degree <= 2 the kernel sums plain monomials and
 *     applies feat_coef[16 t] to tile t's query-side monomials, so each tile's 16 entries must be one
 *     value c_t with c_t * (sum of the tile's slot monomials) equal to the tile's coefficient-weighted
 *     sum (e.g. 1/2 on every slot of a diagonal tile x[4k+r] x[4k+s]; the planner's
 *     tile_coefficients).  wave_tiles must be a count the library is built for
 *     (sta_moment_wave_tiles).
 *   q and k rows are ld_qk elements apart and v rows ldv (a multiple of 32, >= dv); rows are read in
 *     16-byte units, so d times the element size must be a multiple of 16 (pad rows with zero columns
 *     otherwise: zero dimensions only add zero-valued features), and q, k, v must be 16-byte aligned.
 *   d is the staged key width (at most 128).  windows == NULL: rows are d long (ld_qk == d) and the
 *     feature indices are dimensions.  Keys wider than 128 (ld_qk a multiple of 32, 128 <= ld_qk <= 256,
 *     degree <= 4) go through dimension windows: windows [fsplit][4] (device, int32) gives, for every
 *     feature split, the first row dimension of its 4 blocks of 32 dimensions (entries clamped to
 *     [0, ld_qk - 32]); the split stages d = 128 "virtual" dimensions 32 b + j = row dimension
 *     windows[4 fs + b] + j, and its feature quads index those virtual dimensions (the planner assigns
 *     every monomial to one split whose window holds its dimensions).
 *   Degrees 5 .. 8 (d <= 64): STA_PRODUCTS_FP32 and 32 columns only; each quad is then two words,
 *     i0 | b<<8 | i2<<16 | i3<<24 and i4 | i5<<8 | i6<<16 | i7<<24 (feat_quads [fsplit][4][wave_tiles][4][2]),
 *     the features x[i0] x[b+s] x[i2] ... x[i7] (unused factors = d).
 *   grid: bh * fsplit * ceil(dv/columns) workgroups of 256 threads.
 *   products: STA_PRODUCTS_FP32 (fp32 matrix cores; products of the fp32 features exact) or
 *     STA_PRODUCTS_SPLIT_BF16 (each fp32 operand as bf16 hi + lo, three bf16 matrix-core products per
 *     product: about 2^-16 relative error per product, 16x the fp32 matrix-core rate).  Feature values,
 *     the denominator column and all sums stay fp32 either way.
 *   columns: value columns per workgroup, 32 (grid bh * fsplit * ceil(dv/32)) or 64
 *     (sta_moment_columns_ok; grid bh * fsplit).
 *   outputs (fp32, partial over feature splits), in the layout sta_moment_partials_layout gives:
 *     low_num [BH][fsplit][rows][ld], low_den [BH][fsplit][rows], row i stored at row_offset + i.
 */
int sta_moments(const void* q, const void* k, const void* v, int dtype, int64_t bh, int64_t n, int d, int ld_qk,
                int dv, int ldv, int degree, float scale, int chunk, int shift, int fsplit, int wave_tiles, int mixed,
                int products, int columns, const uint32_t* feat_quads, const float* feat_coef,
                const int32_t* windows, float* low_num, float* low_den, void* stream);

/*
 * Wave-specialised form of sta_moments (split-bf16 products, degree <= 3): moments over all keys before
 * each row's *query block* of query_block rows (a multiple of 32, at least 64; blocks offset by shift
 * like the chunks, block b covers rows [b*query_block - shift, (b+1)*query_block - shift)).  Same
 * reference functions as sta_moments; with query_block equal to the article block the residual
 * kernel's in-block keys carry exp(x) whole (sta_block_attention with chunk = query_block).
 *   One workgroup of 512 threads per (head, feature split, group of 16*column_tiles value columns):
 *   4 update waves keep the fp32 state, 4 query waves a frozen split copy refreshed once per block.
 *   feat_quads [fsplit][4][slot_tiles][4] / feat_coef [fsplit][4][slot_tiles][16]: 4 slots of
 *     slot_tiles tiles per feature split (layout and coefficient rules of sta_moments, per-tile query
 *     coefficients at degree <= 2); mixed = 1: slots 2 and 3 hold slot_tiles - 1 real tiles (their
 *     last table tile is padding).  slot_tiles must satisfy sta_moments_ws_ok.
 *   column_tiles: 4 (64 columns per workgroup; ceil(dv/32) must be even) or 2 (32 columns).
 *   handoff: caller-allocated scratch of sta_moments_ws_handoff_bytes(...) bytes, 16-byte aligned (the
 *     per-workgroup copy of the state between the update and the query waves; contents undefined
 *     before and after the call).
 *   q / k / v row rules, outputs and their layout as for sta_moments.
 */
int sta_moments_ws(const void* q, const void* k, const void* v, int dtype, int64_t bh, int64_t n, int d, int dv,
                   int ldv, int degree, float scale, int query_block, int shift, int fsplit, int slot_tiles, int mixed,
                   int column_tiles, const uint32_t* feat_quads, const float* feat_coef, void* handoff,
                   float* low_num, float* low_den, void* stream);

/* 1 when sta_moments_ws runs (d, degree, slot_tiles, column_tiles, dv), else 0. */
int sta_moments_ws_ok(int d, int degree, int slot_tiles, int column_tiles, int dv);

/* Bytes of sta_moments_ws' handoff scratch for bh heads, fsplit splits, slot_tiles, column_tiles, dv. */
int64_t sta_moments_ws_handoff_bytes(int64_t bh, int fsplit, int slot_tiles, int column_tiles, int dv);

/*
 * sta_moments_ws with each head's sequence cut into nseg segments of seg_blocks query blocks (every
 * segment non-empty), one workgroup per (head, segment, feature split, column group), for prefills
 * with too few heads to fill the GPU.  Same outputs (the moment sums of fast_article_attention.py:217-259,
 * at fp32 rounding: a segment's state starts from the earlier segments' total).  Three launches: the
 * update side of every segment from a zero state, writing its total to seg_state; an exclusive scan
 * over the segments; every segment's scan starting from the state before it.
 *   seg_state: caller-allocated scratch of sta_moments_ws_seg_bytes(...) bytes, 16-byte aligned.
 *   handoff: sta_moments_ws_handoff_bytes(bh * nseg, ...) bytes.
 * nseg = 1 is sta_moments_ws (seg_blocks and seg_state unused).
 */
int sta_moments_ws_seg(const void* q, const void* k, const void* v, int dtype, int64_t bh, int64_t n, int d, int dv,
                       int ldv, int degree, float scale, int query_block, int shift, int fsplit, int slot_tiles,
                       int mixed, int column_tiles, const uint32_t* feat_quads, const float* feat_coef, void* handoff,
                       float* low_num, float* low_den, int nseg, int seg_blocks, float* seg_state, void* stream);

/* Bytes of sta_moments_ws_seg's segment-state scratch. */
int64_t sta_moments_ws_seg_bytes(int64_t bh, int fsplit, int slot_tiles, int column_tiles, int dv, int nseg);

/* 1 when sta_moments runs (d, degree, dv, wave_tiles, products) with columns = 64: one workgroup per
 * (head, feature split) covering all value columns (split-bf16 products, 32 < dv <= 64, mixed = 0;
 * one workgroup per compute unit). */
int sta_moment_columns_ok(int d, int degree, int dv, int wave_tiles, int products);

/* 1 when sta_moments runs (d, degree, wave_tiles) with mixed = 1: the feature splits fs >= fsplit/2
 * (fsplit even) then use wave_tiles - 1 tiles per wave (slot wave_tiles of their waves is padding). */
int sta_moment_mixed_ok(int d, int degree, int wave_tiles);

/* Smallest per-wave tile count >= want that sta_moments supports for (d, degree); -1 if none. */
int sta_moment_wave_tiles(int d, int degree, int want);

/* Layout of sta_moments' partial outputs for a sequence of n rows and dv value columns: rows per
 * (head, split) including guard rows, row stride of low_num, and the storage row of sequence row 0. */
int sta_moment_partials_layout(int64_t n, int dv, int64_t* rows, int* ld, int* row_offset);

/* Moment workgroups the kernel keeps resident per compute unit at (d, per-wave tile count): 1 or 2
 * (degree <= 4; sta_moment_occupancy_degree for any degree). */
int sta_moment_occupancy(int d, int wave_tiles);
int sta_moment_occupancy_degree(int d, int degree, int wave_tiles);

/*
 * Persistent moment state update (the decode state; K1's update without the query):
 *   state_num[h][f][c] += sum_{j<n} phi_k(k_j)[f] v_j[c],  state_den[h][f] += sum_{j<n} phi_k(k_j)[f]
 * for rows [0, n) of every head h (head h starts head_rows rows after head h-1 in k and v).
 * Replaces TaylorMomentSketch.update (streaming_taylor_coreset_attention.py:265-280), applied to a whole
 * block of tokens at once (the block completion of a decode step, or a prompt).
 *   Feature table as for sta_moments (wave_tiles tiles of 4 quads per wave) plus feat_rows
 *   [fsplit][4][wave_tiles][16]: the state row of every feature slot in the reference's feature order
 *   (degree 0, 1, ..., each in combinations_with_replacement order), -1 for padding slots.
 *   state_num [BH][n_feat][ld] with ld = 32*ceil(dv/32), state_den [BH][n_feat], fp32, accumulated in
 *   place.  k / v row rules, ld_k and windows (keys wider than 128) as for sta_moments' q / k.
 *   products: STA_PRODUCTS_FP32 or STA_PRODUCTS_SPLIT_BF16 (as for sta_moments; the state and the
 *   sums stay fp32 either way; degrees 5 .. 8 need STA_PRODUCTS_FP32).
 */
int sta_moment_accumulate(const void* k, const void* v, int dtype, int64_t bh, int64_t n, int64_t head_rows, int d,
                          int ld_k, int dv, int ldv, int degree, int fsplit, int wave_tiles,
                          const uint32_t* feat_quads, const float* feat_coef, const int32_t* feat_rows,
                          const int32_t* windows, int n_feat, int products, float* state_num, float* state_den,
                          void* stream);

/*
 * Block form of sta_moment_accumulate for short runs of rows (a decode block completion): the same
 * state update, bit for bit, for split-bf16 products, degree <= 2, d <= 64 (rows d elements apart,
 * no windows) and (wave_tiles, column_tiles) = (2, 2), (4, 2) or (2, 4) (sta_moment_accumulate's
 * feature tables at that tile count).  One workgroup per (head, group of 16 column_tiles value
 * columns; 32 ceil(dv / 32) a multiple of it) stages up to 256 rows at a time once, then runs every
 * feature slice of the state through them (more rows: groups of 256, the state read and written per
 * group).  STA_ERR_UNSUPPORTED outside those limits.
 */
int sta_moment_accumulate_block(const void* k, const void* v, int dtype, int64_t bh, int64_t n, int64_t head_rows,
                                int d, int dv, int ldv, int degree, int fsplit, int wave_tiles, int column_tiles,
                                const uint32_t* feat_quads, const float* feat_coef, const int32_t* feat_rows,
                                int n_feat, float* state_num, float* state_den, void* stream);

/*
 * sta_moment_accumulate on the wave-specialised kernel's update-only pass (split-bf16 products, degree
 * <= 3, d <= 128): 4 update waves per workgroup keep the state of 4 slots of slot_tiles feature tiles x
 * 16 column_tiles columns in matrix-core accumulators, loaded from and stored back to the persistent
 * state through feat_rows; the other 4 waves stage the chunks.  Tables in the layout of sta_moments_ws
 * ([fsplit][4 slots][slot_tiles][...], mixed: slots 2 and 3 one tile less) with the per-feature key-side
 * coefficients; ldv and the state's row stride 32 ceil(dv / 32) multiples of 16 column_tiles.  Same
 * reference function as sta_moment_accumulate (TaylorMomentSketch.update,
 * streaming_taylor_coreset_attention.py:265-280).
 */
int sta_moment_accumulate_ws(const void* k, const void* v, int dtype, int64_t bh, int64_t n, int64_t head_rows, int d,
                             int ld_k, int dv, int ldv, int degree, int fsplit, int slot_tiles, int mixed,
                             int column_tiles, const uint32_t* feat_quads, const float* feat_coef,
                             const int32_t* feat_rows, int n_feat, float* state_num, float* state_den, void* stream);

/*
 * Streaming decode (K5) for S streams in lockstep: ArticleStreamingAttention.update / query
 * (streaming_taylor_coreset_attention.py:576-609).  The state of stream s (fp32, caller-owned):
 *   moments of the tokens of completed blocks   state_num [S][F][ldv], state_den [S][F] (reference order)
 *   the current block's tokens (the buffer)     buf_k [S][block][dk], buf_v [S][block][ldv]
 *   level coresets                              lev_k [S][L][m][dk], lev_v [S][L][m][ldv], lev_w [S][L][m],
 *                                               lev_pos [S][L][m] (sequence positions), m = ceil(block/2)
 * with zero padding columns.  A query returns low + exp over the buffered tokens + weighted exp_{>t}
 * over the occupied levels' items, the reference's low + tail regrouped (the buffered tokens' Taylor
 * part lives in their exact exponential instead of the moments).
 */

/* Row lengths of the decode buffers: dk = 4*ceil(d/4) (32*ceil(d/32) for d > 128), ldv = 32*ceil(dv/32). */
int sta_decode_layout(int d, int dv, int* dk, int* ldv);

/*
 * Moment part of a decode query: part_num[s][p][c] = sum over features f of split p of
 * phi_q(scale*q_s)[f] state_num[s][f][c] (part_den likewise), splits = feature splits per stream.
 * feat_index: the factors of every feature into x = [scale*q, 1] (index d is the constant 1 and fills
 * the unused factors); index_width 4: uint32 [F] packed i0 | i1 << 8 | i2 << 16 | i3 << 24 (d < 255,
 * degree <= 4); index_width 8: uint16 [F][8] (d <= 256, degree <= 8).
 * Replaces TaylorMomentSketch.query (streaming_taylor_coreset_attention.py:282-296).
 */
int sta_decode_moments(const void* q, int dtype, int64_t streams, int d, int dv, float scale, const float* state_num,
                       const float* state_den, int n_feat, const void* feat_index, int index_width, int splits,
                       float* part_num, float* part_den, void* stream);

/*
 * Buffer append and query of a decode step.  flags: 1 APPEND (write k, v [S][d|dv] into buffer slot
 * buf_len), 2 CURRENT (the appended token also counts as a buffered token of this query), 4 QUERY
 * (out[s] = (low + tail numerators) / max(den, eps) in out_dtype; low from sta_decode_moments'
 * partials).  level_mask: bit l set = level l occupied (the completed-block counter).  stats [S][4]
 * (optional): denominator, the reference's low and tail denominators, coreset item count.
 * Replaces MergeReduceCoreset.append / items (streaming_taylor_coreset_attention.py:376-394, :469-490)
 * and the query tail and normalisation of ArticleStreamingAttention.query (:581-609).
 */
int sta_decode_tail(const void* q, const void* k, const void* v, int dtype, int64_t streams, int d, int dv,
                    int degree, float scale, float eps, int flags, float* buf_k, float* buf_v, int block, int buf_len,
                    const float* lev_k, const float* lev_v, const float* lev_w, int n_levels, int level_size,
                    uint64_t level_mask, const float* part_num, const float* part_den, int splits, void* out,
                    int out_dtype, float* stats, void* stream);

/*
 * No counterpart in the reference: a decode step that allocates nothing, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The same launches as sta_decode_moments followed by sta_decode_tail (flags must
 * include QUERY), with the moment partials part_num [S][splits][ldv] and part_den [S][splits] held in a
 * static device array of STA_STATIC_SCRATCH_BYTES per device instead of caller buffers
 * (ldv = 32*ceil(dv/32); S * splits * ldv rounded up to 64, plus S * splits, floats must fit, else
 * STA_ERR_SCRATCH).  state_num == state_den == NULL: no moment state (compressor "none"), the partials
 * are zeroed by a kernel.  Every call on a device shares that device's array: calls that overlap on
 * one device (concurrent streams, or host threads) race; calls on one stream are ordered.  The
 * first call on a device looks up the array's address there (hipGetSymbolAddress).
 */
int64_t sta_static_scratch_bytes(void);
int sta_decode_step_static(const void* q, const void* k, const void* v, int dtype, int64_t streams, int d, int dv,
                           int degree, float scale, float eps, int flags, const float* state_num,
                           const float* state_den, int n_feat, const void* feat_index, int index_width, int splits,
                           float* buf_k, float* buf_v, int block, int buf_len, const float* lev_k, const float* lev_v,
                           const float* lev_w, int n_levels, int level_size, uint64_t level_mask, void* out,
                           int out_dtype, float* stats, void* stream);

/*
 * Block completion: compress the full buffer (call 0) and merge cat(level i-1, previous output) for
 * calls i = 1 .. n_calls-1 (the occupied levels below the counter's lowest zero bit), writing the
 * result as level n_calls-1.  methods [n_calls] (1 sorted_pair, 2 permutation) and the draws dirs
 * [S][n_calls][d], unif [S][n_calls][max_in/2], perms [S][n_calls][max_in] as for sta_compress_nodes;
 * pos0 = sequence position of buffer row 0.  Replaces MergeReduceCoreset.append's compression and
 * _insert_level (streaming_taylor_coreset_attention.py:387-467).
 *   score_f64 = 1 (a float64 caller, whose reference runs its compress calls in float64): dirs and unif
 *   are double, and the projection scores are taken in fp64 from buf_k64 [S][block][dk] / lev_k64
 *   [S][n_levels][level_size][dk], the float64 values of the key rows; lev_k64 rows are written beside
 *   lev_k's.  score_f64 = 0: dirs / unif are float and buf_k64 / lev_k64 are ignored (may be NULL).
 */
int sta_decode_compress(int64_t streams, int d, int dv, const float* buf_k, const float* buf_v, int block, int pos0,
                        float* lev_k, float* lev_v, float* lev_w, int32_t* lev_pos, int n_levels, int level_size,
                        int n_calls, const int32_t* methods, const void* dirs, const void* unif,
                        const int32_t* perms, int max_in, int score_f64, const double* buf_k64, double* lev_k64,
                        void* stream);

/*
 * Block compressor for one batch of coreset nodes (K3), all heads at once.
 * Replaces _compress_one_completed_block (fast_article_attention.py:312-361) for the flat block coreset
 * and MergeReduceCoreset._compress* (streaming_taylor_coreset_attention.py:413-467) for level merges.
 *   batch_nodes[n_batch]: node ids to compute in this launch (their inputs must already exist).
 *   node_desc[n_nodes][8]: kind (0 raw block, 1 merge), a, b (raw: first token; merge: child ids),
 *     n_in, n_out, method (0 copy, 1 sorted_pair, 2 permutation), draw slot, n_out of child a (merge; 0 raw).
 *   dirs [BH][n_draws][D] (normalised projection), unif [BH][n_draws][max_in/2] (pair uniforms),
 *   perms [BH][n_draws][max_in] (randperm draws): the seed-derived draws, replayed by the host.
 *   dtype STA_F64: k is float64 and dirs / unif are double (the draws of a float64 caller); scores are
 *   fp64 products and sums kept whole for the sort, the pair rule is decided in fp64.  Otherwise dirs /
 *   unif are float and scores are fp64 sums of the fp32 products rounded to fp32.
 *   outputs: node_src [BH][n_nodes][cap] (global token index of each kept item), node_w (its weight).
 *   Ancestor scores (levels plans, fp32 / 16-bit keys; anc_levels = 0 and NULLs: off): in a launch that
 *     passes anc [n_nodes][anc_levels] (the draw slots of each raw node's ancestors at levels 1 ..
 *     anc_levels, -1 where that call is not sorted_pair), each raw node's call also projects its key
 *     rows onto those directions and writes level_scores [BH][anc_levels][n]; in later launches (anc
 *     NULL, the same anc_levels and level_scores) a merge node at level 1 .. anc_levels (node_level
 *     [n_nodes]) reads its items' scores there instead of gathering their key rows.  Every score is the
 *     fp64 chain the merge would compute, so the nodes are the same bit for bit.  anc_levels <= 4.
 */
int sta_compress_nodes(const void* k, int dtype, int64_t bh, int64_t n, int d, const int32_t* batch_nodes,
                       int n_batch, const int32_t* node_desc, int n_nodes, int cap, const void* dirs,
                       const void* unif, const int32_t* perms, int n_draws, int max_in, int32_t* node_src,
                       float* node_w, const int32_t* node_level, const int32_t* anc, int anc_levels,
                       float* level_scores, void* stream);

/*
 * Merge nodes of several levels of a levels plan in one launch (K3): the compress calls of
 * MergeReduceCoreset._insert_level's cascade (streaming_taylor_coreset_attention.py:396-411, each call
 * :413-467), the same node values as sta_compress_nodes run level by level.  A workgroup of `groups`
 * thread groups runs `steps` steps with a barrier after each, so a step may read the nodes of the
 * steps before it; in a step each group computes one node:
 *   group_threads 256: groups (<= 4) of 256 threads in lockstep (every group takes the same number of
 *     workgroup barriers per step, whatever its call does); 64: groups (<= 16) of one wave each;
 *   node_table [n_groups][steps][groups]: the node each group computes in each step (-1: none), the
 *     same for every head (grid n_groups x bh).  A node's children must be nodes of an earlier launch
 *     or of an earlier step of the same workgroup (e.g. a subtree: the nodes of one level, then their
 *     parents, ..., its root);
 *   node_level, anc_levels, level_scores: as sta_compress_nodes' later launches (merges at levels 1 ..
 *     anc_levels read the scores their level-0 calls wrote).
 * Other arguments as sta_compress_nodes.  LDS: the call's arrays for every group, groups * (4 M + 256)
 * floats with M = max_in rounded up to 4 (float64: groups * (5 M + 512)); STA_ERR_UNSUPPORTED above
 * 160 KiB.
 */
int sta_compress_merges(const void* k, int dtype, int64_t bh, int64_t n, int d, const int32_t* node_table,
                        int n_groups, int steps, int groups, int group_threads, const int32_t* node_desc,
                        int n_nodes, int cap, const void* dirs, const void* unif, const int32_t* perms, int n_draws,
                        int max_in, int32_t* node_src, float* node_w, const int32_t* node_level, int anc_levels,
                        float* level_scores, void* stream);

/*
 * Segment-mean representatives of completed blocks (the Triton path's coreset).
 * Replaces build_segment_mean_coreset (triton_article_attention.py:189-245).
 *   n_rep = ((N-1)//block) * (block/stride); outputs rep_k [BH][n_rep][D], rep_v [BH][n_rep][Dv] fp32.
 */
int sta_segment_mean(const void* k, const void* v, int dtype, int64_t bh, int64_t n, int d, int dv, int block,
                     int stride, int64_t n_rep, float* rep_k, float* rep_v, void* stream);

/*
 * Fused residual + normalisation per tile of 128 query rows (K2 + K4).
 * Replaces _full_residual_tail / _block_coreset_residual_tail and the combine
 * (fast_article_attention.py:437-514, :596-598), the query side of ArticleStreamingAttention
 * (streaming_taylor_coreset_attention.py:581-599) and _article_direct_kernel
 * (triton_article_attention.py:265-369).
 *   mode: 0 flat block coreset, 1 merge-and-reduce levels, 2 exact residual (compressor "none"),
 *     3 Taylor part only (no residual; used with out_den for the raw low-degree sums).
 *   tiles: tile t covers rows [t*128 - shift, (t+1)*128 - shift); n_tiles = ceil((N+shift)/128).
 *   tile_ptr[n_tiles+1] / tile_nodes: CSR list of the nodes each tile needs.
 *   node_meta[n_nodes][4]: item count, first and last active row, materialized flag (items index
 *     rep_k/rep_v instead of k/v).
 *   low_num / low_den: sta_moments' (or sta_moments_ws') partial outputs (sta_moment_partials_layout),
 *     fsplit splits; chunk: their chunk (sta_moment_chunk) or query block, a multiple of the moment
 *     chunk that divides or is a multiple of the tile rows.
 *   ld_qk / ld_v: row strides (elements) of q, k and of v, multiples of 4 (rows are read in units of
 *     4 elements; pad them with zero columns), bases 16-byte aligned.
 *   rep_k / rep_v (fp32, row strides ld_rep_k / ld_rep_v, multiples of 4): materialized items
 *     (segment means; fp32 inputs only), NULL otherwise.
 *   exp_clamp: 1 evaluates exp(min(x, 80)) as the Triton kernel does.
 *   products: STA_PRODUCTS_FP32 or STA_PRODUCTS_SPLIT_BF16 for the logits q.k and the weighted value
 *     sums (see sta_moments); weights, exponentials and all sums stay fp32.  Degrees 4 .. 8 need
 *     STA_PRODUCTS_FP32 (STA_ERR_UNSUPPORTED otherwise).  d <= 256.
 *   out: [BH][N][Dv] in out_dtype.
 *   out_den: NULL for the normalised output; otherwise out must be fp32 and receives the numerator
 *     and out_den [BH][N] the denominator, unnormalised (the low_num/low_den pair of
 *     low_degree_taylor_causal_sums, fast_article_attention.py:262-285, when mode is 3).
 */
int sta_block_attention(const void* q, const void* k, const void* v, int dtype, int64_t bh, int64_t n, int d,
                        int dv, int ld_qk, int ld_v, int degree, float scale, float eps, int mode, int block, int chunk,
                        int shift, int exp_clamp, int products, const float* low_num, const float* low_den, int fsplit,
                        const int32_t* tile_ptr, const int32_t* tile_nodes, int n_tiles, const int32_t* node_meta,
                        int n_nodes, int cap, const int32_t* node_src, const float* node_w, const float* rep_k,
                        const float* rep_v, int ld_rep_k, int ld_rep_v, int64_t n_rep, void* out, int out_dtype,
                        float* out_den, void* stream);

/*
 * Exact causal softmax attention, FlashAttention-style (online row maximum, no N x N scores).
 * Replaces _flash_causal_kernel / triton_flash_causal_attention (triton_article_attention.py:372-435,
 * :580-637):  out_i = sum_{j<=i} exp(s q_i.k_j - m_i) v_j / max(sum_{j<=i} exp(s q_i.k_j - m_i), 1e-20).
 *   q, k rows are ld_qk elements apart (a multiple of 4, >= d; columns [d, ld_qk) are ignored), v rows
 *   ld_v (a multiple of 4, >= dv); q, k, v 16-byte aligned.  out [BH][N][Dv] dense, dtype out_dtype.
 *   d <= 128, dv <= 256.  fp32 accumulation; products of the inputs are exact (fp32 matrix cores).
 */
int sta_flash_attention(const void* q, const void* k, const void* v, int dtype, int64_t bh, int64_t n, int d,
                        int dv, int ld_qk, int ld_v, float scale, void* out, int out_dtype, void* stream);

/* Rows per block-attention tile and the moment chunk the library uses for a head dimension D (the
 * chunk argument of sta_block_attention is that chunk for sta_moments' partials, the query block for
 * sta_moments_ws' partials). */
int sta_tile_rows(void);
int sta_moment_chunk(int d);

/*
 * Self-test of the matrix-core operand layout assumed by the kernels: computes D = A(16x4) * B(4x16)
 * with one v_mfma_f32_16x16x4_f32 from a[64], b[64] given in the assumed lane layout and writes the
 * 16x16 result row-major to d_out[256].  Device buffers, synchronous.
 */
int sta_selftest_mfma(const float* a, const float* b, float* d_out);

#ifdef __cplusplus
}
#endif

#endif /* STREAMATTN_H */
