"""ORACLE -- test infrastructure only.

CPU restatement of the reference's streaming Taylor+coreset attention hot path, used as the checker
for the HIP kernels.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module; the product path (streaming-attention_amd/) never does.

Each function cites the reference file:line it restates.  Floating-point arithmetic is torch on the
CPU (fp32 where the reference computes in fp32, fp64 for closed-form checks); integer work (sorting,
pair selection, level bookkeeping) is numpy.  The reference's RNG is torch's CPU generator, replayed
here in the reference's own call order (torch 2.10.0, CPU mt19937).

Pinning (see tests/test_oracle.py): exp_taylor known answers; feature counts C(d+l-1, l) and order ==
itertools.combinations_with_replacement; phi_k . phi_q == exp_{<=t} by brute force; moment sums ==
quadratic closed form; compressor="none" == fp64 softmax attention; sorted_pair / random selections,
flat and level-merge outputs == golden vectors written from the reference (tests/golden/); level
invariants (occupancy == binary counter, weight 2^(l+1), weights sum to the tokens compressed); the
blocked online-softmax recursion of the flash baseline == torch.softmax attention for every block size,
and its special cases (one key: out = v_0; equal keys: running mean of v).
"""

from __future__ import annotations

import itertools
import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

Tensor = torch.Tensor


# ----------------------------------------------------------------------------- primitives

def attention_scale(scale: Optional[float], dim: int) -> float:
    """fast_article_attention.py:76-77"""
    return float(1.0 / math.sqrt(dim) if scale is None else scale)


def exp_taylor(x: Tensor, degree: int) -> Tensor:
    """fast_article_attention.py:95-104 (term = term * x / r; out = out + term)."""
    out = torch.ones_like(x)
    term = torch.ones_like(x)
    for r in range(1, degree + 1):
        term = term * x / float(r)
        out = out + term
    return out


def classical_attention(q: Tensor, k: Tensor, v: Tensor, scale: float) -> Tensor:
    """Causal softmax attention in float64 (fast_article_attention.py:116-129 evaluated exactly)."""
    q64, k64, v64 = q.double(), k.double(), v.double()
    n = q.shape[-2]
    logits = (q64 @ k64.transpose(-1, -2)) * scale
    mask = torch.ones(n, n, dtype=torch.bool).tril()
    return torch.softmax(logits.masked_fill(~mask, float("-inf")), dim=-1) @ v64


def flash_attention_blocked(q: Tensor, k: Tensor, v: Tensor, scale: float, block_n: int = 64) -> Tensor:
    """The online-softmax recursion of _flash_causal_kernel (triton_article_attention.py:397-428) in
    float64 for one [N, D] sequence: keys in blocks of block_n; per block the row maximum
    m_new = max(m, max_j s_ij), p_ij = exp(s_ij - m_new), alpha = exp(m - m_new),
    acc = alpha acc + p v, l = alpha l + sum_j p_ij; out = acc / max(l, 1e-20)."""
    q64, k64, v64 = q.double(), k.double(), v.double()
    n = q.shape[0]
    m = torch.full((n,), -math.inf, dtype=torch.float64)
    l = torch.zeros(n, dtype=torch.float64)
    acc = torch.zeros(n, v.shape[-1], dtype=torch.float64)
    rows = torch.arange(n)
    for start in range(0, n, block_n):
        cols = torch.arange(start, min(start + block_n, n))
        s = (q64 @ k64[cols].T) * scale
        s = s.masked_fill(cols[None, :] > rows[:, None], -math.inf)
        m_new = torch.maximum(m, s.max(dim=1).values)
        # rows with every key so far masked keep m = -inf; exp(-inf - -inf) would be NaN, their terms are 0
        finite = torch.isfinite(m_new)
        p = torch.where(finite[:, None], torch.exp(s - torch.where(finite, m_new, 0.0)[:, None]), 0.0)
        alpha = torch.where(finite, torch.exp(torch.where(torch.isfinite(m), m, -math.inf) -
                                              torch.where(finite, m_new, 0.0)), 1.0)
        acc = acc * alpha[:, None] + p @ v64[cols]
        l = l * alpha + p.sum(dim=1)
        m = m_new
    return acc / torch.clamp(l, min=1e-20)[:, None]


def monomials(dim: int, degree: int) -> List[Tuple[int, ...]]:
    """Monomial order: degree-major, combinations_with_replacement within a degree
    (streaming_taylor_coreset_attention.py:170; equal to [1, x, triu row-major] for degree <= 2,
    fast_article_attention.py:167-181)."""
    out: List[Tuple[int, ...]] = []
    for l in range(degree + 1):
        out.extend(itertools.combinations_with_replacement(range(dim), l))
    return out


def inv_multinomial(combo: Tuple[int, ...]) -> float:
    """1 / prod_j alpha_j! (streaming_taylor_coreset_attention.py:78-93)."""
    r = 1.0
    for _, grp in itertools.groupby(combo):
        r /= math.factorial(len(list(grp)))
    return r


def features(x: Tensor, degree: int, key_side: bool) -> Tensor:
    """phi(x) for rows of x: key side carries 1/prod(alpha!), query side none
    (streaming_taylor_coreset_attention.py:184-216; fast_article_attention.py:151-181)."""
    combos = monomials(x.shape[-1], degree)
    cols = []
    for c in combos:
        if not c:
            cols.append(torch.ones(x.shape[:-1], dtype=x.dtype))
            continue
        m = x[..., c[0]]
        for idx in c[1:]:
            m = m * x[..., idx]
        if key_side:
            m = m * inv_multinomial(c)
        cols.append(m)
    return torch.stack(cols, dim=-1)


# ----------------------------------------------------------------------------- low-degree moments

def low_sums_stream(q: Tensor, k: Tensor, v: Tensor, degree: int, scale: float) -> Tuple[Tensor, Tensor]:
    """Token loop with a running F x Dv state (fast_article_attention.py:217-259): this is the
    reference CPU fast path's moment algorithm and the CPU baseline's op sequence."""
    fk = features(k, degree, True)
    fq = features(q * scale, degree, False)
    n, dv = v.shape
    f = fk.shape[-1]
    den_state = torch.zeros(f, dtype=q.dtype)
    num_state = torch.zeros(f, dv, dtype=q.dtype)
    low_den = torch.empty(n, dtype=q.dtype)
    low_num = torch.empty(n, dv, dtype=q.dtype)
    for i in range(n):
        fi = fk[i]
        den_state.add_(fi)
        num_state.add_(fi[:, None] * v[i][None, :])
        qi = fq[i]
        low_den[i] = torch.dot(qi, den_state)
        low_num[i] = qi @ num_state
    return low_num, low_den


def low_sums_direct(q: Tensor, k: Tensor, v: Tensor, degree: int, scale: float) -> Tuple[Tensor, Tensor]:
    """Closed form sum_{j<=i} exp_{<=t}(s q_i.k_j) [v_j, 1] in float64 (what the moments must equal)."""
    x = (q.double() @ k.double().T) * scale
    p = exp_taylor(x, degree).tril()
    return p @ v.double(), p.sum(-1)


# ----------------------------------------------------------------------------- block compressor

def projection_scores(keys: np.ndarray, direction: np.ndarray) -> np.ndarray:
    """<k, dir> accumulated in float64 in index order, rounded once to float32 (the order the HIP
    compressor uses; each fp32*fp32 product is exact in float64).  float64 keys (a float64 caller,
    whose reference compress calls run in float64, fast_article_attention.py:339-341,
    streaming_taylor_coreset_attention.py:441-444): every product rounded to float64, then added, in
    index order, and the float64 score kept whole."""
    k64 = keys.astype(np.float64)
    d64 = direction.astype(np.float64)
    acc = np.zeros(keys.shape[0], dtype=np.float64)
    for a in range(keys.shape[1]):
        acc = acc + k64[:, a] * d64[a]
    return acc if keys.dtype == np.float64 else acc.astype(np.float32)


def sorted_pair_select(src: np.ndarray, w: np.ndarray, scores: np.ndarray, u: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Sorted-pair compression given scores and pair uniforms
    (streaming_taylor_coreset_attention.py:435-467; with unit weights it is the flat rule
    rand < 0.5 / weight 2 of fast_article_attention.py:339-359).  Ties are broken by position."""
    n = src.shape[0]
    order = np.argsort(scores, kind="stable")
    pc = n // 2
    a = order[0 : 2 * pc : 2]
    b = order[1 : 2 * pc : 2]
    wa = w[a].astype(np.float32)
    wb = w[b].astype(np.float32)
    wsum = (wa + wb).astype(np.float32)
    if u.dtype == np.float64:  # float64 draws: the rule in float64 (weights held in float32)
        wa64, wb64 = wa.astype(np.float64), wb.astype(np.float64)
        choose_a = u[:pc] < wa64 / np.maximum(wa64 + wb64, 1e-30)
    else:
        prob = (wa / np.maximum(wsum, np.float32(1e-30))).astype(np.float32)
        choose_a = u[:pc].astype(np.float32) < prob
    out_src = np.where(choose_a, src[a], src[b])
    out_w = wsum
    if n % 2 == 1:
        out_src = np.concatenate([out_src, src[order[-1:]]])
        out_w = np.concatenate([out_w, w[order[-1:]].astype(np.float32)])
    return out_src.astype(np.int64), out_w.astype(np.float32)


def perm_select(src: np.ndarray, w: np.ndarray, perm: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Uniform half-sampling with weight factor n/m (fast_article_attention.py:326-330,
    streaming_taylor_coreset_attention.py:427-433)."""
    n = src.shape[0]
    m = (n + 1) // 2
    factor = np.float32(float(n) / float(m))
    p = perm[:m]
    return src[p].astype(np.int64), (w[p].astype(np.float32) * factor).astype(np.float32)


@dataclass
class CompressCall:
    """One reference compress call: inputs (global token ids, weights), draws and the result."""

    level: int
    src_in: np.ndarray
    w_in: np.ndarray
    method: str  # "sorted_pair" | "perm" | "copy"
    direction: Optional[np.ndarray] = None
    uniforms: Optional[np.ndarray] = None
    perm: Optional[np.ndarray] = None
    src_out: Optional[np.ndarray] = None
    w_out: Optional[np.ndarray] = None


def draw_for_call(g: torch.Generator, n: int, d: int, compressor: str, dtype: torch.dtype = torch.float32):
    """Generator consumption of one compress call on n items
    (fast_article_attention.py:326-348; streaming_taylor_coreset_attention.py:413-456); the direction
    and uniforms are drawn in the keys' dtype, as the reference draws them (float64 for float64 keys)."""
    if compressor == "none" or n <= 1:
        return "copy", None, None, None
    if compressor == "random" or n <= 2:
        return "perm", None, None, torch.randperm(n, generator=g).numpy()
    if compressor != "sorted_pair":
        raise ValueError("compressor must be one of {'sorted_pair', 'random', 'none'}")
    direction = torch.randn(d, generator=g, dtype=dtype)
    direction = direction / torch.clamp(torch.linalg.vector_norm(direction), min=1e-12)
    u = torch.rand(n // 2, generator=g, dtype=dtype)
    return "sorted_pair", direction.numpy(), u.numpy(), None


def _draw_dtype(keys_all: np.ndarray) -> torch.dtype:
    return torch.float64 if keys_all.dtype == np.float64 else torch.float32


def run_call(call: CompressCall, keys_all: np.ndarray, score_fn=projection_scores) -> None:
    if call.method == "copy":
        call.src_out, call.w_out = call.src_in.copy(), call.w_in.copy()
    elif call.method == "perm":
        call.src_out, call.w_out = perm_select(call.src_in, call.w_in, call.perm)
    else:
        scores = score_fn(keys_all[call.src_in], call.direction)
        call.src_out, call.w_out = sorted_pair_select(call.src_in, call.w_in, scores, call.uniforms)


def flat_coreset(k: np.ndarray, block: int, compressor: str, seed: int, score_fn=projection_scores) -> List[CompressCall]:
    """Completed blocks with a later query, each compressed once, generator seeded with `seed`
    (fast_article_attention.py:364-434).  Returns one CompressCall per block (block b's reps are
    active for queries i >= (b+1)*block)."""
    n, d = k.shape
    g = torch.Generator(device="cpu")
    g.manual_seed(int(seed))
    calls = []
    for start in range(0, n, block):
        end = min(start + block, n)
        if end >= n:
            break
        src = np.arange(start, end, dtype=np.int64)
        method, dvec, u, perm = draw_for_call(g, end - start, d, compressor, _draw_dtype(k))
        c = CompressCall(0, src, np.ones(end - start, np.float32), method, dvec, u, perm)
        run_call(c, k, score_fn)
        calls.append(c)
    return calls


@dataclass
class LevelState:
    """Literal merge-and-reduce state (streaming_taylor_coreset_attention.py:332-506)."""

    levels: List[Optional[Tuple[np.ndarray, np.ndarray]]] = field(default_factory=list)
    calls: List[CompressCall] = field(default_factory=list)


def level_block_complete(state: LevelState, g: torch.Generator, block_src: np.ndarray, keys_all: np.ndarray,
                         compressor: str, score_fn=projection_scores) -> None:
    """A full buffer is compressed and inserted at level 0; occupied levels merge cat(old, new) and
    cascade upward (streaming_taylor_coreset_attention.py:387-411, :413-425)."""
    d = keys_all.shape[1]

    def compress(src, w, level):
        method, dvec, u, perm = draw_for_call(g, src.shape[0], d, compressor, _draw_dtype(keys_all))
        c = CompressCall(level, src, w, method, dvec, u, perm)
        run_call(c, keys_all, score_fn)
        state.calls.append(c)
        return c.src_out, c.w_out

    cur = compress(block_src, np.ones(block_src.shape[0], np.float32), 0)
    level = 0
    while True:
        while len(state.levels) <= level:
            state.levels.append(None)
        if state.levels[level] is None:
            state.levels[level] = cur
            return
        old = state.levels[level]
        state.levels[level] = None
        merged_src = np.concatenate([old[0], cur[0]])
        merged_w = np.concatenate([old[1], cur[1]])
        cur = compress(merged_src, merged_w, level + 1)
        level += 1


def level_items(state: LevelState) -> Tuple[np.ndarray, np.ndarray]:
    """Level items in order level 0, 1, ... (streaming_taylor_coreset_attention.py:469-490)."""
    srcs = [lv[0] for lv in state.levels if lv is not None and lv[0].size > 0]
    ws = [lv[1] for lv in state.levels if lv is not None and lv[0].size > 0]
    if not srcs:
        return np.zeros(0, np.int64), np.zeros(0, np.float32)
    return np.concatenate(srcs), np.concatenate(ws)


# ----------------------------------------------------------------------------- forward passes

def _residual(x: Tensor, degree: int) -> Tensor:
    return torch.exp(x) - exp_taylor(x, degree)


def fast_path_forward(q: Tensor, k: Tensor, v: Tensor, *, degree: int = 2, block: int = 128, scale: Optional[float] = None,
                      compressor: str = "sorted_pair", seed: int = 0, query_chunk: int = 2048, eps: float = 1e-12,
                      reference_scores: bool = False, calls_out: Optional[list] = None, low: str = "stream") -> Tensor:
    """The reference CPU fast path for one [N, D] sequence (fast_article_attention.py:522-598):
    stream moments + completed-block reps (chunked q x reps) + exact in-block residual, fp32.
    reference_scores=True orders each compress call as the reference does, by torch's `keys @ direction`
    and argsort (fast_article_attention.py:340-341), instead of the fixed-order scores the HIP kernel
    uses."""
    n, dim = q.shape
    s = attention_scale(scale, dim)
    low_num, low_den = _low_sums(q, k, v, degree, s, low)
    tail_den = torch.zeros(n, dtype=q.dtype)
    tail_num = torch.zeros(n, v.shape[-1], dtype=q.dtype)
    if compressor == "none":
        key_pos = torch.arange(n)
        for st in range(0, n, query_chunk):
            en = min(st + query_chunk, n)
            r = _residual((q[st:en] @ k.T) * s, degree)
            r = r.masked_fill(~(key_pos[None, :] <= torch.arange(st, en)[:, None]), 0.0)
            tail_den[st:en] = r.sum(-1)
            tail_num[st:en] = r @ v
    else:
        score_fn = torch_order_scores if reference_scores else projection_scores
        calls = flat_coreset(k.numpy(), block, compressor, seed, score_fn)
        if calls_out is not None:
            calls_out.extend(calls)
        if calls:
            idx = torch.from_numpy(np.concatenate([c.src_out for c in calls]))
            w = torch.from_numpy(np.concatenate([c.w_out for c in calls]))
            act = torch.cat([torch.full((c.src_out.shape[0],), (int(c.src_in[-1]) + 1), dtype=torch.long) for c in calls])
            rk, rv = k[idx], v[idx]
            for st in range(0, n, query_chunk):
                en = min(st + query_chunk, n)
                r = _residual((q[st:en] @ rk.T) * s, degree)
                r = r.masked_fill(~(torch.arange(st, en)[:, None] >= act[None, :]), 0.0) * w[None, :]
                tail_den[st:en] += r.sum(-1)
                tail_num[st:en] += r @ rv
        for st in range(0, n, block):
            en = min(st + block, n)
            r = _residual((q[st:en] @ k[st:en].T) * s, degree).tril()
            tail_den[st:en] += r.sum(-1)
            tail_num[st:en] += r @ v[st:en]
    return (low_num + tail_num) / torch.clamp((low_den + tail_den)[:, None], min=eps)


def time_fast_path_sample(q: Tensor, k: Tensor, v: Tensor, *, degree: int, block: int, scale: float,
                          compressor: str = "sorted_pair", seed: int = 0, query_chunk: int = 2048,
                          rows: int = 16384) -> Dict[str, float]:
    """Wall time of the reference CPU fast path (fast_article_attention.py:522-598, low_mode="stream")
    for ONE [N, D] sequence, measured on a bounded sample and scaled to the whole sequence:
      * the token loop of the moment scan is timed over the first `rows` tokens (its per-token cost
        does not depend on the position) and scaled by N / rows;
      * the completed-block reps are built for the whole sequence (timed in full);
      * the q x reps residual is timed for the first `rows` query rows -- the reference evaluates every
        query against all reps and masks afterwards, so each query chunk costs the same -- and scaled;
      * the exact in-block residual is timed for the blocks covering the first `rows` rows and scaled.
    Returns seconds per sequence for each part and in total."""
    import time as _time

    n, dim = q.shape
    rows = min(rows, n)
    frac = n / rows
    t0 = _time.perf_counter()
    low_sums_stream(q[:rows], k[:rows], v[:rows], degree, scale)
    t_moments = (_time.perf_counter() - t0) * frac

    t0 = _time.perf_counter()
    calls = flat_coreset(k.numpy(), block, compressor, seed, torch_scores)
    idx = torch.from_numpy(np.concatenate([c.src_out for c in calls]))
    w = torch.from_numpy(np.concatenate([c.w_out for c in calls]))
    act = torch.cat([torch.full((c.src_out.shape[0],), int(c.src_in[-1]) + 1, dtype=torch.long) for c in calls])
    rk, rv = k[idx], v[idx]
    t_reps = _time.perf_counter() - t0

    t0 = _time.perf_counter()
    for st in range(0, rows, query_chunk):
        en = min(st + query_chunk, rows)
        r = _residual((q[st:en] @ rk.T) * scale, degree)
        r = r.masked_fill(~(torch.arange(st, en)[:, None] >= act[None, :]), 0.0) * w[None, :]
        _ = r.sum(-1), r @ rv
    t_tail = (_time.perf_counter() - t0) * frac

    t0 = _time.perf_counter()
    for st in range(0, rows, block):
        en = min(st + block, rows)
        r = _residual((q[st:en] @ k[st:en].T) * scale, degree).tril()
        _ = r.sum(-1), r @ v[st:en]
    t_block = (_time.perf_counter() - t0) * frac
    total = t_moments + t_reps + t_tail + t_block
    return {"moments_s": t_moments, "reps_s": t_reps, "reps_residual_s": t_tail, "inblock_s": t_block, "total_s": total}


def torch_scores(keys: np.ndarray, direction: np.ndarray) -> np.ndarray:
    """`keys @ direction` with torch on the CPU, the reference's own projection
    (fast_article_attention.py:341, streaming_taylor_coreset_attention.py:443)."""
    return (torch.from_numpy(np.ascontiguousarray(keys)) @ torch.from_numpy(direction)).numpy()


def torch_order_scores(keys: np.ndarray, direction: np.ndarray) -> np.ndarray:
    """The rank of every key in torch.argsort(keys @ direction), as float64 scores: a stable sort of
    them is the reference's own order, including the order torch's argsort gives exactly equal scores
    (fast_article_attention.py:341, streaming_taylor_coreset_attention.py:443-444)."""
    order = torch.argsort(torch.from_numpy(np.ascontiguousarray(keys)) @ torch.from_numpy(direction)).numpy()
    rank = np.empty(order.shape[0], dtype=np.float64)
    rank[order] = np.arange(order.shape[0], dtype=np.float64)
    return rank


def _low_sums(q: Tensor, k: Tensor, v: Tensor, degree: int, scale: float, low: str) -> Tuple[Tensor, Tensor]:
    """The moment sums by the reference's token loop ("stream") or their closed form ("direct", for
    feature maps too large to materialise; equal in exact arithmetic, test_stream_moments_equal_closed_form)."""
    if low == "stream":
        return low_sums_stream(q, k, v, degree, scale)
    if low == "direct":
        num, den = low_sums_direct(q, k, v, degree, scale)
        return num.to(q.dtype), den.to(q.dtype)
    raise ValueError("low must be 'stream' or 'direct'")


def levels_forward(q: Tensor, k: Tensor, v: Tensor, *, degree: int = 2, block: int = 128, scale: Optional[float] = None,
                   compressor: str = "sorted_pair", seed: int = 0, eps: float = 1e-12, reference_scores: bool = False,
                   state_out: Optional[LevelState] = None, low: str = "stream") -> Tensor:
    """Streaming semantics of ArticleStreamingAttention for a whole [N, D] sequence
    (streaming_taylor_coreset_attention.py:576-609, :641-687): for every token, update(k_i, v_i) then
    query(q_i).  Queries see the exact moments over keys <= i, the uncompressed buffer (weight 1) and
    the level coresets; a block is compressed as soon as its last token is appended, so that token
    is answered from the compressed levels.  Vectorised per block."""
    n, dim = q.shape
    s = attention_scale(scale, dim)
    low_num, low_den = _low_sums(q, k, v, degree, s, low)
    out = torch.empty(n, v.shape[-1], dtype=q.dtype)
    state = state_out if state_out is not None else LevelState()
    g = torch.Generator(device="cpu")
    g.manual_seed(int(seed))
    score_fn = torch_order_scores if reference_scores else projection_scores
    k_np = k.numpy()

    def tail_for(rows: Tensor, items_src: np.ndarray, items_w: np.ndarray, buf_lo: int, rows_idx: np.ndarray):
        qs = q[rows] * 1.0
        den = torch.zeros(rows.shape[0], dtype=q.dtype)
        num = torch.zeros(rows.shape[0], v.shape[-1], dtype=q.dtype)
        if items_src.size:
            ik = k[torch.from_numpy(items_src)]
            iv = v[torch.from_numpy(items_src)]
            r = _residual((qs @ ik.T) * s, degree) * torch.from_numpy(items_w)[None, :]
            den += r.sum(-1)
            num += r @ iv
        hi = int(rows_idx[-1])
        if compressor == "none":
            buf_lo = 0
        if hi >= buf_lo:
            bk, bv = k[buf_lo : hi + 1], v[buf_lo : hi + 1]
            r = _residual((qs @ bk.T) * s, degree)
            cols = torch.arange(buf_lo, hi + 1)
            r = r.masked_fill(~(cols[None, :] <= torch.from_numpy(rows_idx)[:, None]), 0.0)
            den += r.sum(-1)
            num += r @ bv
        return num, den

    for start in range(0, n, block):
        end = min(start + block, n)
        full = end - start == block
        head_rows = np.arange(start, end - 1 if full else end, dtype=np.int64)
        if compressor == "none":
            isrc, iw = np.zeros(0, np.int64), np.zeros(0, np.float32)
        else:
            isrc, iw = level_items(state)
        if head_rows.size:
            rows = torch.from_numpy(head_rows)
            tn, td = tail_for(rows, isrc, iw, start, head_rows)
            out[rows] = (low_num[rows] + tn) / torch.clamp((low_den[rows] + td)[:, None], min=eps)
        if full:
            last = end - 1
            if compressor != "none":
                level_block_complete(state, g, np.arange(start, end, dtype=np.int64), k_np, compressor, score_fn)
                isrc, iw = level_items(state)
                buf_lo = end
            else:
                buf_lo = 0
            rows = torch.tensor([last])
            tn, td = tail_for(rows, isrc, iw, buf_lo, np.array([last]))
            out[rows] = (low_num[rows] + tn) / torch.clamp((low_den[rows] + td)[:, None], min=eps)
    return out


def segment_mean_coreset(k: Tensor, v: Tensor, block: int, stride: int) -> Tuple[Tensor, Tensor, int]:
    """Segment means of completed blocks with a later query (triton_article_attention.py:189-245)."""
    bh, n, dim = k.shape
    rpb = block // stride
    nb = max(0, (n - 1) // block)
    if nb == 0:
        return k.new_zeros(bh, 0, dim), v.new_zeros(bh, 0, v.shape[-1]), rpb
    use = nb * block
    rk = k[:, :use].reshape(bh, nb, rpb, stride, dim).mean(dim=3).reshape(bh, nb * rpb, dim)
    rv = v[:, :use].reshape(bh, nb, rpb, stride, v.shape[-1]).mean(dim=3).reshape(bh, nb * rpb, v.shape[-1])
    return rk, rv, rpb


def segment_rep_weight(stride: int) -> float:
    """A segment-mean representative stands for `stride` tokens: its residual term is multiplied by the
    stride (triton_article_attention.py:357, `* compress_stride`)."""
    return float(stride)


def segment_rep_active_from(rep_block: Tensor, block: int) -> Tensor:
    """First query row that sees the representatives of block rep_block: the row after the block ends
    (triton_article_attention.py:353-355, `offs_m >= (rep_block + 1) * BLOCK_SIZE`)."""
    return (rep_block + 1) * block


def clamped_exp(x: Tensor) -> Tensor:
    """exp(min(x, 80)), the Triton kernel's guard against overflow (triton_article_attention.py:333, :356)."""
    return torch.exp(torch.clamp(x, max=80.0))


def segment_forward(q: Tensor, k: Tensor, v: Tensor, *, degree: int, block: int, stride: int, scale: Optional[float] = None,
                    eps: float = 1e-12) -> Tensor:
    """Semantics of the fused Triton article kernel for [BH, N, D] in fp64: exp_{<=t} over the whole
    causal prefix, exact residual inside the current block, segment-mean reps of completed blocks with
    weight = stride active for i >= (rep_block+1)*B, exp(min(x, 80)) (triton_article_attention.py:265-369)."""
    bh, n, dim = q.shape
    s = attention_scale(scale, dim)
    q64, k64, v64 = q.double(), k.double(), v.double()
    rk, rv, rpb = segment_mean_coreset(k64, v64, block, stride)
    pos = torch.arange(n)
    x = (q64 @ k64.transpose(-1, -2)) * s
    causal = pos[None, :] <= pos[:, None]
    same = (pos[None, :] // block) == (pos[:, None] // block)
    tay = exp_taylor(x, degree)
    p = torch.where(causal, tay, torch.zeros_like(tay)) + torch.where(causal & same, clamped_exp(x) - tay, torch.zeros_like(tay))
    num = p @ v64
    den = p.sum(-1)
    if rk.shape[1]:
        xr = (q64 @ rk.transpose(-1, -2)) * s
        rep_block = torch.arange(rk.shape[1]) // rpb
        active = pos[:, None] >= segment_rep_active_from(rep_block, block)[None, :]
        r = torch.where(active, clamped_exp(xr) - exp_taylor(xr, degree), torch.zeros_like(xr)) * segment_rep_weight(stride)
        num = num + r @ rv
        den = den + r.sum(-1)
    return num / torch.clamp(den[..., None], min=eps)


def make_data(shape_lead: Tuple[int, ...], n: int, d: int, dv: int, *, radius: float, data: str, seed: int,
              dtype: torch.dtype = torch.float32) -> Tuple[Tensor, Tensor, Tensor]:
    """Synthetic inputs in the reference's draw order: randn q, k, v, then for unit_ball the radii
    rand^(1/d)*r for q then k (fast_article_attention.py:727-758, triton_article_attention.py:645-680)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    sq = tuple(shape_lead) + (n, d)
    sv = tuple(shape_lead) + (n, dv)
    q = torch.randn(sq, dtype=dtype, generator=g)
    k = torch.randn(sq, dtype=dtype, generator=g)
    v = torch.randn(sv, dtype=dtype, generator=g)
    if data == "unit_ball":
        qn = torch.clamp(torch.linalg.vector_norm(q, dim=-1, keepdim=True), min=1e-12)
        kn = torch.clamp(torch.linalg.vector_norm(k, dim=-1, keepdim=True), min=1e-12)
        rq = torch.rand(sq[:-1] + (1,), dtype=dtype, generator=g).pow(1.0 / d) * radius
        rk = torch.rand(sq[:-1] + (1,), dtype=dtype, generator=g).pow(1.0 / d) * radius
        q, k = q / qn * rq, k / kn * rk
    elif data == "unit_sphere":
        q = q / torch.clamp(torch.linalg.vector_norm(q, dim=-1, keepdim=True), min=1e-12) * radius
        k = k / torch.clamp(torch.linalg.vector_norm(k, dim=-1, keepdim=True), min=1e-12) * radius
    return q, k, v


def rel_l2(a: Tensor, b: Tensor) -> float:
    a64, b64 = a.double().cpu(), b.double().cpu()
    return float(torch.linalg.vector_norm(a64 - b64) / torch.clamp(torch.linalg.vector_norm(b64), min=1e-300))


# ----------------------------------------------------------------------------- streaming object

class StreamingAttentionCPU:
    """Per-token restatement of ArticleStreamingAttention (streaming_taylor_coreset_attention.py:523-616)
    on the CPU in the reference's op order: TaylorMomentSketch.update / query (:265-296) with per-degree
    gathered monomials, MergeReduceCoreset.append / _insert_level / _compress (:376-467) with torch's
    `keys @ direction` and argsort, and the query tail over items() (:581-609).  It is the decode CPU
    baseline (one stream, one token per call, as the reference runs) and a token-by-token checker."""

    def __init__(self, dim: int, value_dim: int, *, degree: int, block: int, scale: float,
                 compressor: str = "sorted_pair", seed: int = 0, eps: float = 1e-12) -> None:
        self.dim, self.value_dim, self.degree, self.block = dim, value_dim, degree, block
        self.scale, self.compressor, self.eps = float(scale), compressor, eps
        self.idx: List[Optional[Tensor]] = [None]
        self.coef: List[Tensor] = [torch.ones(1)]
        for l in range(1, degree + 1):
            combos = list(itertools.combinations_with_replacement(range(dim), l))
            self.idx.append(torch.tensor(combos, dtype=torch.long))
            self.coef.append(torch.tensor([inv_multinomial(c) for c in combos], dtype=torch.float32))
        self.den = [torch.zeros(c.shape[0]) for c in self.coef]
        self.num = [torch.zeros(c.shape[0], value_dim) for c in self.coef]
        self.g = torch.Generator(device="cpu")
        self.g.manual_seed(int(seed))
        self.buf_k: List[Tensor] = []
        self.buf_v: List[Tensor] = []
        self.levels: List[Optional[Tuple[Tensor, Tensor, Tensor]]] = []
        self.length = 0

    def _feats(self, x: Tensor, key_side: bool) -> List[Tensor]:
        out = [torch.ones(1)]
        for l in range(1, self.degree + 1):
            m = x[self.idx[l]].prod(dim=-1)
            out.append(m * self.coef[l] if key_side else m)
        return out

    def _compress(self, keys: Tensor, values: Tensor, weights: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
        n = weights.numel()
        if self.compressor == "none" or n <= 1:
            return keys, values, weights
        method, dvec, u, perm = draw_for_call(self.g, n, self.dim, self.compressor, keys.dtype)
        if method == "perm":
            m = (n + 1) // 2
            p = torch.from_numpy(perm[:m]).long()
            return keys[p], values[p], weights[p] * (float(n) / float(m))
        order = torch.argsort(keys @ torch.from_numpy(dvec))
        keys, values, weights = keys[order], values[order], weights[order]
        pc = n // 2
        wa, wb = weights[0: 2 * pc: 2], weights[1: 2 * pc: 2]
        wsum = wa + wb
        choose_a = torch.from_numpy(u) < wa / torch.clamp(wsum, min=1e-30)
        nk = torch.where(choose_a[:, None], keys[0: 2 * pc: 2], keys[1: 2 * pc: 2])
        nv = torch.where(choose_a[:, None], values[0: 2 * pc: 2], values[1: 2 * pc: 2])
        nw = wsum
        if n % 2 == 1:
            nk, nv, nw = torch.cat([nk, keys[-1:]]), torch.cat([nv, values[-1:]]), torch.cat([nw, weights[-1:]])
        return nk, nv, nw

    def update(self, k: Tensor, v: Tensor) -> None:
        for l, f in enumerate(self._feats(k, True)):
            self.den[l].add_(f)
            self.num[l].add_(f[:, None] * v[None, :])
        self.buf_k.append(k.clone())
        self.buf_v.append(v.clone())
        self.length += 1
        if len(self.buf_k) >= self.block:
            keys, values = torch.stack(self.buf_k), torch.stack(self.buf_v)
            self.buf_k.clear()
            self.buf_v.clear()
            blk = self._compress(keys, values, torch.ones(keys.shape[0]))
            level = 0
            while True:
                while len(self.levels) <= level:
                    self.levels.append(None)
                if self.levels[level] is None:
                    self.levels[level] = blk
                    break
                old = self.levels[level]
                self.levels[level] = None
                blk = self._compress(torch.cat([old[0], blk[0]]), torch.cat([old[1], blk[1]]), torch.cat([old[2], blk[2]]))
                level += 1

    def query(self, q: Tensor) -> Tensor:
        den = torch.zeros(())
        num = torch.zeros(self.value_dim)
        for l, f in enumerate(self._feats(q * self.scale, False)):
            den = den + torch.dot(self.den[l], f)
            num = num + f @ self.num[l]
        blocks = []
        if self.buf_k:
            blocks.append((torch.stack(self.buf_k), torch.stack(self.buf_v), torch.ones(len(self.buf_k))))
        blocks += [b for b in self.levels if b is not None and b[2].numel() > 0]
        if blocks:
            keys = torch.cat([b[0] for b in blocks])
            vals = torch.cat([b[1] for b in blocks])
            w = torch.cat([b[2] for b in blocks])
            logits = self.scale * (keys @ q)
            r = w * _residual(logits, self.degree)
            den = den + r.sum()
            num = num + r @ vals
        return num / torch.clamp(den, min=self.eps)


def time_decode_sample(*, dim: int, value_dim: int, degree: int, block: int, scale: float, prefix: int, steps: int,
                       seed: int = 0) -> Dict[str, float]:
    """Seconds per update + query step of the reference's streaming object (StreamingAttentionCPU) for
    ONE stream whose state has the sizes it has after `prefix` tokens: moments filled, the levels of
    the counter prefix // block occupied with block/2-item coresets, prefix % block buffered tokens
    (the per-step cost depends on these sizes, not on the values).  The timed steps include every
    block completion (compress + merges) they reach."""
    import time as _time

    g = torch.Generator().manual_seed(seed)
    st = StreamingAttentionCPU(dim, value_dim, degree=degree, block=block, scale=scale, seed=seed)
    for l in range(len(st.den)):
        st.den[l] = torch.randn(st.den[l].shape, generator=g)
        st.num[l] = torch.randn(st.num[l].shape, generator=g)
    c = prefix // block
    m = (block + 1) // 2
    for lev in range(c.bit_length()):
        st.levels.append(None)
        if (c >> lev) & 1:
            st.levels[lev] = (torch.randn(m, dim, generator=g) * 0.125, torch.randn(m, value_dim, generator=g),
                              torch.full((m,), float(2 ** (lev + 1))))
    for _ in range(prefix % block):
        st.buf_k.append(torch.randn(dim, generator=g) * 0.125)
        st.buf_v.append(torch.randn(value_dim, generator=g))
    st.length = prefix
    xs = torch.randn(steps, 3, max(dim, value_dim), generator=g) * 0.125
    t0 = _time.perf_counter()
    for i in range(steps):
        st.update(xs[i, 1, :dim], xs[i, 2, :value_dim])
        st.query(xs[i, 0, :dim])
    dt = _time.perf_counter() - t0
    return {"s_per_step": dt / steps, "steps": steps, "prefix": prefix}
