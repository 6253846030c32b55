"""Drop-in for the reference's fast Taylor + block-coreset causal attention module
(fast_article_attention.py), executed by hand-written HIP kernels on an AMD Instinct MI355X.

Same public names, keyword arguments, defaults, shapes, stats and exceptions as the reference:

    fast_article_causal_attention(q, k, v, *, degree=2, block_size=128, scale=None,
        compressor="sorted_pair", seed=0, query_chunk_size=2048, low_mode="auto",
        denominator_eps=1e-12, return_stats=False)            (fast_article_attention.py:634-719)

Execution (all on the GPU, no CPU fallback):
  * exact low-degree Taylor moments by a chunked moment scan (K1) plus the closed-form polynomial
    inside each chunk; `low_mode` "auto" / "stream" / "prefix" all select this one exact algorithm;
  * the completed-block sorted_pair / random coreset (K3) with the seed-derived draws replayed in the
    reference's torch CPU generator order;
  * the exp_{>t} residual over the coreset plus the exact in-block residual and the normalisation
    (K2 + K4).
Inputs on the CPU are moved to the first ROCm device and the result is moved back; fp32, bf16 and
fp16 inputs are read natively and computed in fp32 (bf16/fp16 inputs follow the fp32 reference on
the upcast values), the output has q's dtype.
"""

from __future__ import annotations

import argparse
import math
from dataclasses import dataclass
from typing import List, Optional, Tuple, Union

import torch

import _engine
import _plan
from _cli_util import fmt_bytes, pick_device, wall_ms

Tensor = torch.Tensor

__all__ = [
    "FastArticleStats",
    "classical_causal_attention",
    "exp_taylor",
    "fast_article_causal_attention",
    "fast_article_causal_attention_single",
    "low_degree_taylor_causal_sums",
    "low_degree_taylor_causal_sums_prefix",
    "low_degree_taylor_causal_sums_stream",
    "num_taylor_features",
    "safe_relative_l2",
]

# -----------------------------------------------------------------------------------------------
# Small utilities (fast_article_attention.py:48-108)
# -----------------------------------------------------------------------------------------------

_DTYPES = {
    "float32": torch.float32, "fp32": torch.float32, "float": torch.float32,
    "float64": torch.float64, "fp64": torch.float64, "double": torch.float64,
    "bfloat16": torch.bfloat16, "bf16": torch.bfloat16,
    "float16": torch.float16, "fp16": torch.float16, "half": torch.float16,
}


def _resolve_dtype(dtype: Union[str, torch.dtype]) -> torch.dtype:
    if isinstance(dtype, torch.dtype):
        return dtype
    key = str(dtype).lower()
    if key not in _DTYPES:
        raise ValueError(f"Unsupported dtype {dtype!r}; choose one of {sorted(_DTYPES)}")
    return _DTYPES[key]


def _attention_scale(scale: Optional[float], dim: int) -> float:
    """1/sqrt(D) when scale is None (fast_article_attention.py:76-77)."""
    return float(1.0 / math.sqrt(dim)) if scale is None else float(scale)


def exp_taylor(logits: Tensor, degree: int) -> Tensor:
    """sum_{r<=degree} logits^r / r!, built term by term (term = term * x / r)."""
    if degree < 0:
        raise ValueError("degree must be non-negative")
    total = torch.ones_like(logits)
    term = torch.ones_like(logits)
    for r in range(1, degree + 1):
        term = term * logits / float(r)
        total = total + term
    return total


def safe_relative_l2(a: Tensor, b: Tensor, eps: float = 1e-12) -> float:
    return (torch.linalg.vector_norm(a - b) / torch.clamp(torch.linalg.vector_norm(b), min=eps)).item()


@torch.no_grad()
def classical_causal_attention(q: Tensor, k: Tensor, v: Tensor, *, scale: Optional[float] = None) -> Tensor:
    """Exact masked-softmax causal attention for [N,D] tensors: the comparison baseline of the
    reference (fast_article_attention.py:116-129), evaluated with torch on the tensors' device."""
    if q.ndim != 2 or k.ndim != 2 or v.ndim != 2:
        raise ValueError("classical_causal_attention expects q,k,v with shapes [N,D], [N,D], [N,Dv]")
    if q.shape != k.shape or v.shape[0] != k.shape[0]:
        raise ValueError("q and k must match, and v must have the same sequence length")
    n, dim = q.shape
    logits = (q @ k.T) * _attention_scale(scale, dim)
    causal = torch.ones(n, n, device=q.device, dtype=torch.bool).tril()
    return torch.softmax(logits.masked_fill(~causal, float("-inf")), dim=-1) @ v


# -----------------------------------------------------------------------------------------------
# Feature map and low-degree sums
# -----------------------------------------------------------------------------------------------


def num_taylor_features(dim: int, degree: int) -> int:
    """1 + D + D(D+1)/2 features through degree 2 (fast_article_attention.py:137-148)."""
    if degree < 0:
        raise ValueError("degree must be non-negative")
    if degree > 2:
        raise NotImplementedError("fast implementation currently supports degree 0, 1, or 2")
    return _plan.num_features(dim, degree)


def _taylor_features_degree012(x: Tensor, degree: int, *, key_side: bool) -> Tensor:
    """Explicit feature vectors [1, x, x_i x_j (i<=j)] (1/2 on key-side squares); a host-side helper
    for inspection and tests -- the kernels generate these features on the fly."""
    if degree > 2:
        raise NotImplementedError("fast implementation currently supports degree 0, 1, or 2")
    if x.ndim < 2:
        raise ValueError("x must have shape [..., N, D] or [N, D]")
    dim = x.shape[-1]
    parts = [torch.ones(*x.shape[:-1], 1, device=x.device, dtype=x.dtype)]
    if degree >= 1:
        parts.append(x)
    if degree >= 2:
        a, b = torch.triu_indices(dim, dim, device=x.device)
        quad = x[..., a] * x[..., b]
        if key_side:
            quad = quad * torch.where(a == b, 0.5, 1.0).to(device=x.device, dtype=x.dtype)
        parts.append(quad)
    return torch.cat(parts, dim=-1)


def _check_low_inputs(q: Tensor, k: Tensor, v: Tensor, name: str) -> None:
    if q.ndim != 2 or k.ndim != 2 or v.ndim != 2:
        raise ValueError(f"{name} expects [N,D], [N,D], [N,Dv]")
    if q.shape != k.shape or v.shape[0] != k.shape[0]:
        raise ValueError("q and k must match, and v must have the same sequence length")


def _to_gpu(*tensors: Tensor) -> Tuple[List[Tensor], torch.device]:
    """Device the kernels run on: the tensors' own ROCm device, else the first one."""
    home = tensors[0].device
    if home.type == "cuda":
        return [t.contiguous() for t in tensors], home
    if not torch.cuda.is_available():
        raise RuntimeError("streaming-attention HIP kernels need a ROCm GPU; none is visible")
    dev = torch.device("cuda", torch.cuda.current_device())
    return [t.to(dev).contiguous() for t in tensors], dev


def _compute_dtype(t: Tensor) -> torch.dtype:
    """Element type the kernels read: the input's for float32 / bfloat16 / float16; float64 inputs are
    rounded to float32 (the kernels' arithmetic type) and the callers return float64 outputs, while the
    coreset compressor scores the float64 keys with float64 draws (_score_keys)."""
    if t.dtype in (torch.float32, torch.bfloat16, torch.float16):
        return t.dtype
    if t.dtype == torch.float64:
        return torch.float32
    raise ValueError(f"dtype {t.dtype} is not supported (use float64, float32, bfloat16 or float16)")


def _reference_keys(k: Tensor, bh: int, n: int, dim: int, on: bool) -> Optional[Tensor]:
    """For reference_scores=True: the caller's keys in their own dtype as the contiguous CPU
    [B*H, N, D] rows the reference scores (its k[b, h] are views of the caller's tensor, so a contiguous
    CPU tensor is used as it is; other keys are copied to the host).  None when off."""
    if not on:
        return None
    k3 = k.reshape(bh, n, dim)
    if k3.device.type == "cpu" and k3.is_contiguous():
        return k3
    return k3.contiguous().cpu()


def _score_keys(k3: Tensor) -> Optional[Tensor]:
    """The keys the compressor scores for a float64 caller: the float64 keys themselves, since the
    reference runs a float64 caller's compress calls in float64 (float64 directions and uniforms, scores
    keys @ direction in float64; fast_article_attention.py:339-348, streaming_taylor_coreset_attention.py:
    441-457).  None for the other dtypes (their scores come from the rows the kernels read)."""
    return k3.contiguous() if k3.dtype == torch.float64 else None


@torch.no_grad()
def low_degree_taylor_causal_sums(
    q: Tensor, k: Tensor, v: Tensor, *, degree: int = 2, scale: Optional[float] = None, mode: str = "auto"
) -> Tuple[Tensor, Tensor, int]:
    """Exact sum_{j<=i} exp_{<=t}(s q_i.k_j) [v_j, 1] as (low_num [N,Dv], low_den [N], F)
    (fast_article_attention.py:262-285).  Every mode runs the same exact GPU moment scan."""
    if mode not in ("auto", "stream", "prefix"):
        raise ValueError("mode must be one of {'auto', 'stream', 'prefix'}")
    _check_low_inputs(q, k, v, "low_degree_taylor_causal_sums")
    f = num_taylor_features(q.shape[-1], degree)
    s = _attention_scale(scale, q.shape[-1])
    home = q.device
    if q.shape[0] == 0:  # the reference's token loop and cumsum return empty sums
        return q.new_empty((0, v.shape[-1])), q.new_empty((0,)), f
    (qg, kg, vg), _ = _to_gpu(q, k, v)
    dt = _compute_dtype(qg)
    res = _engine.prefill(qg.to(dt)[None], kg.to(dt)[None], vg.to(dt)[None], degree=degree, block=1, scale=s,
                          semantics="taylor")
    low_num = res.out[0].to(device=home, dtype=q.dtype)
    low_den = res.den[0].to(device=home, dtype=q.dtype)
    return low_num, low_den, f


def low_degree_taylor_causal_sums_stream(q, k, v, *, degree: int = 2, scale: Optional[float] = None):
    """(fast_article_attention.py:217-259)"""
    _check_low_inputs(q, k, v, "low_degree_taylor_causal_sums_stream")
    return low_degree_taylor_causal_sums(q, k, v, degree=degree, scale=scale, mode="stream")


def low_degree_taylor_causal_sums_prefix(q, k, v, *, degree: int = 2, scale: Optional[float] = None):
    """(fast_article_attention.py:184-214)"""
    _check_low_inputs(q, k, v, "low_degree_taylor_causal_sums_prefix")
    return low_degree_taylor_causal_sums(q, k, v, degree=degree, scale=scale, mode="prefix")


# -----------------------------------------------------------------------------------------------
# Public fast attention
# -----------------------------------------------------------------------------------------------


@dataclass(frozen=True)
class FastArticleStats:
    """Same fields and formulas as the reference (fast_article_attention.py:293-301, :603-631)."""

    degree: int
    block_size: int
    feature_count: int
    coreset_items: int
    approx_streaming_state_bytes: int
    scratch_low_prefix_bytes: int
    scratch_residual_matrix_bytes: int


def _flat_coreset_items(n: int, block_size: int, compressor: str) -> int:
    if compressor == "none":
        return n
    nbf = (n - 1) // block_size if n > 0 else 0
    return nbf * ((block_size + 1) // 2)


def _stats(n, dim, dv, elem, degree, block_size, compressor, query_chunk_size, low_mode, device_type):
    f = num_taylor_features(dim, degree)
    items = _flat_coreset_items(n, block_size, compressor)
    if compressor == "none":
        resid_scratch = min(query_chunk_size, n) * n * elem
    else:
        reps_scratch = min(query_chunk_size, n) * max(items, 1) * elem
        block_scratch = min(block_size, n) ** 2 * elem
        resid_scratch = max(reps_scratch, block_scratch)
    state = f * (1 + dv) * elem + items * (dim + dv + 1) * elem + min(block_size, n) * (dim + dv) * elem
    resolved = "prefix" if (low_mode == "auto" and device_type == "cuda") else ("stream" if low_mode == "auto" else low_mode)
    low_scratch = f * (1 + dv) * elem if resolved == "stream" else n * f * (1 + dv) * elem
    return FastArticleStats(degree, block_size, f, items, int(state), int(low_scratch), int(resid_scratch))


def _validate_common(degree: int, block_size: int, query_chunk_size: int, low_mode: str) -> None:
    if query_chunk_size <= 0:
        raise ValueError("query_chunk_size must be positive")
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    if degree < 0:
        raise ValueError("degree must be non-negative")
    if degree > 2:
        raise NotImplementedError("fast implementation currently supports degree 0, 1, or 2")
    if low_mode not in ("auto", "stream", "prefix"):
        raise ValueError("mode must be one of {'auto', 'stream', 'prefix'}")


def _check_compressor(compressor: str, n: int, block_size: int) -> None:
    """The reference rejects an unknown compressor only when a completed block with a later query
    exists (fast_article_attention.py:361, reached from :403-413)."""
    if compressor not in _plan.COMPRESSORS and (n - 1) // block_size > 0:
        raise ValueError("compressor must be one of {'sorted_pair', 'random', 'none'}")


def _run_bh(q3, k3, v3, *, degree, block_size, scale, compressor, seed, denominator_eps, out_dtype, draws=None,
            score_keys=None, reference_keys=None):
    semantics = "exact" if compressor == "none" else "flat"
    res = _engine.prefill(
        q3, k3, v3, degree=degree, block=block_size, scale=scale, semantics=semantics, compressor=compressor,
        seed=seed, eps=denominator_eps, out_dtype=out_dtype, draws=draws,
        score_keys=score_keys if semantics == "flat" else None,
        reference_keys=reference_keys if semantics == "flat" else None)
    return res


@torch.no_grad()
def fast_article_causal_attention_single(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    *,
    degree: int = 2,
    block_size: int = 128,
    scale: Optional[float] = None,
    compressor: str = "sorted_pair",
    seed: int = 0,
    query_chunk_size: int = 2048,
    low_mode: str = "auto",
    denominator_eps: float = 1e-12,
    return_stats: bool = False,
    reference_scores: bool = False,
) -> Union[Tensor, Tuple[Tensor, FastArticleStats]]:
    """One [N,D] sequence (fast_article_attention.py:522-631).  reference_scores: order every compress
    call as the reference does on this host (torch's CPU `keys @ direction` and argsort, run on the
    host) instead of the GPU compressor's fixed-order fp64 scores; see fast_article_causal_attention."""
    if q.ndim != 2 or k.ndim != 2 or v.ndim != 2:
        raise ValueError("q,k,v must have shapes [N,D], [N,D], [N,Dv]")
    if q.shape != k.shape:
        raise ValueError(f"q and k must have the same shape, got {tuple(q.shape)} and {tuple(k.shape)}")
    if v.shape[0] != k.shape[0]:
        raise ValueError("v must have the same sequence length as q/k")
    _validate_common(degree, block_size, query_chunk_size, low_mode)
    n, dim = q.shape
    dv = v.shape[-1]
    _check_compressor(compressor, n, block_size)
    home = q.device
    if n == 0:  # nothing to attend: the reference returns an empty [0, Dv] output
        out = q.new_empty((0, dv))
        if not return_stats:
            return out
        return out, _stats(n, dim, dv, q.element_size(), degree, block_size, compressor, query_chunk_size, low_mode,
                           home.type)
    (qg, kg, vg), _ = _to_gpu(q, k, v)
    dt = _compute_dtype(qg)
    res = _run_bh(qg.to(dt)[None], kg.to(dt)[None], vg.to(dt)[None], degree=degree, block_size=block_size,
                  scale=_attention_scale(scale, dim), compressor=compressor, seed=seed,
                  denominator_eps=denominator_eps, out_dtype=dt, score_keys=_score_keys(kg[None]),
                  reference_keys=_reference_keys(k, 1, n, dim, reference_scores))
    out = res.out[0].to(device=home, dtype=q.dtype)
    if not return_stats:
        return out
    return out, _stats(n, dim, dv, q.element_size(), degree, block_size, compressor, query_chunk_size, low_mode,
                       home.type)


@torch.no_grad()
def fast_article_causal_attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    *,
    degree: int = 2,
    block_size: int = 128,
    scale: Optional[float] = None,
    compressor: str = "sorted_pair",
    seed: int = 0,
    query_chunk_size: int = 2048,
    low_mode: str = "auto",
    denominator_eps: float = 1e-12,
    return_stats: bool = False,
    reference_scores: bool = False,
) -> Union[Tensor, Tuple[Tensor, FastArticleStats]]:
    """[N,D] or [B,H,N,D] (fast_article_attention.py:634-719).  All B*H sequences run in one set of
    launches; sequence (b, h) uses seed + b*H + h as in the reference.

    reference_scores (not in the reference; default off): the GPU compressor orders a compress call's
    keys by fp64 projection scores summed in a fixed order, reproducible on any machine.  The reference
    sorts torch's CPU `keys @ direction`, whose fp32 summation order belongs to the host's BLAS, so on
    near-ties (scores a few ulps apart) the two orders can keep different tokens.  With
    reference_scores=True every compress call runs on the host with those same torch calls, in the
    keys' dtype, and the selections are the reference's on this host; the keys are copied to the host
    and the selection takes host time (the moment scan and the residual still run on the GPU)."""
    kwargs = dict(degree=degree, block_size=block_size, scale=scale, compressor=compressor, seed=seed,
                  query_chunk_size=query_chunk_size, low_mode=low_mode, denominator_eps=denominator_eps,
                  return_stats=return_stats, reference_scores=reference_scores)
    if q.ndim == 2:
        return fast_article_causal_attention_single(q, k, v, **kwargs)
    if q.ndim != 4:
        raise ValueError("q/k/v must be [N,D] or [B,H,N,D]")
    if q.shape != k.shape:
        raise ValueError("q and k must have identical shape [B,H,N,D]")
    if v.shape[:3] != q.shape[:3]:
        raise ValueError("v must have shape [B,H,N,Dv]")
    _validate_common(degree, block_size, query_chunk_size, low_mode)
    bsz, heads, n, dim = q.shape
    dv = v.shape[-1]
    _check_compressor(compressor, n, block_size)
    home = q.device
    if bsz * heads == 0 or n == 0:
        out = torch.empty(bsz, heads, n, dv, device=home, dtype=q.dtype)
        if not return_stats:
            return out
        return out, FastArticleStats(degree, block_size, num_taylor_features(dim, degree), 0, 0, 0, 0)
    (qg, kg, vg), _ = _to_gpu(q, k, v)
    dt = _compute_dtype(qg)
    q3 = qg.to(dt).reshape(bsz * heads, n, dim)
    k3 = kg.to(dt).reshape(bsz * heads, n, dim)
    v3 = vg.to(dt).reshape(bsz * heads, n, dv)
    res = _run_bh(q3, k3, v3, degree=degree, block_size=block_size, scale=_attention_scale(scale, dim),
                  compressor=compressor, seed=seed, denominator_eps=denominator_eps, out_dtype=dt,
                  score_keys=_score_keys(kg.reshape(bsz * heads, n, dim)),
                  reference_keys=_reference_keys(k, bsz * heads, n, dim, reference_scores))
    out = res.out.reshape(bsz, heads, n, dv).to(device=home, dtype=q.dtype)
    if not return_stats:
        return out
    return out, _stats(n, dim, dv, q.element_size(), degree, block_size, compressor, query_chunk_size, low_mode,
                       home.type)


# -----------------------------------------------------------------------------------------------
# CLI (same flags and table as fast_article_attention.py:727-894)
# -----------------------------------------------------------------------------------------------


def _make_data(n: int, d: int, dv: int, *, radius: float, data: str, device: torch.device, dtype: torch.dtype,
               seed: int) -> Tuple[Tensor, Tensor, Tensor]:
    """q, k, v ~ N(0,1) in that draw order, then optional projection to the ball / sphere
    (fast_article_attention.py:727-758)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    q = torch.randn(n, d, device=device, dtype=dtype, generator=g)
    k = torch.randn(n, d, device=device, dtype=dtype, generator=g)
    v = torch.randn(n, dv, device=device, dtype=dtype, generator=g)
    if data == "unit_ball":
        qn = torch.clamp(torch.linalg.vector_norm(q, dim=-1, keepdim=True), min=1e-12)
        kn = torch.clamp(torch.linalg.vector_norm(k, dim=-1, keepdim=True), min=1e-12)
        rq = torch.rand(n, 1, device=device, dtype=dtype, generator=g).pow(1.0 / d) * radius
        rk = torch.rand(n, 1, device=device, dtype=dtype, generator=g).pow(1.0 / d) * radius
        q = q / qn * rq
        k = k / kn * rk
    elif data == "unit_sphere":
        q = q / torch.clamp(torch.linalg.vector_norm(q, dim=-1, keepdim=True), min=1e-12) * radius
        k = k / torch.clamp(torch.linalg.vector_norm(k, dim=-1, keepdim=True), min=1e-12) * radius
    elif data != "normal":
        raise ValueError("data must be one of {'unit_ball', 'unit_sphere', 'normal'}")
    return q, k, v


def _demo(args: argparse.Namespace) -> None:
    if args.threads is not None:
        torch.set_num_threads(args.threads)
    device = pick_device(args.device)
    dtype = _resolve_dtype(args.dtype)
    scale = args.scale if args.scale is not None else (1.0 / math.sqrt(args.d) if args.standard_scale else 1.0)
    rows = []
    for n in args.sweep_n:
        q, k, v = _make_data(n, args.d, args.dv, radius=args.radius, data=args.data, device=device, dtype=dtype,
                             seed=args.seed)
        call = lambda rs=False: fast_article_causal_attention(
            q, k, v, degree=args.degree, block_size=args.block_size, scale=scale, compressor=args.compressor,
            seed=args.seed, query_chunk_size=args.query_chunk_size, low_mode=args.low_mode, return_stats=rs)
        exact = classical_causal_attention(q, k, v, scale=scale)
        approx, stats = call(True)
        classical_ms, _ = wall_ms(lambda: classical_causal_attention(q, k, v, scale=scale), args.repeats, device)
        fast_ms, _ = wall_ms(call, args.repeats, torch.device("cuda") if torch.cuda.is_available() else device)
        rows.append([
            str(n), f"{safe_relative_l2(approx, exact):.4g}", f"{(approx - exact).abs().max().item():.4g}",
            f"{classical_ms:.3f}", f"{fast_ms:.3f}", fmt_bytes(stats.approx_streaming_state_bytes),
            fmt_bytes(stats.scratch_low_prefix_bytes), fmt_bytes(stats.scratch_residual_matrix_bytes),
            fmt_bytes(n * n * torch.tensor([], dtype=dtype).element_size()), str(stats.coreset_items),
        ])
    headers = ["n", "rel_l2", "max_abs", "classical_ms", "fast_ms", "approx_state", "low_scratch",
               "resid_scratch", "score_matrix", "coreset_items"]
    print("\n" + " | ".join(headers))
    print(" | ".join(["---"] * len(headers)))
    for r in rows:
        print(" | ".join(r))
    print()


def _parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(description="Fast vectorized Taylor + block-coreset attention benchmark (HIP/MI355X)")
    p.add_argument("--sweep-n", type=int, nargs="+", default=[256, 512, 1024])
    p.add_argument("--d", type=int, default=32)
    p.add_argument("--dv", type=int, default=32)
    p.add_argument("--degree", type=int, default=2)
    p.add_argument("--block-size", type=int, default=128)
    p.add_argument("--compressor", choices=["sorted_pair", "random", "none"], default="sorted_pair")
    p.add_argument("--query-chunk-size", type=int, default=2048)
    p.add_argument("--low-mode", choices=["auto", "stream", "prefix"], default="auto")
    p.add_argument("--threads", type=int, default=None, help="Optional torch.set_num_threads value")
    p.add_argument("--data", choices=["unit_ball", "unit_sphere", "normal"], default="unit_ball")
    p.add_argument("--radius", type=float, default=1.0)
    p.add_argument("--scale", type=float, default=None)
    p.add_argument("--standard-scale", action="store_true", help="Use 1/sqrt(d) when --scale is omitted")
    p.add_argument("--device", default="auto")
    p.add_argument("--dtype", default="float32")
    p.add_argument("--repeats", type=int, default=3)
    p.add_argument("--seed", type=int, default=0)
    return p


if __name__ == "__main__":
    _demo(_parser().parse_args())
