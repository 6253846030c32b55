"""Drop-in for the reference's streaming Taylor + merge-and-reduce coreset module
(streaming_taylor_coreset_attention.py), executed by HIP kernels on an AMD Instinct MI355X.

`article_causal_attention` returns what the reference's per-token loop `update(k_i, v_i); query(q_i)`
returns (streaming_taylor_coreset_attention.py:641-754), computed as one prefill:
  * exact Taylor moments of any degree <= 3 (symmetric monomial basis, key coefficient 1/prod(alpha!));
  * the merge-and-reduce level tree built level-parallel from the same seed-derived draws the
    reference's generator produces, in its call order (one compress per completed block, one per
    cascade merge, merge input = cat(old, new));
  * for token i: the uncompressed buffer (tokens of the current block up to i, weight 1) plus the
    level coresets present after update(k_i) -- so the last token of a block is answered from the
    freshly compressed levels, exactly as in the reference.
"""

from __future__ import annotations

import math
from typing import List, Optional, Tuple, Union

import torch

import _engine
import _plan
from fast_article_attention import _compute_dtype, _to_gpu

Tensor = torch.Tensor

__all__ = ["article_causal_attention", "article_causal_attention_single", "classical_causal_attention",
           "exp_taylor", "safe_relative_l2", "state_size_trace"]


def exp_taylor(logits: Tensor, degree: int) -> Tensor:
    """sum_{l<=degree} logits^l / l! (streaming_taylor_coreset_attention.py:96-105)."""
    if degree < 0:
        raise ValueError("degree must be non-negative")
    total = torch.ones_like(logits)
    term = torch.ones_like(logits)
    for l in range(1, degree + 1):
        term = term * logits / float(l)
        total = total + term
    return total


def safe_relative_l2(a: Tensor, b: Tensor, eps: float = 1e-12) -> float:
    return (torch.linalg.vector_norm(a - b) / torch.clamp(torch.linalg.vector_norm(b), min=eps)).item()


@torch.no_grad()
def classical_causal_attention(q: Tensor, k: Tensor, v: Tensor, *, scale: Optional[float] = None) -> Tensor:
    """Exact causal softmax attention for [N,D] or [B,H,N,D], the comparison baseline
    (streaming_taylor_coreset_attention.py:624-638), evaluated with torch on the tensors' device."""
    if q.shape[-2] != k.shape[-2] or q.shape[:-1] != k.shape[:-1]:
        raise ValueError("q and k must have matching leading dimensions and sequence length")
    if v.shape[:-1] != k.shape[:-1]:
        raise ValueError("v must have the same leading dimensions and sequence length as k")
    dim = q.shape[-1]
    s = float(1.0 / math.sqrt(dim) if scale is None else scale)
    n = q.shape[-2]
    logits = torch.matmul(q, k.transpose(-1, -2).contiguous()) * s
    causal = torch.ones(n, n, device=q.device, dtype=torch.bool).tril()
    return torch.matmul(torch.softmax(logits.masked_fill(~causal, float("-inf")), dim=-1), v)


def _feature_count(dim: int, degree: int, max_monomials: int) -> int:
    total = 0
    for l in range(degree + 1):
        total += math.comb(dim + l - 1, l) if l else 1
        if total > max_monomials:
            raise ValueError(
                f"Requested Taylor feature map has {total:,} monomials through degree {l}, "
                f"exceeding max_monomials={max_monomials:,}. Lower --degree/--d or raise the limit.")
    return total


def state_size_trace(n: int, dim: int, value_dim: int, degree: int, block_size: int, compressor: str,
                     elem: int) -> List[int]:
    """Per-token state bytes after update(k_i): moments plus buffer plus level coresets
    (streaming_taylor_coreset_attention.py:298-306, :495-506, :611-612)."""
    f = _plan.num_features(dim, degree)
    moments = f * (1 + value_dim) * elem
    plan = _plan.levels_plan(n, block_size, compressor) if compressor != "none" else None
    sizes = []
    nb_level_items = []
    level_size = [0] * 64
    # node size per level for a full level (independent of j)
    if plan is not None and plan.level_of is not None and n >= block_size:
        for i in range(plan.n_nodes):
            level_size[int(plan.level_of[i])] = int(plan.meta[i, 0])
    for i in range(n):
        c = (i + 1) // block_size
        buffered = (i + 1) - c * block_size
        if compressor == "none":
            items_bytes = c * block_size * (dim + value_dim + 1) * elem
        else:
            items = sum(level_size[l] for l in range(c.bit_length()) if (c >> l) & 1)
            items_bytes = items * (dim + value_dim + 1) * elem
        sizes.append(moments + buffered * (dim + value_dim) * elem + items_bytes)
    del nb_level_items
    return sizes


@torch.no_grad()
def article_causal_attention_single(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    *,
    degree: int = 2,
    block_size: int = 128,
    scale: Optional[float] = None,
    compressor: str = "sorted_pair",
    seed: int = 0,
    max_monomials: int = 5_000_000,
    return_state_sizes: bool = False,
) -> Union[Tensor, Tuple[Tensor, List[int]]]:
    """One [N,D] sequence (streaming_taylor_coreset_attention.py:641-687)."""
    if q.ndim != 2 or k.ndim != 2 or v.ndim != 2:
        raise ValueError("q, k, v must have shapes [N,D], [N,D], [N,Dv]")
    if q.shape != k.shape:
        raise ValueError(f"q and k must have the same shape, got {tuple(q.shape)} and {tuple(k.shape)}")
    if v.shape[0] != k.shape[0]:
        raise ValueError("v must have same sequence length as q/k")
    out = article_causal_attention(q[None, None], k[None, None], v[None, None], degree=degree,
                                   block_size=block_size, scale=scale, compressor=compressor, seed=seed,
                                   max_monomials=max_monomials, return_state_sizes=return_state_sizes)
    if return_state_sizes:
        o, sizes = out
        return o[0, 0], sizes
    return out[0, 0]


@torch.no_grad()
def article_causal_attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    *,
    degree: int = 2,
    block_size: int = 128,
    scale: Optional[float] = None,
    compressor: str = "sorted_pair",
    seed: int = 0,
    max_monomials: int = 5_000_000,
    return_state_sizes: bool = False,
) -> Union[Tensor, Tuple[Tensor, List[int]]]:
    """[N,D] or [B,H,N,D] (streaming_taylor_coreset_attention.py:690-754); sequence (b, h) uses
    seed + b*H + h.  All sequences run in one set of launches."""
    if q.ndim == 2:
        return article_causal_attention_single(q, k, v, degree=degree, block_size=block_size, scale=scale,
                                               compressor=compressor, seed=seed, max_monomials=max_monomials,
                                               return_state_sizes=return_state_sizes)
    if q.ndim != 4:
        raise ValueError("q/k/v must be [N,D] or [B,H,N,D]")
    if q.shape != k.shape:
        raise ValueError("q and k must have identical shape [B,H,N,D]")
    if v.shape[:3] != q.shape[:3]:
        raise ValueError("v must have shape [B,H,N,Dv]")
    if block_size < 2:
        raise ValueError("block_size must be at least 2")
    if degree < 0:
        raise ValueError("degree must be non-negative")
    bsz, heads, n, dim = q.shape
    dv = v.shape[-1]
    if dim <= 0:
        raise ValueError("dim must be positive")
    _feature_count(dim, degree, max_monomials)
    if compressor not in _plan.COMPRESSORS and n >= block_size:
        raise ValueError("compressor must be one of {'sorted_pair', 'random', 'none'}")
    s = float(1.0 / math.sqrt(dim) if scale is None else scale)
    home = q.device
    (qg, kg, vg), _ = _to_gpu(q, k, v)
    dt = _compute_dtype(qg)
    q3 = qg.to(dt).reshape(bsz * heads, n, dim)
    k3 = kg.to(dt).reshape(bsz * heads, n, dim)
    v3 = vg.to(dt).reshape(bsz * heads, n, dv)
    semantics = "exact" if compressor == "none" else "levels"
    res = _engine.prefill(q3, k3, v3, degree=degree, block=block_size, scale=s, semantics=semantics,
                          compressor=compressor, seed=seed, out_dtype=dt)
    out = res.out.reshape(bsz, heads, n, dv).to(device=home, dtype=q.dtype)
    if not return_state_sizes:
        return out
    one = state_size_trace(n, dim, dv, degree, block_size, compressor, q.element_size())
    return out, one * (bsz * heads)
