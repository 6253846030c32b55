"""Drop-in for the reference's streaming Taylor + merge-and-reduce coreset module
(streaming_taylor_coreset_attention.py), executed by HIP kernels on an AMD Instinct MI355X.

`article_causal_attention` returns what the reference's per-token loop `update(k_i, v_i); query(q_i)`
returns (streaming_taylor_coreset_attention.py:641-754), computed as one prefill:
  * exact Taylor moments of any degree <= 4 (degree 4 for D <= 64; symmetric monomial basis, key
    coefficient 1/prod(alpha!));
  * the merge-and-reduce level tree built level-parallel from the same seed-derived draws the
    reference's generator produces, in its call order (one compress per completed block, one per
    cascade merge, merge input = cat(old, new));
  * for token i: the uncompressed buffer (tokens of the current block up to i, weight 1) plus the
    level coresets present after update(k_i) -- so the last token of a block is answered from the
    freshly compressed levels, exactly as in the reference.

`ArticleStreamingAttention` is the mutable streaming state itself (streaming_taylor_coreset_attention.py
:523-616) with `update(k, v)`, `query(q)`, `state_size_bytes()` and `length`, kept on the GPU (decode
kernels K5).  Beyond the reference it takes `streams=S` for S independent streams advanced in lockstep
(stream s seeded seed + s, the per-sequence seeding of article_causal_attention), and offers `step`
(update + query fused), `extend` (bulk update) and `prefill` (outputs for a prompt plus the state).
"""

from __future__ import annotations

import argparse
import math
import weakref
from dataclasses import dataclass
from typing import List, Optional, Tuple, Union

import torch

import _decode
import _engine
import _plan
from fast_article_attention import _compute_dtype, _reference_keys, _resolve_dtype, _score_keys, _to_gpu

Tensor = torch.Tensor

__all__ = ["ArticleStreamingAttention", "AttentionQueryStats", "CoresetBlock", "article_causal_attention",
           "article_causal_attention_single", "classical_causal_attention", "exp_taylor", "safe_relative_l2",
           "state_size_trace", "coreset_item_trace"]


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


def coreset_item_trace(n: int, block_size: int, compressor: str) -> List[int]:
    """Per-token coreset size (MergeReduceCoreset.num_items after update(k_i): buffered tokens plus the
    occupied levels' items, streaming_taylor_coreset_attention.py:489-493).  compressor "none" keeps
    every token (its levels hold whole blocks, uncompressed)."""
    if compressor == "none":
        return list(range(1, n + 1))
    per_level = [0] * 64  # items of an occupied level (the same for every node of a level)
    plan = _plan.levels_plan(n, block_size, compressor) if n >= block_size else None
    if plan is not None and plan.level_of is not None:
        for i in range(plan.n_nodes):
            per_level[int(plan.level_of[i])] = int(plan.meta[i, 0])
    out = []
    for i in range(n):
        c = (i + 1) // block_size
        out.append((i + 1) - c * block_size + sum(per_level[l] for l in range(c.bit_length()) if (c >> l) & 1))
    return out


def state_size_trace(n: int, dim: int, value_dim: int, degree: int, block_size: int, compressor: str,
                     elem: int) -> List[int]:
    """Per-token state bytes after update(k_i): moments plus buffered tokens (key and value) plus the
    levels' items (key, value, weight) (streaming_taylor_coreset_attention.py:298-306, :495-506,
    :611-612)."""
    moments = _plan.num_features(dim, degree) * (1 + value_dim) * elem
    items = coreset_item_trace(n, block_size, compressor)
    sizes = []
    for i in range(n):
        buffered = (i + 1) % block_size
        levels = items[i] - buffered
        sizes.append(moments + buffered * (dim + value_dim) * elem + levels * (dim + value_dim + 1) * elem)
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
    reference_scores: bool = False,
) -> Union[Tensor, Tuple[Tensor, List[int]]]:
    """One [N,D] sequence (streaming_taylor_coreset_attention.py:641-687); reference_scores as in
    article_causal_attention."""
    if q.ndim != 2 or k.ndim != 2 or v.ndim != 2:
        raise ValueError("q, k, v must have shapes [N,D], [N,D], [N,Dv]")
    if q.shape != k.shape:
        raise ValueError(f"q and k must have the same shape, got {tuple(q.shape)} and {tuple(k.shape)}")
    if v.shape[0] != k.shape[0]:
        raise ValueError("v must have same sequence length as q/k")
    out = article_causal_attention(q[None, None], k[None, None], v[None, None], degree=degree,
                                   block_size=block_size, scale=scale, compressor=compressor, seed=seed,
                                   max_monomials=max_monomials, return_state_sizes=return_state_sizes,
                                   reference_scores=reference_scores)
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
    reference_scores: bool = False,
) -> Union[Tensor, Tuple[Tensor, List[int]]]:
    """[N,D] or [B,H,N,D] (streaming_taylor_coreset_attention.py:690-754); sequence (b, h) uses
    seed + b*H + h.  All sequences run in one set of launches.  reference_scores (not in the reference;
    default off): every compress call of the level cascade runs on the host, ordered by torch's CPU
    `keys @ direction` and argsort in the keys' dtype as the reference orders it on this host, instead of
    the GPU compressor's fixed-order fp64 scores (see fast_article_causal_attention)."""
    if q.ndim == 2:
        return article_causal_attention_single(q, k, v, degree=degree, block_size=block_size, scale=scale,
                                               compressor=compressor, seed=seed, max_monomials=max_monomials,
                                               return_state_sizes=return_state_sizes,
                                               reference_scores=reference_scores)
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
                          compressor=compressor, seed=seed, out_dtype=dt,
                          score_keys=_score_keys(kg.reshape(bsz * heads, n, dim)) if semantics == "levels" else None,
                          reference_keys=_reference_keys(k, bsz * heads, n, dim,
                                                         reference_scores and semantics == "levels"))
    out = res.out.reshape(bsz, heads, n, dv).to(device=home, dtype=q.dtype)
    if not return_state_sizes:
        return out
    one = state_size_trace(n, dim, dv, degree, block_size, compressor, q.element_size())
    return out, one * (bsz * heads)


# -----------------------------------------------------------------------------------------------
# Streaming state (streaming_taylor_coreset_attention.py:229-616)
# -----------------------------------------------------------------------------------------------


@dataclass
class CoresetBlock:
    """Keys, values and weights of a set of coreset items (streaming_taylor_coreset_attention.py:313-329).
    In batched mode every tensor has a leading stream dimension."""

    keys: Tensor
    values: Tensor
    weights: Tensor

    @property
    def size(self) -> int:
        return int(self.weights.shape[-1])


@dataclass
class AttentionQueryStats:
    """streaming_taylor_coreset_attention.py:514-520.  In batched mode the three denominators are
    tensors [S]; coreset_items and state_bytes are per stream (every stream has the same counts)."""

    denominator: Union[float, Tensor]
    low_denominator: Union[float, Tensor]
    tail_denominator: Union[float, Tensor]
    coreset_items: int
    state_bytes: int


def _resolve_gpu(device: Optional[Union[str, torch.device]]) -> torch.device:
    if device is None or str(device) == "auto":
        if not torch.cuda.is_available():
            raise RuntimeError("streaming-attention HIP kernels need a ROCm GPU; none is visible")
        return torch.device("cuda", torch.cuda.current_device())
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError("ArticleStreamingAttention keeps its state on a ROCm GPU; pass a cuda device")
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


def _elem(dtype: torch.dtype) -> int:
    return torch.tensor([], dtype=dtype).element_size()


class _SketchView:
    """The moment sketch of the state (TaylorMomentSketch, streaming_taylor_coreset_attention.py:229-306):
    den_moments / num_moments per degree, in the reference's feature order."""

    def __init__(self, owner: "ArticleStreamingAttention") -> None:
        self._o = weakref.proxy(owner)  # no reference cycle: the object and its state go when it does

    @property
    def length(self) -> int:
        return self._o._st.length

    @property
    def sizes(self) -> List[int]:
        d = self._o.dim
        return [math.comb(d + l - 1, l) if l else 1 for l in range(self._o.degree + 1)]

    def _parts(self, x: Tensor) -> List[Tensor]:
        out, at = [], 0
        for m in self.sizes:
            part = x[:, at: at + m].to(self._o.dtype)
            out.append(part[0] if self._o._single else part)
            at += m
        return out

    @property
    def den_moments(self) -> List[Tensor]:
        return self._parts(self._o._st.full_moments()[0])

    @property
    def num_moments(self) -> List[Tensor]:
        return self._parts(self._o._st.full_moments()[1])

    def state_size_bytes(self, include_feature_map: bool = False) -> int:
        o = self._o
        elem = _elem(o.dtype)
        total = o._st.F * (1 + o.value_dim) * elem
        if include_feature_map:
            for l in range(1, o.degree + 1):
                total += math.comb(o.dim + l - 1, l) * l * 8
            total += o._st.F * elem
        return int(total)


class _CoresetView:
    """The merge-and-reduce coreset of the state (MergeReduceCoreset, streaming_taylor_coreset_attention.py
    :332-506)."""

    def __init__(self, owner: "ArticleStreamingAttention") -> None:
        self._o = weakref.proxy(owner)  # no reference cycle: the object and its state go when it does

    @property
    def length(self) -> int:
        return self._o._st.length

    @property
    def block_size(self) -> int:
        return self._o.block_size

    @property
    def num_compressions(self) -> int:
        return self._o._st.num_compressions

    def _pack(self, keys: Tensor, values: Tensor, weights: Tensor) -> CoresetBlock:
        dt = self._o.dtype
        if self._o._single:
            keys, values, weights = keys[0], values[0], weights[0]
        return CoresetBlock(keys.to(dt), values.to(dt), weights.to(dt))

    @property
    def levels(self) -> List[Optional[CoresetBlock]]:
        st = self._o._st
        if st.exact:
            raise NotImplementedError("compressor='none' keeps every token in one exact buffer; use items()")
        return [None if lv is None else self._pack(lv[0], lv[1], lv[2]) for lv in st.level_items()]

    def level_positions(self) -> List[Optional[Tensor]]:
        """Sequence positions of the items of every level (which tokens were selected)."""
        out = []
        for lv in self._o._st.level_items():
            out.append(None if lv is None else (lv[3][0] if self._o._single else lv[3]))
        return out

    def items(self) -> CoresetBlock:
        """Buffer (weight 1), then levels 0, 1, ... (streaming_taylor_coreset_attention.py:469-490)."""
        st = self._o._st
        bk, bv, _ = st.buffer_items()
        ks, vs, ws = [bk], [bv], [torch.ones(bk.shape[:2], device=bk.device, dtype=torch.float32)]
        if not st.exact:
            for lv in st.level_items():
                if lv is not None:
                    ks.append(lv[0])
                    vs.append(lv[1])
                    ws.append(lv[2])
        return self._pack(torch.cat(ks, 1), torch.cat(vs, 1), torch.cat(ws, 1))

    def num_items(self) -> int:
        return self._o._st.num_items()

    def state_size_bytes(self) -> int:
        o = self._o
        elem = _elem(o.dtype)
        return o._st.reference_state_bytes(elem) - o._st.F * (1 + o.value_dim) * elem


class ArticleStreamingAttention:
    """Streaming causal attention via Taylor moments + residual coreset, state on the GPU
    (streaming_taylor_coreset_attention.py:523-616).

    `update(k, v)` then `query(q)` answers causal self-attention including the current token.  With
    `streams=None` keys are [dim] and outputs [value_dim], as in the reference; with `streams=S` keys
    are [S, dim], queries [S, dim] and outputs [S, value_dim], stream s seeded `seed + s`.

    The state is fp32 whatever `dtype` is: inputs are rounded to `dtype` first (the reference casts
    them to its state dtype) and outputs are returned in `dtype`."""

    def __init__(
        self,
        dim: int,
        value_dim: int,
        *,
        degree: int = 2,
        block_size: int = 128,
        scale: Optional[float] = None,
        compressor: str = "sorted_pair",
        device: Optional[Union[str, torch.device]] = None,
        dtype: Union[str, torch.dtype] = torch.float32,
        seed: int = 0,
        max_monomials: int = 5_000_000,
        denominator_eps: float = 1e-12,
        streams: Optional[int] = None,
    ) -> None:
        if dim <= 0:
            raise ValueError("dim must be positive")
        if degree < 0:
            raise ValueError("degree must be non-negative")
        _feature_count(int(dim), int(degree), int(max_monomials))
        if block_size < 2:
            raise ValueError("block_size must be at least 2")
        self.dim = int(dim)
        self.value_dim = int(value_dim)
        self.degree = int(degree)
        self.block_size = int(block_size)
        self.scale = float(1.0 / math.sqrt(dim) if scale is None else scale)
        self.compressor = str(compressor)
        self.device = _resolve_gpu(device)
        self.dtype = _resolve_dtype(dtype)
        if self.dtype not in (torch.float64, torch.float32, torch.bfloat16, torch.float16):
            raise ValueError(f"dtype {self.dtype} is not supported (float64, float32, bfloat16, float16)")
        # what the kernels read and write: float64 tokens are rounded to float32 (the kernels' arithmetic
        # type) and outputs converted back; sizes and views keep the reference's dtype
        self._kdtype = torch.float32 if self.dtype == torch.float64 else self.dtype
        self.seed = int(seed)
        self.denominator_eps = float(denominator_eps)
        self._single = streams is None
        self.streams = 1 if streams is None else int(streams)
        # a float64 object's compress calls score its float64 keys with float64 draws, as the reference's
        # float64 run does (streaming_taylor_coreset_attention.py:441-457)
        self._st = _decode.decode_state(self.streams, self.dim, self.value_dim, degree=self.degree,
                                       block=self.block_size, scale=self.scale, compressor=self.compressor,
                                       seed=self.seed, device=self.device, eps=self.denominator_eps,
                                       score_f64=self.dtype == torch.float64)
        self.sketch = _SketchView(self)
        self.coreset = _CoresetView(self)

    # ---- input handling ----
    def _rows(self, x: Tensor, width: int, what: str) -> Tensor:
        want = (width,) if self._single else (self.streams, width)
        if tuple(x.shape) != want:
            shape = f"[{width}]" if self._single else f"[{self.streams}, {width}]"
            raise ValueError(f"{what} must have shape {shape}, got {tuple(x.shape)}")
        return x.to(device=self.device, dtype=self._kdtype).reshape(self.streams, width)

    def _keys64(self, key: Tensor) -> Optional[Tensor]:
        """The float64 keys [S, dim] of a float64 object (None otherwise); shapes already checked."""
        if self.dtype != torch.float64:
            return None
        return key.to(device=self.device, dtype=torch.float64).reshape(self.streams, self.dim)

    def _stats_buffer(self, return_stats: bool) -> Optional[Tensor]:
        return torch.empty((self.streams, 4), device=self.device, dtype=torch.float32) if return_stats else None

    def _finish(self, out: Tensor, stats: Optional[Tensor]):
        out = (out[0] if self._single else out).to(self.dtype)
        if stats is None:
            return out
        st = stats.cpu()
        nbytes = self.state_size_bytes(include_feature_map=False)
        if self._single:
            s = AttentionQueryStats(float(st[0, 0]), float(st[0, 1]), float(st[0, 2]), self._st.num_items(), nbytes)
        else:
            s = AttentionQueryStats(st[:, 0], st[:, 1], st[:, 2], self._st.num_items(), nbytes)
        return out, s

    # ---- the reference API ----
    @torch.no_grad()
    def update(self, key: Tensor, value: Tensor) -> None:
        """sketch.update(k, v); coreset.append(k, v) (streaming_taylor_coreset_attention.py:576-579)."""
        self._st.update(self._rows(key, self.dim, "key"), self._rows(value, self.value_dim, "value"),
                        self._keys64(key))

    @torch.no_grad()
    def query(self, query: Tensor, *, return_stats: bool = False) -> Union[Tensor, Tuple[Tensor, AttentionQueryStats]]:
        """low + weighted exp_{>t} tail over items(), divided by clamp(den, eps)
        (streaming_taylor_coreset_attention.py:581-609)."""
        stats = self._stats_buffer(return_stats)
        out = self._st.query(self._rows(query, self.dim, "query"), out_dtype=self._kdtype, stats=stats)
        return self._finish(out, stats)

    def state_size_bytes(self, *, include_feature_map: bool = False) -> int:
        """Bytes of the reference's state of one stream at the reference's dtype
        (streaming_taylor_coreset_attention.py:611-612)."""
        return self._st.reference_state_bytes(_elem(self.dtype), include_feature_map)

    @property
    def length(self) -> int:
        return self._st.length

    # ---- extensions ----
    @torch.no_grad()
    def step(self, query: Tensor, key: Tensor, value: Tensor, *, return_stats: bool = False):
        """update(key, value) then query(query), in two kernel launches (plus the block compression
        when the token completes a block)."""
        stats = self._stats_buffer(return_stats)
        out = self._st.step(self._rows(query, self.dim, "query"), self._rows(key, self.dim, "key"),
                            self._rows(value, self.value_dim, "value"), out_dtype=self._kdtype, stats=stats,
                            k64=self._keys64(key))
        return self._finish(out, stats)

    @torch.no_grad()
    def step_into(self, query: Tensor, key: Tensor, value: Tensor, out: Tensor) -> Tensor:
        """step() into a caller-owned `out` ([value_dim], or [S, value_dim] batched) with no device
        allocation, for serving loops and graph capture: the inputs must already be contiguous device
        tensors of this object's shapes and one dtype; a token that completes a block is refused (call
        step() for it).  The device's static scratch serves one object on one stream at a time: another
        object's (or another stream's) step_into is refused until this one calls release_static()."""
        if self._single:
            query, key, value, o2 = query.view(1, -1), key.view(1, -1), value.view(1, -1), out.view(1, -1)
        else:
            o2 = out
        self._st.step_into(query, key, value, o2)
        return out

    def release_static(self) -> None:
        """Lets another object (or another stream) use step_into on this device: waits for this object's
        allocation-free steps and gives up its claim on the device's static scratch."""
        self._st.release_static()

    @torch.no_grad()
    def extend(self, keys: Tensor, values: Tensor) -> None:
        """update() with every row of keys [P, dim] ([S, P, dim] batched) and values, in bulk."""
        if self._single:
            if keys.ndim != 2 or keys.shape[-1] != self.dim or tuple(values.shape) != (keys.shape[0], self.value_dim):
                raise ValueError("keys / values must have shapes [P, dim] / [P, value_dim]")
            keys, values = keys[None], values[None]
        self._st.extend(keys.to(device=self.device, dtype=self._kdtype),
                        values.to(device=self.device, dtype=self._kdtype),
                        keys.to(device=self.device, dtype=torch.float64) if self.dtype == torch.float64 else None)

    @torch.no_grad()
    def prefill(self, q: Tensor, k: Tensor, v: Tensor) -> Tensor:
        """Outputs of update(k_i, v_i); query(q_i) for every row of a prompt ([P, dim], or [S, P, dim]
        batched), leaving the state after the prompt.  Only on a fresh state."""
        if self._st.length != 0:
            raise ValueError("prefill starts from an empty state; use step() / extend() afterwards")
        one = self._single
        q3 = (q[None] if one else q).to(device=self.device, dtype=self._kdtype).contiguous()
        k3 = (k[None] if one else k).to(device=self.device, dtype=self._kdtype).contiguous()
        k64 = ((k[None] if one else k).to(device=self.device, dtype=torch.float64).contiguous()
               if self.dtype == torch.float64 else None)
        v3 = (v[None] if one else v).to(device=self.device, dtype=self._kdtype).contiguous()
        if (q3.ndim != 3 or q3.shape[0] != self.streams or q3.shape[-1] != self.dim or q3.shape != k3.shape
                or tuple(v3.shape) != (self.streams, q3.shape[1], self.value_dim)):
            raise ValueError("q, k, v must be [P, dim] / [P, value_dim] ([S, P, ...] batched)")
        semantics = "exact" if self.compressor == "none" else "levels"
        res = _engine.prefill(q3, k3, v3, degree=self.degree, block=self.block_size, scale=self.scale,
                              semantics=semantics, compressor=self.compressor, seed=self.seed,
                              eps=self.denominator_eps, out_dtype=self._kdtype,
                              score_keys=k64 if semantics == "levels" else None)
        self._st.extend(k3, v3, k64)
        return (res.out[0] if one else res.out).to(self.dtype)

    def state_dict(self) -> dict:
        """The streams' state for a later resume (no counterpart in the reference): the decode state's
        tensors on the host, counters and generator states, plus this object's settings.  Plain tensors
        and Python scalars, so torch.save / torch.load(weights_only=True) round-trip it."""
        return {"attention": self.state_dict_settings(), "decode": self._st.state_dict()}

    def load_state_dict(self, state: dict) -> None:
        """Resume from state_dict() of an object built with the same settings (the device may differ)."""
        mine = self.state_dict_settings()
        if state["attention"] != mine:
            raise ValueError(f"state settings {state['attention']} do not match this object's {mine}")
        self._st.load_state_dict(state["decode"])

    def state_dict_settings(self) -> dict:
        return {"dim": self.dim, "value_dim": self.value_dim, "degree": self.degree, "block_size": self.block_size,
                "scale": self.scale, "compressor": self.compressor, "dtype": str(self.dtype), "seed": self.seed,
                "denominator_eps": self.denominator_eps, "streams": None if self._single else self.streams}


# ----------------------------------------------------------------------------- small CLI sanity check
# Same flags and printed lines as the reference's (streaming_taylor_coreset_attention.py:762-805).

def _demo(args: argparse.Namespace) -> None:
    device = _resolve_gpu(args.device)
    dtype = _resolve_dtype(args.dtype)
    torch.manual_seed(args.seed)
    q = torch.randn(args.n, args.d, device=device, dtype=dtype)
    k = torch.randn(args.n, args.d, device=device, dtype=dtype)
    v = torch.randn(args.n, args.dv, device=device, dtype=dtype)
    # unit directions scaled to the radius: moderate logits for the low-degree split
    q = q / torch.clamp(torch.linalg.vector_norm(q, dim=-1, keepdim=True), min=1e-12) * args.radius
    k = k / torch.clamp(torch.linalg.vector_norm(k, dim=-1, keepdim=True), min=1e-12) * args.radius
    scale = args.scale if args.scale is not None else 1.0
    exact = classical_causal_attention(q, k, v, scale=scale)
    approx, sizes = article_causal_attention(q, k, v, degree=args.degree, block_size=args.block_size, scale=scale,
                                             compressor=args.compressor, seed=args.seed, return_state_sizes=True)
    print(f"relative_l2={safe_relative_l2(approx, exact):.6g}")
    print(f"max_abs={(approx - exact).abs().max().item():.6g}")
    print(f"final_state_bytes={sizes[-1] if sizes else 0:,}")


def _parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(description="Demo for streaming Taylor+coreset attention (HIP/MI355X)")
    p.add_argument("--n", type=int, default=128)
    p.add_argument("--d", type=int, default=16)
    p.add_argument("--dv", type=int, default=16)
    p.add_argument("--degree", type=int, default=2)
    p.add_argument("--block-size", type=int, default=64)
    p.add_argument("--radius", type=float, default=1.0)
    p.add_argument("--scale", type=float, default=None)
    p.add_argument("--compressor", choices=["sorted_pair", "random", "none"], default="sorted_pair")
    p.add_argument("--device", default=None)
    p.add_argument("--dtype", default="float32")
    p.add_argument("--seed", type=int, default=0)
    return p


if __name__ == "__main__":
    _demo(_parser().parse_args())
