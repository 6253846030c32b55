"""Drop-in for the reference's GPU module (triton_article_attention.py) -- same public API, served by
hand-written HIP kernels for MI355X instead of Triton (there is no Triton in this package).

`triton_article_causal_attention` computes what the reference's fused kernel computes
(triton_article_attention.py:265-369, :447-577): the exact degree-<=2 Taylor term over the whole causal
prefix, the exact residual inside the current article block, and deterministic segment-mean
representatives (weight = compress_stride) for completed blocks with a later query, with
exp(min(x, 80)).  The Taylor term comes from the exact moment scan rather than an O(N^2) sweep.
Accumulation is fp32 (the reference uses tf32 dots); the output dtype is `output_dtype`.
"""

from __future__ import annotations

import argparse
import math
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple, Union

import torch

import _engine
import _native
from _cli_util import event_ms, fmt_bytes
from fast_article_attention import safe_relative_l2  # noqa: F401  (re-exported like the reference)

Tensor = torch.Tensor

__all__ = ["TritonArticleStats", "build_segment_mean_coreset", "torch_classical_causal_attention",
           "triton_article_causal_attention", "triton_flash_causal_attention", "exp_taylor", "safe_relative_l2"]


def _require_backend() -> None:
    """The reference raises ImportError without Triton (triton_article_attention.py:72-77); here the
    backend is the HIP library."""
    _native.lib()


def _require_device(*tensors: Tensor) -> None:
    for x in tensors:
        if not x.is_cuda:
            raise ValueError("HIP kernels require GPU (cuda/ROCm) tensors")


def _ceil_div(a: int, b: int) -> int:
    return (int(a) + int(b) - 1) // int(b)


def _attention_scale(scale: Optional[float], dim: int) -> float:
    return float(1.0 / math.sqrt(dim) if scale is None else scale)


def exp_taylor(x: Tensor, degree: int) -> Tensor:
    total = torch.ones_like(x)
    term = torch.ones_like(x)
    for r in range(1, degree + 1):
        term = term * x / float(r)
        total = total + term
    return total


def torch_classical_causal_attention(q: Tensor, k: Tensor, v: Tensor, *, scale: Optional[float] = None) -> Tensor:
    """Exact torch reference for [N,D] or [B,H,N,D] (triton_article_attention.py:123-143); the
    batched product uses a contiguous right operand."""
    if q.shape != k.shape:
        raise ValueError("q and k must have identical shape")
    if q.ndim == 2:
        n, dim = q.shape
        logits = (q @ k.T.contiguous()) * _attention_scale(scale, dim)
        mask = torch.ones(n, n, device=q.device, dtype=torch.bool).tril()
        return torch.softmax(logits.masked_fill(~mask, float("-inf")), dim=-1) @ v
    if q.ndim == 4:
        b, h, n, dim = q.shape
        if v.shape[:3] != q.shape[:3]:
            raise ValueError("v must have shape [B,H,N,Dv]")
        logits = torch.matmul(q, k.transpose(-1, -2).contiguous()) * _attention_scale(scale, dim)
        mask = torch.ones(n, n, device=q.device, dtype=torch.bool).tril()
        return torch.matmul(torch.softmax(logits.masked_fill(~mask[None, None], float("-inf")), dim=-1), v)
    raise ValueError("q/k/v must be [N,D] or [B,H,N,D]")


def _flatten_bh_qkv(q: Tensor, k: Tensor, v: Tensor) -> Tuple[Tensor, Tensor, Tensor, Tuple[int, ...], bool]:
    """Contiguous [BH,N,D], [BH,N,D], [BH,N,Dv] (triton_article_attention.py:146-162)."""
    if q.shape != k.shape:
        raise ValueError(f"q and k must match, got {tuple(q.shape)} and {tuple(k.shape)}")
    if q.ndim == 2:
        if v.ndim != 2 or v.shape[0] != q.shape[0]:
            raise ValueError("for [N,D] q/k, v must be [N,Dv]")
        return q[None].contiguous(), k[None].contiguous(), v[None].contiguous(), tuple(q.shape), False
    if q.ndim == 4:
        if v.ndim != 4 or v.shape[:3] != q.shape[:3]:
            raise ValueError("for [B,H,N,D] q/k, v must be [B,H,N,Dv]")
        b, h, n, d = q.shape
        return (q.contiguous().view(b * h, n, d), k.contiguous().view(b * h, n, d),
                v.contiguous().view(b * h, n, v.shape[-1]), tuple(q.shape), True)
    raise ValueError("q/k/v must be [N,D] or [B,H,N,D]")


def _restore_shape(out3: Tensor, q_shape: Tuple[int, ...], batched: bool) -> Tensor:
    """[BH, N, Dv] kernel output back to the caller's [B, H, N, Dv], or [N, Dv] for one sequence."""
    return out3.reshape(*q_shape[:-1], out3.shape[-1]) if batched else out3[0]


@dataclass(frozen=True)
class TritonArticleStats:
    """triton_article_attention.py:172-181"""

    degree: int
    block_size: int
    compress_stride: int
    coreset_items_per_sequence: int
    coreset_bytes_per_sequence: int
    kv_bytes_per_sequence: int
    score_matrix_bytes_per_sequence: int
    output_bytes_per_sequence: int


@torch.no_grad()
def build_segment_mean_coreset(k_bhn: Tensor, v_bhn: Tensor, *, block_size: int,
                               compress_stride: int) -> Tuple[Tensor, Tensor, int]:
    """Segment-mean reps [BH,R,D], [BH,R,Dv] of completed blocks with a later query
    (triton_article_attention.py:189-245), computed by the HIP segment-mean kernel.  CPU inputs are
    processed on the first ROCm device and returned on the CPU."""
    if k_bhn.ndim != 3 or v_bhn.ndim != 3:
        raise ValueError("k_bhn and v_bhn must be [BH,N,D] and [BH,N,Dv]")
    if k_bhn.shape[:2] != v_bhn.shape[:2]:
        raise ValueError("k_bhn and v_bhn must have the same [BH,N]")
    if block_size <= 0 or compress_stride <= 0:
        raise ValueError("block_size and compress_stride must be positive")
    if block_size % compress_stride != 0:
        raise ValueError("for the Triton kernel, block_size must be divisible by compress_stride")
    bh, n, dim = k_bhn.shape
    dv = v_bhn.shape[-1]
    rpb = block_size // compress_stride
    nb = max(0, (n - 1) // block_size)
    n_rep = nb * rpb
    home = k_bhn.device
    if n_rep == 0:
        return (torch.empty(bh, 0, dim, device=home, dtype=k_bhn.dtype),
                torch.empty(bh, 0, dv, device=home, dtype=v_bhn.dtype), rpb)
    if home.type == "cuda":
        kg, vg = k_bhn.contiguous(), v_bhn.contiguous()
    else:
        if not torch.cuda.is_available():
            raise RuntimeError("streaming-attention HIP kernels need a ROCm GPU; none is visible")
        kg, vg = k_bhn.cuda().contiguous(), v_bhn.cuda().contiguous()
    if kg.dtype not in _native.DTYPE_CODES or vg.dtype != kg.dtype:
        kg, vg = kg.float(), vg.float()
    rep_k = torch.empty(bh, n_rep, dim, device=kg.device, dtype=torch.float32)
    rep_v = torch.empty(bh, n_rep, dv, device=kg.device, dtype=torch.float32)
    st = _native.lib().sta_segment_mean(kg.data_ptr(), vg.data_ptr(), _native.DTYPE_CODES[kg.dtype], bh, n, dim, dv,
                                        block_size, compress_stride, n_rep, rep_k.data_ptr(), rep_v.data_ptr(),
                                        _native.stream_handle(kg.device))
    _native.check(st, "sta_segment_mean")
    return rep_k.to(device=home, dtype=k_bhn.dtype), rep_v.to(device=home, dtype=v_bhn.dtype), rpb


@torch.no_grad()
def triton_article_causal_attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    *,
    degree: int = 2,
    block_size: int = 128,
    compress_stride: int = 2,
    scale: Optional[float] = None,
    block_m: int = 16,
    block_n: int = 64,
    block_r: int = 64,
    value_block: Optional[int] = None,
    denominator_eps: float = 1.0e-12,
    output_dtype: Optional[torch.dtype] = torch.float32,
    return_stats: bool = False,
) -> Union[Tensor, Tuple[Tensor, TritonArticleStats]]:
    """Same arguments, checks and result as triton_article_attention.py:447-577.  block_m, block_n,
    block_r and value_block are tile hints of the Triton kernel; the HIP kernels use their own fixed
    CDNA4 tiling, so they are accepted and ignored."""
    _require_backend()
    _require_device(q, k, v)
    if degree not in (0, 1, 2):
        raise NotImplementedError("Triton article kernel currently supports degree 0, 1, or 2")
    if block_size <= 0 or compress_stride <= 0:
        raise ValueError("block_size and compress_stride must be positive")
    if block_size % compress_stride != 0:
        raise ValueError("block_size must be divisible by compress_stride")
    q3, k3, v3, original_shape, had_bh = _flatten_bh_qkv(q, k, v)
    bh, n, dim = q3.shape
    dv = v3.shape[-1]
    if dim > 128:
        raise ValueError("this compact kernel supports D <= 128; increase BLOCK_D logic for larger heads")
    if dv > 256:
        raise ValueError("this compact kernel supports Dv <= 256")
    if q3.dtype not in _native.DTYPE_CODES:
        q3, k3 = q3.float(), k3.float()
    if v3.dtype not in _native.DTYPE_CODES:
        v3 = v3.float()
    if not (q3.dtype == k3.dtype == v3.dtype):
        q3, k3, v3 = q3.float(), k3.float(), v3.float()
    out_dtype = output_dtype or torch.float32
    # an output type the kernels do not store (float64) is written as float32 and converted
    k_out = out_dtype if out_dtype in _native.DTYPE_CODES else torch.float32
    res = _engine.prefill(q3, k3, v3, degree=degree, block=block_size, scale=_attention_scale(scale, dim),
                          semantics="segment", stride=compress_stride, exp_clamp=True, eps=denominator_eps,
                          out_dtype=k_out)
    out = _restore_shape(res.out, original_shape, had_bh).to(out_dtype)
    if not return_stats:
        return out
    r = max(0, (n - 1) // block_size) * (block_size // compress_stride)
    ekv = q3.element_size()
    eo = torch.tensor([], dtype=out_dtype).element_size()
    stats = TritonArticleStats(degree, block_size, compress_stride, int(r), int(r * (dim + dv) * ekv),
                               int(n * (dim + dv) * ekv), int(n * n * ekv), int(n * dv * eo))
    return out, stats


@torch.no_grad()
def triton_flash_causal_attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    *,
    scale: Optional[float] = None,
    block_m: int = 16,
    block_n: int = 64,
    value_block: Optional[int] = None,
    output_dtype: Optional[torch.dtype] = torch.float32,
) -> Tensor:
    """Exact causal attention baseline (triton_article_attention.py:580-637): online row maximum, fp32
    accumulation, no N x N score matrix, for [N,D] and [B,H,N,D] tensors; computed by the HIP flash
    kernel.  block_m, block_n and value_block are tile hints of the Triton kernel, accepted and ignored
    (the HIP kernel uses its own CDNA4 tiling)."""
    _require_backend()
    _require_device(q, k, v)
    q3, k3, v3, original_shape, had_bh = _flatten_bh_qkv(q, k, v)
    dim = q3.shape[-1]
    dv = v3.shape[-1]
    if dim > 128:
        raise ValueError("this compact kernel supports D <= 128")
    if dv > 256:
        raise ValueError("this compact kernel supports Dv <= 256")
    if not (q3.dtype == k3.dtype == v3.dtype) or q3.dtype not in _native.DTYPE_CODES:
        q3, k3, v3 = q3.float(), k3.float(), v3.float()
    out_dtype = output_dtype or torch.float32
    out3 = _engine.flash(q3, k3, v3, scale=_attention_scale(scale, dim),
                         out_dtype=out_dtype if out_dtype in _native.DTYPE_CODES else torch.float32)
    return _restore_shape(out3, original_shape, had_bh).to(out_dtype)


# ----------------------------------------------------------------------------- demo / benchmark CLI
# Same flags and table columns as the reference's CLI (triton_article_attention.py:640-855); the
# "triton_*" columns time this module's HIP kernels.

def _make_data(n: int, d: int, dv: int, *, batch: int, heads: int, radius: float, data: str,
               device: torch.device, dtype: torch.dtype, seed: int) -> Tuple[Tensor, Tensor, Tensor]:
    """Inputs in the reference's draw order on `device` (triton_article_attention.py:645-680): randn q, k,
    v of `dtype`; for unit_ball the radii rand^(1/d) r of q then k; unit_sphere scales to radius r."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    lead = (batch, heads) if batch * heads > 1 else ()
    q = torch.randn(*lead, n, d, device=device, dtype=dtype, generator=g)
    k = torch.randn(*lead, n, d, device=device, dtype=dtype, generator=g)
    v = torch.randn(*lead, n, dv, device=device, dtype=dtype, generator=g)

    def unit(x):
        return x / torch.clamp(torch.linalg.vector_norm(x, dim=-1, keepdim=True), min=1e-12)

    if data == "unit_ball":
        rq = torch.rand((*q.shape[:-1], 1), device=device, dtype=dtype, generator=g).pow(1.0 / d) * radius
        rk = torch.rand((*k.shape[:-1], 1), device=device, dtype=dtype, generator=g).pow(1.0 / d) * radius
        q, k = unit(q) * rq, unit(k) * rk
    elif data == "unit_sphere":
        q, k = unit(q) * radius, unit(k) * radius
    elif data != "normal":
        raise ValueError("data must be one of {'unit_ball', 'unit_sphere', 'normal'}")
    return q, k, v


_DTYPES = {"float32": torch.float32, "fp32": torch.float32, "float16": torch.float16, "fp16": torch.float16,
           "half": torch.float16, "bfloat16": torch.bfloat16, "bf16": torch.bfloat16}


def _resolve_dtype(name: str) -> torch.dtype:
    if name.lower() not in _DTYPES:
        raise ValueError(f"unsupported dtype {name!r}; choose one of {sorted(_DTYPES)}")
    return _DTYPES[name.lower()]


def _demo(args: argparse.Namespace) -> None:
    _require_backend()
    if not torch.cuda.is_available():
        raise RuntimeError("a ROCm GPU is required for this benchmark")
    device = torch.device(args.device)
    dtype = _resolve_dtype(args.dtype)
    scale = args.scale if args.scale is not None else (1.0 / math.sqrt(args.d) if args.standard_scale else 1.0)
    headers = ["n", "rel_l2_article", "max_abs_article", "rel_l2_flash", "torch_classical_ms", "triton_flash_ms",
               "triton_article_ms", "coreset_items", "coreset_bytes", "kv_bytes", "score_matrix"]
    print("\n" + " | ".join(headers))
    print(" | ".join(["---"] * len(headers)))
    for n in args.sweep_n:
        q, k, v = _make_data(n, args.d, args.dv, batch=args.batch, heads=args.heads, radius=args.radius,
                             data=args.data, device=device, dtype=dtype, seed=args.seed)
        tiles = dict(block_m=args.block_m, block_n=args.block_n, value_block=args.value_block,
                     output_dtype=torch.float32)
        article_kw = dict(tiles, degree=args.degree, block_size=args.block_size, compress_stride=args.compress_stride,
                          scale=scale, block_r=args.block_r)
        exact = torch_classical_causal_attention(q.float(), k.float(), v.float(), scale=scale)
        flash = triton_flash_causal_attention(q, k, v, scale=scale, **tiles)
        article, stats = triton_article_causal_attention(q, k, v, return_stats=True, **article_kw)
        torch_ms = event_ms(lambda: torch_classical_causal_attention(q.float(), k.float(), v.float(), scale=scale),
                                 args.repeats)
        flash_ms = event_ms(lambda: triton_flash_causal_attention(q, k, v, scale=scale, **tiles), args.repeats)
        article_ms = event_ms(lambda: triton_article_causal_attention(q, k, v, **article_kw), args.repeats)
        print(" | ".join([
            str(n), f"{safe_relative_l2(article, exact):.4g}", f"{(article - exact).abs().max().item():.4g}",
            f"{safe_relative_l2(flash, exact):.4g}", f"{torch_ms:.3f}", f"{flash_ms:.3f}", f"{article_ms:.3f}",
            str(stats.coreset_items_per_sequence), fmt_bytes(stats.coreset_bytes_per_sequence),
            fmt_bytes(stats.kv_bytes_per_sequence), fmt_bytes(stats.score_matrix_bytes_per_sequence),
        ]))


def _parse_args(argv: Optional[Sequence[str]] = None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description="HIP (MI355X) kernels for article-style Taylor + residual-coreset "
                                            "attention, with the exact flash baseline")
    p.add_argument("--sweep-n", type=int, nargs="+", default=[256, 512, 1024, 2048])
    p.add_argument("--d", type=int, default=32)
    p.add_argument("--dv", type=int, default=32)
    p.add_argument("--batch", type=int, default=1)
    p.add_argument("--heads", type=int, default=1)
    p.add_argument("--degree", type=int, default=2, choices=[0, 1, 2])
    p.add_argument("--block-size", type=int, default=128)
    p.add_argument("--compress-stride", type=int, default=2,
                   help="1 disables residual compression and should match exact attention")
    p.add_argument("--block-m", type=int, default=16)
    p.add_argument("--block-n", type=int, default=64)
    p.add_argument("--block-r", type=int, default=64)
    p.add_argument("--value-block", type=int, default=None)
    p.add_argument("--data", choices=["unit_ball", "unit_sphere", "normal"], default="unit_ball")
    p.add_argument("--radius", type=float, default=1.0)
    p.add_argument("--scale", type=float, default=None)
    p.add_argument("--standard-scale", action="store_true", help="Use 1/sqrt(d) when --scale is omitted")
    p.add_argument("--device", default="cuda")
    p.add_argument("--dtype", default="float16", choices=sorted(_DTYPES))
    p.add_argument("--repeats", type=int, default=10)
    p.add_argument("--seed", type=int, default=0)
    return p.parse_args(argv)


if __name__ == "__main__":
    _demo(_parse_args())
