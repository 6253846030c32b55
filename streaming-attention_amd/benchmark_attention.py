"""Drop-in for the reference's benchmark_attention.py: the streaming Taylor + merge-and-reduce coreset
attention against exact causal attention over a sweep of sequence lengths, with the same flags, the
same printed table and the same CSV columns (benchmark_attention.py:204-228, :236-270, :273-306), run
through this package's GPU path.

    python streaming-attention_amd/benchmark_attention.py --sweep-n 256 512 1024 --d 32 --dv 32 \\
        --degree 2 --block-size 128 --csv results.csv

Differences from the reference, all in how numbers are obtained, not in what is reported:
  * the article call is article_causal_attention of this package (HIP kernels; the inputs are moved to
    the GPU when --device is the CPU);
  * the state-size columns come from the per-token size formula (state_size_trace /
    coreset_item_trace, equal to the reference's per-token update loop, benchmark_attention.py:107-136)
    instead of replaying every token through the streaming object.
"""

from __future__ import annotations

import argparse
import csv
import math
import pathlib
import sys
from typing import Dict, List

import torch

_HERE = pathlib.Path(__file__).resolve().parent
if str(_HERE) not in sys.path:
    sys.path.insert(0, str(_HERE))

from _cli_util import fmt_bytes, pick_device, wall_ms  # noqa: E402
from fast_article_attention import _make_data, _resolve_dtype  # noqa: E402
from streaming_taylor_coreset_attention import (  # noqa: E402
    article_causal_attention,
    classical_causal_attention,
    coreset_item_trace,
    safe_relative_l2,
    state_size_trace,
)

# CSV columns, in the reference's order (benchmark_attention.py:204-228)
COLUMNS = ("n", "d", "dv", "degree", "block_size", "compressor", "data", "radius", "scale", "device", "dtype",
           "rel_l2", "max_abs", "mean_abs", "classical_median_ms", "classical_best_ms", "article_median_ms",
           "article_best_ms", "article_final_state_bytes", "article_max_state_bytes", "article_max_coreset_items",
           "classical_kv_bytes", "classical_naive_scores_bytes")


def state_bytes(n: int, d: int, dv: int, *, degree: int, block_size: int, compressor: str, elem: int):
    """(final state bytes, max state bytes, max coreset items) over the n per-token updates."""
    sizes = state_size_trace(n, d, dv, degree, block_size, compressor, elem)
    items = coreset_item_trace(n, block_size, compressor)
    return (sizes[-1], max(sizes), max(items)) if n else (0, 0, 0)


def run_one(args: argparse.Namespace, n: int) -> Dict[str, object]:
    device = pick_device(args.device)
    dtype = _resolve_dtype(args.dtype)
    scale = args.scale if args.scale is not None else (1.0 / math.sqrt(args.d) if args.standard_scale else 1.0)
    q, k, v = _make_data(n, args.d, args.dv, radius=args.radius, data=args.data, device=device, dtype=dtype,
                         seed=args.seed)
    kw = dict(degree=args.degree, block_size=args.block_size, scale=scale, compressor=args.compressor, seed=args.seed)
    with torch.no_grad():
        exact = classical_causal_attention(q, k, v, scale=scale)
        approx = article_causal_attention(q, k, v, **kw).to(exact.device)
        diff = (approx.float() - exact.float()).abs()
        row = {
            "rel_l2": safe_relative_l2(approx, exact),
            "max_abs": diff.max().item(),
            "mean_abs": diff.mean().item(),
        }
    gpu = torch.device("cuda") if torch.cuda.is_available() else device
    row["classical_median_ms"], row["classical_best_ms"] = wall_ms(
        lambda: classical_causal_attention(q, k, v, scale=scale), args.repeats, device)
    row["article_median_ms"], row["article_best_ms"] = wall_ms(
        lambda: article_causal_attention(q, k, v, **kw), args.repeats, gpu)
    elem = torch.tensor([], dtype=dtype).element_size()
    final_b, max_b, max_items = state_bytes(n, args.d, args.dv, degree=args.degree, block_size=args.block_size,
                                            compressor=args.compressor, elem=elem)
    row.update(article_final_state_bytes=final_b, article_max_state_bytes=max_b, article_max_coreset_items=max_items,
               classical_kv_bytes=n * (args.d + args.dv) * elem, classical_naive_scores_bytes=n * n * elem)
    row.update(n=n, d=args.d, dv=args.dv, degree=args.degree, block_size=args.block_size, compressor=args.compressor,
               data=args.data, radius=args.radius, scale=scale, device=str(device),
               dtype=str(dtype).replace("torch.", ""))
    return {c: row[c] for c in COLUMNS}


def print_table(rows: List[Dict[str, object]]) -> None:
    cols = [("n", lambda r: str(r["n"])), ("rel_l2", lambda r: f"{r['rel_l2']:.4g}"),
            ("max_abs", lambda r: f"{r['max_abs']:.4g}"), ("classical_ms", lambda r: f"{r['classical_median_ms']:.3f}"),
            ("article_ms", lambda r: f"{r['article_median_ms']:.3f}"),
            ("article_state", lambda r: fmt_bytes(int(r["article_max_state_bytes"]))),
            ("score_matrix", lambda r: fmt_bytes(int(r["classical_naive_scores_bytes"]))),
            ("coreset_items", lambda r: str(r["article_max_coreset_items"]))]
    print("\n" + " | ".join(h for h, _ in cols))
    print(" | ".join("---" for _ in cols))
    for r in rows:
        print(" | ".join(f(r) for _, f in cols))
    print()


def write_csv(path: pathlib.Path, rows: List[Dict[str, object]]) -> None:
    path.parent.mkdir(parents=True, exist_ok=True)
    with path.open("w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=list(COLUMNS))
        w.writeheader()
        w.writerows(rows)


def parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--sweep-n", type=int, nargs="+", default=[256, 512, 1024])
    p.add_argument("--d", type=int, default=32)
    p.add_argument("--dv", type=int, default=32)
    p.add_argument("--degree", type=int, default=2)
    p.add_argument("--block-size", type=int, default=128)
    p.add_argument("--compressor", choices=["sorted_pair", "random", "none"], default="sorted_pair")
    p.add_argument("--data", choices=["unit_ball", "unit_sphere", "normal"], default="unit_ball")
    p.add_argument("--radius", type=float, default=1.0)
    p.add_argument("--scale", type=float, default=None)
    p.add_argument("--standard-scale", action="store_true", help="Use 1/sqrt(d) when --scale is omitted")
    p.add_argument("--device", default="auto")
    p.add_argument("--dtype", default="float32")
    p.add_argument("--repeats", type=int, default=3)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--csv", type=pathlib.Path, default=None)
    return p


def main(argv=None) -> List[Dict[str, object]]:
    args = parser().parse_args(argv)
    rows = [run_one(args, n) for n in args.sweep_n]
    print_table(rows)
    if args.csv is not None:
        write_csv(args.csv, rows)
        print(f"Wrote {args.csv}")
    return rows


if __name__ == "__main__":
    main()
