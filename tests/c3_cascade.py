"""Shared by the tests of the long-context workload (1 x 32 heads, N = 65536, d = dv = 64, block 256,
merge-and-reduce levels, q / k in the radius-1 ball, v ~ N(0, 1), seed 0): its inputs, and the
oracle's level cascade of one head (every compress call, in the reference's call order,
streaming_taylor_coreset_attention.py:387-411), optionally auditing each call's sort against the
reference's own `keys @ direction` order."""

import functools
from typing import List, Tuple

import numpy as np
import torch

import reference_cpu as orc

N, HEADS, D, DV, BLOCK, SCALE = 65536, 32, 64, 64, 256, 0.125


@functools.lru_cache(maxsize=1)
def inputs() -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return orc.make_data((1, HEADS), N, D, DV, radius=1.0, data="unit_ball", seed=0)


class OrderAudit:
    """score_fn for the oracle's cascade: the fixed-order fp64 scores the HIP compressor uses (these
    drive the selection), with every call's stable sort compared to the sort of the reference's
    `keys @ direction` scores (torch's CPU matmul).  Differences must sit on near-ties."""

    def __init__(self) -> None:
        self.calls = 0
        self.flips = 0  # sorted positions where the two orders differ
        self.calls_with_flips = 0
        self.bad: List[Tuple[int, int]] = []  # (call, position) of a difference away from a near-tie

    def __call__(self, keys: np.ndarray, direction: np.ndarray) -> np.ndarray:
        ours = orc.projection_scores(keys, direction)
        ref = orc.torch_scores(keys, direction)
        ref_order = np.argsort(ref, kind="stable")
        our_order = np.argsort(ours, kind="stable")
        diff, bad = near_tie_flips(ref, ref_order, our_order)
        self.flips += int(diff.size)
        self.calls_with_flips += int(diff.size > 0)
        self.bad += [(self.calls, p) for p in bad]
        self.calls += 1
        return ours


def near_tie_flips(ref_scores, ref_order, our_order, ulps=8):
    """Positions where two sorts differ; each must sit on a near-tie of the reference scores."""
    bad = []
    diff = np.nonzero(ref_order != our_order)[0]
    s_sorted = ref_scores[ref_order]
    for p in diff:
        lo, hi = max(p - 1, 0), min(p + 1, len(s_sorted) - 1)
        gap = min(abs(float(s_sorted[p]) - float(s_sorted[lo])) if lo != p else np.inf,
                  abs(float(s_sorted[hi]) - float(s_sorted[p])) if hi != p else np.inf)
        if gap > ulps * np.spacing(np.float32(abs(s_sorted[p]) + 1e-30)):
            bad.append(int(p))
    return diff, bad


def head_cascade(h: int, score_fn=orc.projection_scores) -> orc.LevelState:
    """Every compress call of head h over the whole sequence (seed h, the per-sequence seed)."""
    k = inputs()[1][0, h].numpy()
    g = torch.Generator(device="cpu")
    g.manual_seed(h)
    state = orc.LevelState()
    for b in range(N // BLOCK):
        orc.level_block_complete(state, g, np.arange(b * BLOCK, (b + 1) * BLOCK, dtype=np.int64), k, "sorted_pair",
                                 score_fn)
    return state
