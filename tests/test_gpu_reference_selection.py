"""reference_scores=True through the public prefill APIs on the GPU: every compress call ordered on the
host by torch's CPU `keys @ direction` and argsort (the reference's order on this host), the moment
scan and the residual on the GPU.  Nodes bit-exact against the oracle's cascade in torch's order on the
same host, outputs within 1e-4 of the oracle's forward with reference_scores=True."""

import numpy as np
import pytest
import torch

import _engine
import fast_article_attention as faa
import reference_cpu as orc
import streaming_taylor_coreset_attention as stc
from conftest import load_golden

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def rel(a, b):
    return orc.rel_l2(torch.as_tensor(a).float().cpu(), torch.as_tensor(b).float().cpu())


def _cases():
    g = load_golden("levels_c1")  # 1024 tokens, d = 32, block 64
    c1 = (torch.from_numpy(g["q"]), torch.from_numpy(g["k"]), torch.from_numpy(g["v"]), 64, 0)
    t = load_golden("selection_near_ties")  # keys in groups of 8 near-duplicates, block 32
    ties = (torch.from_numpy(t["q"]), torch.from_numpy(t["k"]), torch.from_numpy(t["v"]), t.meta["block"],
            t.meta["seed"])
    return {"c1": c1, "near_ties": ties}


@pytest.mark.parametrize("case", ["c1", "near_ties"])
def test_reference_scores_levels(case):
    q, k, v, block, seed = _cases()[case]
    n = q.shape[0]
    print(f"reference scores levels {case}", flush=True)
    res = _engine.prefill(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), degree=2, block=block, scale=1.0,
                          semantics="levels", compressor="sorted_pair", seed=seed, reference_keys=k[None].contiguous())
    out = stc.article_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV), degree=2, block_size=block, scale=1.0,
                                       seed=seed, reference_scores=True)
    # CPU inputs: the caller's own tensor is scored
    out_cpu = stc.article_causal_attention(q, k, v, degree=2, block_size=block, scale=1.0, seed=seed,
                                           reference_scores=True)
    torch.cuda.synchronize()
    state = orc.LevelState()
    ref = orc.levels_forward(q, k, v, degree=2, block=block, scale=1.0, seed=seed, reference_scores=True,
                             state_out=state)
    src, w = res.node_src.cpu().numpy()[0], res.node_w.cpu().numpy()[0]
    plan = res.plan
    for node in range(plan.n_nodes):
        c = state.calls[int(plan.desc[node, 6])]
        size = int(plan.meta[node, 0])
        assert np.array_equal(src[node, :size], c.src_out) and np.array_equal(w[node, :size], c.w_out), node
    assert rel(res.out[0], ref) < 1e-4 and rel(out, ref) < 1e-4
    assert torch.equal(out.cpu(), out_cpu)
    assert n == ref.shape[0]


@pytest.mark.parametrize("case", ["c1", "near_ties"])
def test_reference_scores_flat(case):
    q, k, v, block, seed = _cases()[case]
    print(f"reference scores flat {case}", flush=True)
    out = faa.fast_article_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV), degree=2, block_size=block, scale=1.0,
                                            seed=seed, reference_scores=True)
    calls = []
    ref = orc.fast_path_forward(q, k, v, degree=2, block=block, scale=1.0, seed=seed, reference_scores=True,
                                calls_out=calls)
    res = _engine.prefill(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), degree=2, block=block, scale=1.0,
                          semantics="flat", compressor="sorted_pair", seed=seed, reference_keys=k[None].contiguous())
    torch.cuda.synchronize()
    sizes = res.plan.meta[:, 0]
    src = res.node_src.cpu().numpy()[0]
    for b, c in enumerate(calls):
        assert np.array_equal(src[b, : sizes[b]], c.src_out), b
    assert rel(out, ref) < 1e-4


def test_reference_scores_batched_heads_and_16bit():
    """[B, H, N, D] inputs: sequence (b, h) seeded seed + b*H + h, its rows scored as views of the
    caller's tensor.  bfloat16 inputs run with bfloat16 draws and scores (their selections are pinned
    against the reference's bfloat16 run on the CPU, tests/test_reference_selection.py); here the API
    returns finite bfloat16 outputs."""
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 3, 300, 16, generator=g) * 0.3
    k = torch.randn(2, 3, 300, 16, generator=g) * 0.3
    v = torch.randn(2, 3, 300, 8, generator=g)
    print("reference scores batched", flush=True)
    out = stc.article_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV), degree=2, block_size=32, scale=1.0, seed=4,
                                       reference_scores=True)
    torch.cuda.synchronize()
    for b in range(2):
        for h in range(3):
            ref = orc.levels_forward(q[b, h], k[b, h], v[b, h], degree=2, block=32, scale=1.0, seed=4 + b * 3 + h,
                                     reference_scores=True)
            assert rel(out[b, h], ref) < 1e-4
    qb, kb, vb = q.bfloat16(), k.bfloat16(), v.bfloat16()
    outb = faa.fast_article_causal_attention(qb.to(DEV), kb.to(DEV), vb.to(DEV), degree=2, block_size=32,
                                             scale=1.0, seed=4, reference_scores=True)
    torch.cuda.synchronize()
    assert outb.dtype == torch.bfloat16 and torch.isfinite(outb.float()).all()
