"""The prefill configurations the headline workloads are quoted on, run at their full sizes through the
public API on the GPU, with sampled heads checked against the oracle (the reference's CPU algorithm,
per-sequence seeds seed + b H + h).  Causal outputs of rows [0, m) depend only on the first m tokens,
so at 65536 tokens the oracle checks a prefix of rows of the full-size GPU run.

Tolerances: rel-L2 1e-4 for fp32 inputs; 5e-3 for bf16 inputs and outputs (against the fp32 oracle
on the upcast inputs)."""

import numpy as np
import pytest
import torch

import _engine
import c3_cascade as c3
import fast_article_attention as faa
import reference_cpu as orc
import streaming_taylor_coreset_attention as stc

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def rel(a, b):
    return orc.rel_l2(torch.as_tensor(a).float().cpu(), torch.as_tensor(b).float().cpu())


def test_c2_batched_bf16_flat_and_levels():
    """8 x 16 heads, N = 4096, d = dv = 64, degree 2, block 256, scale 1/8, q, k, v ~ N(0, 1), bf16."""
    b_, h_, n = 8, 16, 4096
    q, k, v = (x.to(torch.bfloat16) for x in orc.make_data((b_, h_), n, 64, 64, radius=1.0, data="normal", seed=0))
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    flat = faa.fast_article_causal_attention(qd, kd, vd, degree=2, block_size=256, scale=0.125,
                                             compressor="sorted_pair", seed=0)
    lev = stc.article_causal_attention(qd, kd, vd, degree=2, block_size=256, scale=0.125, compressor="sorted_pair",
                                       seed=0)
    torch.cuda.synchronize()
    assert flat.shape == (b_, h_, n, 64) and flat.dtype == torch.bfloat16 and lev.dtype == torch.bfloat16
    assert torch.isfinite(flat.float()).all() and torch.isfinite(lev.float()).all()
    for b, h in [(0, 0), (5, 11), (7, 15)]:
        print(f"c2 head ({b}, {h})", flush=True)
        qh, kh, vh = q[b, h].float(), k[b, h].float(), v[b, h].float()
        seed = b * h_ + h
        ref_f = orc.fast_path_forward(qh, kh, vh, degree=2, block=256, scale=0.125, compressor="sorted_pair",
                                      seed=seed)
        ref_l = orc.levels_forward(qh, kh, vh, degree=2, block=256, scale=0.125, compressor="sorted_pair",
                                   seed=seed)
        assert rel(flat[b, h], ref_f) < 5e-3
        assert rel(lev[b, h], ref_l) < 5e-3


def test_c3_long_context_levels():
    """1 x 32 heads, N = 65536, d = dv = 64, degree 2, block 256, scale 1/8, merge-and-reduce levels,
    q, k in the radius-1 ball, v ~ N(0, 1), fp32: every row of head 31 and rows [0, 8192) of head 0
    against the oracle."""
    n, m = c3.N, 8192
    q, k, v = c3.inputs()
    out = stc.article_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV), degree=2, block_size=256, scale=0.125,
                                       compressor="sorted_pair", seed=0)
    torch.cuda.synchronize()
    assert out.shape == (1, 32, n, 64) and torch.isfinite(out).all()
    for h, rows in ((0, m), (31, n)):
        print(f"c3 head {h} rows [0, {rows})", flush=True)
        ref = orc.levels_forward(q[0, h, :rows], k[0, h, :rows], v[0, h, :rows], degree=2, block=256, scale=0.125,
                                 compressor="sorted_pair", seed=h)
        assert rel(out[0, h, :rows], ref) < 1e-4
        if rows == n:  # the last 8192 rows alone (they read the level-6..8 nodes)
            assert rel(out[0, h, n - m:], ref[n - m:]) < 1e-4


def test_c3_every_coreset_node_bit_exact():
    """All 511 level-tree nodes of all 32 heads (kept token and weight of every item, in order) equal
    the oracle's compress calls of the same position in the reference's call order."""
    q, k, v = c3.inputs()
    res = _engine.prefill(q[0].to(DEV), k[0].to(DEV), v[0].to(DEV), degree=2, block=256, scale=0.125,
                          semantics="levels", compressor="sorted_pair", seed=0)
    src = res.node_src.cpu().numpy()
    w = res.node_w.cpu().numpy()
    plan = res.plan
    assert plan.n_nodes == 511 and len(plan.call_sizes) == 511
    slots = [int(plan.desc[node, 6]) for node in range(plan.n_nodes)]
    sizes = [int(plan.meta[node, 0]) for node in range(plan.n_nodes)]
    for h in range(c3.HEADS):
        print(f"c3 nodes head {h}", flush=True)
        calls = c3.head_cascade(h).calls
        for node in range(plan.n_nodes):
            c = calls[slots[node]]
            assert sizes[node] == c.src_out.shape[0]
            assert np.array_equal(src[h, node, : sizes[node]], c.src_out), f"head {h} node {node}"
            assert np.array_equal(w[h, node, : sizes[node]], c.w_out), f"head {h} node {node}"


def test_c4_degree3_levels_full_size():
    """4 x 32 heads, N = 16384, d = 16, dv = 64, degree 3 (969 features), block 128, scale 1, levels,
    q, k in the radius-1.5 ball, fp32: heads (0, 0) and (3, 31) in full against the oracle."""
    b_, h_, n = 4, 32, 16384
    q, k, v = orc.make_data((b_, h_), n, 16, 64, radius=1.5, data="unit_ball", seed=0)
    out = stc.article_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV), degree=3, block_size=128, scale=1.0,
                                       compressor="sorted_pair", seed=0)
    torch.cuda.synchronize()
    assert out.shape == (b_, h_, n, 64) and torch.isfinite(out).all()
    for b, h in [(0, 0), (3, 31)]:
        print(f"c4 head ({b}, {h})", flush=True)
        ref = orc.levels_forward(q[b, h], k[b, h], v[b, h], degree=3, block=128, scale=1.0, compressor="sorted_pair",
                                 seed=b * h_ + h)
        assert rel(out[b, h], ref) < 1e-4


def test_c5_decode_all_streams():
    """64 x 32 = 2048 streams, d = dv = 64, degree 2, block 256, scale 1/8, bf16 q, k, v ~ N(0,1) / 8: a
    4096-token prefix through extend(), then 300 update + query steps (one block completion with its
    compress and merges at token 4352); streams 0 and 2047 against the oracle's level semantics on the
    whole sequence (decode output of token t == row t, stream s seeded s)."""
    s_, prefix, steps = 2048, 4096, 300
    n = prefix + steps
    g = torch.Generator().manual_seed(5)
    q, k, v = ((torch.randn(s_, n, 64, generator=g) * 0.125).to(torch.bfloat16) for _ in range(3))
    st = stc.ArticleStreamingAttention(64, 64, degree=2, block_size=256, scale=0.125, device=DEV,
                                       dtype=torch.bfloat16, seed=0, streams=s_)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    st.extend(kd[:, :prefix], vd[:, :prefix])
    outs = torch.stack([st.step(qd[:, i], kd[:, i], vd[:, i]) for i in range(prefix, n)], dim=1)
    torch.cuda.synchronize()
    assert outs.shape == (s_, steps, 64) and torch.isfinite(outs.float()).all()
    assert st.length == n
    for s in (0, s_ - 1):
        print(f"c5 stream {s}", flush=True)
        ref = orc.levels_forward(q[s].float(), k[s].float(), v[s].float(), degree=2, block=256, scale=0.125,
                                 compressor="sorted_pair", seed=s)
        assert rel(outs[s], ref[prefix:]) < 5e-3


def test_c5_decode_full_prefix():
    """The decode workload's state: 2048 streams with a 32768-token prefix (counter 128: one level-7
    node of 128 items, weight 256), bf16 q, k, v ~ N(0,1) / 8 drawn on the GPU, then 260 steps (the block
    completion at token 33024 merges nothing: level 0 is free); streams 0 and 2047 against the oracle
    on their whole sequences, and the level-7 node's kept tokens and weights bit-exact."""
    s_, prefix, steps = 2048, 32768, 260
    n = prefix + steps
    g = torch.Generator(device=DEV).manual_seed(11)
    qd, kd, vd = ((torch.randn(s_, n, 64, generator=g, device=DEV) * 0.125).to(torch.bfloat16) for _ in range(3))
    st = stc.ArticleStreamingAttention(64, 64, degree=2, block_size=256, scale=0.125, device=DEV,
                                       dtype=torch.bfloat16, seed=0, streams=s_)
    st.extend(kd[:, :prefix], vd[:, :prefix])
    assert st.length == prefix
    pos7 = st.coreset.level_positions()[7].cpu().numpy()
    w7 = st.coreset.levels[7].weights.float().cpu().numpy()
    outs = torch.stack([st.step(qd[:, i], kd[:, i], vd[:, i]) for i in range(prefix, n)], dim=1)
    torch.cuda.synchronize()
    assert outs.shape == (s_, steps, 64) and torch.isfinite(outs.float()).all()
    for s in (0, s_ - 1):
        print(f"c5 full prefix, stream {s}", flush=True)
        q, k, v = qd[s].float().cpu(), kd[s].float().cpu(), vd[s].float().cpu()
        state = orc.LevelState()
        ref = orc.levels_forward(q, k, v, degree=2, block=256, scale=0.125, compressor="sorted_pair", seed=s,
                                 state_out=state)
        assert rel(outs[s], ref[prefix:]) < 5e-3
        # the level-7 node after the prefix: the 255th compress call (128 blocks: 255 calls)
        c = state.calls[254]
        assert c.level == 7
        assert np.array_equal(pos7[s], c.src_out) and np.array_equal(w7[s], c.w_out)
