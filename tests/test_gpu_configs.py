"""The prefill configurations the headline workloads are quoted on, run at their full sizes through the
public API on the GPU, with sampled heads checked against the oracle (the reference's CPU algorithm,
per-sequence seeds seed + b H + h).  Causal outputs of rows [0, m) depend only on the first m tokens,
so at 65536 tokens the oracle checks a prefix of rows of the full-size GPU run.

Tolerances: rel-L2 1e-4 for fp32 inputs; 5e-3 for bf16 inputs and outputs (against the fp32 oracle
on the upcast inputs)."""

import pytest
import torch

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


def test_c3_long_context_levels_prefix_rows():
    """1 x 32 heads, N = 65536, d = dv = 64, degree 2, block 256, scale 1/8, merge-and-reduce levels,
    q, k in the radius-1 ball, v ~ N(0, 1), fp32: rows [0, 8192) of heads 0 and 31 against the oracle."""
    n, m = 65536, 8192
    q, k, v = orc.make_data((1, 32), n, 64, 64, radius=1.0, data="unit_ball", seed=0)
    out = stc.article_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV), degree=2, block_size=256, scale=0.125,
                                       compressor="sorted_pair", seed=0)
    torch.cuda.synchronize()
    assert out.shape == (1, 32, n, 64) and torch.isfinite(out).all()
    for h in (0, 31):
        print(f"c3 head {h} rows [0, {m})", flush=True)
        ref = orc.levels_forward(q[0, h, :m], k[0, h, :m], v[0, h, :m], degree=2, block=256, scale=0.125,
                                 compressor="sorted_pair", seed=h)
        assert rel(out[0, h, :m], ref) < 1e-4


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
    """64 x 32 = 2048 streams, d = dv = 64, degree 2, block 256, scale 1/8, bf16 q, k, v ~ N(0, 1) / 8: a
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
