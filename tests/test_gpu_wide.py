"""Keys wider than 128 dimensions and Taylor degrees 4 .. 8, on the GPU against the oracle.

Keys wider than the 128 staged dimensions go through dimension windows (every feature split stages the
4 blocks of 32 dimensions its monomials use); degrees 5 .. 8 run the fp32-product scan with two-word
feature quads; degree 4 reaches the reference's default max_monomials (5,000,000 features, D = 102).
The reference's CPU fast path and streaming object have no key-width bound
(fast_article_attention.py:137-181, :552-565; streaming_taylor_coreset_attention.py:139, :150-178).
Where the feature map is too large for the oracle's token loop, the oracle's moment sums come from their
closed form (low="direct"), which the oracle tests pin against the token loop."""

import numpy as np
import pytest
import torch

import _engine
import fast_article_attention as faa
import reference_cpu as orc
import streaming_taylor_coreset_attention as stc

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def rel(a, b):
    return orc.rel_l2(torch.as_tensor(a).float().cpu(), torch.as_tensor(b).float().cpu())


@pytest.mark.parametrize("d", [160, 192, 256])
def test_wide_keys_prefill_flat_levels_exact(d):
    """Degree 2 with 160 / 192 / 256-dimensional keys: the fast path (flat coreset), the level API and
    compressor "none" (classical attention) against the oracle."""
    n, dv = 600, 32
    print(f"wide keys prefill d={d}", flush=True)
    q, k, v = orc.make_data((1, 2), n, d, dv, radius=1.0, data="unit_ball", seed=11)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kw = dict(degree=2, block_size=64, scale=1.0, compressor="sorted_pair", seed=5)
    flat = faa.fast_article_causal_attention(qd, kd, vd, **kw)
    lev = stc.article_causal_attention(qd, kd, vd, **kw)
    exact = faa.fast_article_causal_attention(qd, kd, vd, degree=2, block_size=64, scale=1.0, compressor="none")
    torch.cuda.synchronize()
    for h in range(2):
        args = (q[0, h], k[0, h], v[0, h])
        ref_f = orc.fast_path_forward(*args, degree=2, block=64, scale=1.0, compressor="sorted_pair", seed=5 + h)
        ref_l = orc.levels_forward(*args, degree=2, block=64, scale=1.0, compressor="sorted_pair", seed=5 + h)
        assert rel(flat[0, h], ref_f) < 1e-4
        assert rel(lev[0, h], ref_l) < 1e-4
        assert rel(exact[0, h], orc.classical_attention(*args, 1.0)) < 2e-5


@pytest.mark.parametrize("d", [192, 256])
def test_wide_keys_decode(d):
    """Streaming decode with 192 / 256-dimensional keys: extend() over a prompt (windowed state
    accumulation), then step() token by token through block completions, against the oracle's level
    semantics; the state moments against the fp64 feature sums."""
    s_, n, dv, prompt = 2, 330, 24, 150
    print(f"wide keys decode d={d}", flush=True)
    q, k, v = orc.make_data((s_,), n, d, dv, radius=1.0, data="unit_ball", seed=12)
    st = stc.ArticleStreamingAttention(d, dv, degree=2, block_size=64, scale=1.0, device=DEV, seed=0, streams=s_)
    st.extend(k[:, :prompt].to(DEV), v[:, :prompt].to(DEV))
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    outs = torch.stack([st.step(qd[:, i], kd[:, i], vd[:, i]) for i in range(prompt, n)], dim=1)
    den, num = st._st.full_moments()
    torch.cuda.synchronize()
    for s in range(s_):
        ref = orc.levels_forward(q[s], k[s], v[s], degree=2, block=64, scale=1.0, compressor="sorted_pair", seed=s)
        assert rel(outs[s], ref[prompt:]) < 1e-4
        fk = orc.features(k[s].double(), 2, True)
        assert rel(den[s], fk.sum(0)) < 2e-5
        assert rel(num[s], fk.T @ v[s].double()) < 2e-5


@pytest.mark.parametrize("d,degree", [(8, 5), (16, 5), (8, 6), (4, 8)])
def test_high_degree_levels_and_decode(d, degree):
    """Taylor degrees 5 .. 8: the level API (prefill) and the streaming object (extend, then steps)
    against the oracle's level semantics with the general feature map."""
    n, dv, prompt = 420, 16, 200
    print(f"high degree d={d} degree={degree}", flush=True)
    q, k, v = orc.make_data((), n, d, dv, radius=1.0, data="unit_ball", seed=13)
    ref = orc.levels_forward(q, k, v, degree=degree, block=64, scale=1.0, compressor="sorted_pair", seed=0)
    out = stc.article_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV), degree=degree, block_size=64, scale=1.0,
                                       compressor="sorted_pair", seed=0)
    st = stc.ArticleStreamingAttention(d, dv, degree=degree, block_size=64, scale=1.0, device=DEV, seed=0)
    st.extend(k[:prompt].to(DEV), v[:prompt].to(DEV))
    outs = torch.stack([st.step(q[i].to(DEV), k[i].to(DEV), v[i].to(DEV)) for i in range(prompt, n)])
    torch.cuda.synchronize()
    assert rel(out, ref) < 1e-4
    assert rel(outs, ref[prompt:]) < 1e-4


def test_degree4_up_to_the_default_feature_limit():
    """Degree 4 with d = 100 (4,598,126 features, under the default max_monomials of 5,000,000): the raw
    Taylor sums against their closed form, the level API against the oracle, and decode steps; d = 103
    exceeds max_monomials and raises the reference's ValueError."""
    d, n, dv = 100, 200, 16
    print("degree 4 d=100", flush=True)
    q, k, v = orc.make_data((), n, d, dv, radius=1.0, data="unit_ball", seed=14)
    res = _engine.prefill(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), degree=4, block=1, scale=1.0,
                          semantics="taylor")
    num, den = orc.low_sums_direct(q, k, v, 4, 1.0)
    assert rel(res.out[0], num) < 1e-4 and rel(res.den[0], den) < 1e-4
    assert res.feature_count == 4598126
    out = stc.article_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV), degree=4, block_size=64, scale=1.0, seed=0)
    ref = orc.levels_forward(q, k, v, degree=4, block=64, scale=1.0, seed=0, low="direct")
    assert rel(out, ref) < 1e-4
    st = stc.ArticleStreamingAttention(d, dv, degree=4, block_size=64, scale=1.0, device=DEV, seed=0)
    st.extend(k[:130].to(DEV), v[:130].to(DEV))
    outs = torch.stack([st.step(q[i].to(DEV), k[i].to(DEV), v[i].to(DEV)) for i in range(130, n)])
    torch.cuda.synchronize()
    assert rel(outs, ref[130:]) < 1e-4
    with pytest.raises(ValueError, match="max_monomials"):
        stc.ArticleStreamingAttention(103, dv, degree=4, device=DEV)


def test_degree3_wide_keys_levels():
    """Degree 3 with 160-dimensional keys (708,561 features in 4 windows) through the level API."""
    d, n, dv = 160, 260, 16
    print("degree 3 d=160", flush=True)
    q, k, v = orc.make_data((), n, d, dv, radius=1.0, data="unit_ball", seed=15)
    out = stc.article_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV), degree=3, block_size=64, scale=1.0, seed=0)
    torch.cuda.synchronize()
    ref = orc.levels_forward(q, k, v, degree=3, block=64, scale=1.0, seed=0, low="direct")
    assert rel(out, ref) < 1e-4


def test_limits_beyond_the_kernels():
    """Beyond the kernels: degree 9, degree 5 above d = 64, degree 4 above d = 128 (NotImplementedError);
    D above 256 (ValueError)."""
    q, k, v = orc.make_data((), 70, 8, 8, radius=1.0, data="unit_ball", seed=1)
    with pytest.raises(NotImplementedError):
        stc.article_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV), degree=9, block_size=16)
    with pytest.raises(NotImplementedError):
        stc.ArticleStreamingAttention(68, 8, degree=5, device=DEV, max_monomials=10 ** 9)
    with pytest.raises(NotImplementedError):
        stc.ArticleStreamingAttention(130, 8, degree=4, device=DEV, max_monomials=10 ** 9)
    with pytest.raises(ValueError):
        stc.ArticleStreamingAttention(260, 8, degree=2, device=DEV)
    wide = torch.zeros(1, 1, 40, 260, device=DEV)
    with pytest.raises(ValueError):
        faa.fast_article_causal_attention(wide, wide, wide[..., :8].contiguous(), degree=2, block_size=16)
    assert np.isfinite(stc.article_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV), degree=8, block_size=16,
                                                    scale=1.0).cpu().numpy()).all()
