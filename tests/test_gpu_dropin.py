"""Drop-in coverage beyond the headline shapes, on the GPU against the oracle: compress calls above 1024
items (blocks of 2048 and 4096, flat and levels, prefill and decode), value widths above 256 (column
groups), float64 inputs (compress calls drawn and scored in float64, everything else computed on the
float32 rounding, outputs float64), and the benchmark_attention.py CSV columns."""

import csv

import numpy as np
import pytest
import torch

import _engine
import benchmark_attention as bench_mod
import fast_article_attention as faa
import reference_cpu as orc
import streaming_taylor_coreset_attention as stc
import triton_article_attention as taa

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def rel(a, b):
    return orc.rel_l2(torch.as_tensor(a).float().cpu(), torch.as_tensor(b).float().cpu())


@pytest.mark.parametrize("block,n,semantics", [(2048, 2 * 2048 + 300, "flat"), (2048, 4 * 2048 + 77, "levels"),
                                               (4096, 2 * 4096 + 5, "levels"), (1500, 3 * 1500 + 11, "levels")])
def test_large_blocks_match_the_oracle(block, n, semantics):
    """Compress calls on up to 4096 items: every node's kept tokens and weights bit-exact against the
    oracle's compress calls, outputs within 1e-4."""
    print(f"large block {block} n={n} {semantics}", flush=True)
    q, k, v = orc.make_data((), n, 32, 32, radius=1.0, data="unit_ball", seed=3)
    res = _engine.prefill(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), degree=2, block=block, scale=1.0,
                          semantics=semantics, compressor="sorted_pair", seed=7)
    torch.cuda.synchronize()
    if semantics == "flat":
        ref = orc.fast_path_forward(q, k, v, degree=2, block=block, scale=1.0, compressor="sorted_pair", seed=7)
        calls = orc.flat_coreset(k.numpy(), block, "sorted_pair", 7, orc.projection_scores)
    else:
        state = orc.LevelState()
        ref = orc.levels_forward(q, k, v, degree=2, block=block, scale=1.0, compressor="sorted_pair", seed=7,
                                 state_out=state)
        calls = state.calls
    assert rel(res.out[0], ref) < 1e-4
    src, w = res.node_src.cpu().numpy()[0], res.node_w.cpu().numpy()[0]
    nodes = [node for node in range(res.plan.n_nodes) if int(res.plan.meta[node, 0]) > 0]
    assert len(nodes) == len(calls)
    for node in nodes:
        size, slot = int(res.plan.meta[node, 0]), int(res.plan.desc[node, 6])
        assert size == calls[slot].src_out.shape[0]
        assert np.array_equal(src[node, :size], calls[slot].src_out), f"node {node}"
        assert np.array_equal(w[node, :size], calls[slot].w_out), f"node {node}"


def test_large_block_decode_matches_the_oracle():
    """Streaming decode with block 2048 (compress calls on 2048 items): a 4200-token prefix through
    extend(), then 60 steps, against the oracle's level semantics."""
    s_, prefix, steps, block = 3, 4200, 60, 2048
    n = prefix + steps
    q, k, v = orc.make_data((s_,), n, 16, 24, radius=1.0, data="unit_ball", seed=4)
    st = stc.ArticleStreamingAttention(16, 24, degree=2, block_size=block, scale=1.0, device=DEV, seed=0, streams=s_)
    st.extend(k[:, :prefix].to(DEV), v[:, :prefix].to(DEV))
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    outs = torch.stack([st.step(qd[:, i], kd[:, i], vd[:, i]) for i in range(prefix, n)], dim=1)
    torch.cuda.synchronize()
    for s in range(s_):
        ref = orc.levels_forward(q[s], k[s], v[s], degree=2, block=block, scale=1.0, compressor="sorted_pair", seed=s)
        assert rel(outs[s], ref[prefix:]) < 1e-4


@pytest.mark.parametrize("api", ["flat", "levels"])
def test_value_width_above_256(api):
    """dv = 300 runs as column groups of 256 + 44: equal to the oracle, and each group equal to a
    separate call on its columns."""
    q, k, v = orc.make_data((1, 2), 700, 16, 300, radius=1.0, data="unit_ball", seed=5)
    fn = faa.fast_article_causal_attention if api == "flat" else stc.article_causal_attention
    out = fn(q.to(DEV), k.to(DEV), v.to(DEV), degree=2, block_size=64, scale=1.0, compressor="sorted_pair", seed=2)
    narrow = fn(q.to(DEV), k.to(DEV), v[..., 256:].contiguous().to(DEV), degree=2, block_size=64, scale=1.0,
                compressor="sorted_pair", seed=2)
    torch.cuda.synchronize()
    assert out.shape == (1, 2, 700, 300)
    assert torch.equal(out[..., 256:], narrow)
    ref_fn = orc.fast_path_forward if api == "flat" else orc.levels_forward
    for h in range(2):
        ref = ref_fn(q[0, h], k[0, h], v[0, h], degree=2, block=64, scale=1.0, compressor="sorted_pair", seed=2 + h)
        assert rel(out[0, h], ref) < 1e-4


def test_streaming_value_width_above_256():
    """ArticleStreamingAttention with value_dim 600 (column groups of 256 + 256 + 88, every group fed the
    same keys and seeds): prefill, extend and steps through block completions against the oracle's level
    semantics; every group keeps the same coreset; the moments, the level items and a save / resume
    cover all 600 columns; step_into refuses (one kernel call's columns only)."""
    s_, n, d, dv, block, prompt = 2, 330, 16, 600, 64, 150
    print("streaming value width 600", flush=True)
    q, k, v = orc.make_data((s_,), n, d, dv, radius=1.0, data="unit_ball", seed=8)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    st = stc.ArticleStreamingAttention(d, dv, degree=2, block_size=block, scale=1.0, device=DEV, seed=0, streams=s_)
    out_p = st.prefill(qd[:, :100], kd[:, :100], vd[:, :100])
    st.extend(kd[:, 100:prompt], vd[:, 100:prompt])
    outs = torch.stack([st.step(qd[:, i], kd[:, i], vd[:, i]) for i in range(prompt, n - 20)], dim=1)
    saved = st.state_dict()
    st2 = stc.ArticleStreamingAttention(d, dv, degree=2, block_size=block, scale=1.0, device=DEV, seed=0, streams=s_)
    st2.load_state_dict(saved)
    tail1 = torch.stack([st.step(qd[:, i], kd[:, i], vd[:, i]) for i in range(n - 20, n)], dim=1)
    tail2 = torch.stack([st2.step(qd[:, i], kd[:, i], vd[:, i]) for i in range(n - 20, n)], dim=1)
    den, num = st._st.full_moments()
    torch.cuda.synchronize()
    assert out_p.shape == (s_, 100, dv) and outs.shape == (s_, n - 20 - prompt, dv)
    assert torch.equal(tail1, tail2)
    groups = st._st.groups
    assert [g.dv for g in groups] == [256, 256, 88]
    for lv in range(len(groups[0].level_items())):
        items = [g.level_items()[lv] for g in groups]
        if items[0] is not None:
            assert all(torch.equal(it[3], items[0][3]) and torch.equal(it[2], items[0][2]) for it in items)
    for s in range(s_):
        ref = orc.levels_forward(q[s], k[s], v[s], degree=2, block=block, scale=1.0, compressor="sorted_pair", seed=s)
        assert rel(out_p[s], ref[:100]) < 1e-4
        assert rel(outs[s], ref[prompt: n - 20]) < 1e-4
        assert rel(tail1[s], ref[n - 20:]) < 1e-4
        fk = orc.features(k[s].double(), 2, True)
        assert rel(num[s], fk.T @ v[s].double()) < 2e-5 and rel(den[s], fk.sum(0)) < 2e-5
    items = st.coreset.items()
    assert items.values.shape[-1] == dv
    with pytest.raises(ValueError, match="column groups"):
        st.step_into(qd[:, 0].contiguous(), kd[:, 0].contiguous(), vd[:, 0].contiguous(),
                     torch.empty(s_, dv, device=DEV))


def _nodes_equal_calls(res, calls):
    src, w = res.node_src.cpu().numpy()[0], res.node_w.cpu().numpy()[0]
    nodes = [node for node in range(res.plan.n_nodes) if int(res.plan.meta[node, 0]) > 0]
    assert len(nodes) == len(calls)
    for node in nodes:
        size, slot = int(res.plan.meta[node, 0]), int(res.plan.desc[node, 6])
        assert np.array_equal(src[node, :size], calls[slot].src_out), f"node {node}"
        assert np.array_equal(w[node, :size], calls[slot].w_out), f"node {node}"
    return src


@pytest.mark.parametrize("semantics", ["flat", "levels"])
def test_float64_selections_follow_the_float64_draws(semantics):
    """float64 keys: the compressor draws float64 directions and uniforms and scores the float64 keys
    in fp64, as the reference's float64 run does: every node bit-exact against the oracle's float64
    compress calls (which differ from the float32 run's), outputs within 1e-4 of the oracle's float64
    forward."""
    n, block = 1100, 64
    q, k, v = orc.make_data((), n, 16, 16, radius=1.0, data="unit_ball", seed=6, dtype=torch.float64)
    kd = k[None].to(DEV).contiguous()
    res = _engine.prefill(q[None].float().to(DEV), k[None].float().to(DEV), v[None].float().to(DEV), degree=2,
                          block=block, scale=1.0, semantics=semantics, compressor="sorted_pair", seed=3,
                          score_keys=kd)
    res32 = _engine.prefill(q[None].float().to(DEV), k[None].float().to(DEV), v[None].float().to(DEV), degree=2,
                            block=block, scale=1.0, semantics=semantics, compressor="sorted_pair", seed=3)
    torch.cuda.synchronize()
    if semantics == "flat":
        calls = orc.flat_coreset(k.numpy(), block, "sorted_pair", 3, orc.projection_scores)
        ref = orc.fast_path_forward(q, k, v, degree=2, block=block, scale=1.0, compressor="sorted_pair", seed=3)
    else:
        state = orc.LevelState()
        ref = orc.levels_forward(q, k, v, degree=2, block=block, scale=1.0, compressor="sorted_pair", seed=3,
                                 state_out=state)
        calls = state.calls
    assert calls[0].direction.dtype == np.float64 and calls[0].uniforms.dtype == np.float64
    src64 = _nodes_equal_calls(res, calls)
    assert not np.array_equal(src64, res32.node_src.cpu().numpy()[0]), "float64 and float32 draws selected alike"
    assert rel(res.out[0], ref) < 1e-4


def test_float64_public_apis():
    """float64 q, k, v through the public APIs: float64 outputs within 1e-4 of the oracle's float64
    forward (whose compress calls draw and score in float64); the streaming object (prefill, extend,
    step) keeps the float64 levels of the oracle's cascade; the Triton-semantics API (segment means,
    no draws) equals its float32 run on the rounded inputs."""
    n = 700
    q, k, v = orc.make_data((), n, 16, 16, radius=1.0, data="unit_ball", seed=6, dtype=torch.float64)
    kw = dict(degree=2, block_size=64, scale=1.0, compressor="sorted_pair", seed=1)
    for fn, ref_fn in ((faa.fast_article_causal_attention, orc.fast_path_forward),
                       (stc.article_causal_attention, orc.levels_forward)):
        out64 = fn(q.to(DEV), k.to(DEV), v.to(DEV), **kw)
        assert out64.dtype == torch.float64
        ref = ref_fn(q, k, v, degree=2, block=64, scale=1.0, compressor="sorted_pair", seed=1)
        assert rel(out64, ref) < 1e-4
        # host float64 tensors too (moved to the GPU and back)
        assert torch.equal(fn(q, k, v, **kw), out64.cpu())
    state = orc.LevelState()
    ref = orc.levels_forward(q, k, v, degree=2, block=64, scale=1.0, compressor="sorted_pair", seed=1,
                             state_out=state)
    # the streaming object with dtype float64: prefill 300 rows, extend 200, then step token by token
    st = stc.ArticleStreamingAttention(16, 16, degree=2, block_size=64, scale=1.0, device=DEV,
                                       dtype=torch.float64, seed=1)
    out_p = st.prefill(q[:300].to(DEV), k[:300].to(DEV), v[:300].to(DEV))
    st.extend(k[300:500].to(DEV), v[300:500].to(DEV))
    outs = torch.stack([st.step(q[i].to(DEV), k[i].to(DEV), v[i].to(DEV)) for i in range(500, n)])
    torch.cuda.synchronize()
    assert out_p.dtype == torch.float64 and outs.dtype == torch.float64
    assert rel(out_p, ref[:300]) < 1e-4 and rel(outs, ref[500:]) < 1e-4
    got = [lv for lv in st._st.level_items()]
    want = state.levels
    assert len([g for g in got if g is not None]) == len([w for w in want if w is not None])
    for lvl, item in enumerate(got):
        if item is None:
            assert lvl >= len(want) or want[lvl] is None
            continue
        keys, _, w, pos = item
        assert np.array_equal(pos[0].cpu().numpy(), want[lvl][0]), f"level {lvl}"
        assert np.array_equal(w[0].cpu().numpy(), want[lvl][1]), f"level {lvl}"
        assert torch.equal(st._st.lev_k64[0, lvl, :, :16].cpu(), k[torch.from_numpy(want[lvl][0])])
    assert st.state_size_bytes() == st._st.reference_state_bytes(8) == 2 * st._st.reference_state_bytes(4)
    # save / resume of a float64 stream keeps its float64 key rows
    sd = st.state_dict()
    st2 = stc.ArticleStreamingAttention(16, 16, degree=2, block_size=64, scale=1.0, device=DEV,
                                        dtype=torch.float64, seed=1)
    st2.load_state_dict(sd)
    nb = st._st.buf_len
    assert torch.equal(st2._st.lev_k64, st._st.lev_k64)
    assert torch.equal(st2._st.buf_k64[:, :nb], st._st.buf_k64[:, :nb])
    assert torch.equal(st2.step(q[0].to(DEV), k[0].to(DEV), v[0].to(DEV)), st.step(q[0].to(DEV), k[0].to(DEV),
                                                                                      v[0].to(DEV)))
    with pytest.raises(ValueError):
        st.step_into(q[0].float().to(DEV), k[0].float().to(DEV), v[0].float().to(DEV),
                     torch.empty(16, device=DEV))
    # the Triton-semantics API upcasts float64 like the reference, and writes float64 outputs
    q32, k32, v32 = q.float(), k.float(), v.float()
    o = taa.triton_article_causal_attention(q[None, None].to(DEV), k[None, None].to(DEV), v[None, None].to(DEV),
                                            block_size=64, scale=1.0, output_dtype=torch.float64)
    o32 = taa.triton_article_causal_attention(q32[None, None].to(DEV), k32[None, None].to(DEV),
                                              v32[None, None].to(DEV), block_size=64, scale=1.0)
    assert o.dtype == torch.float64 and torch.equal(o, o32.double())


def test_benchmark_csv_has_the_reference_columns(tmp_path):
    out = tmp_path / "bench.csv"
    rows = bench_mod.main(["--sweep-n", "256", "600", "--d", "16", "--dv", "16", "--block-size", "64",
                           "--repeats", "1", "--csv", str(out)])
    with out.open() as fh:
        got = list(csv.DictReader(fh))
    assert list(got[0].keys()) == list(bench_mod.COLUMNS) and len(got) == 2
    for r in rows:
        assert r["rel_l2"] < 0.5 and r["article_median_ms"] > 0 and r["classical_median_ms"] > 0
    # state columns: the per-token trace of the streaming object
    st = stc.ArticleStreamingAttention(16, 16, degree=2, block_size=64, scale=1.0, device=DEV)
    q, k, v = faa._make_data(600, 16, 16, radius=1.0, data="unit_ball", device=DEV, dtype=torch.float32, seed=0)
    sizes, items = [], []
    for i in range(600):
        st.update(k[i], v[i])
        sizes.append(st.state_size_bytes())
        items.append(st.coreset.num_items())
    assert rows[1]["article_final_state_bytes"] == sizes[-1]
    assert rows[1]["article_max_state_bytes"] == max(sizes)
    assert rows[1]["article_max_coreset_items"] == max(items)
