"""Pins the CPU oracle (oracle/reference_cpu.py) before it is trusted as the checker:
known answers, closed forms, brute force, the reference's golden vectors, and planted mistakes."""

import itertools
import math

import numpy as np
import pytest
import torch

import reference_cpu as orc

TOL_FP32 = dict(rel=2e-6)


def rel(a, b):
    return orc.rel_l2(torch.as_tensor(a), torch.as_tensor(b))


# --------------------------------------------------------------------------- primitives

def test_exp_taylor_known_values():
    # test_streaming_attention.py:24-28
    y = orc.exp_taylor(torch.tensor([0.0, 1.0, -1.0]), 3)
    assert torch.allclose(y, torch.tensor([1.0, 8.0 / 3.0, 1.0 / 3.0]))


def test_exp_taylor_matches_reference_values(golden):
    g = golden("features")
    assert np.array_equal(orc.exp_taylor(torch.from_numpy(g["x"]), 3).numpy(), g["taylor3"])


@pytest.mark.parametrize("d,t,expect", [(64, 2, 2145), (32, 2, 561), (16, 3, 969), (8, 0, 1), (5, 1, 6)])
def test_feature_counts(d, t, expect):
    assert len(orc.monomials(d, t)) == expect
    assert expect == sum(math.comb(d + l - 1, l) for l in range(t + 1))


def test_feature_order_is_combinations_with_replacement():
    combos = orc.monomials(6, 3)
    expected = [()] + [c for l in (1, 2, 3) for c in itertools.combinations_with_replacement(range(6), l)]
    assert combos == expected
    # degree-2 block equals torch.triu_indices row-major order (fast_article_attention.py:173)
    r, c = torch.triu_indices(6, 6)
    assert [x for x in combos if len(x) == 2] == list(zip(r.tolist(), c.tolist()))


def test_features_match_reference_fast_path(golden):
    g = golden("features")
    x = torch.from_numpy(g["x"])
    assert np.array_equal(orc.features(x, 2, True).numpy(), g["key2"])
    assert np.array_equal(orc.features(x, 2, False).numpy(), g["query2"])


@pytest.mark.parametrize("degree", [0, 1, 2, 3, 4])
def test_feature_inner_product_is_truncated_exp(degree):
    g = torch.Generator().manual_seed(degree)
    q = torch.randn(9, 5, generator=g, dtype=torch.float64)
    k = torch.randn(7, 5, generator=g, dtype=torch.float64)
    lhs = orc.features(q, degree, False) @ orc.features(k, degree, True).T
    rhs = orc.exp_taylor(q @ k.T, degree)
    assert torch.allclose(lhs, rhs, rtol=1e-12, atol=1e-12)


def test_inv_multinomial_values():
    assert orc.inv_multinomial(()) == 1.0
    assert orc.inv_multinomial((2, 2)) == 0.5
    assert orc.inv_multinomial((1, 1, 1)) == pytest.approx(1 / 6)
    assert orc.inv_multinomial((0, 0, 3)) == 0.5
    assert orc.inv_multinomial((0, 1, 2)) == 1.0


# --------------------------------------------------------------------------- moments

@pytest.mark.parametrize("degree", [0, 1, 2, 3])
def test_stream_moments_equal_closed_form(degree):
    g = torch.Generator().manual_seed(10 + degree)
    q = torch.randn(40, 6, generator=g, dtype=torch.float64) * 0.4
    k = torch.randn(40, 6, generator=g, dtype=torch.float64) * 0.4
    v = torch.randn(40, 3, generator=g, dtype=torch.float64)
    num, den = orc.low_sums_stream(q, k, v, degree, 0.7)
    num2, den2 = orc.low_sums_direct(q, k, v, degree, 0.7)
    assert torch.allclose(num, num2, rtol=1e-10, atol=1e-10)
    assert torch.allclose(den, den2, rtol=1e-10, atol=1e-10)


def test_stream_moments_match_reference(golden):
    g = golden("flat_c1")
    q, k, v = (torch.from_numpy(g[x]) for x in "qkv")
    num, den = orc.low_sums_stream(q, k, v, 2, 1.0)
    assert rel(num, g["low_num"]) < 1e-6
    assert rel(den, g["low_den"]) < 1e-6


def test_make_data_matches_reference(golden):
    g = golden("flat_c1")
    q, k, v = orc.make_data((), 1024, 32, 32, radius=1.0, data="unit_ball", seed=0)
    assert np.array_equal(q.numpy(), g["q"]) and np.array_equal(k.numpy(), g["k"]) and np.array_equal(v.numpy(), g["v"])


# --------------------------------------------------------------------------- flash baseline recursion

@pytest.mark.parametrize("block_n", [1, 7, 16, 64, 1000])
def test_flash_recursion_equals_softmax_attention(block_n):
    # the blocked online-softmax recursion (triton_article_attention.py:397-428) against torch.softmax
    g = torch.Generator().manual_seed(block_n)
    q = torch.randn(150, 12, generator=g) * 2.0  # logits of tens: the running maximum moves
    k = torch.randn(150, 12, generator=g) * 2.0
    v = torch.randn(150, 5, generator=g)
    out = orc.flash_attention_blocked(q, k, v, 1.5, block_n)
    assert rel(out, orc.classical_attention(q, k, v, 1.5)) < 1e-12


def test_flash_recursion_special_cases():
    g = torch.Generator().manual_seed(1)
    v = torch.randn(40, 3, generator=g)
    q = torch.randn(40, 4, generator=g)
    k = torch.ones(40, 4)  # equal keys: uniform weights over each prefix
    out = orc.flash_attention_blocked(q, k, v, 1.0, 16)
    expect = torch.cumsum(v.double(), 0) / torch.arange(1, 41, dtype=torch.float64)[:, None]
    assert torch.allclose(out, expect, rtol=1e-12, atol=1e-12)
    assert torch.equal(out[0], v[0].double())  # row 0 sees key 0 only
    # logits of 1000 and 2000: no overflow, each row takes its largest visible key
    qb = torch.tensor([[1.0, 0.0]] * 3)
    kb = torch.tensor([[0.0, 0.0], [1000.0, 0.0], [2000.0, 0.0]])
    out = orc.flash_attention_blocked(qb, kb, v[:3], 1.0, 2)
    assert torch.allclose(out, v[:3].double())


# --------------------------------------------------------------------------- exact residual

def test_none_compressor_reconstructs_classical():
    # test_fast_article_attention.py:10-29 with the reference tolerances
    torch.manual_seed(0)
    q = torch.randn(64, 8) * 0.1
    k = torch.randn(64, 8) * 0.1
    v = torch.randn(64, 7)
    out = orc.fast_path_forward(q, k, v, degree=2, block=16, scale=1.0, compressor="none")
    exact = orc.classical_attention(q, k, v, 1.0)
    assert rel(out, exact) < 2e-6
    assert (out.double() - exact).abs().max().item() < 3e-6


def test_none_compressor_matches_reference_output(golden):
    g = golden("flat_c1")
    q, k, v = (torch.from_numpy(g[x]) for x in "qkv")
    out = orc.fast_path_forward(q, k, v, degree=2, block=128, scale=1.0, compressor="none")
    assert rel(out, g["out_none"]) < 1e-6
    assert rel(out, g["exact"]) < 1e-5


# --------------------------------------------------------------------------- flat coreset

def _golden_calls(g, prefix, count):
    return [{k[len(f"{prefix}call{i}_"):]: g[k] for k in g if k.startswith(f"{prefix}call{i}_")} for i in range(count)]


def _normalise(raw):
    d = torch.from_numpy(raw)
    return (d / torch.clamp(torch.linalg.vector_norm(d), min=1e-12)).numpy()


@pytest.mark.parametrize("comp", ["sorted_pair", "random"])
def test_flat_draws_and_selection_match_reference(golden, comp):
    g = golden("flat_c1")
    k = g["k"]
    ref_calls = _golden_calls(g, f"{comp}_", int(g[f"{comp}_ncalls"]))
    calls = orc.flat_coreset(k, 128, comp, 0, score_fn=orc.torch_scores)
    assert len(calls) == len(ref_calls) == 7
    for c, rc in zip(calls, ref_calls):
        if comp == "sorted_pair":
            assert np.array_equal(c.direction, _normalise(rc["direction_raw"]))
            assert np.array_equal(c.uniforms, rc["uniforms"])
            assert np.array_equal(orc.torch_scores(k[c.src_in], c.direction), rc["scores"])
        else:
            assert np.array_equal(c.perm, rc["perm"])
    idx = np.concatenate([c.src_out for c in calls])
    assert np.array_equal(idx, g[f"{comp}_rep_idx"])
    assert np.array_equal(np.concatenate([c.w_out for c in calls]), g[f"{comp}_rep_w"])
    act = np.concatenate([np.full(c.src_out.shape[0], c.src_in[-1] + 1) for c in calls])
    assert np.array_equal(act, g[f"{comp}_rep_active"])


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


def test_fixed_order_scores_agree_with_reference_order(golden):
    """The HIP compressor's fixed-order fp64 scores sort exactly like the reference's MKL fp32 scores,
    except at near-ties (audited)."""
    total_diff = 0
    checked = 0
    for name, prefix in (("flat_c1", "sorted_pair_"), ("flat_oddblock", ""), ("levels_c1", ""), ("levels_deg3", ""),
                         ("levels_oddblock", "")):
        g = golden(name)
        k = g["k"]
        block = int(g.meta["block"])
        for ci, rc in enumerate(_golden_calls(g, prefix, int(g[f"{prefix}ncalls"]))):
            if "scores" not in rc:
                continue
            ref_scores = rc["scores"]
            ref_order = rc["order"]
            if "src_in" in rc:  # level cascade: the compress input as token ids
                rows = k[rc["src_in"]]
            else:  # flat: call ci is block ci
                rows = k[ci * block:(ci + 1) * block]
            checked += 1
            ours = orc.projection_scores(rows, _normalise(rc["direction_raw"]))
            our_order = np.argsort(ours, kind="stable")
            diff, bad = near_tie_flips(ref_scores, ref_order, our_order)
            total_diff += diff.size
            assert not bad, f"{name}: order differs away from a near-tie at {bad}"
    assert checked > 40
    assert total_diff == 0  # none expected at these sizes


@pytest.mark.parametrize("seed", [0, 3, 11])
def test_float64_selections_follow_float64_draws_and_torch_order(seed):
    """float64 keys: the oracle's compress calls draw float64 directions and uniforms (the reference
    draws in the keys' dtype, fast_article_attention.py:339, :348; streaming_taylor_coreset_attention.py:
    441, :456), its fixed-order fp64 scores sort exactly like torch's float64 `keys @ direction`, and the
    selections differ from the float32 run's (a float32 draw for float64 keys is a different draw,
    not a rounding)."""
    q, k, v = orc.make_data((), 2048 + 37, 24, 8, radius=1.0, data="unit_ball", seed=seed, dtype=torch.float64)
    k64 = k.numpy()
    for build in (lambda kk, fn: orc.flat_coreset(kk, 128, "sorted_pair", seed, fn),
                  lambda kk, fn: _level_calls(kk, 128, seed, fn)):
        fixed = build(k64, orc.projection_scores)
        torch_order = build(k64, orc.torch_scores)
        f32 = build(k64.astype(np.float32), orc.projection_scores)
        assert fixed[0].direction.dtype == np.float64 and fixed[0].uniforms.dtype == np.float64
        assert len(fixed) == len(torch_order) == len(f32)
        for a, b in zip(fixed, torch_order):
            assert np.array_equal(a.src_out, b.src_out) and np.array_equal(a.w_out, b.w_out)
        assert any(not np.array_equal(a.src_out, c.src_out) for a, c in zip(fixed, f32))


def _level_calls(k_np, block, seed, score_fn):
    state = orc.LevelState()
    g = torch.Generator().manual_seed(seed)
    for start in range(0, k_np.shape[0] - block + 1, block):
        orc.level_block_complete(state, g, np.arange(start, start + block, dtype=np.int64), k_np, "sorted_pair",
                                 score_fn)
    return state.calls


def test_flat_fixed_order_selection_equals_reference(golden):
    for name, comp_prefix in (("flat_c1", "sorted_pair_"), ("flat_oddblock", "")):
        g = golden(name)
        block = int(g.meta["block"])
        calls = orc.flat_coreset(g["k"], block, "sorted_pair", int(g.meta["seed"]))
        idx = np.concatenate([c.src_out for c in calls])
        assert np.array_equal(idx, g[f"{comp_prefix}rep_idx"])
        assert np.array_equal(np.concatenate([c.w_out for c in calls]), g[f"{comp_prefix}rep_w"])


@pytest.mark.parametrize("comp", ["sorted_pair", "random"])
def test_flat_forward_matches_reference(golden, comp):
    g = golden("flat_c1")
    q, k, v = (torch.from_numpy(g[x]) for x in "qkv")
    out = orc.fast_path_forward(q, k, v, degree=2, block=128, scale=1.0, compressor=comp, seed=0)
    assert rel(out, g[f"{comp}_out"]) < 1e-6


def test_flat_oddblock_forward(golden):
    g = golden("flat_oddblock")
    q, k, v = (torch.from_numpy(g[x]) for x in "qkv")
    out = orc.fast_path_forward(q, k, v, degree=2, block=33, scale=1.0, compressor="sorted_pair", seed=9)
    assert rel(out, g["out"]) < 1e-6
    assert sorted(set(g["rep_w"].tolist())) == [1.0, 2.0]  # odd tail keeps weight 1


def test_flat_bh_seeds(golden):
    g = golden("flat_bh")
    q, k, v = (torch.from_numpy(g[x]) for x in "qkv")
    bsz, heads = q.shape[:2]
    for b in range(bsz):
        for h in range(heads):
            out = orc.fast_path_forward(q[b, h], k[b, h], v[b, h], degree=2, block=32, scale=None,
                                        compressor="sorted_pair", seed=7 + b * heads + h)
            assert rel(out, g["out"][b, h]) < 1e-6


# --------------------------------------------------------------------------- merge-and-reduce levels

LEVEL_CASES = ["levels_c1", "levels_random", "levels_deg3", "levels_oddblock", "levels_block2"]


@pytest.mark.parametrize("name", LEVEL_CASES)
def test_level_cascade_matches_reference(golden, name):
    g = golden(name)
    m = g.meta
    q, k, v = (torch.from_numpy(g[x]) for x in "qkv")
    state = orc.LevelState()
    out = orc.levels_forward(q, k, v, degree=m["degree"], block=m["block"], scale=m["scale"],
                             compressor=m["compressor"], seed=m["seed"], state_out=state)
    ref_calls = [c for c in _golden_calls(g, "", int(g["ncalls"]))]
    # every compress call: same inputs (order and weights), same kept items and weights
    assert len(state.calls) == len(ref_calls)
    for c, rc in zip(state.calls, ref_calls):
        assert np.array_equal(c.src_in, rc["src_in"]) and np.array_equal(c.w_in, rc["w_in"])
        assert np.array_equal(c.src_out, rc["src_out"]), f"{name}: selection differs"
        assert np.array_equal(c.w_out, rc["w_out"])
    assert rel(out, g["out"]) < 2e-6


def test_level_invariants(golden):
    g = golden("levels_c1")
    m = g.meta
    state = orc.LevelState()
    q, k, v = (torch.from_numpy(g[x]) for x in "qkv")
    orc.levels_forward(q, k, v, degree=2, block=m["block"], scale=1.0, seed=0, state_out=state)
    nb = m["n"] // m["block"]
    for lev, node in enumerate(state.levels):
        present = node is not None
        assert present == bool((nb >> lev) & 1)
        if present:
            assert node[0].shape[0] == m["block"] // 2
            assert np.all(node[1] == 2.0 ** (lev + 1))
    items_w = sum(float(n[1].sum()) for n in state.levels if n is not None)
    assert items_w == nb * m["block"]  # weight is conserved


def test_levels_without_compression_is_exact():
    # test_streaming_attention.py:10-21: degree 3, block > n, unit-norm q, k
    torch.manual_seed(0)
    q = torch.randn(24, 6)
    k = torch.randn(24, 6)
    v = torch.randn(24, 5)
    q = q / q.norm(dim=-1, keepdim=True)
    k = k / k.norm(dim=-1, keepdim=True)
    out = orc.levels_forward(q, k, v, degree=3, block=25, scale=1.0)
    assert torch.allclose(out.double(), orc.classical_attention(q, k, v, 1.0), atol=3e-6, rtol=3e-6)


# --------------------------------------------------------------------------- segment means

def test_segment_mean_matches_reference(golden):
    g = golden("segment_mean")
    rk, rv, rpb = orc.segment_mean_coreset(torch.from_numpy(g["k"]), torch.from_numpy(g["v"]), 8, 2)
    assert rpb == int(g["reps_per_block"]) == 4
    assert rk.shape == (2, 8, 4) and rv.shape == (2, 8, 5)  # test_triton_article_attention.py:29-39
    assert torch.allclose(rk, torch.from_numpy(g["rep_k"]), atol=1e-7)
    assert torch.allclose(rv, torch.from_numpy(g["rep_v"]), atol=1e-7)


def test_segment_forward_stride1_is_exact():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 40, 8, generator=g) * 0.3
    k = torch.randn(2, 40, 8, generator=g) * 0.3
    v = torch.randn(2, 40, 4, generator=g)
    out = orc.segment_forward(q, k, v, degree=2, block=8, stride=1, scale=1.0)
    assert rel(out, orc.classical_attention(q, k, v, 1.0)) < 1e-12


def _segment_constant(n, d, dv, stride, seed, amp=0.8):
    """q random; k and v constant inside every stride segment [s*stride, (s+1)*stride), so a segment's
    mean is each of its tokens."""
    g = torch.Generator().manual_seed(seed)
    nseg = -(-n // stride)
    q = torch.randn(2, n, d, generator=g, dtype=torch.float64) * amp
    k = (torch.randn(2, nseg, d, generator=g, dtype=torch.float64) * amp).repeat_interleave(stride, dim=1)[:, :n]
    v = torch.randn(2, nseg, dv, generator=g, dtype=torch.float64).repeat_interleave(stride, dim=1)[:, :n]
    return q, k, v


@pytest.mark.parametrize("block,stride,n,degree", [(8, 2, 45, 2), (16, 4, 70, 2), (16, 8, 64, 1), (12, 3, 50, 0),
                                                   (8, 8, 33, 2)])
def test_segment_forward_segment_constant_is_exact(block, stride, n, degree):
    """With keys and values constant inside every stride segment, a segment-mean representative
    weighted by the stride stands in exactly for the stride tokens it averages, and the completed
    blocks' representatives cover exactly the keys before the row's block: the Triton semantics at any
    stride then equal causal softmax attention (logits far below the clamp at 80)."""
    q, k, v = _segment_constant(n, 8, 5, stride, seed=block + stride + n)
    out = orc.segment_forward(q, k, v, degree=degree, block=block, stride=stride, scale=1.0)
    assert rel(out, orc.classical_attention(q, k, v, 1.0)) < 1e-12


def test_segment_forward_clamp_closed_form():
    """exp(min(x, 80)) on both residual terms, checked against a hand evaluation (d = dv = 1, scale 1,
    block 2, stride 2, degree 2, n = 3):
      keys 9, 11, 10; values 1, 3, -1; queries 0.5, 9, 9.
      row 0: only key 0 -> v0.
      row 1 (logits 81, 99, both clamped): Taylor over keys 0, 1 plus the exact in-block residual ->
             (e^80 v0 + e^80 v1) / (2 e^80).
      row 2 (logits 81, 99, 90): Taylor over keys 0..2, in-block residual of key 2 (clamped to 80), and
             block 0's one representative (key 10, value 2, logit 90 clamped, weight 2):
             (T(81) v0 + T(99) v1 + e^80 v2 + 2 (e^80 - T(90)) 2) / (T(81) + T(99) + e^80 + 2 (e^80 - T(90))),
             T(x) = 1 + x + x^2 / 2."""
    T = lambda x: 1.0 + x + x * x / 2.0
    e80 = math.exp(80.0)
    k = torch.tensor([[[9.0], [11.0], [10.0]]], dtype=torch.float64)
    v = torch.tensor([[[1.0], [3.0], [-1.0]]], dtype=torch.float64)
    q = torch.tensor([[[0.5], [9.0], [9.0]]], dtype=torch.float64)
    out = orc.segment_forward(q, k, v, degree=2, block=2, stride=2, scale=1.0)[0, :, 0]
    row0 = 1.0
    row1 = (e80 * 1.0 + e80 * 3.0) / (2 * e80)
    num2 = T(81) * 1.0 + T(99) * 3.0 + e80 * -1.0 + 2 * (e80 - T(90)) * 2.0
    den2 = T(81) + T(99) + e80 + 2 * (e80 - T(90))
    expect = torch.tensor([row0, row1, num2 / den2], dtype=torch.float64)
    assert torch.allclose(out, expect, rtol=1e-12, atol=0)
    assert abs(float(out[1]) - 2.0) < 1e-12 and abs(float(out[2]) - 1.0) < 1e-9  # the clamp equalises


@pytest.mark.parametrize("mistake", ["weight_one", "active_one_block_early", "active_one_block_late", "no_clamp"])
def test_planted_segment_mistakes_are_caught(monkeypatch, mistake):
    """Each plausible slip in the Triton semantics fails one of the two pins above."""
    if mistake == "weight_one":
        monkeypatch.setattr(orc, "segment_rep_weight", lambda stride: 1.0)
    elif mistake == "active_one_block_early":
        monkeypatch.setattr(orc, "segment_rep_active_from", lambda rb, block: rb * block)
    elif mistake == "active_one_block_late":
        monkeypatch.setattr(orc, "segment_rep_active_from", lambda rb, block: (rb + 2) * block)
    else:
        monkeypatch.setattr(orc, "clamped_exp", torch.exp)
    failed = []
    try:
        test_segment_forward_segment_constant_is_exact(8, 2, 45, 2)
    except AssertionError:
        failed.append("segment_constant")
    try:
        test_segment_forward_clamp_closed_form()
    except AssertionError:
        failed.append("clamp")
    assert failed, f"planted mistake {mistake} passed both pins"


# --------------------------------------------------------------------------- planted mistakes

def test_planted_pair_rule_mistake_is_caught(golden, monkeypatch):
    """Swapping the kept element of each pair must break the golden selections."""
    g = golden("levels_c1")
    q, k, v = (torch.from_numpy(g[x]) for x in "qkv")
    real = orc.sorted_pair_select

    def flipped(src, w, scores, u):
        return real(src, w, scores, 1.0 - u)

    monkeypatch.setattr(orc, "sorted_pair_select", flipped)
    state = orc.LevelState()
    orc.levels_forward(q, k, v, degree=2, block=64, scale=1.0, seed=0, state_out=state)
    ref0 = g["call0_src_out"]
    assert not np.array_equal(state.calls[0].src_out, ref0)


def test_planted_taylor_mistake_is_caught(golden, monkeypatch):
    """Dropping the quadratic Taylor term must break the reference moment sums."""
    g = golden("flat_c1")
    q, k, v = (torch.from_numpy(g[x]) for x in "qkv")
    real = orc.features
    monkeypatch.setattr(orc, "features", lambda x, deg, ks: real(x, min(deg, 1), ks))
    num, den = orc.low_sums_stream(q, k, v, 2, 1.0)
    assert rel(den, g["low_den"]) > 1e-4


def test_streaming_object_matches_levels_forward():
    """The per-token restatement of the reference's streaming object (reference-style torch projection
    and argsort) gives the vectorised level semantics' outputs."""
    n, d, dv, block = 200, 6, 4, 16
    q, k, v = orc.make_data((), n, d, dv, radius=1.0, data="unit_ball", seed=2)
    ref = orc.levels_forward(q, k, v, degree=2, block=block, scale=0.8, seed=5, reference_scores=True)
    st = orc.StreamingAttentionCPU(d, dv, degree=2, block=block, scale=0.8, seed=5)
    outs = []
    for i in range(n):
        st.update(k[i], v[i])
        outs.append(st.query(q[i]))
    assert orc.rel_l2(torch.stack(outs), ref) < 1e-5


def test_decode_timing_sample_runs():
    t = orc.time_decode_sample(dim=8, value_dim=8, degree=2, block=16, scale=0.5, prefix=100, steps=40)
    assert t["s_per_step"] > 0 and t["steps"] == 40
