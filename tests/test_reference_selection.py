"""Reference-order selections (reference_scores=True; sta_host_select in libstadraws.so), on the CPU.

The HIP compressor orders a compress call's keys by fp64 projection scores summed in a fixed order.
The reference sorts torch's CPU `keys @ direction` (fast_article_attention.py:340-341,
streaming_taylor_coreset_attention.py:443-444), whose summation order belongs to the host's BLAS, in
the keys' own dtype with draws and pair rule in that dtype.  sta_host_select runs every compress call
of a node plan on the host with those torch calls.  Pinned here by:
  * the reference's own selections written by tests/golden/make_golden.py: every golden case in
    float32, the float64 / bfloat16 / float16 runs, and keys whose projections nearly tie (rows
    repeated with one coordinate moved by one ulp), where the BLAS order decides which token survives;
  * the headline workload (32 heads x 65536 tokens, 511 compress calls per head): every node equals the
    oracle's level cascade in torch's own order (c3_cascade with reference_cpu.torch_order_scores: the
    ranks of torch.argsort(keys @ direction); a stable sort of torch's scores is not that order where
    two scores tie exactly, as two keys of head 5's compress call 184 do).
The near-tie and 16-bit orders belong to the BLAS code path of the host that wrote the golden file, so
those comparisons run on a host with the same CPU model only (the oracle comparisons run anywhere)."""

import pathlib

import numpy as np
import pytest
import torch

import _plan
import c3_cascade as c3
import reference_cpu as orc
from conftest import load_golden

DTYPES = {"f64": torch.float64, "bf16": torch.bfloat16, "f16": torch.float16}


def _cpu_model() -> str:
    for line in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
        if line.startswith("model name"):
            return line.split(":", 1)[1].strip()
    return "unknown"


def _same_host(g) -> bool:
    return g.meta.get("cpu_model") == _cpu_model()


def _level_nodes_equal(plan, src, w, call_src, call_w):
    """Every node of a levels plan against the call with its slot in the reference's call order."""
    for node in range(plan.n_nodes):
        slot = int(plan.desc[node, 6])
        size = int(plan.meta[node, 0])
        assert np.array_equal(src[node, :size], call_src(slot)), f"node {node} (call {slot})"
        assert np.array_equal(w[node, :size].astype(np.float64), np.asarray(call_w(slot), dtype=np.float64)), \
            f"node {node} (call {slot}) weights"


def _flat_items(plan, src, w):
    nb = len(plan.batches[0])
    sizes = plan.meta[:, 0]
    return (np.concatenate([src[b, : sizes[b]] for b in range(nb)]),
            np.concatenate([w[b, : sizes[b]] for b in range(nb)]))


@pytest.mark.parametrize("name", ["levels_c1", "levels_random", "levels_deg3", "levels_oddblock", "levels_block2"])
def test_golden_level_selections(name):
    g = load_golden(name)
    m = g.meta
    k = torch.from_numpy(g["k"])[None].contiguous()
    plan = _plan.levels_plan(k.shape[1], m["block"], m["compressor"])
    src, w = _plan.reference_selection(plan, (m["seed"],), k, m["compressor"])
    _level_nodes_equal(plan, src[0], w[0], lambda s: g[f"call{s}_src_out"], lambda s: g[f"call{s}_w_out"])


@pytest.mark.parametrize("name,prefix,comp", [("flat_c1", "sorted_pair_", "sorted_pair"),
                                              ("flat_c1", "random_", "random"),
                                              ("flat_oddblock", "", "sorted_pair")])
def test_golden_flat_selections(name, prefix, comp):
    g = load_golden(name)
    k = torch.from_numpy(g["k"])[None].contiguous()
    plan = _plan.flat_plan(k.shape[1], g.meta["block"], comp)
    src, w = _plan.reference_selection(plan, (g.meta["seed"],), k, comp)
    idx, ws = _flat_items(plan, src[0], w[0])
    assert np.array_equal(idx, g[f"{prefix}rep_idx"]) and np.array_equal(ws, g[f"{prefix}rep_w"])


@pytest.mark.parametrize("tag", list(DTYPES))
def test_selections_in_the_keys_dtype(tag):
    """float64, bfloat16 and float16 keys: the draws, scores and pair rule in that dtype reproduce the
    reference's run in it (levels and flat).  The float64 run's order is also checked against the oracle
    (fp64 scores in dimension order, ties far apart in float64)."""
    g = load_golden("selection_dtypes")
    case = next(c for c in g.meta["cases"] if c["tag"] == tag)
    dt = DTYPES[tag]
    k = torch.from_numpy(g[f"{tag}_k"]).to(dt)[None].contiguous()
    assert torch.equal(k.double()[0], torch.from_numpy(g[f"{tag}_k"]))  # the stored keys are exact
    n, block, seed = case["n"], case["block"], case["seed"]
    lp = _plan.levels_plan(n, block, "sorted_pair")
    src, w = _plan.reference_selection(lp, (seed,), k, "sorted_pair")
    fp = _plan.flat_plan(n, block, "sorted_pair")
    fsrc, fw = _plan.reference_selection(fp, (seed,), k, "sorted_pair")
    if tag == "f64" or _same_host(g):
        assert int(g[f"{tag}_levels_ncalls"]) == len(lp.call_sizes)
        _level_nodes_equal(lp, src[0], w[0], lambda s: g[f"{tag}_levels_call{s}_src_out"],
                           lambda s: g[f"{tag}_levels_call{s}_w_out"])
        idx, ws = _flat_items(fp, fsrc[0], fw[0])
        assert np.array_equal(idx, g[f"{tag}_flat_rep_idx"])
        assert np.array_equal(ws.astype(np.float64), g[f"{tag}_flat_rep_w"])
    if tag == "f64":
        state = orc.LevelState()
        gen = torch.Generator(device="cpu")
        gen.manual_seed(seed)
        keys = k[0].numpy()
        for b in range(n // block):
            orc.level_block_complete(state, gen, np.arange(b * block, (b + 1) * block, dtype=np.int64), keys,
                                     "sorted_pair")
        _level_nodes_equal(lp, src[0], w[0], lambda s: state.calls[s].src_out, lambda s: state.calls[s].w_out)


def test_near_ties_follow_the_reference_order():
    """Keys in groups of 8 near-duplicates: torch's CPU score order decides every pair inside a group,
    and some scores tie exactly (torch.argsort then orders them its own way).  The host selection equals
    the oracle's cascade in torch's order (this host) and, on the golden file's host, the reference's
    own run; the fixed-order selection differs from it somewhere."""
    g = load_golden("selection_near_ties")
    m = g.meta
    k = torch.from_numpy(g["k"])[None].contiguous()
    n, block, seed = m["n"], m["block"], m["seed"]
    lp = _plan.levels_plan(n, block, "sorted_pair")
    src, w = _plan.reference_selection(lp, (seed,), k, "sorted_pair")
    keys = g["k"]

    def cascade(score_fn):
        state = orc.LevelState()
        gen = torch.Generator(device="cpu")
        gen.manual_seed(seed)
        for b in range(n // block):
            orc.level_block_complete(state, gen, np.arange(b * block, (b + 1) * block, dtype=np.int64), keys,
                                     "sorted_pair", score_fn)
        return state.calls

    ref_calls = cascade(orc.torch_order_scores)
    _level_nodes_equal(lp, src[0], w[0], lambda s: ref_calls[s].src_out, lambda s: ref_calls[s].w_out)
    fixed = cascade(orc.projection_scores)
    differ = sum(not np.array_equal(a.src_out, b.src_out) for a, b in zip(ref_calls, fixed))
    print(f"near ties: {differ} of {len(fixed)} compress calls keep other tokens in the fixed order")
    fp = _plan.flat_plan(n, block, "sorted_pair")
    fsrc, fw = _plan.reference_selection(fp, (seed,), k, "sorted_pair")
    idx, ws = _flat_items(fp, fsrc[0], fw[0])
    flat_ref = orc.flat_coreset(keys, block, "sorted_pair", seed, orc.torch_order_scores)
    assert np.array_equal(idx, np.concatenate([c.src_out for c in flat_ref]))
    if _same_host(g):
        assert differ > 0, "the near-tie keys no longer separate the two orders"
        _level_nodes_equal(lp, src[0], w[0], lambda s: g[f"levels_call{s}_src_out"],
                           lambda s: g[f"levels_call{s}_w_out"])
        assert np.array_equal(idx, g["flat_rep_idx"]) and np.array_equal(ws, g["flat_rep_w"])


def test_c3_reference_order_equals_the_torch_order_cascade():
    """All 511 nodes of all 32 heads of the headline workload equal the oracle's cascade in the order of
    torch's CPU `keys @ direction` and argsort on this host."""
    _, k, _ = c3.inputs()
    plan = _plan.levels_plan(c3.N, c3.BLOCK, "sorted_pair")
    src, w = _plan.reference_selection(plan, _plan.sequence_seeds(0, c3.HEADS), k[0].contiguous(), "sorted_pair")
    for h in range(c3.HEADS):
        calls = c3.head_cascade(h, orc.torch_order_scores).calls
        _level_nodes_equal(plan, src[h], w[h], lambda s: calls[s].src_out, lambda s: calls[s].w_out)


def test_host_select_refuses_bad_plans():
    k = torch.zeros(1, 64, 4)
    plan = _plan.levels_plan(64, 16, "sorted_pair")
    dr, desc = _plan.draws_for(plan, (0,), 4, "sorted_pair", dtype=torch.float32)
    import _native

    bad = desc.copy()
    bad[-1, 1] = plan.n_nodes - 1  # a merge whose child is itself
    with pytest.raises(_native.NativeError, match="merge"):
        _native.host_select(k, True, bad, plan.n_nodes, plan.cap, dr.dirs, dr.unif, dr.perms)
    bad = desc.copy()
    bad[0, 1] = 60  # a raw block past the sequence's end
    with pytest.raises(_native.NativeError, match="raw node"):
        _native.host_select(k, True, bad, plan.n_nodes, plan.cap, dr.dirs, dr.unif, dr.perms)
    with pytest.raises(ValueError):
        _native.host_select(k.double(), True, desc, plan.n_nodes, plan.cap, dr.dirs, dr.unif, dr.perms)
