"""GPU parity of the streaming decode path (ArticleStreamingAttention on the HIP decode kernels K5,
through the C ABI): per-token update / query outputs against the reference's own outputs (golden
fixtures) and the oracle, the level coresets bit-exact (kept token and weight of every item), the
batched step / extend / prefill forms against the prefill kernels, the moment sketch against the
closed-form feature sums, and the query statistics against the reference's low / tail split.
Tolerances: fp32 rel-L2 <= 1e-4, bf16 inputs <= 5e-3."""

import numpy as np
import pytest
import torch

import _decode
import _engine
import _native
import reference_cpu as orc
import streaming_taylor_coreset_attention as stc

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
FP32_TOL = 1e-4
BF16_TOL = 5e-3
# moment sums of the state accumulation with split-bf16 products (about 2^-16 relative per product)
MOM_TOL = 2e-5
LEVEL_CASES = ["levels_c1", "levels_random", "levels_deg3", "levels_oddblock", "levels_block2"]


def rel(a, b):
    return orc.rel_l2(torch.as_tensor(a).float().cpu(), torch.as_tensor(b).float().cpu())


def t(x):
    return torch.from_numpy(np.ascontiguousarray(x))


def level_node(plan, lev, j):
    ids = np.nonzero(plan.level_of[: plan.n_nodes] == lev)[0]
    return int(ids[j])


def final_level_nodes(plan, n, block):
    """{level: node id} of the levels occupied after n tokens (counter c = n // block)."""
    c = n // block
    return {lev: level_node(plan, lev, (c >> lev) - 1) for lev in range(c.bit_length()) if (c >> lev) & 1}


@pytest.mark.parametrize("name", LEVEL_CASES)
def test_decode_matches_reference_goldens(golden, name):
    """update(k_i, v_i); query(q_i) token by token == the reference's outputs; the final levels are
    the reference's compress outputs (positions and weights, bit-exact)."""
    g = golden(name)
    m = g.meta
    q, k, v = (t(g[x]) for x in "qkv")
    n = q.shape[0]
    st = stc.ArticleStreamingAttention(m["d"], m["dv"], degree=m["degree"], block_size=m["block"], scale=m["scale"],
                                       compressor=m["compressor"], device=DEV, seed=m["seed"])
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    outs = []
    for i in range(n):
        st.update(kd[i], vd[i])
        outs.append(st.query(qd[i]))
    out = torch.stack(outs)
    assert rel(out, g["out"]) < FP32_TOL
    assert st.length == n

    plan = _engine._plan.levels_plan(n, m["block"], m["compressor"])
    pos = st.coreset.level_positions()
    levels = st.coreset.levels
    for lev, node in final_level_nodes(plan, n, m["block"]).items():
        slot = int(plan.desc[node, 6])
        assert np.array_equal(pos[lev].cpu().numpy(), g[f"call{slot}_src_out"]), f"level {lev}"
        assert np.array_equal(levels[lev].weights.cpu().numpy(), g[f"call{slot}_w_out"])
        assert torch.equal(levels[lev].keys.cpu(), k[pos[lev].cpu().long()])
    occupied = [lev for lev, lv in enumerate(levels) if lv is not None]
    assert occupied == sorted(final_level_nodes(plan, n, m["block"]))


def _data(streams, n, d, dv, seed, dtype=torch.float32, scale_in=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(streams, n, d, generator=g) * scale_in).to(dtype)
    k = (torch.randn(streams, n, d, generator=g) * scale_in).to(dtype)
    v = torch.randn(streams, n, dv, generator=g).to(dtype)
    return q, k, v


BATCH_CASES = [
    # streams, n, d, dv, block, degree, compressor, scale, dtype, input scale
    (5, 700, 32, 48, 64, 2, "sorted_pair", 0.3, torch.float32, 1.0),
    (3, 400, 16, 64, 33, 3, "sorted_pair", 0.5, torch.float32, 1.0),
    (4, 300, 8, 8, 16, 2, "random", 1.0, torch.float32, 0.5),
    (2, 130, 12, 5, 2, 1, "sorted_pair", 1.0, torch.float32, 0.5),
    (3, 200, 64, 64, 32, 2, "none", 0.125, torch.float32, 1.0),
    (6, 600, 64, 64, 128, 2, "sorted_pair", 0.125, torch.bfloat16, 1.0),
    (2, 300, 128, 130, 64, 2, "sorted_pair", None, torch.float32, 1.0),
]


@pytest.mark.parametrize("streams,n,d,dv,block,degree,comp,scale,dtype,xs", BATCH_CASES)
def test_batched_step_matches_prefill(streams, n, d, dv, block, degree, comp, scale, dtype, xs):
    """step() per token over S streams == the prefill kernels on the same [1, S, N, D] input (stream s
    seeded seed + s); the final levels hold the prefill's selected tokens, bit-exact."""
    q, k, v = _data(streams, n, d, dv, seed=n + d, dtype=dtype, scale_in=xs)
    seed = 7
    ref = stc.article_causal_attention(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), degree=degree,
                                       block_size=block, scale=scale, compressor=comp, seed=seed)[0]
    st = stc.ArticleStreamingAttention(d, dv, degree=degree, block_size=block, scale=scale, compressor=comp,
                                       device=DEV, dtype=dtype, seed=seed, streams=streams)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    outs = torch.stack([st.step(qd[:, i], kd[:, i], vd[:, i]) for i in range(n)], dim=1)
    assert outs.dtype == dtype
    tol = BF16_TOL if dtype == torch.bfloat16 else FP32_TOL
    assert rel(outs, ref) < tol
    if comp != "none":
        s = float(1.0 / np.sqrt(d)) if scale is None else scale
        res = _engine.prefill(q.to(DEV), k.to(DEV), v.to(DEV), degree=degree, block=block, scale=s,
                              semantics="levels", compressor=comp, seed=seed)
        src = res.node_src.cpu().numpy()
        w = res.node_w.cpu().numpy()
        pos = st.coreset.level_positions()
        lw = st.coreset.levels
        for lev, node in final_level_nodes(res.plan, n, block).items():
            size = int(res.plan.meta[node, 0])
            assert np.array_equal(pos[lev].cpu().numpy(), src[:, node, :size]), f"level {lev}"
            assert np.array_equal(lw[lev].weights.float().cpu().numpy(), w[:, node, :size])


@pytest.mark.parametrize("prefix", [0, 1, 64, 333])
def test_extend_then_step(prefix):
    """extend() over a prefix (any length, partial blocks included) then step() == prefill rows."""
    streams, n, d, dv, block = 3, 520, 16, 16, 64
    q, k, v = _data(streams, n, d, dv, seed=prefix)
    ref = stc.article_causal_attention(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), degree=2,
                                       block_size=block, scale=0.5, seed=11)[0]
    st = stc.ArticleStreamingAttention(d, dv, degree=2, block_size=block, scale=0.5, device=DEV, seed=11,
                                       streams=streams)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    lo = 0
    if prefix == 333:  # a partly filled buffer first
        st.extend(kd[:, :40], vd[:, :40])
        lo = 40
    st.extend(kd[:, lo:prefix], vd[:, lo:prefix])
    assert st.length == prefix
    outs = torch.stack([st.step(qd[:, i], kd[:, i], vd[:, i]) for i in range(prefix, n)], dim=1)
    assert rel(outs, ref[:, prefix:]) < FP32_TOL


@pytest.mark.parametrize("how", ["extend", "prefill"])
def test_extend_padded_keys_with_values_in_place(how):
    """d = 6 needs a zero-padded copy of the keys (16-byte rows) while dv = 32 rows could be read in
    place: the values must then be copied next to the key copy (rows [0, nb B) of the whole blocks), for
    a prompt that ends in a partial block.  The following steps == the prefill rows."""
    streams, n, p, d, dv, block = 3, 120, 40, 6, 32, 16
    q, k, v = _data(streams, n, d, dv, seed=17, scale_in=0.5)
    ref = stc.article_causal_attention(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), degree=2,
                                       block_size=block, scale=0.5, seed=3)[0]
    st = stc.ArticleStreamingAttention(d, dv, degree=2, block_size=block, scale=0.5, device=DEV, seed=3,
                                       streams=streams)
    qd, kd, vd = q.to(DEV).contiguous(), k.to(DEV).contiguous(), v.to(DEV).contiguous()
    if how == "extend":
        st.extend(kd[:, :p].contiguous(), vd[:, :p].contiguous())
    else:
        head = st.prefill(qd[:, :p].contiguous(), kd[:, :p].contiguous(), vd[:, :p].contiguous())
        assert rel(head, ref[:, :p]) < FP32_TOL
    assert st.length == p
    den, num = st._st.full_moments()
    phi = orc.features(k[:, :p].double(), 2, key_side=True)  # [S, p, F]
    assert rel(den.cpu(), phi.sum(1)) < 1e-6
    assert rel(num.cpu(), phi.transpose(1, 2) @ v[:, :p].double()) < MOM_TOL
    outs = torch.stack([st.step(qd[:, i], kd[:, i], vd[:, i]) for i in range(p, n)], dim=1)
    assert rel(outs, ref[:, p:]) < FP32_TOL


def test_prefill_then_step_bf16():
    """prefill() of a prompt returns the prompt's outputs and leaves the state for decoding
    (the decode workload's regime: q, k, v ~ N(0,1)/8, bf16, scale 1/8, block 256)."""
    streams, n, p, d = 4, 900, 600, 64
    q, k, v = _data(streams, n, d, d, seed=5, dtype=torch.bfloat16, scale_in=0.125)
    ref = stc.article_causal_attention(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), degree=2,
                                       block_size=256, seed=0)[0]
    st = stc.ArticleStreamingAttention(d, d, degree=2, block_size=256, device=DEV, dtype=torch.bfloat16,
                                       streams=streams)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    head = st.prefill(qd[:, :p], kd[:, :p], vd[:, :p])
    assert rel(head, ref[:, :p]) < BF16_TOL
    outs = torch.stack([st.step(qd[:, i], kd[:, i], vd[:, i]) for i in range(p, n)], dim=1)
    assert rel(outs, ref[:, p:]) < BF16_TOL


def test_decode_vs_oracle_single_stream():
    n, d, dv, block = 300, 8, 8, 16
    q, k, v = orc.make_data((), n, d, dv, radius=1.0, data="unit_ball", seed=9)
    ref = orc.levels_forward(q, k, v, degree=2, block=block, scale=1.0, seed=4)
    st = stc.ArticleStreamingAttention(d, dv, degree=2, block_size=block, scale=1.0, device=DEV, seed=4)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    out = torch.stack([st.step(qd[i], kd[i], vd[i]) for i in range(n)])
    assert rel(out, ref) < FP32_TOL
    # the oracle's literal level state after the same tokens
    state = orc.LevelState()
    orc.levels_forward(q, k, v, degree=2, block=block, scale=1.0, seed=4, state_out=state)
    pos = st.coreset.level_positions()
    for lev, lv in enumerate(state.levels):
        if lv is None:
            assert lev >= len(pos) or pos[lev] is None
        else:
            assert np.array_equal(pos[lev].cpu().numpy(), lv[0]) and np.array_equal(
                st.coreset.levels[lev].weights.cpu().numpy(), lv[1])


def test_decode_degree4_vs_oracle():
    """Degree-4 decode: per-token outputs and the sketch moments (reference feature order) against the
    oracle; the 4-factor decode feature table and 4-term Taylor tail."""
    n, d, dv, block = 150, 6, 8, 16
    q, k, v = orc.make_data((), n, d, dv, radius=1.0, data="unit_ball", seed=21)
    ref = orc.levels_forward(q, k, v, degree=4, block=block, scale=1.0, seed=5)
    st = stc.ArticleStreamingAttention(d, dv, degree=4, block_size=block, scale=1.0, device=DEV, seed=5)
    st.extend(k[:40].to(DEV), v[:40].to(DEV))
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    out = torch.stack([st.step(qd[i], kd[i], vd[i]) for i in range(40, n)])
    assert rel(out, ref[40:]) < FP32_TOL
    phi = orc.features(k.double(), 4, key_side=True)
    den = torch.cat([x.cpu().double() for x in st.sketch.den_moments])
    num = torch.cat([x.cpu().double() for x in st.sketch.num_moments])
    assert [x.shape[0] for x in st.sketch.den_moments] == [1, 6, 21, 56, 126]
    assert rel(den, phi.sum(0)) < 1e-6
    assert rel(num, phi.T @ v.double()) < MOM_TOL


@pytest.mark.parametrize("products", [_native.PRODUCTS_SPLIT_BF16, _native.PRODUCTS_FP32])
def test_sketch_moments_closed_form(monkeypatch, products):
    """den_moments / num_moments (reference order, per degree) == sum_j phi_k(k_j) [1, v_j] in fp64, with
    either product form of the state accumulation (the denominators are fp32 sums either way)."""
    monkeypatch.setattr(_decode, "ACCUMULATE_PRODUCTS", products)
    n, d, dv = 150, 6, 5
    g = torch.Generator().manual_seed(2)
    k = torch.randn(n, d, generator=g) * 0.5
    v = torch.randn(n, dv, generator=g)
    st = stc.ArticleStreamingAttention(d, dv, degree=3, block_size=32, device=DEV)
    st.extend(k[:100].to(DEV), v[:100].to(DEV))
    for i in range(100, n):
        st.update(k[i].to(DEV), v[i].to(DEV))
    phi = orc.features(k.double(), 3, key_side=True)
    den = torch.cat([x.cpu().double() for x in st.sketch.den_moments])
    num = torch.cat([x.cpu().double() for x in st.sketch.num_moments])
    assert [x.shape[0] for x in st.sketch.den_moments] == [1, 6, 21, 56]
    assert rel(den, phi.sum(0)) < 1e-6
    assert rel(num, phi.T @ v.double()) < (1e-6 if products == _native.PRODUCTS_FP32 else MOM_TOL)


@pytest.mark.parametrize("S,n,head_rows,d,dv,degree,dtype", [
    (3, 300, 320, 16, 24, 2, torch.float32), (2, 257, 257, 64, 64, 2, torch.float32),
    (2, 200, 256, 128, 100, 2, torch.float32), (2, 190, 192, 16, 64, 3, torch.float32),
    (2, 300, 300, 64, 64, 2, torch.bfloat16), (1, 70, 80, 8, 8, 0, torch.float32),
    (1, 90, 96, 12, 40, 1, torch.float32)])
def test_accumulate_ws_matches_chunked_and_closed_form(monkeypatch, S, n, head_rows, d, dv, degree, dtype):
    """The state accumulation on the wave-specialised update-only pass (sta_moment_accumulate_ws) and on
    the chunked kernel, from the same nonzero state: both equal the fp64 closed form
    state0 + sum_j phi_k(k_j) [v_j, 1] in the reference's feature order (split-bf16 products)."""
    print(f"accumulate ws S={S} n={n} rows={head_rows} d={d} dv={dv} degree={degree} {dtype}", flush=True)
    g = torch.Generator().manual_seed(n + d)
    states = {}
    monkeypatch.setattr(_decode, "ACCUMULATE_WS_MIN_ROWS", 1)
    for ws in (True, False):
        monkeypatch.setattr(_decode, "ACCUMULATE_WS", ws)
        st = _decode.DecodeState(S, d, dv, degree=degree, block=64, scale=1.0, compressor="sorted_pair", seed=0,
                                 device=DEV)
        if ws:
            assert st._acc_table_ws(st.dk) is not None
            k = torch.zeros(S, head_rows, st.dk)
            k[:, :, :d] = torch.randn(S, head_rows, d, generator=g) * 0.4
            v = torch.zeros(S, head_rows, st.ldv)
            v[:, :, :dv] = torch.randn(S, head_rows, dv, generator=g)
            k, v = k.to(dtype), v.to(dtype)
            num0 = torch.randn(S, st.F, st.ldv, generator=g)
            num0[..., dv:] = 0
            den0 = torch.randn(S, st.F, generator=g)
        st.state_num.copy_(num0.to(DEV))
        st.state_den.copy_(den0.to(DEV))
        st._accumulate(k.to(DEV).contiguous(), v.to(DEV).contiguous(), n, head_rows, st.state_num, st.state_den)
        torch.cuda.synchronize()
        states[ws] = (st.state_num.cpu().double(), st.state_den.cpu().double())
    for s in range(S):
        phi = orc.features(k[s, :n, :d].double(), degree, key_side=True)
        want_num = num0[s].double()[:, :dv] + phi.T @ v[s, :n, :dv].double()
        want_den = den0[s].double() + phi.sum(0)
        for ws in (True, False):
            num, den = states[ws]
            assert rel(num[s][:, :dv], want_num) < MOM_TOL, (ws, s)
            assert rel(den[s], want_den) < 1e-6, (ws, s)
            assert torch.all(num[s][:, dv:] == 0)


@pytest.mark.parametrize("S,n,head_rows,d,dv,degree,dtype,tiles,cols", [
    (3, 256, 256, 64, 64, 2, torch.float32, 4, 32), (2, 300, 320, 16, 24, 2, torch.float32, 4, 32),
    (2, 100, 128, 64, 100, 2, torch.float32, 2, 64), (2, 257, 260, 48, 64, 1, torch.bfloat16, 4, 32),
    (1, 33, 40, 8, 8, 0, torch.float32, 2, 64), (2, 256, 256, 64, 64, 2, torch.bfloat16, 2, 64),
    (1, 600, 600, 32, 64, 2, torch.float16, 4, 32), (3, 256, 256, 64, 64, 2, torch.float32, 2, 32),
    (2, 520, 520, 64, 64, 2, torch.float32, 2, 64)])
def test_accumulate_block_matches_chunked(monkeypatch, S, n, head_rows, d, dv, degree, dtype, tiles, cols):
    """The block accumulation (sta_moment_accumulate_block: rows staged once per workgroup, every feature
    slice run through them) gives the chunked kernel's state bit for bit from the same nonzero state
    (runs of 1 to 3 groups of 256 rows, 1 to 4 column groups of 32 or 64 columns, 2 and 4 tiles per
    wave), and the fp64 closed form state0 + sum_j phi_k(k_j) [v_j, 1]."""
    print(f"accumulate block S={S} n={n} rows={head_rows} d={d} dv={dv} degree={degree} {dtype} nt={tiles} "
          f"cols={cols}", flush=True)
    g = torch.Generator().manual_seed(n + d + 1)
    states = {}
    monkeypatch.setattr(_decode, "ACCUMULATE_WS", False)
    monkeypatch.setattr(_decode, "ACCUMULATE_BLOCK_TILES", tiles)
    monkeypatch.setattr(_decode, "ACCUMULATE_BLOCK_COLUMNS", cols)
    for blk in (True, False):
        monkeypatch.setattr(_decode, "ACCUMULATE_BLOCK", blk)
        st = _decode.DecodeState(S, d, dv, degree=degree, block=64, scale=1.0, compressor="sorted_pair", seed=0,
                                 device=DEV)
        if blk:
            assert st._acc_table_block(st.dk) is not None
            k = torch.zeros(S, head_rows, st.dk)
            k[:, :, :d] = torch.randn(S, head_rows, d, generator=g) * 0.4
            v = torch.zeros(S, head_rows, st.ldv)
            v[:, :, :dv] = torch.randn(S, head_rows, dv, generator=g)
            k, v = k.to(dtype), v.to(dtype)
            num0 = torch.randn(S, st.F, st.ldv, generator=g)
            num0[..., dv:] = 0
            den0 = torch.randn(S, st.F, generator=g)
        else:
            assert st._acc_table_block(st.dk) is None
        st.state_num.copy_(num0.to(DEV))
        st.state_den.copy_(den0.to(DEV))
        st._accumulate(k.to(DEV).contiguous(), v.to(DEV).contiguous(), n, head_rows, st.state_num, st.state_den)
        torch.cuda.synchronize()
        states[blk] = (st.state_num.cpu(), st.state_den.cpu())
    assert torch.equal(states[True][0], states[False][0]) and torch.equal(states[True][1], states[False][1])
    for s in range(S):
        phi = orc.features(k[s, :n, :d].double(), degree, key_side=True)
        want_num = num0[s].double()[:, :dv] + phi.T @ v[s, :n, :dv].double()
        want_den = den0[s].double() + phi.sum(0)
        num, den = (x.double() for x in states[True])
        assert rel(num[s][:, :dv], want_num) < MOM_TOL and rel(den[s], want_den) < 1e-6, s
        assert torch.all(num[s][:, dv:] == 0)


def test_query_stats_split():
    """return_stats: denominator = low + tail, with the reference's split: low over every token (the
    sketch holds the buffered tokens too), tail over items() = buffer (weight 1) + levels."""
    n, d, dv, block, s = 77, 8, 4, 16, 0.7
    q, k, v = orc.make_data((), n, d, dv, radius=1.0, data="unit_ball", seed=3)
    st = stc.ArticleStreamingAttention(d, dv, degree=2, block_size=block, scale=s, device=DEV, seed=1)
    st.extend(k[: n - 1].to(DEV), v[: n - 1].to(DEV))
    st.update(k[n - 1].to(DEV), v[n - 1].to(DEV))
    out, stats = st.query(q[n - 1].to(DEV), return_stats=True)
    x = (k.double() @ q[n - 1].double()) * s
    low = orc.exp_taylor(x, 2).sum().item()
    items = st.coreset.items()
    xi = (items.keys.cpu().double() @ q[n - 1].double()) * s
    tail = (items.weights.cpu().double() * (torch.exp(xi) - orc.exp_taylor(xi, 2))).sum().item()
    assert abs(stats.low_denominator - low) < 1e-5 * abs(low)
    assert abs(stats.tail_denominator - tail) < 2e-5 * abs(low + tail)
    assert abs(stats.denominator - (low + tail)) < 1e-5 * abs(low + tail)
    assert stats.coreset_items == items.size == (n % block) + (block // 2) * bin(n // block).count("1")
    assert stats.state_bytes == st.state_size_bytes()


def test_state_size_matches_trace():
    """state_size_bytes() after every token == the reference's state-size formula."""
    n, d, dv, block = 100, 4, 3, 8
    q, k, v = orc.make_data((), n, d, dv, radius=1.0, data="unit_ball", seed=1)
    trace = stc.state_size_trace(n, d, dv, 2, block, "sorted_pair", 4)
    st = stc.ArticleStreamingAttention(d, dv, degree=2, block_size=block, scale=1.0, device=DEV)
    for i in range(n):
        st.update(k[i].to(DEV), v[i].to(DEV))
        assert st.state_size_bytes() == trace[i]
        assert st.coreset.num_items() == (i + 1) % block + (block // 2) * bin((i + 1) // block).count("1")


def test_decode_errors():
    st = stc.ArticleStreamingAttention(8, 4, device=DEV)
    with pytest.raises(ValueError):
        st.update(torch.zeros(7, device=DEV), torch.zeros(4, device=DEV))
    with pytest.raises(ValueError):
        st.query(torch.zeros(2, 8, device=DEV))
    with pytest.raises(ValueError):
        stc.ArticleStreamingAttention(8, 4, block_size=1, device=DEV)
    bad = stc.ArticleStreamingAttention(4, 2, block_size=2, compressor="bogus", device=DEV)
    bad.update(torch.zeros(4, device=DEV), torch.zeros(2, device=DEV))
    with pytest.raises(ValueError):
        bad.update(torch.zeros(4, device=DEV), torch.zeros(2, device=DEV))
    lib = _native.lib()
    assert lib.sta_decode_compress(1, 4, 2, None, None, 2, 0, None, None, None, None, 1, 1, 1, None, None, None,
                                   None, 2, 0, None, None, None) == _native.STA_ERR_ARG


@pytest.mark.parametrize("comp,dtype", [("sorted_pair", torch.float32), ("random", torch.bfloat16),
                                        ("none", torch.float32)])
def test_state_dict_resume_is_bit_exact(comp, dtype):
    """state_dict() after 300 tokens (with draws reserved ahead), torch.save / torch.load(weights_only=True),
    load_state_dict() into a fresh object: the next 400 steps (block completions and merges included)
    equal those of the original object bit for bit, and so do the final levels."""
    import io
    S, d, dv, block = 5, 24, 20, 32
    g = torch.Generator().manual_seed(3)
    q, k, v = ((torch.randn(S, 700, w, generator=g) * 0.3).to(dtype) for w in (d, d, dv))
    kw = dict(degree=2, block_size=block, scale=0.5, compressor=comp, device=DEV, dtype=dtype, seed=11, streams=S)
    a = stc.ArticleStreamingAttention(d, dv, **kw)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    a.extend(kd[:, :290], vd[:, :290])
    for i in range(290, 300):
        a.step(qd[:, i], kd[:, i], vd[:, i])
    a._st.reserve_draws(100)
    buf = io.BytesIO()
    torch.save(a.state_dict(), buf)
    buf.seek(0)
    b = stc.ArticleStreamingAttention(d, dv, **kw)
    b.load_state_dict(torch.load(buf, weights_only=True))
    assert b.length == a.length == 300
    out_a = torch.stack([a.step(qd[:, i], kd[:, i], vd[:, i]) for i in range(300, 700)], dim=1)
    out_b = torch.stack([b.step(qd[:, i], kd[:, i], vd[:, i]) for i in range(300, 700)], dim=1)
    assert torch.equal(out_a, out_b)
    if comp != "none":
        for la, lb in zip(a.coreset.level_positions(), b.coreset.level_positions()):
            assert (la is None and lb is None) or torch.equal(la, lb)
    with pytest.raises(ValueError):
        stc.ArticleStreamingAttention(d, dv, **dict(kw, seed=12)).load_state_dict(a.state_dict())
