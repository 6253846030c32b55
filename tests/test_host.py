"""Host-side checks of the product that need no GPU: the C-ABI library loads and exports every symbol
the header declares; the seed-derived draws the product replays equal the reference's; level-tree
plans follow the reference's cascade; the Python API raises the reference's exceptions."""

import itertools
import pathlib
import re

import numpy as np
import pytest
import torch

import _native
import reference_cpu as orc
import _plan
import fast_article_attention as faa
import streaming_taylor_coreset_attention as stc
import triton_article_attention as taa

ROOT = pathlib.Path(__file__).resolve().parents[1]


def header_symbols():
    text = (ROOT / "include" / "streamattn.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int64_t|int|const char\*)\s+(sta_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_header_symbols():
    lib = _native.load_library()
    syms = header_symbols()
    assert len(syms) >= 10
    for s in syms:
        assert hasattr(lib, s), s
    assert set(syms) == set(_native.EXPORTED_SYMBOLS)
    assert lib.sta_version() >= 100
    assert lib.sta_tile_rows() == _plan.TILE_ROWS
    for d in (8, 64, 65, 128):
        assert lib.sta_moment_chunk(d) == _plan.moment_chunk(d)
    assert lib.sta_status_string(0) == b"ok"
    lim = _native.limits()
    assert lim == {"max_d": 256, "max_dv": 256, "max_degree": 8, "max_compress_in": 4096}


def test_library_rejects_bad_arguments_without_touching_a_device():
    lib = _native.load_library()
    # null pointers / bad sizes are refused before any launch
    assert lib.sta_moments(None, None, None, 0, 1, 1, 4, 4, 1, 32, 2, 1.0, 32, 0, 1, 9, 0, 0, 32, None, None, None,
                           None, None, None) == _native.STA_ERR_ARG
    assert lib.sta_moments(16, 16, 16, 0, 1, 64, 64, 64, 64, 64, 2, 1.0, 32, 0, 8, 5, 0, 2, 32, 16, 16, None, 16, 16,
                           None) == _native.STA_ERR_ARG  # unknown products mode
    for mixed, products, columns, dv in [(1, 1, 64, 64), (0, 0, 64, 64), (0, 1, 64, 32), (0, 1, 48, 64)]:
        assert lib.sta_moments(16, 16, 16, 0, 1, 64, 64, 64, dv, 64, 2, 1.0, 32, 0, 8, 5, mixed, products, columns,
                               16, 16, None, 16, 16, None) == _native.STA_ERR_ARG  # 64 columns: split, unmixed, 32 < dv <= 64
    # row stride without windows must be d; windows need the staged width 128, a whole number of 32-wide
    # blocks up to 256 and degree <= 4; degree 5 .. 8 runs fp32 products only
    args = dict(q=16, d=64, ld=64, degree=2, products=1, win=None)

    def mom(**kw):
        a = dict(args, **kw)
        nt = max(lib.sta_moment_wave_tiles(min(a["d"], 128), min(a["degree"], 8), 4), 4)
        return lib.sta_moments(a["q"], 16, 16, 0, 1, 64, a["d"], a["ld"], 64, 64, a["degree"], 1.0, 32, 0, 8, nt, 0,
                               a["products"], 32, 16, 16, a["win"], 16, 16, None)
    assert mom(ld=96) == _native.STA_ERR_ARG
    assert mom(d=128, ld=200, win=16) == _native.STA_ERR_ARG
    assert mom(d=128, ld=288, win=16) == _native.STA_ERR_ARG
    assert mom(d=64, ld=256, win=16) == _native.STA_ERR_ARG
    assert mom(d=160, ld=160) == _native.STA_ERR_UNSUPPORTED
    assert mom(degree=5, products=1) == _native.STA_ERR_UNSUPPORTED
    assert mom(degree=9, products=0) == _native.STA_ERR_UNSUPPORTED
    assert lib.sta_moment_columns_ok(64, 2, 64, 5, 1) == 1
    assert lib.sta_moment_columns_ok(64, 2, 64, 5, 0) == 0 and lib.sta_moment_columns_ok(64, 3, 64, 5, 1) == 0
    assert lib.sta_moment_columns_ok(64, 2, 32, 5, 1) == 0 and lib.sta_moment_columns_ok(64, 2, 64, 4, 1) == 0
    assert lib.sta_compress_nodes(None, 0, 1, 1, 1, None, 1, None, 1, 1, None, None, None, 0, 2, None, None,
                                  None, None, 0, None, None) == _native.STA_ERR_ARG
    # merge launches: the compress_nodes checks, then the round layout and the LDS of every wave
    def merges(dtype=0, steps=2, groups=4, gt=64, max_in=256, k=16):
        return lib.sta_compress_merges(k, dtype, 1, 64, 8, 16, 1, steps, groups, gt, 16, 3, 2, None, None, None, 0,
                                       max_in, 16, 16, None, 0, None, None)
    assert merges(k=None) == _native.STA_ERR_ARG
    assert merges(dtype=9) == _native.STA_ERR_DTYPE
    assert merges(steps=0) == _native.STA_ERR_ARG and merges(groups=0) == _native.STA_ERR_ARG
    assert merges(gt=128) == _native.STA_ERR_ARG and merges(groups=17) == _native.STA_ERR_ARG
    assert merges(gt=256, groups=5) == _native.STA_ERR_ARG
    assert merges(groups=16, max_in=4096) == _native.STA_ERR_UNSUPPORTED
    assert lib.sta_segment_mean(1, 1, 0, 1, 10, 4, 4, 8, 3, 0, 1, 1, None) == _native.STA_ERR_SHAPE
    # flash: null pointers, D beyond the limit, strides not whole 4-element units, misaligned rows
    assert lib.sta_flash_attention(None, 16, 16, 0, 1, 8, 4, 4, 4, 4, 1.0, 16, 0, None) == _native.STA_ERR_ARG
    assert lib.sta_flash_attention(16, 16, 16, 0, 1, 8, 129, 4, 132, 4, 1.0, 16, 0, None) == _native.STA_ERR_UNSUPPORTED
    assert lib.sta_flash_attention(16, 16, 16, 0, 1, 8, 4, 300, 4, 300, 1.0, 16, 0, None) == _native.STA_ERR_UNSUPPORTED
    assert lib.sta_flash_attention(16, 16, 16, 0, 1, 8, 6, 4, 6, 4, 1.0, 16, 0, None) == _native.STA_ERR_ARG
    assert lib.sta_flash_attention(8, 16, 16, 0, 1, 8, 4, 4, 4, 4, 1.0, 16, 0, None) == _native.STA_ERR_ARG
    assert lib.sta_flash_attention(16, 16, 16, 7, 1, 8, 4, 4, 4, 4, 1.0, 16, 0, None) == _native.STA_ERR_DTYPE
    assert lib.sta_flash_attention(16, 16, 16, 0, 0, 8, 4, 4, 4, 4, 1.0, 16, 0, None) == _native.STA_ERR_SHAPE


def _norm(raw):
    d = torch.from_numpy(raw)
    return (d / torch.clamp(torch.linalg.vector_norm(d), min=1e-12)).numpy()


@pytest.mark.parametrize("comp", ["sorted_pair", "random"])
def test_flat_draw_replay_matches_reference(golden, comp):
    g = golden("flat_c1")
    plan = _plan.flat_plan(1024, 128, comp)
    draws, desc = _plan.draws_for(plan, (0,), 32, comp)
    assert draws.n_calls == int(g[f"{comp}_ncalls"]) == 7
    for c in range(7):
        if comp == "sorted_pair":
            assert np.array_equal(draws.dirs[0, c], _norm(g[f"{comp}_call{c}_direction_raw"]))
            assert np.array_equal(draws.unif[0, c, :64], g[f"{comp}_call{c}_uniforms"])
            assert desc[c, 5] == _plan.METHOD_SORTED_PAIR
        else:
            assert np.array_equal(draws.perms[0, c, :128], g[f"{comp}_call{c}_perm"])
            assert desc[c, 5] == _plan.METHOD_PERM


@pytest.mark.parametrize("name", ["levels_c1", "levels_random", "levels_deg3", "levels_oddblock", "levels_block2"])
def test_level_draw_replay_and_cascade_match_reference(golden, name):
    g = golden(name)
    m = g.meta
    plan = _plan.levels_plan(m["n"], m["block"], m["compressor"])
    draws, desc = _plan.draws_for(plan, (m["seed"],), m["d"], m["compressor"])
    n_calls = int(g["ncalls"])
    assert plan.call_sizes == [int(g[f"call{c}_src_in"].shape[0]) for c in range(n_calls)]
    for c in range(n_calls):
        if f"call{c}_direction_raw" in g:
            assert np.array_equal(draws.dirs[0, c], _norm(g[f"call{c}_direction_raw"]))
            assert np.array_equal(draws.unif[0, c, : g[f"call{c}_uniforms"].shape[0]], g[f"call{c}_uniforms"])
        if f"call{c}_perm" in g:
            assert np.array_equal(draws.perms[0, c, : g[f"call{c}_perm"].shape[0]], g[f"call{c}_perm"])
    # merge inputs are cat(old, new) of the two children, in that order
    slot_of = {int(plan.desc[i, 6]): i for i in range(plan.n_nodes)}
    for c in range(n_calls):
        node = slot_of[c]
        kind, a, b, n_in = (int(x) for x in plan.desc[node, :4])
        if kind == _plan.KIND_RAW:
            assert np.array_equal(g[f"call{c}_src_in"], np.arange(a, a + n_in))
        else:
            ca, cb = int(plan.desc[a, 6]), int(plan.desc[b, 6])
            assert np.array_equal(g[f"call{c}_src_in"], np.concatenate([g[f"call{ca}_src_out"], g[f"call{cb}_src_out"]]))


def test_level_plan_intervals_follow_binary_counter():
    n, B = 5000, 64
    plan = _plan.levels_plan(n, B, "sorted_pair")
    # for every row, the visible nodes are exactly those of the counter (i+1)//B
    for i in range(0, n, 37):
        c = (i + 1) // B
        vis = {int(x) for x in np.nonzero((plan.meta[:, 1] <= i) & (plan.meta[:, 2] >= i) & (plan.meta[:, 0] > 0))[0]}
        expect = set()
        for lev in range(c.bit_length()):
            if (c >> lev) & 1:
                j = (c >> lev) - 1
                expect.add(int(np.nonzero((plan.level_of == lev))[0][0]) + j)
        assert vis == expect, i
        t = (i + plan.shift) // _plan.TILE_ROWS
        assert vis <= set(plan.tile_nodes[plan.tile_ptr[t]:plan.tile_ptr[t + 1]].tolist())


def _quad_factors(words):
    """(i0, b, extra factors...) of a packed quad: one word (degree <= 4) or two (degree 5 .. 8)."""
    w = [int(x) for x in words]
    ids = [w[0] & 255, (w[0] >> 8) & 255, (w[0] >> 16) & 255, w[0] >> 24]
    if len(w) > 1:
        ids += [w[1] & 255, (w[1] >> 8) & 255, (w[1] >> 16) & 255, w[1] >> 24]
    return ids


def _quad_features(ft):
    """(monomial, coef) of every feature slot of a quad table: monomial = sorted factors without the
    constant index d; slots beyond the constant (index > d) are reported as None."""
    out = []
    for q, words in enumerate(ft.quads.reshape(-1, ft.qw)):
        i0, b, *extra = _quad_factors(words)
        for s in range(4):
            ids = (i0, b + s, *extra)
            coef = float(ft.coef[4 * q + s])
            mono = None if max(ids) > ft.d else tuple(sorted(i for i in ids if i != ft.d))
            out.append((mono, coef))
    return out


@pytest.mark.parametrize("d,degree", [(5, 3), (64, 2), (32, 2), (16, 3), (8, 0), (12, 1), (128, 2), (6, 2), (6, 4),
                                      (16, 4), (8, 5), (16, 5), (6, 8), (4, 7), (72, 4)])
def test_feature_tiles_cover_the_monomial_basis(d, degree):
    ft = _plan.feature_tiles(d, degree)
    assert ft.count == _plan.num_features(d, degree)
    assert ft.qw == (2 if degree >= 5 else 1)
    assert ft.quads.shape == (4 * ft.n_tiles * ft.qw,) and ft.coef.shape == (16 * ft.n_tiles,)
    feats = _quad_features(ft)
    live = sorted((m, np.float32(c).item()) for m, c in feats if c != 0.0)
    expect = sorted((m, np.float32(orc.inv_multinomial(m)).item()) for m in orc.monomials(d, degree))
    assert live == expect
    # every slot reads inside the staged row: factors up to d + 3 (the constant, then zero padding);
    # padding quads take the zero x[d + 1] as first factor
    for words in ft.quads.reshape(-1, ft.qw):
        i0, b, *extra = _quad_factors(words)
        assert b % 4 == 0 and b + 3 <= ft.d + 3
        assert max(extra) <= ft.d and i0 <= ft.d + 1


@pytest.mark.parametrize("d,degree", [(64, 2), (32, 2), (128, 2), (8, 0), (12, 1), (16, 2), (4, 2)])
def test_tile_coefficients_preserve_every_tile_polynomial(d, degree):
    """The per-tile coefficient table of the split-product moment scan (degree <= 2) gives every tile
    the same polynomial as the per-feature table: checked by evaluating both on random x (x[d] = 1,
    x[d+1..d+3] = 0), over the padded work split too."""
    ft = _plan.feature_tiles(d, degree)
    opts = ((2, 2), (4, 2), (5, 2), (9, 2), (16, 1))
    ms = _plan.moment_split(ft, 3, 64, opts)
    rng = np.random.default_rng(d + degree)
    for quads, coef in ((ft.quads, ft.coef), (ms.quads, ms.coef)):
        tc = _plan.tile_coefficients(quads, coef, d)
        q = quads.reshape(-1, 4).astype(np.int64)
        per_tile = tc.reshape(-1, 16)
        assert np.all(per_tile == per_tile[:, :1])  # uniform over a tile
        assert set(np.unique(per_tile).tolist()) <= {0.0, 0.5, 1.0}
        for _ in range(3):
            x = np.concatenate([rng.standard_normal(d), [1.0, 0.0, 0.0, 0.0]])
            i0, b, i2, i3 = q & 255, (q >> 8) & 255, (q >> 16) & 255, (q >> 24) & 255
            mono = np.stack([x[i0] * x[b + s] * x[i2] * x[i3] for s in range(4)], axis=-1).reshape(-1, 16)
            want = (mono * coef.reshape(-1, 16)).sum(1)
            got = per_tile[:, 0] * mono.sum(1)
            np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    # planted mistakes: a diagonal coefficient of 1 instead of 1/2 has no uniform tile coefficient, and
    # degree 3 tiles are rejected
    if degree == 2:
        bad = ft.coef.copy().reshape(-1, 4, 4)
        q = ft.quads.reshape(-1, 4)
        diag = [t for t in range(q.shape[0]) if all((int(q[t, r]) & 255) == ((int(q[t, 0]) >> 8) & 255) + r
                                                    for r in range(4))]
        assert len(diag) == d // 4
        bad[diag[0], 1, 1] = 1.0
        with pytest.raises(ValueError):
            _plan.tile_coefficients(ft.quads, bad.reshape(-1), d)
    with pytest.raises(ValueError):
        ft3 = _plan.feature_tiles(16, 3)
        _plan.tile_coefficients(ft3.quads, ft3.coef, 16)


def test_feature_tiles_limits():
    with pytest.raises(NotImplementedError):
        _plan.feature_tiles(68, 5)  # degree 5 .. 8 only for d <= 64
    with pytest.raises(NotImplementedError):
        _plan.feature_tiles(8, 9)
    with pytest.raises(NotImplementedError):
        _plan.feature_tiles(160, 2)  # wider than the staged rows: window_tiles
    with pytest.raises(NotImplementedError):
        _plan.window_tiles(160, 5)
    ft = _plan.feature_tiles(16, 4)
    assert ft.count == 4845 and 16 * ft.n_tiles >= 4845


@pytest.mark.parametrize("d,degree", [(160, 2), (256, 2), (192, 1), (256, 0), (160, 3)])
def test_window_tiles_cover_the_monomial_basis(d, degree):
    """Keys wider than 128: every monomial of the d row dimensions sits in exactly one slot of one
    window, with its coefficient; a slot's virtual factors map through its window's blocks to the
    slot's monomial; each window holds 4 distinct 32-dimension blocks."""
    wt = _plan.window_tiles(d, degree)
    assert wt.count == _plan.num_features(d, degree)
    seen = {}
    for blocks, ft in zip(wt.blocks, wt.tiles):
        assert len(set(blocks)) == 4 and all(b % 32 == 0 and b + 32 <= d for b in blocks)
        real = lambda v: blocks[v // 32] + v % 32 if v < 128 else None  # noqa: E731
        for slot, (mono, coef) in enumerate(_quad_features(ft)):
            if coef == 0.0:
                continue
            got = ft.combo(slot)
            assert got is not None and tuple(sorted(real(v) for v in mono)) == got
            assert np.float32(coef) == np.float32(orc.inv_multinomial(got))
            assert got not in seen
            seen[got] = coef
    assert len(seen) == _plan.num_features(d, degree)
    rows = _plan.reference_rank(np.asarray([list(m) + [-1] * (max(degree, 1) - len(m)) for m in seen], dtype=np.int32),
                                np.asarray([len(m) for m in seen], dtype=np.int8), d, degree)
    assert np.array_equal(np.sort(rows), np.arange(len(seen)))


def test_feature_tiles_padding_is_small():
    ft = _plan.feature_tiles(64, 2)  # the long-context workload's basis
    assert ft.n_tiles == 141  # 135 for a dense packing of 2145 features


def test_moment_split_balances_waves():
    opts = ((2, 2), (4, 2), (5, 2), (9, 2), (16, 1))
    ft = _plan.feature_tiles(64, 2)
    ms = _plan.moment_split(ft, 32, 64, opts)  # 32 heads, d = dv = 64, degree 2
    assert (ms.fsplit, ms.csplit, ms.wave_tiles) == (8, 2, 5)
    assert 32 * ms.fsplit * ms.csplit <= 512
    for d, degree, bh, dv in [(64, 2, 128, 64), (16, 3, 128, 64), (32, 2, 1, 32), (4, 0, 1, 5), (40, 2, 1, 256)]:
        ft = _plan.feature_tiles(d, degree)
        ms = _plan.moment_split(ft, bh, dv, opts)
        sizes = np.diff(ms.tile_off)
        assert ms.tile_off[0] == 0 and ms.tile_off[-1] == ft.n_tiles
        assert len(sizes) == 4 * ms.fsplit and sizes.min() >= 0 and sizes.max() <= ms.wave_tiles
        assert ms.wave_tiles in [o for o, _ in opts] and ms.csplit == -(-dv // 32)
        # the padded table holds every real tile exactly once, padding has coefficient 0
        tab = ms.quads.reshape(4 * ms.fsplit, ms.wave_tiles, 4)
        cf = ms.coef.reshape(4 * ms.fsplit, ms.wave_tiles, 16)
        real = np.concatenate([tab[j, :sizes[j]] for j in range(len(sizes))]).reshape(-1)
        assert np.array_equal(real, ft.quads)
        assert all(np.all(cf[j, sizes[j]:] == 0) for j in range(len(sizes)))
    # mixed tile counts: half the feature splits run one tile less per wave
    ft = _plan.feature_tiles(64, 2)
    ms = _plan.moment_split(ft, 32, 64, ((2, 2), (4, 2), (5, 2), (9, 1), (16, 1)), mixed_nts=(4, 5))
    assert (ms.fsplit, ms.csplit, ms.wave_tiles, ms.mixed) == (8, 2, 5, True)
    sizes = np.diff(ms.tile_off)
    half = 2 * ms.fsplit
    assert sizes[:half].max() <= 5 and sizes[half:].max() <= 4 and sizes.sum() == ft.n_tiles == 141
    # every real tile sits inside the slots its wave runs
    q = ms.quads.reshape(4 * ms.fsplit, ms.wave_tiles, 4)
    c = ms.coef.reshape(4 * ms.fsplit, ms.wave_tiles, 16)
    assert np.all(c[half:, ms.wave_tiles - 1] == 0)
    got = sorted(tuple(q[j, i]) for j in range(4 * ms.fsplit) for i in range(sizes[j]))
    assert got == sorted(tuple(x) for x in ft.quads.reshape(-1, 4))
    # 64-column workgroups (split products): one per compute unit, 8 feature splits of 5 tiles per wave
    ms = _plan.moment_split(ft, 32, 64, ((2, 2), (4, 2), (5, 2), (9, 1), (16, 1)), mixed_nts=(4, 5), wide_nts=(5,))
    assert (ms.fsplit, ms.csplit, ms.wave_tiles, ms.mixed, ms.columns) == (8, 1, 5, False, 64)
    assert np.diff(ms.tile_off).sum() == 141 and np.diff(ms.tile_off).max() <= 5


def test_library_moment_tile_options():
    lib = _native.load_library()
    for d, degree in [(64, 2), (16, 3), (128, 2), (100, 3)]:
        opts = [lib.sta_moment_wave_tiles(d, degree, w) for w in range(1, 17)]
        assert all(o >= w for o, w in zip(opts, range(1, 17)))
        assert opts[-1] == 16
    assert lib.sta_moment_wave_tiles(64, 2, 9) == 9
    assert lib.sta_moment_wave_tiles(64, 2, 17) == -1
    assert lib.sta_moment_occupancy(64, 5) == 2 and lib.sta_moment_occupancy(64, 16) == 1
    assert lib.sta_moment_occupancy(128, 5) == 1


# --------------------------------------------------------------------------- reference error behaviour

def _qkv(n=10, d=4, dv=3):
    return torch.randn(n, d), torch.randn(n, d), torch.randn(n, dv)


def test_fast_path_argument_errors():
    q, k, v = _qkv()
    with pytest.raises(ValueError):
        faa.fast_article_causal_attention(q[None], k, v)
    with pytest.raises(ValueError):
        faa.fast_article_causal_attention(q, k[:, :3], v)
    with pytest.raises(ValueError):
        faa.fast_article_causal_attention(q, k, v[:5])
    with pytest.raises(ValueError):
        faa.fast_article_causal_attention(q, k, v, query_chunk_size=0)
    with pytest.raises(ValueError):
        faa.fast_article_causal_attention(q, k, v, block_size=0)
    with pytest.raises(NotImplementedError):
        faa.fast_article_causal_attention(q, k, v, degree=3)
    with pytest.raises(ValueError):
        faa.fast_article_causal_attention(q, k, v, low_mode="bogus")
    with pytest.raises(ValueError):
        faa.fast_article_causal_attention(q[None, None], k[None, None], v[None, None, :5])
    with pytest.raises(ValueError):
        faa.low_degree_taylor_causal_sums(q, k, v, mode="bogus")
    with pytest.raises(NotImplementedError):
        faa.num_taylor_features(4, 3)
    with pytest.raises(ValueError):
        faa.exp_taylor(torch.zeros(2), -1)


@pytest.mark.parametrize("d,degree,bh,dv,ct", [(64, 2, 32, 64, 4), (64, 2, 128, 64, 4), (16, 3, 128, 64, 4), (32, 2, 1, 32, 2),
                                                (64, 2, 3, 100, 4), (128, 2, 8, 96, 2)])
def test_moment_split_ws_covers_every_tile_once(d, degree, bh, dv, ct):
    """The wave-specialised kernel's table: 4 slots per feature split, slots within their tile budget
    (slot_tiles, one less in slots 2 and 3 when mixed), every feature tile exactly once, padding slots
    with coefficient 0."""
    ft = _plan.feature_tiles(d, degree)
    ms = _plan.moment_split_ws(ft, bh, dv, (2, 3, 4, 5), ct)
    sizes = np.diff(ms.tile_off)
    assert sizes.size == 4 * ms.fsplit and sizes.sum() == ft.n_tiles
    caps = np.array([ms.wave_tiles - (1 if ms.mixed and j % 4 >= 2 else 0) for j in range(sizes.size)])
    assert (sizes <= caps).all() and (sizes >= 0).all()
    q = ms.quads.reshape(-1, ms.wave_tiles, 4)
    c = ms.coef.reshape(-1, ms.wave_tiles, 16)
    got = np.concatenate([q[j, : sizes[j]] for j in range(sizes.size)]).reshape(-1)
    assert np.array_equal(got, ft.quads)
    for j in range(sizes.size):
        assert not c[j, sizes[j]:].any()
    assert ms.csplit == -(-dv // (16 * ct)) and ms.columns == 16 * ct


def test_empty_sequences_return_empty_outputs_on_the_host():
    """N = 0: the reference returns empty outputs (its token loop and chunk loops do not run); nothing
    is launched, so this holds without a GPU."""
    q, k, v = torch.zeros(0, 6), torch.zeros(0, 6), torch.zeros(0, 3)
    out = faa.fast_article_causal_attention(q, k, v)
    assert out.shape == (0, 3) and out.dtype == torch.float32
    out, st = faa.fast_article_causal_attention_single(q, k, v, return_stats=True)
    assert out.shape == (0, 3) and st.coreset_items == 0 and st.feature_count == 28
    num, den, f = faa.low_degree_taylor_causal_sums(q, k, v)
    assert num.shape == (0, 3) and den.shape == (0,) and f == 28
    out4 = faa.fast_article_causal_attention(q[None, None], k[None, None], v[None, None])
    assert out4.shape == (1, 1, 0, 3)


def test_streaming_argument_errors():
    q, k, v = _qkv()
    with pytest.raises(ValueError):
        stc.article_causal_attention(q, k, v, block_size=1)
    with pytest.raises(ValueError):
        stc.article_causal_attention(q, k, v, degree=4, max_monomials=10)
    with pytest.raises(ValueError):
        stc.article_causal_attention(q, k, v, block_size=4, compressor="bogus")


def test_triton_api_argument_errors():
    q, k, v = _qkv()
    with pytest.raises((ImportError, ValueError)):
        taa.triton_article_causal_attention(q, k, v)  # CPU tensors (test_triton_article_attention.py:17-26)
    with pytest.raises(ValueError):
        taa.build_segment_mean_coreset(k[None], v[None], block_size=8, compress_stride=3)
    with pytest.raises((ImportError, ValueError)):
        taa.triton_flash_causal_attention(q, k, v)  # CPU tensors


def test_stats_formulas_match_reference(golden):
    g = golden("flat_bh")
    ref = g["stats"].tolist()
    st = faa._stats(200, 16, 8, 4, 2, 32, "sorted_pair", 2048, "stream", "cpu")
    assert [st.degree, st.block_size, st.feature_count, st.coreset_items, st.approx_streaming_state_bytes,
            st.scratch_low_prefix_bytes, st.scratch_residual_matrix_bytes] == ref


# --------------------------------------------------------------------------- decode host logic

def test_library_decode_entries_reject_bad_arguments():
    lib = _native.load_library()
    assert lib.sta_moment_accumulate(None, None, 0, 1, 1, 1, 4, 4, 1, 32, 2, 1, 9, None, None, None, None, 15, 1,
                                     None, None, None) == _native.STA_ERR_ARG
    assert lib.sta_decode_moments(None, 0, 1, 4, 4, 1.0, None, None, 15, None, 4, 1, None, None,
                                  None) == _native.STA_ERR_ARG
    assert lib.sta_decode_moments(16, 0, 1, 4, 4, 1.0, 16, 16, 15, 16, 6, 1, 16, 16,
                                  None) == _native.STA_ERR_ARG  # index width 4 or 8
    assert lib.sta_decode_tail(None, None, None, 0, 1, 4, 4, 2, 1.0, 1e-12, 8, None, None, 16, 0, None, None, None, 0,
                               8, 0, None, None, 1, None, 0, None, None) == _native.STA_ERR_ARG
    assert lib.sta_decode_compress(1, 4, 2, None, None, 2, 0, None, None, None, None, 1, 1, 1, None, None, None,
                                   None, 2, 0, None, None, None) == _native.STA_ERR_ARG
    assert lib.sta_decode_compress(1, 4, 2, 16, 16, 2, 0, 16, 16, 16, 16, 1, 1, 1, 16, 16, 16,
                                   16, 2, 1, None, None, None) == _native.STA_ERR_ARG  # float64 scoring needs its rows
    assert _native.decode_layout(6, 5) == (8, 32)
    assert _native.decode_layout(64, 130) == (64, 160)
    assert _native.decode_layout(130, 8) == (160, 32)  # wide keys in whole 32-dimension blocks


@pytest.mark.parametrize("d,degree", [(4, 2), (5, 3), (64, 2), (16, 3), (3, 0), (7, 1), (6, 4), (16, 4), (6, 6),
                                      (4, 8), (256, 2), (255, 1)])
def test_feature_index_is_reference_order(d, degree):
    idx = _plan.feature_index(d, degree)
    combos = orc.monomials(d, degree)
    assert idx.shape[0] == len(combos)
    if _plan.feature_index_width(d, degree) == 4:
        assert idx.dtype == np.uint32 and idx.ndim == 1
        for f, c in enumerate(combos):
            full = list(c) + [d] * (4 - len(c))
            assert int(idx[f]) == full[0] | (full[1] << 8) | (full[2] << 16) | (full[3] << 24)
    else:
        assert idx.dtype == np.uint16 and idx.shape[1] == 8 and (degree > 4 or d >= 255)
        for f, c in enumerate(combos):
            assert idx[f].tolist() == list(c) + [d] * (8 - len(c))


@pytest.mark.parametrize("width,d,degree,bh,dv", [(64, 64, 2, 2048, 64), (8, 6, 3, 1, 5), (16, 16, 3, 96, 64),
                                                  (8, 5, 2, 3, 16), (128, 128, 2, 2, 130), (4, 4, 1, 7, 3),
                                                  (8, 7, 5, 3, 16), (8, 8, 6, 1, 8), (160, 150, 2, 4, 16),
                                                  (256, 256, 2, 2, 64)])
def test_split_state_rows_cover_reference_features(width, d, degree, bh, dv):
    """Every reference feature of dimension d has exactly one slot in the accumulate table; each slot's
    monomial (the quad's factors, through the split's window for keys wider than 128) is that
    feature's monomial."""
    if width > 128:
        wt = _plan.window_tiles(width, degree)
        ft = _plan.window_feature_tiles(wt)
        ms = _plan.moment_split_windows(wt, bh, dv, ((5, 1), (16, 1)))
    else:
        ft = _plan.feature_tiles(width, degree)
        opts = (((2, 2), (4, 2), (5, 2), (9, 2), (16, 1)) if degree < 3 else
                ((4, 1),) if degree >= 5 else ((4, 2), (8, 1), (16, 1)))
        ms = _plan.moment_split(ft, bh, dv, opts)
    rows = _plan.split_state_rows(ft, ms, d)
    order = _plan.reference_feature_order(d, degree)
    inv = {f: c for c, f in order.items()}
    assert sorted(r for r in rows if r >= 0) == list(range(_plan.num_features(d, degree)))
    quads = ms.quads.reshape(-1, 4, ft.qw)  # [parts * wave_tiles, 4, words]
    coef = ms.coef.reshape(-1, 16)
    for slot, r in enumerate(rows):
        if r < 0:
            continue
        tile, q, s = slot // 16, (slot % 16) // 4, slot % 4
        i0, b, *extra = _quad_factors(quads[tile, q])
        fac = [f for f in (i0, b + s, *extra) if f < ft.d]
        if ms.win is not None:  # virtual dimension 32 j + i of split fs = row dimension win[4 fs + j] + i
            fs = tile // (4 * ms.wave_tiles)
            fac = [int(ms.win[4 * fs + f // 32]) + f % 32 for f in fac]
        assert tuple(sorted(fac)) == inv[r]
        assert coef[tile, slot % 16] == np.float32(orc.inv_multinomial(inv[r]))


@pytest.mark.parametrize("block,comp", [(16, "sorted_pair"), (33, "sorted_pair"), (2, "sorted_pair"), (32, "random")])
def test_completion_calls_follow_the_level_plan(block, comp):
    """Concatenating the per-completion call sizes of blocks 1..C gives the level plan's call order."""
    c = 37
    sizes = []
    for b in range(c):
        sizes += _plan.completion_call_sizes(b, block, comp)
    assert sizes == _plan.levels_plan(c * block, block, comp).call_sizes


@pytest.mark.parametrize("d,deg", [(16, 3), (32, 3), (5, 3), (16, 4), (6, 4)])
def test_window_cover_holds_every_monomial_once_in_fewer_quads(d, deg):
    """The degree-3 / 4 window cover: every monomial of the degree (the oracle's list) in exactly one
    window, each window a quad the kernel can read (deg - 1 shared factors, one aligned 4-element
    block), and no more windows than rows cut at multiples of 4 (the packing it replaced)."""
    cover = _plan._window_cover(d, deg)
    held = [m for _, got in cover for m in got]
    assert sorted(held) == sorted(m for m in orc.monomials(d, deg) if len(m) == deg)
    assert len(held) == len(set(held))
    for (fixed, m), got in cover:
        assert len(fixed) == deg - 1 and list(fixed) == sorted(fixed) and 1 <= len(got) <= 4
        for mono in got:
            rest = list(mono)
            for f in fixed:
                rest.remove(f)
            assert len(rest) == 1 and rest[0] // 4 == m
    rows = sum(-(-(d - 4 * (pre[-1] // 4)) // 4) for pre in itertools.combinations_with_replacement(range(d), deg - 1))
    assert len(cover) <= rows
    if (d, deg) == (16, 3):
        assert len(cover) == 208 and _plan.feature_tiles(16, 3).n_tiles == 64


def test_static_scratch_owner_registry():
    """One decode state on one stream per device may use the static scratch; others are refused until
    the owner releases it (the allocation-free step's overlap guard; CPU logic only)."""
    import _decode

    reg = _decode.StaticScratchOwners()
    reg.claim(0, owner=1, stream=0x10)
    reg.claim(0, owner=1, stream=0x10)  # the owner again, same stream
    reg.claim(1, owner=2, stream=0x20)  # another device is independent
    with pytest.raises(ValueError, match="another decode state"):
        reg.claim(0, owner=2, stream=0x10)
    with pytest.raises(ValueError, match="another stream"):
        reg.claim(0, owner=1, stream=0x11)
    assert not reg.release(0, owner=2)
    assert reg.release(0, owner=1)
    reg.claim(0, owner=2, stream=0x11)
    assert reg.holder(0) == (2, 0x11)


@pytest.mark.parametrize("n,block,gt,groups,bottom", [(64 * 256, 64, 256, 4, 16), (64 * 37, 64, 256, 4, 16),
                                                     (5000, 16, 256, 2, 4), (4096, 256, 256, 1, 1),
                                                     (128 * 1000, 128, 256, 4, 8), (64 * 256, 64, 64, 0, 16),
                                                     (5000, 16, 64, 0, 4), (128 * 1000, 128, 64, 0, 8)])
def test_merge_launches(n, block, gt, groups, bottom):
    """Subtree launches of a levels plan: every merge node once, after its children (an earlier launch
    or an earlier step of its own workgroup); log2(bottom) + 1 levels per launch, a level's nodes taken
    `groups` at a time by 256-thread groups (one step per level with one wave per node); the LDS of a
    workgroup's groups limits their number."""
    plan = _plan.levels_plan(n, block, "sorted_pair")
    _, desc = _plan.draws_for(plan, (0,), 8, "sorted_pair")
    ls = _plan.merge_launches(plan, block, False, group_threads=gt, groups=groups, bottom=bottom)
    _plan.check_merge_launches(plan, desc, ls)
    merge_levels = len(plan.batches) - 1
    assert sum(ln.levels[1] - ln.levels[0] + 1 for ln in ls) == merge_levels
    b0 = min(bottom, 1 << (len(plan.batches[1]) - 1).bit_length())
    assert ls[0].levels[1] - ls[0].levels[0] + 1 == min(b0.bit_length(), merge_levels)
    assert ls[0].groups == (b0 if gt == 64 else min(groups, b0))
    assert all(ln.groups * ln.group_threads <= 1024 for ln in ls)
    if gt == 64:
        assert all(ln.steps == ln.levels[1] - ln.levels[0] + 1 for ln in ls)
    # groups limited by LDS: 4096-item calls need 66 KiB each
    big = _plan.levels_plan(8192 * 4, 4096, "sorted_pair")
    assert _plan.merge_launches(big, 4096, False, group_threads=gt, groups=4, bottom=16)[0].groups == 2
    # a schedule that computes a parent in the step of its children, or leaves a merge out, is refused
    bad = [_plan.MergeLaunch(ln.table.copy(), ln.groups, ln.steps, ln.levels, ln.group_threads) for ln in ls]
    t = bad[0].table
    last = t.shape[1] - 1
    if last > 0:
        t[0, last, 0], t[0, 0, 0] = t[0, 0, 0], t[0, last, 0]
        with pytest.raises(ValueError):
            _plan.check_merge_launches(plan, desc, bad)
    with pytest.raises(ValueError):
        _plan.check_merge_launches(plan, desc, ls[:-1])
    assert _plan.merge_launches(_plan.flat_plan(5000, 64, "sorted_pair"), 64, False) == []


def test_ancestor_table_slots():
    """Each level-0 node's ancestor at level l is node (l, j >> l), whose draw slot the table holds; off
    for flat plans, random compressors (permutation calls) and single-level plans."""
    plan = _plan.levels_plan(64 * 37, 64, "sorted_pair")
    _, desc = _plan.draws_for(plan, (0,), 8, "sorted_pair")
    a, level_of, anc = _plan.ancestor_table(plan, desc)
    assert len(plan.batches) - 1 == 5 and a == 4 and anc.shape == (plan.n_nodes, a)
    first = [int(b[0]) for b in plan.batches]
    for j in range(len(plan.batches[0])):
        for l in range(1, a + 1):
            if (j >> l) < len(plan.batches[l]):
                assert anc[first[0] + j, l - 1] == desc[first[l] + (j >> l), 6]
            else:
                assert anc[first[0] + j, l - 1] == -1
    assert (anc[first[1]:] == -1).all() and list(level_of[first[2]: first[2] + 2]) == [2, 2]
    for p2, comp in ((_plan.flat_plan(5000, 64, "sorted_pair"), "sorted_pair"),
                     (_plan.levels_plan(5000, 64, "random"), "random"),
                     (_plan.levels_plan(100, 64, "sorted_pair"), "sorted_pair")):
        _, dsc = _plan.draws_for(p2, (0,), 8, comp)
        assert _plan.ancestor_table(p2, dsc)[0] == 0
