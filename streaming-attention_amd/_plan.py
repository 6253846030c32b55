"""Host-side plans for the HIP kernels: feature tables, seed-derived draws, coreset node DAGs and the
per-tile node lists.  Everything here is a pure function of sizes and seeds (never of q/k/v), so it
is computed once per configuration and cached.

Random draws follow the reference's torch CPU generator call order exactly:
  * flat block coreset: one generator seeded with `seed`; for every completed block that has a later
    query, in block order: sorted_pair -> randn(d), rand(B//2); random (or sorted_pair with n <= 2)
    -> randperm(n)   (fast_article_attention.py:339, :348, :328, :335, :395-419);
  * merge-and-reduce levels: one generator seeded with `seed` at construction; one compress call per
    completed block and one per cascade merge, in the order the binary counter produces them
    (streaming_taylor_coreset_attention.py:367-368, :387-411, :427-467).
The projection direction is normalised with the same torch ops as the reference
(fast_article_attention.py:340), so it is bit-identical.
"""

from __future__ import annotations

import heapq
import itertools
import math
import threading
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

import _native

TILE_ROWS = 128  # must equal sta_tile_rows()
NODE_DESC = 8
NODE_META = 4
METHOD_COPY, METHOD_SORTED_PAIR, METHOD_PERM = 0, 1, 2
KIND_RAW, KIND_MERGE = 0, 1
MODE_FLAT, MODE_LEVELS, MODE_EXACT, MODE_TAYLOR = 0, 1, 2, 3
COMPRESSORS = ("sorted_pair", "random", "none")

_lock = threading.Lock()
_cache: Dict[tuple, object] = {}


def _cached(key, build):
    with _lock:
        hit = _cache.get(key)
    if hit is not None:
        return hit
    val = build()
    with _lock:
        if len(_cache) > 256:
            _cache.clear()
        _cache[key] = val
    return val


def moment_chunk(d: int) -> int:
    """Tokens per moment chunk (must equal sta_moment_chunk)."""
    return 32


def num_features(d: int, degree: int) -> int:
    return sum(math.comb(d + l - 1, l) if l > 0 else 1 for l in range(degree + 1))


def _factorial_inverse(combo: Tuple[int, ...]) -> float:
    """1 / prod_j alpha_j! for a non-decreasing multi-index."""
    inv = 1.0
    for _, run in itertools.groupby(combo):
        inv /= math.factorial(len(list(run)))
    return inv


# ----------------------------------------------------------------------------- feature tiles


def _window_cover(d: int, deg: int) -> List[Tuple[Tuple[Tuple[int, ...], int], List[Tuple[int, ...]]]]:
    """The degree-`deg` monomials in x[0..d) assigned to quad windows: a window (fixed, m) holds the 4
    monomials fixed + (v,) for v in [4 m, 4 m + 4) (fixed: deg - 1 non-decreasing factors), the form a
    quad of the moment kernel reads (the shared factors and one aligned 4-element block).  Every
    monomial lies in up to deg windows (its value in each factor position as the varying one); the cover
    takes windows greedily by the number of still uncovered monomials they hold (ties: the smallest key),
    which leaves fewer padding slots than one row per prefix when the rows are short (d = 16, degree 3:
    208 windows for 816 monomials against 260 rows' quads)."""
    mons = list(itertools.combinations_with_replacement(range(d), deg))
    wins: Dict[Tuple[Tuple[int, ...], int], List[int]] = {}
    mon_w: List[List[Tuple[Tuple[int, ...], int]]] = [[] for _ in mons]
    for i, mono in enumerate(mons):
        seen = set()
        for t in range(deg):
            key = (mono[:t] + mono[t + 1:], mono[t] // 4)
            if key in seen:
                continue
            seen.add(key)
            wins.setdefault(key, []).append(i)
            mon_w[i].append(key)
    cnt = {k: len(v) for k, v in wins.items()}
    heap = [(-c, k) for k, c in cnt.items()]
    heapq.heapify(heap)
    covered = [False] * len(mons)
    out = []
    while heap:
        negc, key = heapq.heappop(heap)
        c = cnt[key]
        if c == 0:
            continue
        if -negc != c:  # stale entry: requeue with the current count
            heapq.heappush(heap, (-c, key))
            continue
        got = [i for i in wins[key] if not covered[i]]
        for i in got:
            covered[i] = True
            for k2 in mon_w[i]:
                cnt[k2] -= 1
        out.append((key, [mons[i] for i in got]))
    assert all(covered)
    return out

MOM_WAVES = 4  # waves per moment workgroup (sta_moments)
OCC2_SPEEDUP = 1.2  # per-tile throughput of two resident moment workgroups per CU vs one
WIDE_COST = 1.2  # time per tile of a 64-column workgroup (split products) vs a 32-column one alone
MOM_MAX_WAVE_TILES = 16  # largest per-wave tile count the kernel is instantiated for
COVER_MAX_MONOMIALS = 50_000  # largest degree-3 / 4 monomial set packed by the window cover (<= 0.5 s)


@dataclass(frozen=True)
class FeatureTiles:
    """The monomial basis through `degree` laid out for the moment kernel: tiles of 16 features made of
    4 quads; quad q of tile t is quads[(4 t + q) * qw : (4 t + q + 1) * qw], packed i0 | b << 8 | i2 << 16 |
    i3 << 24 (qw = 1, degree <= 4) and a second word i4 | i5 << 8 | i6 << 16 | i7 << 24 (qw = 2, degree
    5 .. 8), and holds the features x[i0] * x[b + s] * x[i2] * ... (the degree - 2 extra factors), s = 0..3,
    with b a multiple of 4 and x[d] = 1 (so i0 = i2 = ... = d reduces the degree).
    coef[16 t + 4 q + s] is the key-side coefficient 1/prod(alpha!) of feature s of the quad, 0 where
    b + s is not a valid last factor (padding; x[b + s] is then 0 or the constant 1).

    Same set of monomials as the reference's feature map (fast_article_attention.py:151-181,
    streaming_taylor_coreset_attention.py:118-216); the order differs, which the moment sums do not
    depend on.  Monomials sharing all factors but the last form a row (last factor >= the others); a
    row is cut at multiples of 4, so every quad is one 16-byte LDS read in the kernel.  Padding costs
    about 4% more tiles than a dense packing at d = 64, degree 2."""

    d: int
    degree: int
    count: int
    n_tiles: int
    quads: np.ndarray  # uint32 [n_tiles * 4 * qw]
    coef: np.ndarray  # float32 [n_tiles * 16]
    # the monomial of every slot: mono_len [n_tiles * 16] its degree (-1 for padding), mono [n_tiles * 16,
    # max(degree, 1)] its factors ascending in the first mono_len columns (-1 after)
    mono_len: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int8))
    mono: np.ndarray = field(default_factory=lambda: np.zeros((0, 1), np.int32))
    qw: int = 1  # 32-bit words per quad

    def combo(self, slot: int) -> Optional[Tuple[int, ...]]:
        """The sorted multi-index of a slot (None for padding)."""
        n = int(self.mono_len[slot])
        return None if n < 0 else tuple(int(x) for x in self.mono[slot, :n])


def quad_words(degree: int) -> int:
    """32-bit words per feature quad of a degree (the moment kernel's mom_quad_words)."""
    return 2 if degree >= 5 else 1


def _pack_quad(i0: int, b: int, extras: Tuple[int, ...], one: int, qw: int) -> List[int]:
    """Words of a quad: i0 | b << 8 | e0 << 16 | e1 << 24 [, e2 | e3 << 8 | e4 << 16 | e5 << 24]; unused
    extra factors are `one` (the constant x[d] = 1)."""
    ex = list(extras) + [one] * (4 * qw - 2 - len(extras))
    words = [i0 | (b << 8) | (ex[0] << 16) | (ex[1] << 24)]
    if qw == 2:
        words.append(ex[2] | (ex[3] << 8) | (ex[4] << 16) | (ex[5] << 24))
    return words


class _Quads:
    """Quads under construction as arrays: i0 [n], b [n], extras [n, 6] (unused = the constant index),
    coef [n, 4], per-slot monomials mono [n, 4, width] ascending with -1 after mono_len [n, 4] (-1 for
    padding slots)."""

    def __init__(self, width: int) -> None:
        self.width = max(width, 1)
        self.parts: List[Tuple[np.ndarray, ...]] = []

    def add_arrays(self, i0, b, extras, coef, mono, mono_len) -> None:
        n = i0.shape[0]
        ex = np.full((n, 6), -1, dtype=np.int32)
        ex[:, : extras.shape[1]] = extras
        mo = np.full((n, 4, self.width), -1, dtype=np.int32)
        mo[:, :, : mono.shape[2]] = mono
        self.parts.append((i0.astype(np.int32), b.astype(np.int32), ex, coef.astype(np.float64), mo,
                           mono_len.astype(np.int8)))

    def add_lists(self, quads: List[Tuple[int, int, Tuple[int, ...]]], coefs: List[List[float]],
                  combos: List[Optional[Tuple[int, ...]]]) -> None:
        if not quads:
            return
        n = len(quads)
        i0 = np.asarray([q[0] for q in quads])
        b = np.asarray([q[1] for q in quads])
        ex = np.full((n, 6), -1, dtype=np.int32)
        for i, q in enumerate(quads):
            ex[i, : len(q[2])] = q[2]
        mo = np.full((n, 4, self.width), -1, dtype=np.int32)
        ml = np.full((n, 4), -1, dtype=np.int8)
        for i, c in enumerate(combos):
            if c is not None:
                ml[i // 4, i % 4] = len(c)
                mo[i // 4, i % 4, : len(c)] = c
        self.add_arrays(i0, b, ex, np.asarray(coefs, dtype=np.float64).reshape(n, 4), mo, ml)

    def cat(self):
        if not self.parts:
            return (np.zeros(0, np.int32), np.zeros(0, np.int32), np.zeros((0, 6), np.int32),
                    np.zeros((0, 4)), np.zeros((0, 4, self.width), np.int32), np.zeros((0, 4), np.int8))
        return tuple(np.concatenate([p[i] for p in self.parts]) for i in range(6))


def _row_quads(qs: _Quads, d: int, prefixes: np.ndarray) -> int:
    """Quads of the rows prefix + (c,), c from the prefix's last factor to d - 1, for every sorted prefix
    row of `prefixes` [P, L] (L >= 1), built with numpy: the row is cut at multiples of 4; a slot's
    coefficient is 1/prod(alpha!) of its monomial.  Returns the number of features."""
    pn, ln = prefixes.shape
    if pn == 0:
        return 0
    lo = prefixes[:, -1].astype(np.int64)
    nq = (d - 1) // 4 - lo // 4 + 1
    rowid = np.repeat(np.arange(pn), nq)
    k = np.arange(int(nq.sum())) - np.repeat(np.cumsum(nq) - nq, nq)
    b = (lo[rowid] // 4) * 4 + 4 * k
    c = b[:, None] + np.arange(4)[None, :]
    valid = (c >= lo[rowid][:, None]) & (c < d)
    # 1/prod(alpha!) of the prefix and the run length of its last factor
    run = np.ones(pn, dtype=np.int64)
    prod = np.ones(pn, dtype=np.float64)
    for j in range(1, ln):
        run = np.where(prefixes[:, j] == prefixes[:, j - 1], run + 1, 1)
        prod *= run
    base = 1.0 / prod
    coef = np.where(c == lo[rowid][:, None], (base / (run + 1))[rowid][:, None], base[rowid][:, None])
    coef = np.where(valid, coef, 0.0)
    mono = np.concatenate([np.broadcast_to(prefixes[rowid][:, None, :], (rowid.shape[0], 4, ln)), c[:, :, None]], axis=2)
    mono_len = np.where(valid, ln + 1, -1)
    qs.add_arrays(prefixes[rowid, 0], b, prefixes[rowid, 1:], coef, mono, mono_len)
    return int(valid.sum())


def _rows_to_tiles(d: int, degree: int, qs: _Quads, count: int, reorder: bool) -> FeatureTiles:
    """Tiles of 4 quads from the quads in order.  reorder: first every run of 4 quads that share (b,
    extras) and take 4 consecutive first factors i0 = 4k .. 4k+3, then the remaining quads in order.  In
    the kernel's update a tile's 16 lanes then read 4 distinct key rows per factor (x[i0] by quad,
    x[b + s] by slot), a pattern the transposed key rows serve without LDS bank conflicts, and the query
    reads one 16-byte block x[b..b+3] per token for all 4 quads."""
    one = d
    qw = quad_words(degree)
    i0, b, ex, coef, mono, mono_len = qs.cat()
    nq = i0.shape[0]
    ex = np.where(ex < 0, one, ex)
    order = np.arange(nq)
    if reorder and nq:
        real = i0 != one
        idx = np.nonzero(real)[0]
        # group the real quads by (extras, b, i0 >> 2); a group of 4 distinct i0 is a run
        keys = [i0[idx]] + [i0[idx] >> 2, b[idx]] + [ex[idx, j] for j in range(6)]
        srt = idx[np.lexsort(keys)]
        gk = np.stack([ex[srt, j] for j in range(6)] + [b[srt], i0[srt] >> 2], axis=1)
        new_grp = np.ones(srt.shape[0], dtype=bool)
        new_grp[1:] = np.any(gk[1:] != gk[:-1], axis=1)
        gid = np.cumsum(new_grp) - 1
        gsize = np.bincount(gid)
        first_pos = np.full(gsize.shape[0], nq, dtype=np.int64)
        np.minimum.at(first_pos, gid, srt)
        in_run = gsize[gid] == 4
        run_members = srt[in_run]
        run_gid = gid[in_run]
        # runs in the order of their first quad, members by i0
        run_order = np.lexsort((i0[run_members], first_pos[run_gid]))
        head = run_members[run_order]
        rest_mask = np.ones(nq, dtype=bool)
        rest_mask[head] = False
        order = np.concatenate([head, np.nonzero(rest_mask)[0]])
    i0, b, ex, coef, mono, mono_len = i0[order], b[order], ex[order], coef[order], mono[order], mono_len[order]
    n_tiles = -(-nq // 4)
    pad = np.asarray(_pack_quad(one + 1, d // 4 * 4, (), one, qw), dtype=np.uint32)
    q = np.tile(pad, n_tiles * 4)
    if nq:
        w0 = (i0 | (b << 8) | (ex[:, 0] << 16) | (ex[:, 1] << 24)).astype(np.uint32)
        if qw == 2:
            w1 = (ex[:, 2] | (ex[:, 3] << 8) | (ex[:, 4] << 16) | (ex[:, 5] << 24)).astype(np.uint32)
            q[: 2 * nq] = np.stack([w0, w1], axis=1).reshape(-1)
        else:
            q[:nq] = w0
    c = np.zeros(n_tiles * 16, dtype=np.float32)
    c[: 4 * nq] = coef.reshape(-1)
    ml = np.full(n_tiles * 16, -1, dtype=np.int8)
    ml[: 4 * nq] = mono_len.reshape(-1)
    mo = np.full((n_tiles * 16, qs.width), -1, dtype=np.int32)
    mo[: 4 * nq] = mono.reshape(-1, qs.width)
    return FeatureTiles(d, degree, count, n_tiles, q, c, ml, mo, qw)


def feature_tiles(d: int, degree: int) -> FeatureTiles:
    """Feature tiles of the basis through `degree` of x[0 .. d) for a staged key width d <= 128 (degree
    5 .. 8: d <= 64; wider keys: window_tiles)."""
    if degree > 8 or d > 128 or (degree >= 5 and d > 64):
        raise NotImplementedError("the HIP feature map supports degree <= 4 with D <= 128 (wider keys through "
                                  "dimension windows) and degree 5 .. 8 with D <= 64")

    def build():
        one = d
        quads: List[Tuple[int, int, Tuple[int, ...]]] = []
        coefs: List[List[float]] = []
        slot_combos: List[Optional[Tuple[int, ...]]] = []
        count = 0

        def add_row(prefix: Tuple[int, ...], lo: int, hi: int, with_const: bool) -> None:
            """Features prefix + (c,) for lo <= c < hi (and the constant feature `prefix` when
            with_const, stored at c = d), in quads of 4-aligned c."""
            nonlocal count
            last = d if with_const else hi - 1
            if last < lo:
                return
            i0 = prefix[0] if len(prefix) >= 1 else one
            extras = tuple(prefix[1:])
            for b in range((lo // 4) * 4, last + 1, 4):
                if not any(lo <= c < hi or (with_const and c == d) for c in range(b, b + 4)):
                    continue  # no feature in this quad (degree 0: only the constant's quad is kept)
                cs = []
                for s_ in range(4):
                    c = b + s_
                    if lo <= c < hi:
                        cs.append(_factorial_inverse(tuple(sorted(prefix + (c,)))))
                        slot_combos.append(tuple(sorted(prefix + (c,))))
                        count += 1
                    elif with_const and c == d:
                        cs.append(_factorial_inverse(prefix))
                        slot_combos.append(tuple(prefix))
                        count += 1
                    else:
                        cs.append(0.0)
                        slot_combos.append(None)
                quads.append((i0, b, extras))
                coefs.append(cs)

        # degree 0 and 1: x_c for c < d plus the constant, all with prefix ()
        add_row((), 0, d if degree >= 1 else 0, True)
        if degree >= 2:
            for a in range(d):
                add_row((a,), a, d, False)
        # degrees 3 and 4: the window cover (fewer padding slots than rows cut at multiples of 4); rows
        # (built with numpy) for large sets, where the greedy cover takes seconds of host time, and for
        # degrees 5 .. 8
        qs = _Quads(degree)
        big_rows = []
        for deg in range(3, degree + 1):
            if deg >= 5 or math.comb(d + deg - 1, deg) > COVER_MAX_MONOMIALS:
                big_rows.append(deg)
                continue
            for (fixed, m), got in _window_cover(d, deg):
                mine = set(got)
                cs = []
                for s_ in range(4):
                    mono = tuple(sorted(fixed + (4 * m + s_,))) if 4 * m + s_ < d else None
                    if mono is not None and mono in mine:
                        cs.append(_factorial_inverse(mono))
                        slot_combos.append(mono)
                        count += 1
                    else:  # padding, or a monomial another window holds
                        cs.append(0.0)
                        slot_combos.append(None)
                quads.append((fixed[0] if fixed else one, 4 * m, tuple(fixed[1:])))
                coefs.append(cs)
        qs.add_lists(quads, coefs, slot_combos)
        for deg in big_rows:
            pre = np.asarray(list(itertools.combinations_with_replacement(range(d), deg - 1)), dtype=np.int64)
            count += _row_quads(qs, d, pre.reshape(-1, deg - 1))
        return _rows_to_tiles(d, degree, qs, count, reorder=degree <= 4)

    return _cached(("ftiles", d, degree), build)


# ----------------------------------------------------------------------------- dimension windows
WINDOW_BLOCK = 32  # dimensions per window block
WINDOW_BLOCKS = 4  # blocks per window (128 staged dimensions)


@dataclass(frozen=True)
class WindowTiles:
    """The basis through `degree` (<= 4) of keys wider than the 128 staged dimensions: every monomial is
    assigned to one window of 4 blocks of 32 row dimensions holding all its factors, and each window's
    monomials are tiled over the window's 128 virtual dimensions (virtual 32 b + j = row dimension
    blocks[b] + j).  tiles[w] is window w's FeatureTiles (virtual indices, constant x[128] = 1; combos in
    ROW dimensions); blocks[w] the first row dimension of each of its 4 blocks."""

    d: int  # row width (a multiple of 32)
    degree: int
    count: int
    blocks: Tuple[Tuple[int, ...], ...]
    tiles: Tuple[FeatureTiles, ...]

    @property
    def n_tiles(self) -> int:
        return sum(t.n_tiles for t in self.tiles)


def window_tiles(d: int, degree: int) -> WindowTiles:
    """Windows for a row width d > 128 (a multiple of 32, at most 256) and degree <= 4.  The block sets
    (the distinct 32-dimension blocks of a monomial's factors, at most `degree` of them) are covered
    greedily by 4-block windows, each set assigned to the first window that covers it (most monomials
    first); every window's monomials form rows by their leading factors as in feature_tiles."""
    if d % WINDOW_BLOCK or d <= 128 or degree > 4:
        raise NotImplementedError("dimension windows need a row width above 128 (a multiple of 32) and degree <= 4")

    def build():
        nb = d // WINDOW_BLOCK
        vd = WINDOW_BLOCK * WINDOW_BLOCKS
        sets = [frozenset(c) for r in range(1, min(degree, nb) + 1) for c in itertools.combinations(range(nb), r)]

        def weight(sset):  # monomials whose distinct blocks are exactly sset
            k = len(sset)
            return sum(math.comb(WINDOW_BLOCK * k + l - 1, l) for l in range(k, degree + 1)) if k else 1

        left = set(sets)
        chosen: List[Tuple[Tuple[int, ...], List[frozenset]]] = []
        cands = list(itertools.combinations(range(nb), WINDOW_BLOCKS))
        while left:
            best = max(cands, key=lambda w: (sum(weight(x) for x in left if x <= set(w)), tuple(-i for i in w)))
            got = [x for x in left if x <= set(best)]
            left -= set(got)
            chosen.append((best, got))
        if not chosen:  # degree 0: the constant feature alone
            chosen.append((tuple(range(WINDOW_BLOCKS)), []))
        tiles = []
        count = 0
        for wi, (wblocks, got) in enumerate(chosen):
            vpos = {b: k for k, b in enumerate(wblocks)}
            mine = set(got)

            def virt(dim):
                return WINDOW_BLOCK * vpos[dim // WINDOW_BLOCK] + dim % WINDOW_BLOCK

            # the window's monomials (row dimensions, sorted), then rows by leading factors in virtual order
            rows: Dict[Tuple[int, ...], List[int]] = {}
            real_of: Dict[Tuple[int, ...], Tuple[int, ...]] = {}
            dims = [b * WINDOW_BLOCK + j for b in wblocks for j in range(WINDOW_BLOCK)]
            for l in range(1, degree + 1):
                for mono in itertools.combinations_with_replacement(dims, l):
                    if frozenset(m // WINDOW_BLOCK for m in mono) not in mine:
                        continue
                    v = tuple(sorted(virt(m) for m in mono))
                    rows.setdefault(v[:-1], []).append(v[-1])
                    real_of[v] = mono
            quads, coefs, combos = [], [], []
            if wi == 0:
                rows.setdefault((), [])  # the constant feature (x[vd] = 1) lives in window 0's () row
            n = 0
            for prefix in sorted(rows):
                cs_set = set(rows[prefix])
                with_const = prefix == () and wi == 0
                lasts = sorted(cs_set | ({vd} if with_const else set()))
                for b in sorted({4 * (c // 4) for c in lasts}):
                    cf = []
                    for s_ in range(4):
                        c = b + s_
                        if c in cs_set:
                            v = tuple(sorted(prefix + (c,)))
                            cf.append(_factorial_inverse(v))
                            combos.append(real_of[v])
                            n += 1
                        elif with_const and c == vd:
                            cf.append(1.0)
                            combos.append(())
                            n += 1
                        else:
                            cf.append(0.0)
                            combos.append(None)
                    quads.append((prefix[0] if prefix else vd, b, tuple(prefix[1:])))
                    coefs.append(cf)
            qs = _Quads(degree)
            qs.add_lists(quads, coefs, combos)
            tiles.append(_rows_to_tiles(vd, degree, qs, n, reorder=True))
            count += n
        assert count == num_features(d, degree), (count, num_features(d, degree))
        return WindowTiles(d, degree, count, tuple(tuple(b * WINDOW_BLOCK for b in w) for w, _ in chosen),
                           tuple(tiles))

    return _cached(("wtiles", d, degree), build)


def reference_feature_order(d: int, degree: int) -> Dict[Tuple[int, ...], int]:
    """Index of every sorted multi-index in the reference's feature order: degree 0, 1, ..., t, each
    degree in itertools.combinations_with_replacement(range(d), l) order
    (streaming_taylor_coreset_attention.py:160-176, fast_article_attention.py:151-181)."""

    def build():
        order: Dict[Tuple[int, ...], int] = {(): 0}
        for l in range(1, degree + 1):
            for combo in itertools.combinations_with_replacement(range(d), l):
                order[combo] = len(order)
        return order

    return _cached(("reforder", d, degree), build)


def feature_index_width(d: int, degree: int) -> int:
    """Factor slots per feature of feature_index (sta_decode_moments' index_width): 4 (8-bit factors
    packed in a uint32) for d < 255 and degree <= 4, else 8 (uint16 factors)."""
    return 4 if d < 255 and degree <= 4 else 8


def feature_index(d: int, degree: int) -> np.ndarray:
    """The factors of every reference feature f as indices into x = [x_0 .. x_{d-1}, 1] (index d is the
    constant 1 filling the unused factors): uint32 [F] packed i0 | i1 << 8 | i2 << 16 | i3 << 24 when
    feature_index_width is 4, else uint16 [F, 8]."""
    if degree > 8:
        raise NotImplementedError("the HIP feature map supports degree <= 8")

    def build():
        order = reference_feature_order(d, degree)
        if feature_index_width(d, degree) == 4:
            out = np.zeros(len(order), dtype=np.uint32)
            for combo, f in order.items():
                idx = list(combo) + [d] * (4 - len(combo))
                out[f] = idx[0] | (idx[1] << 8) | (idx[2] << 16) | (idx[3] << 24)
            return out
        out16 = np.full((len(order), 8), d, dtype=np.uint16)
        for combo, f in order.items():
            out16[f, : len(combo)] = combo
        return out16

    return _cached(("findex", d, degree), build)


@dataclass(frozen=True)
class MomentSplit:
    """Work split of the moment kernel: `fsplit` feature splits x `csplit` column groups of `columns`
    (32 or 64) value columns per head,
    4 waves per workgroup, every wave holding exactly `wave_tiles` tiles.  quads/coef are the feature
    table in the kernel's layout [fsplit][4][wave_tiles][4 quads | 16 coefficients]; wave j (= 4 fs + w)
    holds the real tiles [tile_off[j], tile_off[j+1]) followed by padding tiles (coefficient 0)."""

    fsplit: int
    csplit: int
    wave_tiles: int
    tile_off: np.ndarray  # int32 [fsplit * 4 + 1]
    quads: np.ndarray  # uint32 [fsplit * 4 * wave_tiles * 4]
    coef: np.ndarray  # float32 [fsplit * 4 * wave_tiles * 16]
    mixed: bool = False  # splits fs >= fsplit / 2 run wave_tiles - 1 tiles per wave
    columns: int = 32  # value columns per workgroup
    win: Optional[np.ndarray] = None  # int32 [fsplit * 4]: each split's window blocks (keys wider than 128)


def moment_split(ft: FeatureTiles, bh: int, dv: int, nt_options: Tuple[Tuple[int, int], ...],
                 compute_units: int = 256, mixed_nts: Tuple[int, ...] = (),
                 wide_nts: Tuple[int, ...] = ()) -> MomentSplit:
    """Choose (fsplit, wave_tiles, mixed) minimising rounds-of-workgroups x tiles-per-wave on a GPU with
    `compute_units` compute units; nt_options lists (per-wave tile count, workgroups resident per
    compute unit) pairs the library supports, mixed_nts the tile counts it also runs mixed (the feature
    splits fs >= fsplit / 2 hold one tile less per wave; every compute unit then pairs a full and a
    short workgroup), wide_nts the tile counts it runs with 64 value columns per workgroup (one
    workgroup per compute unit, every feature value generated once for all 64 columns: WIDE_COST per
    tile against one 32-column tile alone on a compute unit).  Ties go to fewer feature splits (fewer
    partial sums)."""

    def build():
        t = ft.n_tiles
        csplit = -(-dv // 32)
        opts = sorted(nt_options)
        best = None
        for fsplit in range(1, t + 1):
            need = -(-t // (MOM_WAVES * fsplit))
            cand = next(((o, occ) for o, occ in opts if o >= need), None)
            if cand is None:
                continue
            nt, occ = cand
            rounds = -(-(bh * fsplit * csplit) // (compute_units * occ))
            # a compute unit time-shares its resident workgroups; two waves per SIMD overlap one wave's
            # VALU/LDS work with the other's matrix-core work (measured 1.2x per tile at d = 64)
            speed = OCC2_SPEEDUP if occ == 2 else 1.0
            for mixed in (False, True):
                if mixed and (nt not in mixed_nts or fsplit % 2 or csplit != 2 or occ != 2
                              or 2 * fsplit * (2 * nt - 1) < t):
                    continue
                cost = rounds * (nt - 0.5 if mixed else nt) * occ / speed
                if best is None or cost < best[0] - 1e-9:
                    best = (cost, fsplit, nt, mixed, 32)
            wide = next((o for o in sorted(wide_nts) if o >= need), None)
            if wide is not None:
                cost = -(-(bh * fsplit) // compute_units) * wide * WIDE_COST
                if best is None or cost < best[0] - 1e-9:
                    best = (cost, fsplit, wide, False, 64)
            if need == 1:
                break
        if best is None:
            raise ValueError(f"no supported per-wave tile count for {t} feature tiles (options {opts})")
        _, fsplit, nt, mixed, columns = best
        csplit = -(-dv // columns)
        parts = fsplit * MOM_WAVES
        if mixed:
            caps = [nt if j < parts // 2 else nt - 1 for j in range(parts)]
            sizes = list(caps)
            excess = sum(caps) - t
            j = parts - 1
            while excess > 0:
                if sizes[j] > 0:
                    sizes[j] -= 1
                    excess -= 1
                j = j - 1 if j > 0 else parts - 1
        else:
            base, extra = divmod(t, parts)
            sizes = [base + (1 if i < extra else 0) for i in range(parts)]
        off = np.zeros(parts + 1, dtype=np.int32)
        off[1:] = np.cumsum(sizes)
        # zero-valued padding slots
        pad = np.asarray(_pack_quad(ft.d + 1, ft.d // 4 * 4, (), ft.d, ft.qw), dtype=np.uint32)
        quads = np.tile(pad, (parts, nt, 4, 1))
        coef = np.zeros((parts, nt, 16), dtype=np.float32)
        tiles_q = ft.quads.reshape(t, 4, ft.qw)
        tiles_c = ft.coef.reshape(t, 16)
        for j in range(parts):
            cnt = sizes[j]
            quads[j, :cnt] = tiles_q[off[j]:off[j] + cnt]
            coef[j, :cnt] = tiles_c[off[j]:off[j] + cnt]
        return MomentSplit(fsplit, csplit, nt, off, quads.reshape(-1), coef.reshape(-1), mixed, columns)

    return _cached(("msplit", ft.d, ft.degree, bh, dv, tuple(nt_options), compute_units, tuple(mixed_nts),
                    tuple(wide_nts)), build)


def window_feature_tiles(wt: WindowTiles) -> FeatureTiles:
    """The windows' tiles as one table (virtual indices, row-dimension combos), window after window."""

    def build():
        qw = wt.tiles[0].qw
        return FeatureTiles(WINDOW_BLOCK * WINDOW_BLOCKS, wt.degree, wt.count, wt.n_tiles,
                            np.concatenate([t.quads for t in wt.tiles]), np.concatenate([t.coef for t in wt.tiles]),
                            np.concatenate([t.mono_len for t in wt.tiles]), np.concatenate([t.mono for t in wt.tiles]),
                            qw)

    return _cached(("wft", wt.d, wt.degree), build)


def moment_split_windows(wt: WindowTiles, bh: int, dv: int, nt_options: Tuple[Tuple[int, int], ...],
                         compute_units: int = 256) -> MomentSplit:
    """Work split of the moment kernel for keys wider than 128: every feature split holds the tiles of
    one window (its table entry win[4 fs .. 4 fs + 3] names the window's blocks), window w taking
    ceil(tiles_w / (4 wave_tiles)) splits with its tiles balanced over their waves; wave_tiles
    minimises rounds of workgroups x tiles per wave as in moment_split.  The table's tile ranges index
    window_feature_tiles(wt)."""

    def build():
        csplit = -(-dv // 32)
        best = None
        for nt, occ in sorted(nt_options):
            splits = [-(-t.n_tiles // (MOM_WAVES * nt)) for t in wt.tiles]
            fsplit = sum(splits)
            rounds = -(-(bh * fsplit * csplit) // (compute_units * occ))
            cost = rounds * nt * occ / (OCC2_SPEEDUP if occ == 2 else 1.0)
            if best is None or cost < best[0] - 1e-9:
                best = (cost, nt, splits)
        if best is None:
            raise ValueError("no supported per-wave tile count for the windowed feature tiles")
        _, nt, splits = best
        fsplit = sum(splits)
        parts = fsplit * MOM_WAVES
        qw = wt.tiles[0].qw
        ft = window_feature_tiles(wt)
        pad = np.asarray(_pack_quad(ft.d + 1, ft.d // 4 * 4, (), ft.d, qw), dtype=np.uint32)
        quads = np.tile(pad, (parts, nt, 4, 1))
        coef = np.zeros((parts, nt, 16), dtype=np.float32)
        win = np.zeros(fsplit * 4, dtype=np.int32)
        off = np.zeros(parts + 1, dtype=np.int32)
        tiles_q = ft.quads.reshape(ft.n_tiles, 4, qw)
        tiles_c = ft.coef.reshape(ft.n_tiles, 16)
        fs, base, j = 0, 0, 0
        for w, t in enumerate(wt.tiles):
            nparts = MOM_WAVES * splits[w]
            b_, extra = divmod(t.n_tiles, nparts)
            for p_ in range(nparts):
                cnt = b_ + (1 if p_ < extra else 0)
                quads[j, :cnt] = tiles_q[base:base + cnt]
                coef[j, :cnt] = tiles_c[base:base + cnt]
                base += cnt
                off[j + 1] = base
                j += 1
            for _ in range(splits[w]):
                win[4 * fs: 4 * fs + 4] = wt.blocks[w]
                fs += 1
        assert j == parts and base == ft.n_tiles
        return MomentSplit(fsplit, csplit, nt, off, quads.reshape(-1), coef.reshape(-1), False, 32, win)

    return _cached(("msplit_win", wt.d, wt.degree, bh, dv, tuple(nt_options), compute_units), build)


def moment_split_ws(ft: FeatureTiles, bh: int, dv: int, slot_options: Tuple[int, ...], column_tiles: int,
                    compute_units: int = 256, allow_mixed: bool = True) -> MomentSplit:
    """Work split of the wave-specialised moment kernel (sta_moments_ws): `fsplit` feature splits x
    `csplit` groups of 16 * column_tiles value columns per head, one workgroup of 4 update and 4 query
    waves per compute unit; a feature split holds 4 slots of `wave_tiles` tiles (mixed: slots 2 and 3
    one tile less).  A SIMD runs the update wave of slot w and the query wave of slot (w + 2) & 3, so a
    workgroup's time is proportional to 2 * wave_tiles - mixed; the choice minimises rounds of
    workgroups times that, ties to fewer feature splits.  Same table layout as moment_split, with the
    4 slots in place of the 4 waves."""

    def build():
        t = ft.n_tiles
        csplit = -(-dv // (16 * column_tiles))
        best = None
        for nts in sorted(slot_options):
            for mixed in (False, True):
                if mixed and (nts < 2 or not allow_mixed):
                    continue
                per = 4 * nts - (2 if mixed else 0)
                fsplit = -(-t // per)
                rounds = -(-(bh * fsplit * csplit) // compute_units)
                cost = rounds * (2 * nts - (1 if mixed else 0))
                key = (cost, fsplit, mixed)
                if best is None or key < best[0]:
                    best = (key, fsplit, nts, mixed)
        if best is None:
            raise ValueError("no tile count for the wave-specialised moment kernel")
        _, fsplit, nts, mixed = best
        parts = fsplit * 4
        caps = [nts - (1 if mixed and (j % 4) >= 2 else 0) for j in range(parts)]
        # fill the slots in order, the last ones short when the tiles run out (padding tiles: coefficient 0)
        sizes, left = [], t
        per_fs = sum(caps[:4])
        base_fs, extra = divmod(t, fsplit)
        for fs in range(fsplit):
            want = base_fs + (1 if fs < extra else 0)  # balance the real tiles over the feature splits
            for j in range(4):
                cap = caps[4 * fs + j]
                take = min(cap, want, left)
                sizes.append(take)
                want -= take
                left -= take
        assert left == 0 and per_fs >= base_fs + (1 if extra else 0)
        off = np.zeros(parts + 1, dtype=np.int32)
        off[1:] = np.cumsum(sizes)
        pad_quad = (ft.d + 1) | ((ft.d // 4 * 4) << 8) | (ft.d << 16) | (ft.d << 24)
        quads = np.full((parts, nts, 4), pad_quad, dtype=np.uint32)
        coef = np.zeros((parts, nts, 16), dtype=np.float32)
        tiles_q = ft.quads.reshape(t, 4)
        tiles_c = ft.coef.reshape(t, 16)
        for j in range(parts):
            cnt = sizes[j]
            quads[j, :cnt] = tiles_q[off[j]:off[j] + cnt]
            coef[j, :cnt] = tiles_c[off[j]:off[j] + cnt]
        return MomentSplit(fsplit, csplit, nts, off, quads.reshape(-1), coef.reshape(-1), mixed, 16 * column_tiles)

    return _cached(("msplit_ws", ft.d, ft.degree, bh, dv, tuple(slot_options), column_tiles, compute_units,
                    allow_mixed), build)


def ws_segments(n: int, shift: int, query_block: int, bh: int, ft: FeatureTiles, dv: int,
                slot_options: Tuple[int, ...], column_tiles: int, compute_units: int = 256,
                min_blocks: int = 2) -> Tuple[int, int]:
    """(nseg, seg_blocks) for sta_moments_ws_seg: when the workgroups of the whole-sequence scan at the
    split a busy GPU would use (bh x fsplit x csplit) leave compute units idle, each head's scan is cut
    into nseg segments of seg_blocks query blocks (at least min_blocks), every segment non-empty;
    (1, 0) otherwise."""
    full = moment_split_ws(ft, max(bh, compute_units), dv, slot_options, column_tiles)
    grid = bh * full.fsplit * full.csplit
    blocks = -(-(n + shift) // query_block)
    want = min(compute_units // max(grid, 1), blocks // min_blocks)
    if grid >= compute_units or want <= 1:
        return 1, 0
    seg_blocks = -(-blocks // want)
    return -(-blocks // seg_blocks), seg_blocks


def tile_coefficients(quads: np.ndarray, coef: np.ndarray, d: int) -> np.ndarray:
    """The coefficient table of the split-product moment scan at degree <= 2 (moments.hip,
    mom_query_split): every tile's 16 entries set to one value c_t with

        c_t * sum over the tile's 16 slots of monomial(slot) == sum over slots of coef(slot) * monomial(slot)

    as polynomials in x (x[d] = 1, x[d + 1 ..] = 0).  The kernel then accumulates plain monomials and
    applies c_t once per tile and query token.  Degree <= 2 tiles are of three kinds: 16 distinct
    monomials of coefficient 1 (c_t = 1); a diagonal tile x[4k + r] x[4k + s], whose slot pairs (r, s),
    (s, r) both hold the monomial of coefficient 1 and whose diagonal holds coefficient 1/2 (c_t = 1/2);
    zero-valued padding (c_t = 0).  Raises ValueError for a table without such a c_t per tile (degree
    >= 3, or d not a multiple of 4)."""
    q = np.asarray(quads, dtype=np.int64).reshape(-1, 4)
    c = np.asarray(coef, dtype=np.float64).reshape(-1, 16)
    out = np.zeros(c.shape, dtype=np.float32)
    for t in range(q.shape[0]):
        want: Dict[Tuple[int, ...], float] = {}
        cnt: Dict[Tuple[int, ...], int] = {}
        for qi in range(4):
            pq = int(q[t, qi])
            i0, b, i2, i3 = pq & 255, (pq >> 8) & 255, (pq >> 16) & 255, (pq >> 24) & 255
            for s_ in range(4):
                ids = (i0, b + s_, i2, i3)
                if max(ids) > d:
                    continue  # a factor x[d + 1 ..] = 0
                mono = tuple(sorted(i for i in ids if i != d))
                want[mono] = want.get(mono, 0.0) + float(c[t, 4 * qi + s_])
                cnt[mono] = cnt.get(mono, 0) + 1
        vals = {want[m] / cnt[m] for m in cnt}
        if len(vals) > 1:
            raise ValueError(f"tile {t} has no uniform coefficient: {sorted(vals)}")
        out[t] = vals.pop() if vals else 0.0
    return out.reshape(np.asarray(coef).shape)


def reference_rank(mono: np.ndarray, mono_len: np.ndarray, d: int, degree: int) -> np.ndarray:
    """Index of every monomial (rows of mono, factors ascending in the first mono_len columns) in the
    reference's feature order for dimension d: degree 0, 1, ..., each in
    itertools.combinations_with_replacement(range(d), l) order (streaming_taylor_coreset_attention.py:
    160-176).  A sorted multiset a_1 <= .. <= a_l is the strictly increasing b_i = a_i + i - 1 in
    range(n), n = d + l - 1, whose lexicographic rank is sum_i [C(n - b_{i-1} - 1, l - i + 1) -
    C(n - b_i, l - i + 1)] (b_0 = -1).  -1 where mono_len < 0."""
    top = d + degree + 1
    pas = np.zeros((top + 1, degree + 2), dtype=np.int64)
    pas[:, 0] = 1
    for n_ in range(1, top + 1):
        pas[n_, 1:] = pas[n_ - 1, 1:] + pas[n_ - 1, :-1]
    offset = np.zeros(degree + 2, dtype=np.int64)
    for l in range(1, degree + 2):
        offset[l] = offset[l - 1] + (math.comb(d + l - 2, l - 1) if l - 1 > 0 else 1)
    out = np.full(mono_len.shape[0], -1, dtype=np.int64)
    for l in range(0, degree + 1):
        sel = np.nonzero(mono_len == l)[0]
        if sel.size == 0:
            continue
        if l == 0:
            out[sel] = 0
            continue
        n_ = d + l - 1
        bb = mono[sel, :l].astype(np.int64) + np.arange(l)[None, :]
        prev = np.concatenate([np.full((sel.size, 1), -1, dtype=np.int64), bb[:, :-1]], axis=1)
        rank = np.zeros(sel.size, dtype=np.int64)
        for i in range(l):
            k = l - i
            rank += pas[n_ - prev[:, i] - 1, k] - pas[n_ - bb[:, i], k]
        out[sel] = offset[l] + rank
    return out


def split_state_rows(ft: FeatureTiles, ms: MomentSplit, d: int) -> np.ndarray:
    """int32 [fsplit * 4 * wave_tiles * 16]: the reference-order feature row (for the true dimension d
    <= ft.d, or the row dimensions of a windowed table) of every feature slot of the split's table, -1
    for padding slots and for monomials that involve a padding dimension >= d (their keys are zero
    there)."""

    def build():
        ml = ft.mono_len.astype(np.int64)
        inside = np.all((ft.mono < d) | (np.arange(ft.mono.shape[1])[None, :] >= ml[:, None]), axis=1)
        slot_row = np.where(inside & (ml >= 0), reference_rank(ft.mono, np.where(inside, ml, -1), d, ft.degree), -1)
        parts = ms.tile_off.shape[0] - 1
        rows = np.full((parts, ms.wave_tiles, 16), -1, dtype=np.int32)
        for j in range(parts):
            a, b = int(ms.tile_off[j]), int(ms.tile_off[j + 1])
            rows[j, : b - a] = slot_row[16 * a: 16 * b].reshape(b - a, 16)
        got = np.sort(rows[rows >= 0])
        assert got.size == num_features(d, ft.degree) and np.array_equal(got, np.arange(got.size))
        return rows.reshape(-1)

    return _cached(("srows", ft.d, ft.degree, d, ms.fsplit, ms.wave_tiles, ms.tile_off.tobytes(),
                    ms.win.tobytes() if ms.win is not None else b""), build)


# ----------------------------------------------------------------------------- draws

def _compressed_size(n_in: int, compressor: str) -> int:
    if compressor == "none" or n_in <= 1:
        return n_in
    return (n_in + 1) // 2


@dataclass
class Draws:
    """Seed-derived randomness of every compress call, per sequence, in reference call order."""

    dirs: np.ndarray  # float32 [BH, n_calls, d] (float64 for a float64 caller)
    unif: np.ndarray  # float32 [BH, n_calls, max_in // 2] (float64 likewise)
    perms: np.ndarray  # int32 [BH, n_calls, max_in]
    n_calls: int
    max_in: int


def _draw_one_call(g: torch.Generator, n_in: int, d: int, compressor: str, dtype: torch.dtype = torch.float32):
    """Consume the generator exactly as one reference compress call on n_in items does (directions and
    uniforms in `dtype`, the keys' dtype of the reference call)."""
    if compressor == "none" or n_in <= 1:
        return METHOD_COPY, None, None, None
    if compressor not in ("random", "sorted_pair"):
        raise ValueError("compressor must be one of {'sorted_pair', 'random', 'none'}")
    if compressor == "random" or n_in <= 2:
        perm = torch.randperm(n_in, generator=g)
        return METHOD_PERM, None, None, perm.numpy().astype(np.int32)
    direction = torch.randn(d, generator=g, dtype=dtype)
    direction = direction / torch.clamp(torch.linalg.vector_norm(direction), min=1e-12)
    u = torch.rand(n_in // 2, generator=g, dtype=dtype)
    table = torch.float64 if dtype == torch.float64 else torch.float32  # 16-bit values held exactly
    return METHOD_SORTED_PAIR, direction.to(table).numpy(), u.to(table).numpy(), None


def _call_method(n_in: int, compressor: str) -> int:
    if compressor == "none" or n_in <= 1:
        return METHOD_COPY
    if compressor not in ("random", "sorted_pair"):
        raise ValueError("compressor must be one of {'sorted_pair', 'random', 'none'}")
    return METHOD_PERM if compressor == "random" or n_in <= 2 else METHOD_SORTED_PAIR


def _collect_draws(seeds: List[int], call_sizes: List[int], d: int, compressor: str,
                   f64: bool = False, dtype: Optional[torch.dtype] = None) -> Tuple[Draws, List[int]]:
    """Draws of every sequence over the compress calls of call_sizes, replayed natively (the same
    generator calls as _draw_one_call, per sequence on its own generator, sequences in parallel); f64:
    directions and uniforms drawn as float64 (a float64 caller's); dtype, when given: drawn in that
    dtype (float64 tables for float64, float32 tables otherwise)."""
    methods = [_call_method(n_in, compressor) for n_in in call_sizes]
    max_in = max(max(call_sizes) if call_sizes else 2, 2)
    dirs, unif, perms = _native.host_draws(seeds, call_sizes, d, compressor, max_in, f64=f64, dtype=dtype)
    return Draws(dirs, unif, perms, len(call_sizes), max_in), methods


def _collect_draws_py(seeds: List[int], call_sizes: List[int], d: int, compressor: str,
                      f64: bool = False, dtype: Optional[torch.dtype] = None) -> Tuple[Draws, List[int]]:
    """The same draws one generator call at a time through torch's Python API."""
    n_calls = len(call_sizes)
    max_in = max(max(call_sizes) if call_sizes else 2, 2)
    bh = len(seeds)
    tdt = dtype if dtype is not None else (torch.float64 if f64 else torch.float32)
    ft = np.float64 if tdt == torch.float64 else np.float32
    dirs = np.zeros((bh, max(n_calls, 1), d), dtype=ft)
    unif = np.zeros((bh, max(n_calls, 1), max_in // 2), dtype=ft)
    perms = np.zeros((bh, max(n_calls, 1), max_in), dtype=np.int32)
    methods: List[int] = []
    for h, seed in enumerate(seeds):
        g = torch.Generator(device="cpu")
        g.manual_seed(int(seed))
        for c, n_in in enumerate(call_sizes):
            method, dvec, u, perm = _draw_one_call(g, n_in, d, compressor,
                                                   tdt)
            if h == 0:
                methods.append(method)
            if dvec is not None:
                dirs[h, c] = dvec
                unif[h, c, : u.shape[0]] = u
            if perm is not None:
                perms[h, c, : perm.shape[0]] = perm
    return Draws(dirs, unif, perms, n_calls, max_in), methods


# ----------------------------------------------------------------------------- node DAGs

@dataclass
class NodePlan:
    mode: int
    n: int
    block: int
    shift: int
    n_nodes: int
    cap: int
    desc: np.ndarray  # int32 [n_nodes, NODE_DESC]
    meta: np.ndarray  # int32 [n_nodes, NODE_META]: size, lo, hi, materialized
    batches: List[np.ndarray]  # node ids per compress launch, in dependency order
    tile_ptr: np.ndarray  # int32 [n_tiles + 1]
    tile_nodes: np.ndarray  # int32
    n_tiles: int
    call_sizes: List[int] = field(default_factory=list)  # n_in of each draw slot (call order)
    level_of: Optional[np.ndarray] = None  # level of each node (levels mode)


def _tile_lists(meta: np.ndarray, n: int, shift: int) -> Tuple[np.ndarray, np.ndarray, int]:
    n_tiles = -(-(n + shift) // TILE_ROWS)
    tiles: List[np.ndarray] = []
    nodes: List[np.ndarray] = []
    for node in range(meta.shape[0]):
        size, lo, hi = int(meta[node, 0]), int(meta[node, 1]), int(meta[node, 2])
        if size <= 0 or lo > hi:
            continue
        t0 = (lo + shift) // TILE_ROWS
        t1 = (hi + shift) // TILE_ROWS
        tiles.append(np.arange(t0, t1 + 1, dtype=np.int64))
        nodes.append(np.full(t1 - t0 + 1, node, dtype=np.int64))
    if tiles:
        tt = np.concatenate(tiles)
        nn = np.concatenate(nodes)
        order = np.lexsort((nn, tt))
        tt, nn = tt[order], nn[order]
    else:
        tt = np.zeros(0, np.int64)
        nn = np.zeros(0, np.int64)
    counts = np.bincount(tt, minlength=n_tiles)
    ptr = np.zeros(n_tiles + 1, dtype=np.int32)
    ptr[1:] = np.cumsum(counts)
    return ptr, nn.astype(np.int32), n_tiles


def flat_plan(n: int, block: int, compressor: str) -> NodePlan:
    """Flat block coreset (fast_article_attention.py:364-434): block b (every block with a later
    query) is compressed once; its reps are active for rows >= (b+1)*B."""

    def build():
        if compressor == "none":
            return exact_plan(n)
        nbf = (n - 1) // block if n > 0 else 0
        cap = max(1, _compressed_size(block, compressor))
        desc = np.zeros((max(nbf, 1), NODE_DESC), dtype=np.int32)
        meta = np.zeros((max(nbf, 1), NODE_META), dtype=np.int32)
        call_sizes = []
        for b in range(nbf):
            m = _compressed_size(block, compressor)
            desc[b] = [KIND_RAW, b * block, 0, block, m, 0, b, 0]
            meta[b] = [m, (b + 1) * block, n - 1, 0]
            call_sizes.append(block)
        if nbf == 0:
            meta[0] = [0, 1, 0, 0]
        ptr, tn, nt = _tile_lists(meta[:nbf], n, 0)
        batches = [np.arange(nbf, dtype=np.int32)] if nbf else []
        return NodePlan(MODE_FLAT, n, block, 0, max(nbf, 1), cap, desc, meta, batches, ptr, tn, nt, call_sizes)

    return _cached(("flat", n, block, compressor), build)


def exact_plan(n: int) -> NodePlan:
    def build():
        desc = np.zeros((1, NODE_DESC), dtype=np.int32)
        meta = np.array([[0, 1, 0, 0]], dtype=np.int32)
        ptr, tn, nt = _tile_lists(meta[:0], n, 0)
        return NodePlan(MODE_EXACT, n, 1, 0, 1, 1, desc, meta, [], ptr, tn, nt, [])

    return _cached(("exact", n), build)


def levels_plan(n: int, block: int, compressor: str) -> NodePlan:
    """Merge-and-reduce level tree computed level-parallel.  node(0, j) = compress(block j);
    node(l, j) = compress(cat(node(l-1, 2j), node(l-1, 2j+1))).  After c completed blocks level l holds
    node(l, (c >> l) - 1) iff bit l of c is set, so a node (l, j) with j even is visible to the rows
    whose counter (i+1)//B lies in [(j+1) 2^l, (j+2) 2^l - 1]; nodes with odd j are merge inputs only."""

    def build():
        if compressor == "none":
            return exact_plan(n)
        nb = n // block
        counts = []
        l = 0
        while (nb >> l) > 0:
            counts.append(nb >> l)
            l += 1
        offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64) if counts else np.zeros(1, np.int64)
        n_nodes = int(offs[-1]) if counts else 0
        nid = lambda lev, j: int(offs[lev] + j)

        sizes = [0] * n_nodes
        n_in_of = [0] * n_nodes
        for lev, cnt in enumerate(counts):
            for j in range(cnt):
                i = nid(lev, j)
                n_in_of[i] = block if lev == 0 else sizes[nid(lev - 1, 2 * j)] + sizes[nid(lev - 1, 2 * j + 1)]
                sizes[i] = _compressed_size(n_in_of[i], compressor)

        # reference call order: block c completes -> node(0, c-1), then one merge per carry
        slot = [0] * n_nodes
        call_sizes: List[int] = []
        for c in range(1, nb + 1):
            lev, j = 0, c - 1
            while True:
                i = nid(lev, j)
                slot[i] = len(call_sizes)
                call_sizes.append(n_in_of[i])
                if j % 2 == 1:  # the level was occupied: merge into the next level
                    lev, j = lev + 1, j // 2
                else:
                    break

        cap = max([1] + sizes)
        desc = np.zeros((max(n_nodes, 1), NODE_DESC), dtype=np.int32)
        meta = np.zeros((max(n_nodes, 1), NODE_META), dtype=np.int32)
        level_of = np.zeros(max(n_nodes, 1), dtype=np.int32)
        for lev, cnt in enumerate(counts):
            for j in range(cnt):
                i = nid(lev, j)
                if lev == 0:
                    desc[i] = [KIND_RAW, j * block, 0, n_in_of[i], sizes[i], 0, slot[i], 0]
                else:
                    a_ = nid(lev - 1, 2 * j)
                    desc[i] = [KIND_MERGE, a_, nid(lev - 1, 2 * j + 1), n_in_of[i], sizes[i], 0, slot[i], sizes[a_]]
                level_of[i] = lev
                if j % 2 == 0:
                    lo = (j + 1) * (1 << lev) * block - 1
                    hi = min((j + 2) * (1 << lev) * block - 2, n - 1)
                else:
                    lo, hi = 1, 0
                meta[i] = [sizes[i], lo, hi, 0]
        if n_nodes == 0:
            meta[0] = [0, 1, 0, 0]
        ptr, tn, nt = _tile_lists(meta[:n_nodes], n, 1)
        batches = [np.arange(offs[lev], offs[lev] + counts[lev], dtype=np.int32) for lev in range(len(counts))]
        return NodePlan(MODE_LEVELS, n, block, 1, max(n_nodes, 1), cap, desc, meta, batches, ptr, tn, nt, call_sizes, level_of)

    return _cached(("levels", n, block, compressor), build)


CMP_MAX_ANC = 4  # ancestor levels a level-0 compress call can score (sta_compress_nodes / _leaves)


def ancestor_table(plan: NodePlan, desc: np.ndarray,
                   max_levels: int = CMP_MAX_ANC) -> Tuple[int, Optional[np.ndarray], Optional[np.ndarray]]:
    """Ancestor scores of a levels plan (sta_compress_nodes): (anc_levels, node_level int32 [n_nodes], anc
    int32 [n_nodes, anc_levels]) where anc[node (0, j), l - 1] is the draw slot of node (l, j >> l), the
    call that later sorts block j's surviving tokens at level l, or -1 where that call is not
    sorted_pair; rows of merge nodes are -1.  (0, None, None) when the plan has no merge levels or its
    level-0 calls do not project (desc: the plan's descriptors with methods filled in)."""
    if plan.mode != MODE_LEVELS or plan.level_of is None or len(plan.batches) < 2 or max_levels < 1:
        return 0, None, None
    levels = len(plan.batches)
    a_lev = min(levels - 1, max_levels, CMP_MAX_ANC)
    first = [int(b[0]) for b in plan.batches]
    counts = [len(b) for b in plan.batches]
    if not np.all(desc[first[0]: first[0] + counts[0], 5] == METHOD_SORTED_PAIR):
        return 0, None, None
    anc = np.full((plan.n_nodes, a_lev), -1, dtype=np.int32)
    for l in range(1, a_lev + 1):
        j = np.arange(counts[0]) >> l
        ok = j < counts[l]
        node = first[l] + np.minimum(j, counts[l] - 1)
        slot = np.where(ok & (desc[node, 5] == METHOD_SORTED_PAIR), desc[node, 6], -1)
        anc[first[0]: first[0] + counts[0], l - 1] = slot
    return a_lev, plan.level_of.astype(np.int32), anc


CMP_MAX_D = 256  # key width of the compressor's direction buffer (csrc/compress.hip)


def compress_region_floats(max_in: int, f64: bool) -> int:
    """LDS floats of one compress call's arrays (cmp_smem_floats without ancestor directions)."""
    m = (max_in + 3) & ~3
    return (2 if f64 else 1) * m + 3 * m + (2 if f64 else 1) * CMP_MAX_D


@dataclass
class MergeLaunch:
    """One sta_compress_merges launch: table int32 [workgroups, steps, groups] of node ids (-1: idle),
    groups of group_threads threads (64: one wave per node; 256: lockstep groups)."""
    table: np.ndarray
    groups: int
    steps: int
    levels: Tuple[int, int]  # first and last tree level it computes
    group_threads: int = 256

    @property
    def workgroups(self) -> int:
        return int(self.table.shape[0])


def merge_launches(plan: NodePlan, max_in: int, f64: bool, group_threads: int = 256, groups: int = 4,
                   bottom: int = 16, lds_bytes: int = 160 * 1024) -> List[MergeLaunch]:
    """The merge levels of a levels plan as sta_compress_merges launches of subtrees.  A launch starting
    at level l0 gives each workgroup B = 2^k consecutive nodes (l0, j) (at most `bottom`) and the B >> r
    nodes (l0 + r, j) above them for k + 1 levels (fewer at the top); its G groups take a level's nodes
    G at a time, one step each (64-thread groups: G = B, one step per level; 256-thread groups: G <=
    `groups`, at most 1024 threads).  A workgroup's LDS (G call regions) stays within lds_bytes.  Every
    node's children are then computed by an earlier launch or an earlier step of its own workgroup.
    Empty for plans without merge levels."""
    if plan.mode != MODE_LEVELS or len(plan.batches) < 2:
        return []
    region = compress_region_floats(max_in, f64) * 4
    cap_g = 1
    limit = min(16, bottom) if group_threads == 64 else min(groups, 1024 // group_threads)
    while cap_g * 2 <= limit and cap_g * 2 * region <= lds_bytes:
        cap_g *= 2
    counts = [len(b) for b in plan.batches]
    launches: List[MergeLaunch] = []
    l0 = 1
    while l0 < len(counts):
        b = 1
        while b < min(bottom if group_threads != 64 else cap_g, counts[l0]):
            b *= 2
        g = b if group_threads == 64 else min(cap_g, b)
        depth = min(b.bit_length(), len(counts) - l0)
        per_level = [-(-(b >> r) // g) for r in range(depth)]
        n_wg = -(-counts[l0] // b)
        table = np.full((n_wg, sum(per_level), g), -1, dtype=np.int32)
        base = 0
        for r in range(depth):
            per = b >> r
            for j in range(counts[l0 + r]):
                q = j % per
                table[j // per, base + q // g, q % g] = plan.batches[l0 + r][j]
            base += per_level[r]
        launches.append(MergeLaunch(table, g, int(sum(per_level)), (l0, l0 + depth - 1), group_threads))
        l0 += depth
    return launches


def check_merge_launches(plan: NodePlan, desc: np.ndarray, launches: List[MergeLaunch]) -> None:
    """Every merge node exactly once, after both its children (raw nodes: the first launch; merges: an
    earlier launch, or an earlier step of the same workgroup).  Raises ValueError otherwise."""
    done = np.zeros(plan.n_nodes, dtype=bool)
    done[plan.batches[0]] = True
    seen = np.zeros(plan.n_nodes, dtype=bool)
    for ln in launches:
        before = done.copy()
        for w in range(ln.workgroups):
            mine = before.copy()
            for r in range(ln.steps):
                nodes = [int(x) for x in ln.table[w, r] if x >= 0]
                for node in nodes:
                    if desc[node, 0] != KIND_MERGE or seen[node]:
                        raise ValueError(f"merge launch lists node {node} twice or a raw node")
                    a, b = int(desc[node, 1]), int(desc[node, 2])
                    if not (mine[a] and mine[b]):
                        raise ValueError(f"merge node {node} is scheduled before its children {a}, {b}")
                    seen[node] = True
                for node in nodes:
                    mine[node] = True
                    done[node] = True
    merges = desc[: plan.n_nodes, 0] == KIND_MERGE
    if not np.array_equal(seen, merges):
        raise ValueError("merge launches leave merge nodes out")


def segment_plan(n: int, block: int, stride: int) -> Tuple[NodePlan, int, int]:
    """Segment-mean reps of completed blocks with a later query (triton_article_attention.py:189-245,
    active for i >= (rep_block+1)*B with weight = stride, :353-357)."""

    def build():
        rpb = block // stride
        nbk = max(0, (n - 1) // block)
        n_rep = nbk * rpb
        nn = max(nbk, 1)
        desc = np.zeros((nn, NODE_DESC), dtype=np.int32)
        meta = np.zeros((nn, NODE_META), dtype=np.int32)
        for b in range(nbk):
            meta[b] = [rpb, (b + 1) * block, n - 1, 1]
        if nbk == 0:
            meta[0] = [0, 1, 0, 1]
        ptr, tn, nt = _tile_lists(meta[:nbk], n, 0)
        plan = NodePlan(MODE_FLAT, n, block, 0, nn, max(rpb, 1), desc, meta, [], ptr, tn, nt, [])
        return plan, n_rep, rpb

    return _cached(("segment", n, block, stride), build)


def draws_for(plan: NodePlan, seeds: Tuple[int, ...], d: int, compressor: str,
              f64: bool = False, dtype: Optional[torch.dtype] = None) -> Tuple[Draws, np.ndarray]:
    """Draw table for every sequence plus the node descriptors with their compress method filled in
    (f64: float64 directions and uniforms; dtype, when given: drawn in that dtype)."""

    def build():
        draws, methods = _collect_draws(list(seeds), plan.call_sizes, d, compressor, f64, dtype)
        desc = plan.desc.copy()
        if plan.mode in (MODE_FLAT, MODE_LEVELS) and plan.call_sizes:
            for i in range(desc.shape[0]):
                if plan.meta[i, 0] == 0 and desc[i, 3] == 0:
                    continue
                desc[i, 5] = methods[desc[i, 6]]
        return draws, desc

    return _cached(("draws", plan.mode, plan.n, plan.block, tuple(seeds), d, compressor, bool(f64), dtype), build)


def reference_selection(plan: NodePlan, seeds: Tuple[int, ...], keys: torch.Tensor, compressor: str,
                        threads: int = 0) -> Tuple[np.ndarray, np.ndarray]:
    """Node tables (node_src int32, node_w float32 [S, n_nodes, cap]) of a flat or levels plan with every
    compress call ordered as the reference orders it: torch's CPU `keys @ direction` and argsort in the
    keys' dtype on the draws of that dtype (sta_host_select).  keys: contiguous CPU [S, N, d] in the
    caller's dtype and layout."""
    if plan.mode not in (MODE_FLAT, MODE_LEVELS) or not plan.batches:
        raise ValueError("reference_selection needs a flat or levels plan with compress calls")
    s_, n, d = keys.shape
    if n != plan.n or len(seeds) != s_:
        raise ValueError("keys do not match the plan and seeds")
    dr, desc = draws_for(plan, tuple(seeds), d, compressor, dtype=keys.dtype)
    return _native.host_select(keys, plan.mode == MODE_LEVELS, desc, plan.n_nodes, plan.cap, dr.dirs, dr.unif,
                               dr.perms, threads)


def completion_call_sizes(blocks_before: int, block: int, compressor: str) -> List[int]:
    """Input sizes of the compress calls made when block number blocks_before + 1 completes: the
    block itself, then one merge per occupied level below the counter's lowest zero bit
    (streaming_taylor_coreset_attention.py:387-411); every level holds compressed_size(block) items."""
    m = _compressed_size(block, compressor)
    carries = 0
    c = blocks_before
    while c & 1:
        carries += 1
        c >>= 1
    return [block] + [2 * m] * carries


def sequence_seeds(seed: int, bh: int) -> Tuple[int, ...]:
    """Per-sequence seeds seed + b*H + h (fast_article_attention.py:693,
    streaming_taylor_coreset_attention.py:743), i.e. seed + flattened (b, h) index."""
    return tuple(int(seed) + i for i in range(bh))
