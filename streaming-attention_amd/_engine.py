"""Launch sequence of the prefill path on one ROCm device:

    K1 moments (sta_moments)  ->  K3 compress, one launch per tree level (sta_compress_nodes)
                              ->  K2+K4 block attention with the normalisation (sta_block_attention)

All launches go to torch's current stream of the input device.  Device buffers are torch tensors
allocated here (the C ABI never allocates); plan arrays and draw tables are cached per device.
"""

from __future__ import annotations

import os
import threading
from dataclasses import dataclass
from typing import Callable, Dict, Optional, Tuple

import numpy as np
import torch

import _native
import _plan

SEMANTICS = ("flat", "levels", "exact", "segment", "taylor")

# Matrix-core products of the moment scan (sta_moments): fp32 operands carried as bf16 hi + lo with three
# bf16 products each (about 2^-16 relative error per product; the moment sums agree with the fp32
# products to a few 1e-6 relative), or plain fp32 products (PRODUCTS_FP32).
MOMENT_PRODUCTS = _native.PRODUCTS_SPLIT_BF16
# Run the level / block compressor on a second stream (STA_OVERLAP_COMPRESS=1) instead of the caller's
# stream.  Off by default: the moment scan fills every compute unit's registers, so the compressor
# cannot run beside it, and a compressor launch that starts first delays the scan's workgroups
# (32 x 65536 tokens: 9.49 ms per prefill on two streams, 9.38 ms on one; 1 head: 0.618 / 0.609 ms).
OVERLAP_COMPRESS = os.environ.get("STA_OVERLAP_COMPRESS", "0") != "0"
# Levels plans: the level-0 compress calls also score their key rows for their ancestors' calls
# (sta_compress_nodes' ancestor scores), so the merges read 4 bytes per item instead of a key row.
# The nodes are the same bit for bit either way (STA_ANCESTOR_SCORES=0 keeps the gathers).
ANCESTOR_SCORES = os.environ.get("STA_ANCESTOR_SCORES", "1") != "0"
# levels scored that way (at most 4): each costs the level-0 calls one more fp64 chain per row, and pays
# where a level's gathers are large
ANCESTOR_LEVELS = int(os.environ.get("STA_ANCESTOR_LEVELS", "3"))
# only for key rows of at least this many bytes: a short row's gather costs the merges little, and the
# extra chains cost the level-0 calls more (1x32x65536, d = 64 fp32: 0.393 -> 0.375 ms; 4x32x16384,
# d = 16: 0.26 -> 0.30 ms)
ANCESTOR_MIN_ROW_BYTES = 256
# Levels plans: the merge levels as subtree launches (sta_compress_merges): a workgroup takes up to 16
# nodes of one level and the nodes above them, computing a level's nodes in steps with a barrier between
# (32 x 65536 tokens: 8 merge levels in 2 launches instead of 8).  "group": four 256-thread groups in
# lockstep, one node each per step; "wave": one wave per node, 16 waves; "auto": waves for compress calls
# of at most 128 items (a wave sorts them in a quarter of the work of 256), groups above
# (32 x 65536 tokens, 256-item calls: 9 launches 372-379 us, groups 355-372, waves 418-432;
# 4 x 32 x 16384, 128-item calls: 9 launches 258-261 us, groups 271-281, waves 238-250);
# "0": sta_compress_nodes level by level.  The nodes are the same bit for bit either way.  "auto" also
# keeps the level-by-level launches when the first subtree launch would have fewer workgroups than the
# device has compute units (few heads: a subtree's levels run one after another on a few units, where
# a level's own launch spreads its nodes over all of them; compressor of 1 x 65536 tokens 0.150 ->
# 0.119 ms, 16 x 65536 0.251 -> 0.230 ms; 32 x 65536 keeps the subtrees, 0.332 against 0.338 ms).
MERGE_LAUNCHES = os.environ.get("STA_MERGE_LAUNCHES", "auto")
MERGE_GROUPS = int(os.environ.get("STA_MERGE_GROUPS", "4"))  # 256-thread groups per workgroup
MERGE_BOTTOM = int(os.environ.get("STA_MERGE_BOTTOM", "16"))  # nodes of a subtree's lowest level

_side_streams: Dict[str, "torch.cuda.Stream"] = {}
_cu_counts: Dict[int, int] = {}


def _compute_units(dev: torch.device) -> int:
    """Compute units of the device (cached per device index)."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _cu_counts:
        _cu_counts[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return _cu_counts[idx]


def _side_stream(dev: torch.device) -> "torch.cuda.Stream":
    key = str(dev)
    with _dev_lock:
        st = _side_streams.get(key)
        if st is None:
            st = torch.cuda.Stream(device=dev)  # default priority
            _side_streams[key] = st
    return st


# The wave-specialised moment kernel (sta_moments_ws: update and query waves, 64 value columns per
# workgroup, the queries answered against the state before their article block) for split products at
# degree <= 3 whenever the article block is a whole number (>= 2) of moment chunks; sta_moments
# otherwise.  A/B on one MI355X in one session (moment scan / whole step):
#   1 x 32 heads x 65536, fp32, degree 2, block 256:    6.89 -> 6.38 ms / 9.75 -> 9.61 ms
#   8 x 16 heads x 4096, bf16, degree 2, block 256:     2.29 -> 1.68 ms / 3.41 -> 2.83 ms
#   4 x 32 heads x 16384, fp32, degree 3, block 128:    6.13 -> 4.28 ms / 7.88 -> 6.18 ms
# STA_MOMENT_WS=never / always overrides the choice (a prefill's moment_kernel argument too).
MOMENT_WS_POLICY = os.environ.get("STA_MOMENT_WS", "auto")  # "auto" | "always" | "never"
# Sequence segments of the wave-specialised scan when the heads alone leave compute units idle
# (STA_WS_SEGMENTS=0: never).
WS_SEGMENTS = os.environ.get("STA_WS_SEGMENTS", "1") != "0"


def use_moments_ws(element_size: int, degree: int) -> bool:
    return MOMENT_WS_POLICY not in ("never", "0")


def ws_query_block(semantics: str, block: int) -> Optional[int]:
    """Query block of sta_moments_ws for a prefill, or None for sta_moments: the article block where the
    residual kernel's in-block keys start at the block (flat, levels, segment), any block where every
    key is in the residual (exact)."""
    if semantics in ("flat", "levels", "segment"):
        return block if block % 32 == 0 and block >= 64 else None
    if semantics == "exact":
        return 256
    return None  # raw Taylor sums: the residual kernel adds the polynomial over the query block's keys


# Offer the planner the 64-column moment workgroups (split products, 32 < dv <= 64).  Off: on 32 heads x
# 65536 tokens (d = dv = 64) they take 9.6 ms against 8.4 ms for two 32-column workgroups per compute
# unit; the feature work they save (17 % of the VALU) is less than one wave per SIMD loses in latency.
MOMENT_WIDE = False

# The same choice for the residual / combine kernel (sta_block_attention): logits and weighted value sums,
# when coreset items take part.  Without them (compressor "none", the raw Taylor sums, or sequences no
# longer than a block) the result is exact attention and keeps fp32 products: the reference holds those
# cases to 2e-6 / 3e-6 of softmax attention (test_fast_article_attention.py:10-29,
# test_streaming_attention.py:10-21), which split products in this kernel exceed (about 5e-6).
RESIDUAL_PRODUCTS = _native.PRODUCTS_SPLIT_BF16
EXACT_SEMANTICS = ("exact", "taylor")

_dev_lock = threading.Lock()
_dev_cache: Dict[tuple, object] = {}


def _on_device(key: tuple, device: torch.device, build: Callable[[], object]):
    full = key + (str(device),)
    with _dev_lock:
        hit = _dev_cache.get(full)
    if hit is not None:
        return hit
    val = build()
    with _dev_lock:
        if len(_dev_cache) > 128:
            _dev_cache.clear()
        _dev_cache[full] = val
    return val


def _i32(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(device)


def _f32(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)


def _unit_width(width: int, element_size: int) -> int:
    """Smallest row length >= width that is a whole number of 16-byte units."""
    per_unit = 16 // element_size
    return -(-width // per_unit) * per_unit


STAGED_D = 128  # key dimensions the moment kernels stage whole; wider keys go through dimension windows
MAX_D_HIGH_DEGREE = 64  # degree 5 .. 8


def check_kernel_limits(d: int, degree: int) -> None:
    """The HIP kernels' key width and degree limits (sta_limits), with the reference's exception types:
    ValueError for the key width, NotImplementedError for the degree."""
    lim = _native.limits()
    if d > lim["max_d"]:
        raise ValueError(f"the HIP kernels support D <= {lim['max_d']}")
    if degree > lim["max_degree"]:
        raise NotImplementedError(f"the HIP kernels support Taylor degree <= {lim['max_degree']}")
    if degree >= 5 and d > MAX_D_HIGH_DEGREE:
        raise NotImplementedError(f"the HIP kernels support Taylor degree >= 5 for D <= {MAX_D_HIGH_DEGREE}")
    if degree >= 4 and d > STAGED_D:
        raise NotImplementedError(f"the HIP kernels support Taylor degree 4 for D <= {STAGED_D}")


def _padded_rows(t: torch.Tensor, width: int) -> torch.Tensor:
    """t itself when its rows already have `width` elements and it is 16-byte aligned, else a copy
    zero-padded to `width` columns."""
    if t.shape[-1] == width and t.data_ptr() % 16 == 0:
        return t
    out = torch.zeros(t.shape[:-1] + (width,), device=t.device, dtype=t.dtype)
    out[..., : t.shape[-1]] = t
    return out


class KernelTimer:
    """Records HIP events around each launch on the launch stream (for measured per-kernel times).
    `only`: the launch names to time (None: all); the others run without events (each timed launch
    adds a pair of event records to the stream, a few microseconds of GPU time)."""

    def __init__(self, only: Optional[Tuple[str, ...]] = None) -> None:
        self.events: Dict[str, list] = {}
        self.only = None if only is None else frozenset(only)

    def wrap(self, name: str, fn: Callable[[], None]) -> None:
        if self.only is not None and name not in self.only:
            fn()
            return
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        self.events.setdefault(name, []).append((s, e))

    def totals_ms(self) -> Dict[str, Tuple[float, int]]:
        torch.cuda.synchronize()
        out = {}
        for name, evs in self.events.items():
            out[name] = (sum(s.elapsed_time(e) for s, e in evs), len(evs))
        return out


def _run(timer: Optional[KernelTimer], name: str, fn: Callable[[], None]) -> None:
    if timer is None:
        fn()
    else:
        timer.wrap(name, fn)


@dataclass
class PrefillResult:
    out: torch.Tensor
    node_src: Optional[torch.Tensor]
    node_w: Optional[torch.Tensor]
    plan: _plan.NodePlan
    feature_count: int
    fsplit: int
    den: Optional[torch.Tensor] = None  # raw denominator (semantics "taylor")
    moment_kernel: str = ""  # the moment-scan kernel that ran: "moments_ws_kernel" or "moments_kernel"


def prefill(
    q3: torch.Tensor,
    k3: torch.Tensor,
    v3: torch.Tensor,
    *,
    degree: int,
    block: int,
    scale: float,
    semantics: str,
    compressor: str = "sorted_pair",
    seed: int = 0,
    eps: float = 1e-12,
    out_dtype: torch.dtype = torch.float32,
    stride: int = 1,
    exp_clamp: bool = False,
    draws: Optional[_plan.Draws] = None,
    timer: Optional[KernelTimer] = None,
    products: Optional[int] = None,
    residual_products: Optional[int] = None,
    moment_kernel: Optional[str] = None,
    score_keys: Optional[torch.Tensor] = None,
    reference_keys: Optional[torch.Tensor] = None,
) -> PrefillResult:
    """Run the whole prefill for contiguous [BH, N, D] device tensors of one dtype.  moment_kernel:
    "ws" (sta_moments_ws where it applies), "chunked" (sta_moments) or None (use_moments_ws).
    score_keys: the float64 keys of a float64 caller ([BH, N, D], contiguous, on the device; k3 is
    their float32 rounding): the compressor then draws its directions and uniforms as float64 and
    scores these keys in fp64, as the reference's float64 run does.
    reference_keys: the caller's keys in their own dtype as a contiguous CPU [BH, N, D] tensor: the
    compress calls then run on the host in the reference's own score order (torch's CPU
    `keys @ direction` and argsort, _plan.reference_selection) instead of the HIP compressor."""
    if semantics not in SEMANTICS:
        raise ValueError(f"semantics must be one of {SEMANTICS}")
    for t in (q3, k3, v3):
        _native.require_device(t)
    if not (q3.dtype == k3.dtype == v3.dtype) or q3.dtype not in _native.DTYPE_CODES:
        raise ValueError("q, k, v must share one of the dtypes float32, bfloat16, float16")
    lib = _native.lib()
    dev = q3.device
    bh, n, d = q3.shape
    dv = v3.shape[-1]
    lim = _native.limits()
    if score_keys is not None:
        _native.require_device(score_keys)
        if score_keys.dtype != torch.float64 or tuple(score_keys.shape) != (bh, n, d) or \
                not score_keys.is_contiguous():
            raise ValueError("score_keys must be the contiguous float64 [BH, N, D] keys")
    if reference_keys is not None:
        if reference_keys.device.type != "cpu" or not reference_keys.is_contiguous() or \
                tuple(reference_keys.shape) != (bh, n, d) or reference_keys.dtype not in _native.DRAW_TYPES:
            raise ValueError("reference_keys must be the caller's contiguous CPU [BH, N, D] keys")
        if draws is not None:
            raise ValueError("reference_keys take the draws of their own dtype; explicit draws do not apply")
    check_kernel_limits(d, degree)
    if dv > lim["max_dv"]:
        # value columns are independent given the keys (the denominator and the coreset selections do
        # not depend on v): wide values run as column groups of at most max_dv, every group recomputing
        # the same denominator and selections
        parts = [prefill(q3, k3, v3[..., c0: c0 + lim["max_dv"]].contiguous(), degree=degree, block=block,
                         scale=scale, semantics=semantics, compressor=compressor, seed=seed, eps=eps,
                         out_dtype=out_dtype, stride=stride, exp_clamp=exp_clamp, draws=draws, timer=timer,
                         products=products, residual_products=residual_products, moment_kernel=moment_kernel,
                         score_keys=score_keys, reference_keys=reference_keys)
                 for c0 in range(0, dv, lim["max_dv"])]
        first = parts[0]
        return PrefillResult(torch.cat([r.out for r in parts], dim=-1), first.node_src, first.node_w, first.plan,
                             first.feature_count, first.fsplit, first.den, first.moment_kernel)
    if semantics == "segment" and q3.dtype != torch.float32:
        # segment means are fp32 and the residual kernel reads them with the inputs in one format
        q3, k3, v3 = q3.float(), k3.float(), v3.float()
    dt = _native.DTYPE_CODES[q3.dtype]
    odt = _native.DTYPE_CODES[out_dtype]
    stream = _native.stream_handle(dev)
    chunk = _plan.moment_chunk(d)

    raw = semantics == "taylor"
    if semantics in ("exact", "taylor"):
        plan = _plan.exact_plan(n)
    elif semantics == "flat":
        plan = _plan.flat_plan(n, block, compressor)
    elif semantics == "levels":
        plan = _plan.levels_plan(n, block, compressor)
    else:
        plan, n_rep, _rpb = _plan.segment_plan(n, block, stride)
    shift = plan.shift
    mode = _plan.MODE_TAYLOR if raw else plan.mode
    if plan.call_sizes and max(plan.call_sizes) > lim["max_compress_in"]:
        raise ValueError(f"block_size {block} needs compress calls on {max(plan.call_sizes)} items; "
                         f"the HIP compressor handles at most {lim['max_compress_in']}")

    # the moment kernel reads rows in 16-byte units: q/k padded with zero dimensions to a whole unit
    # (zero dimensions only add zero-valued features), v to whole 32-column groups; keys wider than the
    # 128 staged dimensions to whole 32-dimension window blocks
    windowed = d > STAGED_D
    dm = -(-d // _plan.WINDOW_BLOCK) * _plan.WINDOW_BLOCK if windowed else _unit_width(d, q3.element_size())
    wt = _plan.window_tiles(dm, degree) if windowed else None
    ft = _plan.window_feature_tiles(wt) if windowed else _plan.feature_tiles(dm, degree)
    k1_products = MOMENT_PRODUCTS if products is None else int(products)
    if degree >= 5:
        k1_products = _native.PRODUCTS_FP32  # the degree 5 .. 8 scan runs fp32 products
    qblock = ws_query_block(semantics, block) if (k1_products == _native.PRODUCTS_SPLIT_BF16 and degree <= 3 and
                                                  not windowed and
                                                  (use_moments_ws(q3.element_size(), degree) if moment_kernel is None
                                                   else moment_kernel == "ws")) else None
    ws_ct = 4 if (-(-dv // 32)) % 2 == 0 else 2
    ws_opts = _native.moment_ws_slot_tiles(dm, degree, ws_ct, dv) if qblock else ()
    nseg, seg_blocks = 1, 0
    if ws_opts:
        # few heads: cut each head's scan into segments of whole query blocks (sta_moments_ws_seg)
        nseg, seg_blocks = _plan.ws_segments(n, shift, qblock, bh, ft, dv, ws_opts, ws_ct) if WS_SEGMENTS else (1, 0)
        ms = _plan.moment_split_ws(ft, bh * nseg, dv, ws_opts, ws_ct)
        chunk = qblock
    elif windowed:
        qblock = None
        ms = _plan.moment_split_windows(wt, bh, dv, _native.moment_wave_tile_options(STAGED_D, degree))
    else:
        qblock = None
        ms = _plan.moment_split(ft, bh, dv, _native.moment_wave_tile_options(dm, degree),
                                mixed_nts=_native.moment_mixed_tiles(dm, degree),
                                wide_nts=_native.moment_wide_tiles(dm, degree, dv, k1_products) if MOMENT_WIDE else ())
    fsplit = ms.fsplit
    # split products at degree <= 2 apply one coefficient per tile on the query side
    tile_coef = k1_products == _native.PRODUCTS_SPLIT_BF16 and degree <= 2
    fidx, fcoef, fwin = _on_device(
        ("mtable", dm, degree, bh, dv, ms.mixed, ms.wave_tiles, ms.fsplit, tile_coef, ms.columns, qblock is not None),
        dev,
        lambda: (_i32(ms.quads, dev),
                 _f32(_plan.tile_coefficients(ms.quads, ms.coef, ft.d) if tile_coef else ms.coef, dev),
                 _i32(ms.win, dev) if ms.win is not None else None))

    # ---- host side first: every validation error is raised before anything is launched ----
    pkey = (plan.mode, plan.n, plan.block, compressor if semantics != "segment" else stride)
    meta_d, tptr_d, tnodes_d = _on_device(
        ("plan",) + pkey, dev,
        lambda: (_i32(plan.meta, dev), _i32(plan.tile_ptr, dev), _i32(np.maximum(plan.tile_nodes, 0) if plan.tile_nodes.size else np.zeros(1, np.int32), dev)),
    )
    f64 = score_keys is not None
    host_select = reference_keys is not None and semantics in ("flat", "levels") and bool(plan.batches)
    if host_select:
        # every compress call on the host, in the reference's score order; the tables go up like an input
        src_np, w_np = _plan.reference_selection(plan, _plan.sequence_seeds(seed, bh), reference_keys, compressor)
        host_nodes = (torch.from_numpy(src_np).to(dev), torch.from_numpy(w_np).to(dev))
    if semantics != "segment" and plan.batches and not host_select:
        seeds = _plan.sequence_seeds(seed, bh)
        fdraw = (lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float64)).to(dev)) if f64 else \
            (lambda a: _f32(a, dev))
        if draws is None:
            dr, desc = _plan.draws_for(plan, seeds, d, compressor, f64)
            dirs_d, unif_d, perms_d, desc_d = _on_device(
                ("draws",) + pkey + (seeds, d, f64), dev,
                lambda: (fdraw(dr.dirs), fdraw(dr.unif), _i32(dr.perms, dev), _i32(desc, dev)),
            )
        else:
            dr = draws
            n_calls = max(len(plan.call_sizes), 1)
            need = max(plan.call_sizes)
            if (dr.dirs.shape != (bh, n_calls, d) or dr.max_in < need or dr.unif.shape != (bh, n_calls, dr.max_in // 2)
                    or dr.perms.shape != (bh, n_calls, dr.max_in)):
                raise ValueError("explicit draws do not match the compress-call layout of this configuration")
            if (dr.dirs.dtype == np.float64) != f64:
                raise ValueError("explicit draws must be float64 exactly when score_keys are given")
            _, desc = _plan.draws_for(plan, seeds[:1], d, compressor)
            dirs_d, unif_d, perms_d, desc_d = (fdraw(dr.dirs), fdraw(dr.unif), _i32(dr.perms, dev), _i32(desc, dev))
        batches_d = _on_device(("batches",) + pkey, dev, lambda: [_i32(b, dev) for b in plan.batches])
        # levels: the level-0 calls also score their rows for their ancestors' calls, which then read
        # one score per item instead of gathering key rows (float64 scoring keeps the gathers)
        anc_levels, anc_d, level_d = 0, None, None
        if ANCESTOR_SCORES and not f64 and d * k3.element_size() >= ANCESTOR_MIN_ROW_BYTES:
            anc_levels, level_of, anc = _plan.ancestor_table(plan, desc, ANCESTOR_LEVELS)
            if anc_levels:
                anc_d, level_d = _on_device(("anc", anc_levels) + pkey, dev,
                                            lambda: (_i32(anc, dev), _i32(level_of, dev)))
        merge_l = []
        if MERGE_LAUNCHES in ("group", "wave", "auto") and plan.mode == _plan.MODE_LEVELS:
            wave = MERGE_LAUNCHES == "wave" or (MERGE_LAUNCHES == "auto" and dr.max_in <= 128)
            gt = 64 if wave else 256

            def build_merges():
                launches = _plan.merge_launches(plan, dr.max_in, f64, group_threads=gt, groups=MERGE_GROUPS,
                                                bottom=MERGE_BOTTOM)
                _plan.check_merge_launches(plan, desc, launches)
                return [(ln, _i32(ln.table, dev)) for ln in launches]

            merge_l = _on_device(("merges", gt, MERGE_GROUPS, MERGE_BOTTOM, dr.max_in, f64) + pkey, dev, build_merges)
            if MERGE_LAUNCHES == "auto" and merge_l and merge_l[0][0].workgroups * bh < _compute_units(dev):
                merge_l = []

    lrows, lld, _ = _native.moment_partials_layout(n, dv)
    low_num = torch.empty((bh, fsplit, lrows, lld), device=dev, dtype=torch.float32)
    low_den = torch.empty((bh, fsplit, lrows), device=dev, dtype=torch.float32)

    mq, mk, mv = _padded_rows(q3, dm), _padded_rows(k3, dm), _padded_rows(v3, -(-dv // 32) * 32)

    if qblock is not None:
        hbytes = lib.sta_moments_ws_handoff_bytes(bh * nseg, fsplit, ms.wave_tiles, ws_ct, dv)
        handoff = torch.empty((max(hbytes, 16) // 4,), device=dev, dtype=torch.float32)
        seg_state = (torch.empty((lib.sta_moments_ws_seg_bytes(bh, fsplit, ms.wave_tiles, ws_ct, dv, nseg) // 4,),
                                 device=dev, dtype=torch.float32) if nseg > 1 else None)

        def k1():
            st = lib.sta_moments_ws_seg(
                mq.data_ptr(), mk.data_ptr(), mv.data_ptr(), dt, bh, n, dm, dv, mv.shape[-1], degree,
                float(scale), qblock, shift, fsplit, ms.wave_tiles, int(ms.mixed), ws_ct,
                fidx.data_ptr(), fcoef.data_ptr(), handoff.data_ptr(), low_num.data_ptr(), low_den.data_ptr(),
                nseg, seg_blocks, _native.ptr(seg_state), stream)
            _native.check(st, "sta_moments_ws_seg")
    else:
        def k1():
            st = lib.sta_moments(
                mq.data_ptr(), mk.data_ptr(), mv.data_ptr(), dt, bh, n, ft.d, dm, dv, mv.shape[-1], degree,
                float(scale), chunk, shift,
                fsplit, ms.wave_tiles, int(ms.mixed), k1_products, ms.columns,
                fidx.data_ptr(), fcoef.data_ptr(), _native.ptr(fwin), low_num.data_ptr(), low_den.data_ptr(),
                stream)
            _native.check(st, "sta_moments")

    # The compressor needs only the keys and the draws: with OVERLAP_COMPRESS it goes on a second stream
    # (default priority), released before the moment scan is queued.
    main = torch.cuda.current_stream(dev)
    side = _side_stream(dev) if (OVERLAP_COMPRESS and semantics != "segment" and plan.batches and
                                 not host_select) else main
    if side is not main:
        side.wait_stream(main)

    _run(timer, "moments", k1)

    node_src = node_w = None
    rep_k = rep_v = None
    n_rep_arg = 0
    if semantics == "segment":
        n_rep_arg = n_rep
        if n_rep > 0:
            rep_k = torch.empty((bh, n_rep, d), device=dev, dtype=torch.float32)
            rep_v = torch.empty((bh, n_rep, dv), device=dev, dtype=torch.float32)

            def k_seg():
                st = lib.sta_segment_mean(k3.data_ptr(), v3.data_ptr(), dt, bh, n, d, dv, block, stride, n_rep,
                                          rep_k.data_ptr(), rep_v.data_ptr(), stream)
                _native.check(st, "sta_segment_mean")

            _run(timer, "segment_mean", k_seg)
            rep_k, rep_v = _padded_rows(rep_k, -(-d // 4) * 4), _padded_rows(rep_v, -(-dv // 4) * 4)
            rpb = block // stride
            src_np = np.arange(plan.n_nodes * plan.cap, dtype=np.int32).reshape(plan.n_nodes, plan.cap)
            src_np = np.where(src_np < n_rep, src_np, 0).astype(np.int32)
            node_src, node_w = _on_device(
                ("segnodes", n, block, stride, bh), dev,
                lambda: (_i32(np.broadcast_to(src_np, (bh,) + src_np.shape).copy(), dev),
                         torch.full((bh, plan.n_nodes, plan.cap), float(stride), device=dev, dtype=torch.float32)),
            )
            del rpb
    elif host_select:
        node_src, node_w = host_nodes
    elif plan.batches:
        node_src = torch.empty((bh, plan.n_nodes, plan.cap), device=dev, dtype=torch.int32)
        node_w = torch.empty((bh, plan.n_nodes, plan.cap), device=dev, dtype=torch.float32)
        lscore = torch.empty((bh, anc_levels, n), device=dev, dtype=torch.float32) if anc_levels else None
        if side is not main:
            node_src.record_stream(side)
            node_w.record_stream(side)
            if lscore is not None:
                lscore.record_stream(side)
        with torch.cuda.stream(side):
            k3_stream = _native.stream_handle(dev)
            # with merge launches: the level-0 batch alone, then the subtrees
            for bi, bd in enumerate(batches_d[:1] if merge_l else batches_d):
                def k3_launch(bd=bd, first=bi == 0):
                    st = lib.sta_compress_nodes(
                        (score_keys if f64 else k3).data_ptr(), _native.STA_F64 if f64 else dt, bh, n, d,
                        bd.data_ptr(), int(bd.numel()), desc_d.data_ptr(),
                        plan.n_nodes, plan.cap, dirs_d.data_ptr(), unif_d.data_ptr(), perms_d.data_ptr(),
                        dr.dirs.shape[1], dr.max_in, node_src.data_ptr(), node_w.data_ptr(),
                        _native.ptr(level_d), _native.ptr(anc_d) if first else None, anc_levels,
                        _native.ptr(lscore), k3_stream)
                    _native.check(st, "sta_compress_nodes")

                _run(timer, "compress", k3_launch)
            for ln, table_d in merge_l:
                def k3_merges(ln=ln, table_d=table_d):
                    st = lib.sta_compress_merges(
                        (score_keys if f64 else k3).data_ptr(), _native.STA_F64 if f64 else dt, bh, n, d,
                        table_d.data_ptr(), ln.workgroups, ln.steps, ln.groups, ln.group_threads, desc_d.data_ptr(),
                        plan.n_nodes, plan.cap, dirs_d.data_ptr(), unif_d.data_ptr(), perms_d.data_ptr(),
                        dr.dirs.shape[1], dr.max_in, node_src.data_ptr(), node_w.data_ptr(),
                        _native.ptr(level_d), anc_levels, _native.ptr(lscore), k3_stream)
                    _native.check(st, "sta_compress_merges")

                _run(timer, "compress", k3_merges)
        if side is not main:
            main.wait_stream(side)

    if raw:
        out = torch.empty((bh, n, dv), device=dev, dtype=torch.float32)
        out_den = torch.empty((bh, n), device=dev, dtype=torch.float32)
    else:
        out = torch.empty((bh, n, dv), device=dev, dtype=out_dtype)
        out_den = None
    n_nodes_arg = plan.n_nodes if (node_src is not None) else 0

    if residual_products is not None:
        k2_products = int(residual_products)
    elif semantics in EXACT_SEMANTICS or (n_nodes_arg == 0 and n_rep_arg == 0) or degree > 3:
        # no coreset item (the result is exact attention), or degree >= 4 (the fp32-product kernel's Taylor)
        k2_products = _native.PRODUCTS_FP32
    else:
        k2_products = RESIDUAL_PRODUCTS

    def k24():
        st = lib.sta_block_attention(
            mq.data_ptr(), mk.data_ptr(), mv.data_ptr(), dt, bh, n, d, dv, dm, mv.shape[-1], degree, float(scale),
            float(eps), mode, block, chunk, shift, 1 if exp_clamp else 0,
            k2_products, low_num.data_ptr(), low_den.data_ptr(),
            fsplit, tptr_d.data_ptr(), tnodes_d.data_ptr(), plan.n_tiles, meta_d.data_ptr(), n_nodes_arg, plan.cap,
            _native.ptr(node_src), _native.ptr(node_w), _native.ptr(rep_k), _native.ptr(rep_v),
            rep_k.shape[-1] if rep_k is not None else 0, rep_v.shape[-1] if rep_v is not None else 0, n_rep_arg,
            out.data_ptr(), odt, _native.ptr(out_den), stream)
        _native.check(st, "sta_block_attention")

    _run(timer, "block_attention", k24)
    return PrefillResult(out, node_src, node_w, plan, ft.count, fsplit, out_den,
                         "moments_ws_kernel" if qblock is not None else "moments_kernel")


def flash(q3: torch.Tensor, k3: torch.Tensor, v3: torch.Tensor, *, scale: float,
          out_dtype: torch.dtype = torch.float32, timer: Optional[KernelTimer] = None) -> torch.Tensor:
    """Exact causal softmax attention of contiguous [BH, N, D] device tensors of one dtype
    (sta_flash_attention); rows are zero-padded to whole 4-element units when D or Dv is not."""
    for t in (q3, k3, v3):
        _native.require_device(t)
    if not (q3.dtype == k3.dtype == v3.dtype) or q3.dtype not in _native.DTYPE_CODES:
        raise ValueError("q, k, v must share one of the dtypes float32, bfloat16, float16")
    bh, n, d = q3.shape
    dv = v3.shape[-1]
    odt = out_dtype if out_dtype in _native.DTYPE_CODES else torch.float32
    out = torch.empty((bh, n, dv), device=q3.device, dtype=odt)
    if bh == 0 or n == 0:
        return out.to(out_dtype)
    dq, dvp = -(-d // 4) * 4, -(-dv // 4) * 4
    mq, mk, mv = _padded_rows(q3, dq), _padded_rows(k3, dq), _padded_rows(v3, dvp)
    lib = _native.lib()

    def launch():
        st = lib.sta_flash_attention(mq.data_ptr(), mk.data_ptr(), mv.data_ptr(), _native.DTYPE_CODES[q3.dtype],
                                     bh, n, d, dv, dq, dvp, float(scale), out.data_ptr(), _native.DTYPE_CODES[odt],
                                     _native.stream_handle(q3.device))
        _native.check(st, "sta_flash_attention")

    _run(timer, "flash", launch)
    return out if odt == out_dtype else out.to(out_dtype)
