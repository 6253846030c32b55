"""Batched streaming decode state on one ROCm device: S independent streams (stream s seeded seed + s)
advancing in lockstep, the state of the reference's ArticleStreamingAttention
(streaming_taylor_coreset_attention.py:523-616) for each of them.

Device state (fp32, see csrc/decode.hip):
  state_num [S, F, ldv], state_den [S, F]   moments of the tokens of completed blocks, reference order
  buf_k [S, cap, dk], buf_v [S, cap, ldv]   the tokens of the current block (cap = block; for
                                            compressor "none" every token, cap grows)
  lev_k [S, L, m, dk], lev_v [S, L, m, ldv], lev_w [S, L, m], lev_pos [S, L, m]   level coresets
Host state: length (tokens per stream), blocks (completed blocks = the level-occupancy counter),
buf_len, and one torch CPU generator per stream that the compress calls draw from in the reference's
order (randn(d) + rand(n//2) per sorted_pair call, randperm(n) for n <= 2 or "random").

A float64 stream (score_f64) also keeps the float64 values of the buffered and level key rows
(buf_k64 [S, cap, dk], lev_k64 [S, L, m, dk]) and draws its directions and uniforms as float64: its
compress calls score and select as the reference's float64 run does; every other computation reads the
float32 rows.

Per decode step (update then query of one token per stream): sta_decode_moments (state read) and
sta_decode_tail (append + buffer / level items + combine).  When the token completes a block:
sta_moment_accumulate (buffer -> state) and sta_decode_compress (buffer -> level 0 and the merge
cascade), then the query.
"""

from __future__ import annotations

import os
from collections import deque
from dataclasses import dataclass
from typing import Deque, Dict, List, Optional, Tuple

import numpy as np
import torch

import _engine
import _native
import _plan

M_SORTED_PAIR, M_PERM = _plan.METHOD_SORTED_PAIR, _plan.METHOD_PERM


@dataclass
class _CompletionDraws:
    blocks_before: int
    n_calls: int
    methods: torch.Tensor  # int32 [n_calls]
    dirs: torch.Tensor  # float32 [S, n_calls, d] (float64 for a float64 stream)
    unif: torch.Tensor  # float32 [S, n_calls, max_in // 2] (likewise)
    perms: torch.Tensor  # int32 [S, n_calls, max_in]


ACCUMULATE_PRODUCTS = _native.PRODUCTS_SPLIT_BF16
# block completions and extend() on the wave-specialised kernel's update-only pass where it applies
# (split products, degree <= 3, d <= 128); STA_ACCUMULATE_WS=0 keeps the chunked accumulation kernel
ACCUMULATE_WS = os.environ.get("STA_ACCUMULATE_WS", "1") != "0"
ACCUMULATE_WS_MIN_ROWS = 512
# Shorter runs of rows (a block completion) through the block accumulation (sta_moment_accumulate_block:
# the rows staged once per workgroup, every feature slice of the state run through them with the next
# slice's loads in flight; split products, degree <= 2, d <= 64) with this many tiles per wave;
# STA_ACCUMULATE_BLOCK=0 keeps the chunked kernel (the state is the same bit for bit).
ACCUMULATE_BLOCK = os.environ.get("STA_ACCUMULATE_BLOCK", "1") != "0"
ACCUMULATE_BLOCK_TILES = int(os.environ.get("STA_ACCUMULATE_BLOCK_TILES", "2"))
# value columns per workgroup: 64 (every key feature generated once per stream) where the state's rows
# are whole groups of 64, else 32
ACCUMULATE_BLOCK_COLUMNS = int(os.environ.get("STA_ACCUMULATE_BLOCK_COLUMNS", "64"))


class StaticScratchOwners:
    """Who uses each device's static scratch (sta_decode_step_static keeps the moment partials in one
    library array per device, so calls that overlap on a device overwrite each other's partials).  A
    decode state claims its device's scratch for one stream at its first allocation-free step; a call
    from another state, or from the same state on another stream, is refused until the owner releases
    it (which first waits for the owner's stream, so the owner's last call has finished)."""

    def __init__(self) -> None:
        self._owner: Dict[int, Tuple[int, int]] = {}  # device index -> (owner id, stream handle)

    def claim(self, device: int, owner: int, stream: int) -> None:
        held = self._owner.get(device)
        if held is not None and held != (owner, stream):
            what = "another decode state" if held[0] != owner else f"this decode state on another stream ({held[1]:#x})"
            raise ValueError(f"the static scratch of device {device} is in use by {what}; calls that overlap on "
                             f"one device would overwrite each other's partials: release_static() the owner first")
        self._owner[device] = (owner, stream)

    def release(self, device: int, owner: int) -> bool:
        """Drops `owner`'s claim on `device`; True when it held one."""
        if self._owner.get(device, (None,))[0] == owner:
            del self._owner[device]
            return True
        return False

    def holder(self, device: int) -> Optional[Tuple[int, int]]:
        return self._owner.get(device)


STATIC_OWNERS = StaticScratchOwners()


class DecodeState:
    def __init__(self, streams: int, dim: int, value_dim: int, *, degree: int, block: int, scale: float,
                 compressor: str, seed: int, device: torch.device, eps: float = 1e-12,
                 score_f64: bool = False) -> None:
        if streams <= 0:
            raise ValueError("streams must be positive")
        if dim <= 0 or value_dim <= 0:
            raise ValueError("dim and value_dim must be positive")
        if block < 2:
            raise ValueError("block_size must be at least 2")
        lim = _native.limits()
        if value_dim > lim["max_dv"]:
            raise ValueError(f"the HIP decode kernels support Dv <= {lim['max_dv']}")
        if degree < 0:
            raise ValueError("degree must be non-negative")
        _engine.check_kernel_limits(dim, degree)
        if device.type != "cuda":
            raise ValueError("the HIP decode state lives on a ROCm GPU device")
        self.S, self.d, self.dv = int(streams), int(dim), int(value_dim)
        self.degree, self.block, self.scale = int(degree), int(block), float(scale)
        self.compressor, self.seed, self.eps = str(compressor), int(seed), float(eps)
        self.device = device
        self._dev_index = device.index if device.index is not None else torch.cuda.current_device()
        self.exact = self.compressor == "none"
        # matrix-core products of the state accumulation (block completions, extend): split-bf16 as in the
        # prefill moment scan (the state and every sum stay fp32); fp32 products at degree 5 .. 8
        self.products = ACCUMULATE_PRODUCTS if self.degree <= 4 else _native.PRODUCTS_FP32
        self.m = (self.block + 1) // 2
        if not self.exact and max(self.block, 2 * self.m) > lim["max_compress_in"]:
            raise ValueError(f"block_size {block} exceeds the HIP compressor's {lim['max_compress_in']} items")
        self.dk, self.ldv = _native.decode_layout(self.d, self.dv)
        self.F = _plan.num_features(self.d, self.degree)
        self.lib = _native.lib()

        dev, S = device, self.S
        f32 = dict(device=dev, dtype=torch.float32)
        self.state_num = torch.zeros((S, self.F, self.ldv), **f32)
        self.state_den = torch.zeros((S, self.F), **f32)
        self.cap = self.block
        self.buf_k = torch.zeros((S, self.cap, self.dk), **f32)
        self.buf_v = torch.zeros((S, self.cap, self.ldv), **f32)
        self.L = 0
        self.lev_k = torch.zeros((S, 1, 1, self.dk), **f32)
        self.lev_v = torch.zeros((S, 1, 1, self.ldv), **f32)
        self.lev_w = torch.zeros((S, 1, 1), **f32)
        self.lev_pos = torch.zeros((S, 1, 1), device=dev, dtype=torch.int32)
        # float64 key rows of a float64 stream (the compressor's scores); none for compressor "none"
        self.score_f64 = bool(score_f64) and not self.exact
        f64 = dict(device=dev, dtype=torch.float64)
        self.buf_k64 = torch.zeros((S, self.cap, self.dk), **f64) if self.score_f64 else None
        self.lev_k64 = torch.zeros((S, 1, 1, self.dk), **f64) if self.score_f64 else None
        self.length = 0
        self.blocks = 0
        self.buf_len = 0
        self.num_compressions = 0
        # stream s draws from its own CPU generator seeded seed + s, continued block after block
        self._gens = _native.DrawSet([self.seed + s for s in range(S)])
        self._draws: Deque[_CompletionDraws] = deque()

        # moment query: feature factors in reference order, splits to fill the GPU
        self.findex_width = _plan.feature_index_width(self.d, self.degree)
        fi = _plan.feature_index(self.d, self.degree)
        self.findex = torch.from_numpy(fi.view(np.int32) if fi.dtype == np.uint32 else fi.view(np.int16)).to(dev)
        self.splits = max(1, min(-(-2048 // S), self.F // 64 if self.F >= 64 else 1))
        self.part_num = torch.zeros((S, self.splits, self.ldv), **f32)
        self.part_den = torch.zeros((S, self.splits), **f32)
        self._acc_tables: Dict[int, tuple] = {}
        self.timer = None  # optional _engine.KernelTimer: HIP events around every launch

    def _launch(self, name: str, fn) -> None:
        if self.timer is None:
            fn()
        else:
            self.timer.wrap(name, fn)

    # ------------------------------------------------------------------ helpers
    def _stream(self) -> int:
        return _native.stream_handle(self.device)

    def _acc_table(self, width: int):
        """Moment-accumulate tables for rows `width` elements long: (split, quads, coef, rows, windows,
        staged width); keys wider than the 128 staged dimensions through dimension windows."""
        if width not in self._acc_tables:
            if width > _engine.STAGED_D:
                wt = _plan.window_tiles(width, self.degree)
                ft = _plan.window_feature_tiles(wt)
                ms = _plan.moment_split_windows(wt, self.S, self.dv,
                                                _native.moment_wave_tile_options(_engine.STAGED_D, self.degree))
            else:
                ft = _plan.feature_tiles(width, self.degree)
                ms = _plan.moment_split(ft, self.S, self.dv, _native.moment_wave_tile_options(width, self.degree))
            rows = _plan.split_state_rows(ft, ms, self.d)
            dev = self.device
            self._acc_tables[width] = (
                ms,
                torch.from_numpy(ms.quads.view(np.int32)).to(dev),
                torch.from_numpy(ms.coef).to(dev),
                torch.from_numpy(rows).to(dev),
                torch.from_numpy(ms.win).to(dev) if ms.win is not None else None,
                ft.d,
            )
        return self._acc_tables[width]

    def _acc_table_ws(self, width: int):
        """Tables of the wave-specialised accumulation (sta_moment_accumulate_ws) for rows `width` elements
        long, or None where it does not apply (fp32 products, degree >= 4, keys wider than the staged
        128 dimensions): (split, column tiles, quads, coef, rows)."""
        key = ("ws", width)
        if key not in self._acc_tables:
            entry = None
            ct = 4 if (-(-self.dv // 32)) % 2 == 0 else 2
            if (ACCUMULATE_WS and self.products == _native.PRODUCTS_SPLIT_BF16 and self.degree <= 3
                    and width <= _engine.STAGED_D):
                opts = _native.moment_ws_slot_tiles(width, self.degree, ct, self.dv)
                if opts:
                    ft = _plan.feature_tiles(width, self.degree)
                    ms = _plan.moment_split_ws(ft, self.S, self.dv, opts, ct)
                    rows = _plan.split_state_rows(ft, ms, self.d)
                    dev = self.device
                    entry = (ms, ct, torch.from_numpy(ms.quads.view(np.int32)).to(dev),
                             torch.from_numpy(ms.coef).to(dev), torch.from_numpy(rows).to(dev))
            self._acc_tables[key] = entry
        return self._acc_tables[key]

    def _block_column_tiles(self) -> int:
        ldo = 32 * (-(-self.dv // 32))
        return 4 if ACCUMULATE_BLOCK_COLUMNS == 64 and ldo % 64 == 0 and ACCUMULATE_BLOCK_TILES == 2 else 2

    def _acc_table_block(self, width: int):
        """Tables of the block accumulation (sta_moment_accumulate_block) for rows `width` elements long
        (the chunked kernel's table layout at ACCUMULATE_BLOCK_TILES tiles per wave), or None where it
        does not apply: (split, quads, coef, rows)."""
        key = ("block", width, ACCUMULATE_BLOCK_TILES)
        if key not in self._acc_tables:
            entry = None
            if (ACCUMULATE_BLOCK and self.products == _native.PRODUCTS_SPLIT_BF16 and self.degree <= 2
                    and width <= 64):
                opts = tuple(o for o in _native.moment_wave_tile_options(width, self.degree)
                             if o[0] == ACCUMULATE_BLOCK_TILES)
                if opts:
                    ft = _plan.feature_tiles(width, self.degree)
                    ms = _plan.moment_split(ft, self.S, self.dv, opts)
                    rows = _plan.split_state_rows(ft, ms, self.d)
                    dev = self.device
                    entry = (ms, torch.from_numpy(ms.quads.view(np.int32)).to(dev), torch.from_numpy(ms.coef).to(dev),
                             torch.from_numpy(rows).to(dev))
            self._acc_tables[key] = entry
        return self._acc_tables[key]

    def _accumulate(self, k: torch.Tensor, v: torch.Tensor, n: int, head_rows: int, state_num: torch.Tensor,
                    state_den: torch.Tensor, row_off: int = 0) -> None:
        """state += moments of rows [row_off, row_off + n) of k [S, head_rows, width] / v [S, head_rows, ldv]
        (contiguous, width a whole number of 16-byte units, ldv a multiple of 32)."""
        if n <= 0:
            return
        width = k.shape[-1]
        assert k.is_contiguous() and v.is_contiguous() and k.shape[1] == head_rows == v.shape[1]
        kp = k.data_ptr() + row_off * width * k.element_size()
        vp = v.data_ptr() + row_off * v.shape[-1] * v.element_size()
        # the wave-specialised pass pays for its state load / store and pipeline fill over long runs of
        # rows (extend); a block completion's rows go to the chunked kernel (c5: 256 rows of 2048 streams
        # 1.8 against 2.6 ms; 4096 rows 23.2 against 10.0 ms)
        ws = self._acc_table_ws(width) if n >= ACCUMULATE_WS_MIN_ROWS else None
        if ws is not None:
            ms, ct, quads, coef, rows = ws

            def run_ws():
                st = self.lib.sta_moment_accumulate_ws(
                    kp, vp, _native.DTYPE_CODES[k.dtype], self.S, n, head_rows, width, width, self.dv, v.shape[-1],
                    self.degree, ms.fsplit, ms.wave_tiles, int(ms.mixed), ct, quads.data_ptr(), coef.data_ptr(),
                    rows.data_ptr(), self.F, state_num.data_ptr(), state_den.data_ptr(), self._stream())
                _native.check(st, "sta_moment_accumulate_ws")

            self._launch("moment_accumulate", run_ws)
            return
        blk = self._acc_table_block(width)
        if blk is not None:
            ms, quads, coef, rows = blk

            def run_block():
                st = self.lib.sta_moment_accumulate_block(
                    kp, vp, _native.DTYPE_CODES[k.dtype], self.S, n, head_rows, width, self.dv, v.shape[-1],
                    self.degree, ms.fsplit, ms.wave_tiles, self._block_column_tiles(), quads.data_ptr(),
                    coef.data_ptr(), rows.data_ptr(), self.F, state_num.data_ptr(), state_den.data_ptr(),
                    self._stream())
                _native.check(st, "sta_moment_accumulate_block")

            self._launch("moment_accumulate", run_block)
            return
        ms, quads, coef, rows, win, staged = self._acc_table(width)

        def run():
            st = self.lib.sta_moment_accumulate(
                kp, vp, _native.DTYPE_CODES[k.dtype], self.S, n, head_rows, staged, width, self.dv,
                v.shape[-1], self.degree, ms.fsplit, ms.wave_tiles, quads.data_ptr(), coef.data_ptr(), rows.data_ptr(),
                _native.ptr(win), self.F, self.products, state_num.data_ptr(), state_den.data_ptr(), self._stream())
            _native.check(st, "sta_moment_accumulate")

        self._launch("moment_accumulate", run)

    def _ensure_levels(self, need: int) -> None:
        if need <= self.L:
            return
        new_l = max(need, 2 * self.L, 4)
        S, m = self.S, self.m
        f32 = dict(device=self.device, dtype=torch.float32)
        lk = torch.zeros((S, new_l, m, self.dk), **f32)
        lv = torch.zeros((S, new_l, m, self.ldv), **f32)
        lw = torch.zeros((S, new_l, m), **f32)
        lp = torch.zeros((S, new_l, m), device=self.device, dtype=torch.int32)
        lk64 = torch.zeros((S, new_l, m, self.dk), device=self.device, dtype=torch.float64) if self.score_f64 else None
        if self.L:
            lk[:, : self.L] = self.lev_k
            lv[:, : self.L] = self.lev_v
            lw[:, : self.L] = self.lev_w
            lp[:, : self.L] = self.lev_pos
            if lk64 is not None:
                lk64[:, : self.L] = self.lev_k64
        self.lev_k, self.lev_v, self.lev_w, self.lev_pos, self.L = lk, lv, lw, lp, new_l
        if lk64 is not None:
            self.lev_k64 = lk64

    def _grow_buffer(self) -> None:
        new_cap = 2 * self.cap
        f32 = dict(device=self.device, dtype=torch.float32)
        bk = torch.zeros((self.S, new_cap, self.dk), **f32)
        bv = torch.zeros((self.S, new_cap, self.ldv), **f32)
        bk[:, : self.cap] = self.buf_k
        bv[:, : self.cap] = self.buf_v
        self.buf_k, self.buf_v, self.cap = bk, bv, new_cap

    # ------------------------------------------------------------------ draws
    def _draw_completion(self, blocks_before: int) -> _CompletionDraws:
        sizes = _plan.completion_call_sizes(blocks_before, self.block, self.compressor)
        n_calls = len(sizes)
        max_in = max(self.block, 2 * self.m)
        methods = [_plan._call_method(n_in, self.compressor) for n_in in sizes]
        dirs, unif, perms = self._gens.next(sizes, self.d, self.compressor, max_in, f64=self.score_f64)
        dev = self.device
        return _CompletionDraws(
            blocks_before, n_calls, torch.tensor(methods, dtype=torch.int32).to(dev), torch.from_numpy(dirs).to(dev),
            torch.from_numpy(unif).to(dev), torch.from_numpy(perms).to(dev))

    def reserve_draws(self, tokens: int) -> int:
        """Draw ahead, on the host, the compress calls of every block completion within the next
        `tokens` tokens (they depend only on the seeds); returns the number of completions queued."""
        if self.exact:
            return 0
        queued_to = self.blocks + len(self._draws)
        last = (self.length + tokens) // self.block
        for c in range(queued_to, last):
            self._draws.append(self._draw_completion(c))
        return len(self._draws)

    def _take_draws(self) -> _CompletionDraws:
        if self._draws:
            dr = self._draws.popleft()
            assert dr.blocks_before == self.blocks
            return dr
        return self._draw_completion(self.blocks)

    # ------------------------------------------------------------------ block completion
    def _complete_block(self, accumulate: bool = True) -> None:
        """The buffer holds a full block: moments += buffer, then compress + cascade into the levels."""
        if accumulate:
            self._accumulate(self.buf_k, self.buf_v, self.block, self.cap, self.state_num, self.state_den)
        dr = self._take_draws()
        self._ensure_levels(dr.n_calls)

        def run():
            st = self.lib.sta_decode_compress(
                self.S, self.d, self.dv, self.buf_k.data_ptr(), self.buf_v.data_ptr(), self.block,
                self.length - self.block, self.lev_k.data_ptr(), self.lev_v.data_ptr(), self.lev_w.data_ptr(),
                self.lev_pos.data_ptr(), self.L, self.m, dr.n_calls, dr.methods.data_ptr(), dr.dirs.data_ptr(),
                dr.unif.data_ptr(), dr.perms.data_ptr(), dr.perms.shape[-1], int(self.score_f64),
                _native.ptr(self.buf_k64), _native.ptr(self.lev_k64), self._stream())
            _native.check(st, "sta_decode_compress")

        self._launch("decode_compress", run)
        self.num_compressions += dr.n_calls
        self.blocks += 1
        self.buf_len = 0

    # ------------------------------------------------------------------ kernels
    def _check_rows(self, x: torch.Tensor, width: int, what: str) -> torch.Tensor:
        if x.shape != (self.S, width):
            raise ValueError(f"{what} must have shape [{self.S}, {width}], got {tuple(x.shape)}")
        if x.device != self.device:
            x = x.to(self.device)
        if x.dtype not in _native.DTYPE_CODES:
            x = x.float()
        return x.contiguous()

    def _tail(self, q, k, v, flags: int, out_dtype: torch.dtype, stats: Optional[torch.Tensor]):
        dt_src = q if q is not None else k
        dt = _native.DTYPE_CODES[dt_src.dtype]
        out = None
        if flags & _native.DEC_QUERY:
            out = torch.empty((self.S, self.dv), device=self.device, dtype=out_dtype)

        def run():
            st = self.lib.sta_decode_tail(
                _native.ptr(q), _native.ptr(k), _native.ptr(v), dt, self.S, self.d, self.dv, self.degree, self.scale,
                self.eps, flags, self.buf_k.data_ptr(), self.buf_v.data_ptr(), self.cap, self.buf_len,
                self.lev_k.data_ptr(), self.lev_v.data_ptr(), self.lev_w.data_ptr(), self.L, self.m,
                self.blocks if not self.exact else 0, self.part_num.data_ptr(), self.part_den.data_ptr(), self.splits,
                _native.ptr(out), _native.DTYPE_CODES[out_dtype], _native.ptr(stats), self._stream())
            _native.check(st, "sta_decode_tail")

        self._launch("decode_tail", run)
        return out

    def _moments(self, q: torch.Tensor) -> None:
        if self.exact:
            return  # the state stays zero: every token is answered exactly from the buffer

        def run():
            st = self.lib.sta_decode_moments(
                q.data_ptr(), _native.DTYPE_CODES[q.dtype], self.S, self.d, self.dv, self.scale,
                self.state_num.data_ptr(), self.state_den.data_ptr(), self.F, self.findex.data_ptr(),
                self.findex_width, self.splits, self.part_num.data_ptr(), self.part_den.data_ptr(), self._stream())
            _native.check(st, "sta_decode_moments")

        self._launch("decode_moments", run)

    def _put_k64(self, k64: Optional[torch.Tensor], lo: int, hi: int) -> None:
        """Buffer rows [lo, hi) of a float64 stream take the float64 keys k64 [S, hi - lo, d]."""
        if not self.score_f64:
            return
        if k64 is None or k64.dtype != torch.float64 or tuple(k64.shape) != (self.S, hi - lo, self.d):
            raise ValueError(f"a float64 stream needs the float64 keys [{self.S}, {hi - lo}, {self.d}]")
        self.buf_k64[:, lo:hi, : self.d] = k64.to(self.device)

    # ------------------------------------------------------------------ public operations
    def update(self, k: torch.Tensor, v: torch.Tensor, k64: Optional[torch.Tensor] = None) -> None:
        """Append one token per stream (MergeReduceCoreset.append + TaylorMomentSketch.update); k64
        [S, d]: the float64 keys of a float64 stream."""
        k = self._check_rows(k, self.d, "key")
        v = self._check_rows(v, self.dv, "value").to(k.dtype)
        if self.exact and self.buf_len == self.cap:
            self._grow_buffer()
        self._put_k64(None if k64 is None else k64[:, None], self.buf_len, self.buf_len + 1)
        self._tail(None, k, v, _native.DEC_APPEND, torch.float32, None)
        self.buf_len += 1
        self.length += 1
        if not self.exact and self.buf_len == self.block:
            self._complete_block()

    def query(self, q: torch.Tensor, out_dtype: torch.dtype = torch.float32,
              stats: Optional[torch.Tensor] = None) -> torch.Tensor:
        q = self._check_rows(q, self.d, "query")
        self._moments(q)
        return self._tail(q, None, None, _native.DEC_QUERY, out_dtype, stats)

    def step(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out_dtype: torch.dtype = torch.float32,
             stats: Optional[torch.Tensor] = None, k64: Optional[torch.Tensor] = None) -> torch.Tensor:
        """update(k, v) then query(q) for every stream, fused into two launches unless the token
        completes a block (k64: as for update)."""
        completes = (not self.exact and self.buf_len + 1 == self.block) or (self.exact and self.buf_len == self.cap)
        if completes:
            self.update(k, v, k64)
            return self.query(q, out_dtype, stats)
        q = self._check_rows(q, self.d, "query")
        k = self._check_rows(k, self.d, "key").to(q.dtype)
        v = self._check_rows(v, self.dv, "value").to(q.dtype)
        self._put_k64(None if k64 is None else k64[:, None], self.buf_len, self.buf_len + 1)
        self._moments(q)
        out = self._tail(q, k, v, _native.DEC_APPEND | _native.DEC_CURRENT | _native.DEC_QUERY, out_dtype, stats)
        self.buf_len += 1
        self.length += 1
        return out

    def step_into(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                  stats: Optional[torch.Tensor] = None) -> torch.Tensor:
        """step(q, k, v) written into the caller's `out` [S, dv] without any device allocation: one
        sta_decode_step_static call (the moment partials live in the library's static scratch).  The
        inputs must already be contiguous [S, d] / [S, dv] device tensors of one supported dtype; a token
        that completes a block (compress, merges, host draws) is refused: use step() for it."""
        if (not self.exact and self.buf_len + 1 == self.block) or (self.exact and self.buf_len == self.cap):
            raise ValueError("step_into cannot complete a block; call step() for this token")
        if self.score_f64:
            raise ValueError("step_into takes float32 / bfloat16 / float16 tokens; a float64 stream uses step()")
        for x, width, what in ((q, self.d, "query"), (k, self.d, "key"), (v, self.dv, "value")):
            if x.shape != (self.S, width) or x.device != self.device or not x.is_contiguous():
                raise ValueError(f"{what} must be a contiguous [{self.S}, {width}] tensor on {self.device}")
        if not (q.dtype == k.dtype == v.dtype) or q.dtype not in _native.DTYPE_CODES:
            raise ValueError("q, k, v must share one of the dtypes float32, bfloat16, float16")
        if out.shape != (self.S, self.dv) or out.device != self.device or not out.is_contiguous() or \
                out.dtype not in _native.DTYPE_CODES:
            raise ValueError(f"out must be a contiguous [{self.S}, {self.dv}] float32/bfloat16/float16 tensor "
                             f"on {self.device}")
        flags = _native.DEC_APPEND | _native.DEC_CURRENT | _native.DEC_QUERY
        stream = self._stream()
        STATIC_OWNERS.claim(self._dev_index, id(self), stream)
        self._static_stream = stream

        def run():
            st = self.lib.sta_decode_step_static(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), _native.DTYPE_CODES[q.dtype], self.S, self.d, self.dv,
                self.degree, self.scale, self.eps, flags,
                None if self.exact else self.state_num.data_ptr(), None if self.exact else self.state_den.data_ptr(),
                self.F, self.findex.data_ptr(), self.findex_width, self.splits, self.buf_k.data_ptr(),
                self.buf_v.data_ptr(), self.cap,
                self.buf_len, self.lev_k.data_ptr(), self.lev_v.data_ptr(), self.lev_w.data_ptr(), self.L, self.m,
                self.blocks if not self.exact else 0, out.data_ptr(), _native.DTYPE_CODES[out.dtype],
                _native.ptr(stats), self._stream())
            _native.check(st, "sta_decode_step_static")

        self._launch("decode_step_static", run)
        self.buf_len += 1
        self.length += 1
        return out

    def release_static(self) -> None:
        """Gives up this state's claim on its device's static scratch after waiting for the stream of its
        allocation-free steps, so that another state (or another stream) may use step_into."""
        if STATIC_OWNERS.holder(self._dev_index) == (id(self), getattr(self, "_static_stream", None)):
            torch.cuda.ExternalStream(self._static_stream, device=self.device).synchronize()
        STATIC_OWNERS.release(self._dev_index, id(self))

    def __del__(self) -> None:
        try:
            if STATIC_OWNERS.holder(self._dev_index) is not None:
                self.release_static()
        except Exception:
            pass

    def extend(self, k: torch.Tensor, v: torch.Tensor, k64: Optional[torch.Tensor] = None) -> None:
        """update() for every token of k [S, P, d] / v [S, P, dv], in bulk: whole blocks go to the state
        in one moment-accumulate launch and are compressed block by block (k64 [S, P, d]: the float64
        keys of a float64 stream)."""
        if k.ndim != 3 or k.shape[0] != self.S or k.shape[2] != self.d:
            raise ValueError(f"keys must have shape [{self.S}, P, {self.d}], got {tuple(k.shape)}")
        if self.score_f64 and (k64 is None or tuple(k64.shape) != tuple(k.shape)):
            raise ValueError(f"a float64 stream needs the float64 keys [{self.S}, P, {self.d}]")
        if v.shape != (self.S, k.shape[1], self.dv):
            raise ValueError(f"values must have shape [{self.S}, {k.shape[1]}, {self.dv}], got {tuple(v.shape)}")
        k = k.to(self.device)
        v = v.to(self.device)
        if k.dtype not in _native.DTYPE_CODES:
            k = k.float()
        v = v.to(k.dtype)
        p_total = k.shape[1]
        i = 0

        def to_buffer(lo: int, hi: int) -> None:
            n = hi - lo
            while self.exact and self.buf_len + n > self.cap:
                self._grow_buffer()
            self.buf_k[:, self.buf_len: self.buf_len + n, : self.d] = k[:, lo:hi].float()
            self.buf_v[:, self.buf_len: self.buf_len + n, : self.dv] = v[:, lo:hi].float()
            if self.score_f64:
                self._put_k64(k64[:, lo:hi], self.buf_len, self.buf_len + n)
            self.buf_len += n
            self.length += n

        if self.exact:
            to_buffer(0, p_total)
            return
        # 1. top up a partly filled buffer
        if self.buf_len > 0:
            n = min(p_total, self.block - self.buf_len)
            to_buffer(0, n)
            i = n
            if self.buf_len == self.block:
                self._complete_block()
        # 2. whole blocks: one moment-accumulate launch, then block-by-block compression
        nb = (p_total - i) // self.block
        if nb > 0:
            esize = k.element_size()
            unit = _plan.WINDOW_BLOCK if self.d > _engine.STAGED_D else 16 // esize
            width = -(-self.d // unit) * unit
            lo, hi = i, i + nb * self.block
            if width == self.d and k.is_contiguous() and k.data_ptr() % 16 == 0:
                kp, koff = k, lo  # read in place
            else:
                kp, koff = torch.zeros((self.S, hi - lo, width), device=self.device, dtype=k.dtype), 0
                kp[..., : self.d] = k[:, lo:hi]
            # v in place only next to k in place: both are then read at row lo of [S, p_total, .] rows
            if kp is k and self.ldv == self.dv and v.is_contiguous() and v.data_ptr() % 16 == 0:
                vp = v
            else:
                vp = torch.zeros((self.S, kp.shape[1], self.ldv), device=self.device, dtype=k.dtype)
                vp[:, koff: koff + hi - lo, : self.dv] = v[:, lo:hi]
            self._accumulate(kp, vp, hi - lo, kp.shape[1], self.state_num, self.state_den, row_off=koff)
            for b in range(nb):
                to_buffer(lo + b * self.block, lo + (b + 1) * self.block)
                self._complete_block(accumulate=False)
            i = hi
        # 3. the rest starts a new buffer
        if i < p_total:
            to_buffer(i, p_total)

    # ------------------------------------------------------------------ inspection
    def full_moments(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """(den [S, F], num [S, F, dv]) over every token so far, reference feature order (the
        reference's sketch state: completed blocks plus the buffer)."""
        num = self.state_num.clone()
        den = self.state_den.clone()
        self._accumulate(self.buf_k, self.buf_v, self.buf_len, self.cap, num, den)
        return den, num[..., : self.dv]

    def level_items(self) -> List[Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]]]:
        """Per level: (keys [S, m, d], values [S, m, dv], weights [S, m], positions [S, m]) or None."""
        out = []
        top = self.blocks.bit_length()
        for l in range(top):
            if self.exact or not (self.blocks >> l) & 1:
                out.append(None)
            else:
                out.append((self.lev_k[:, l, :, : self.d], self.lev_v[:, l, :, : self.dv], self.lev_w[:, l],
                            self.lev_pos[:, l]))
        return out

    def buffer_items(self) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(keys [S, n, d], values [S, n, dv], positions [n]) of the uncompressed buffer."""
        n = self.buf_len
        pos = torch.arange(self.length - n, self.length, device=self.device, dtype=torch.int32)
        return self.buf_k[:, :n, : self.d], self.buf_v[:, :n, : self.dv], pos

    def num_items(self) -> int:
        if self.exact:
            return self.length
        return self.buf_len + self.m * bin(self.blocks).count("1")

    def reference_state_bytes(self, elem: int, include_feature_map: bool = False,
                              value_dim: Optional[int] = None) -> int:
        """ArticleStreamingAttention.state_size_bytes of one stream for element size `elem`
        (streaming_taylor_coreset_attention.py:298-306, :495-506, :611-612); value_dim: the object's
        whole value width when this state holds one column group of it."""
        d, dv = self.d, self.dv if value_dim is None else int(value_dim)
        total = self.F * (1 + dv) * elem
        if include_feature_map:
            for l in range(1, self.degree + 1):
                total += (_plan.num_features(d, l) - _plan.num_features(d, l - 1)) * l * 8
            total += self.F * elem
        buffered = self.length - (self.length // self.block) * self.block
        total += buffered * (d + dv) * elem
        completed = self.length // self.block
        items = completed * self.block if self.exact else self.m * bin(completed).count("1")
        total += items * (d + dv + 1) * elem
        return int(total)

    # ------------------------------------------------------------------ save / resume
    def _config(self) -> Dict[str, object]:
        return {"streams": self.S, "dim": self.d, "value_dim": self.dv, "degree": self.degree, "block": self.block,
                "scale": self.scale, "compressor": self.compressor, "seed": self.seed, "eps": self.eps,
                "score_f64": self.score_f64}

    def state_dict(self) -> Dict[str, object]:
        """The streams' whole state on the host: configuration, counters, moments, buffered tokens, level
        coresets, each stream's generator state and any reserved completion draws.  Plain tensors, ints,
        floats and strings, so torch.save / torch.load(weights_only=True) round-trip it."""
        torch.cuda.synchronize(self.device)
        levels = {}
        if self.L:
            levels = {"lev_k": self.lev_k.cpu(), "lev_v": self.lev_v.cpu(), "lev_w": self.lev_w.cpu(),
                      "lev_pos": self.lev_pos.cpu()}
        draws = [{"blocks_before": dr.blocks_before, "n_calls": dr.n_calls, "methods": dr.methods.cpu(),
                  "dirs": dr.dirs.cpu(), "unif": dr.unif.cpu(), "perms": dr.perms.cpu()} for dr in self._draws]
        return {
            "format": 1,
            "config": self._config(),
            "length": self.length, "blocks": self.blocks, "buf_len": self.buf_len,
            "num_compressions": self.num_compressions, "levels_allocated": self.L,
            "state_num": self.state_num.cpu(), "state_den": self.state_den.cpu(),
            "buf_k": self.buf_k[:, : self.buf_len].cpu(), "buf_v": self.buf_v[:, : self.buf_len].cpu(),
            **levels,
            **({"buf_k64": self.buf_k64[:, : self.buf_len].cpu(),
                "lev_k64": self.lev_k64[:, : self.L].cpu()} if self.score_f64 else {}),
            "generators": self._gens.get_state(),
            "draws": draws,
        }

    def load_state_dict(self, sd: Dict[str, object]) -> None:
        """Resume from state_dict(): the configuration must match this object's."""
        if sd.get("format") != 1:
            raise ValueError("unknown decode state format")
        if sd["config"] != self._config():
            raise ValueError(f"decode state configuration {sd['config']} does not match {self._config()}")
        dev = self.device
        buf_len = int(sd["buf_len"])
        while self.cap < buf_len:
            self._grow_buffer()
        self.state_num.copy_(sd["state_num"].to(dev))
        self.state_den.copy_(sd["state_den"].to(dev))
        self.buf_k.zero_()
        self.buf_v.zero_()
        self.buf_k[:, :buf_len] = sd["buf_k"].to(dev)
        self.buf_v[:, :buf_len] = sd["buf_v"].to(dev)
        n_lev = int(sd["levels_allocated"])
        if n_lev:
            self._ensure_levels(n_lev)
            self.lev_k.zero_()
            self.lev_v.zero_()
            self.lev_w.zero_()
            self.lev_pos.zero_()
            self.lev_k[:, :n_lev] = sd["lev_k"].to(dev)
            self.lev_v[:, :n_lev] = sd["lev_v"].to(dev)
            self.lev_w[:, :n_lev] = sd["lev_w"].to(dev)
            self.lev_pos[:, :n_lev] = sd["lev_pos"].to(dev)
        if self.score_f64:
            self.buf_k64.zero_()
            self.buf_k64[:, :buf_len] = sd["buf_k64"].to(dev)
            if n_lev:
                self.lev_k64.zero_()
                self.lev_k64[:, :n_lev] = sd["lev_k64"].to(dev)
        self.length, self.blocks, self.buf_len = int(sd["length"]), int(sd["blocks"]), buf_len
        self.num_compressions = int(sd["num_compressions"])
        self._gens.set_state(sd["generators"])
        self._draws = deque(_CompletionDraws(int(d["blocks_before"]), int(d["n_calls"]), d["methods"].to(dev),
                                             d["dirs"].to(dev), d["unif"].to(dev), d["perms"].to(dev))
                            for d in sd["draws"])

    def device_bytes(self) -> int:
        """Bytes of device memory this state holds."""
        ts = [self.state_num, self.state_den, self.buf_k, self.buf_v, self.lev_k, self.lev_v, self.lev_w,
              self.lev_pos, self.part_num, self.part_den, self.findex]
        if self.score_f64:
            ts += [self.buf_k64, self.lev_k64]
        return int(sum(t.numel() * t.element_size() for t in ts))


class ColumnGroups:
    """Value widths above the decode kernels' max_dv: one DecodeState per group of at most max_dv value
    columns, every group fed the same keys with the same seeds.  A stream's selections, denominators
    and statistics depend on its keys and draws only, so every group keeps the same coreset (the same
    tokens and weights) and the groups' outputs concatenate to the whole value width; the key-side work
    (feature moments of the denominators, compression) runs once per group.  The reference's streaming
    object has no value-width bound (streaming_taylor_coreset_attention.py:523-575)."""

    def __init__(self, streams: int, dim: int, value_dim: int, **kw) -> None:
        w = _native.limits()["max_dv"]
        if value_dim <= w:
            raise ValueError("ColumnGroups is for value widths above the kernels' max_dv; use DecodeState")
        self.bounds = [(c0, min(c0 + w, value_dim)) for c0 in range(0, value_dim, w)]
        self.groups = [DecodeState(streams, dim, c1 - c0, **kw) for c0, c1 in self.bounds]
        self.dv = int(value_dim)

    def __getattr__(self, name: str):
        # counters, shapes and key-side state are the same in every group: group 0's
        if name in ("groups", "bounds", "dv"):
            raise AttributeError(name)
        return getattr(self.groups[0], name)

    @property
    def timer(self):
        return self.groups[0].timer

    @timer.setter
    def timer(self, t) -> None:
        for g in self.groups:
            g.timer = t

    def _cols(self, v: Optional[torch.Tensor]) -> List[Optional[torch.Tensor]]:
        if v is None:
            return [None] * len(self.groups)
        if v.shape[-1] != self.dv:
            raise ValueError(f"values must have {self.dv} columns, got {v.shape[-1]}")
        return [v[..., c0:c1].contiguous() for c0, c1 in self.bounds]

    def reserve_draws(self, tokens: int) -> int:
        return [g.reserve_draws(tokens) for g in self.groups][0]

    def update(self, k: torch.Tensor, v: torch.Tensor, k64: Optional[torch.Tensor] = None) -> None:
        for g, vg in zip(self.groups, self._cols(v)):
            g.update(k, vg, k64)

    def query(self, q: torch.Tensor, out_dtype: torch.dtype = torch.float32,
              stats: Optional[torch.Tensor] = None) -> torch.Tensor:
        return torch.cat([g.query(q, out_dtype, stats if i == 0 else None) for i, g in enumerate(self.groups)], -1)

    def step(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out_dtype: torch.dtype = torch.float32,
             stats: Optional[torch.Tensor] = None, k64: Optional[torch.Tensor] = None) -> torch.Tensor:
        return torch.cat([g.step(q, k, vg, out_dtype, stats if i == 0 else None, k64)
                          for i, (g, vg) in enumerate(zip(self.groups, self._cols(v)))], -1)

    def release_static(self) -> None:
        for g in self.groups:
            g.release_static()

    def step_into(self, q, k, v, out, stats=None):
        raise ValueError(f"step_into writes one kernel call's columns: value_dim {self.dv} runs as column groups; "
                         f"use step()")

    def extend(self, k: torch.Tensor, v: torch.Tensor, k64: Optional[torch.Tensor] = None) -> None:
        for g, vg in zip(self.groups, self._cols(v)):
            g.extend(k, vg, k64)

    def full_moments(self) -> Tuple[torch.Tensor, torch.Tensor]:
        parts = [g.full_moments() for g in self.groups]
        return parts[0][0], torch.cat([p[1] for p in parts], -1)

    def level_items(self):
        per = [g.level_items() for g in self.groups]
        out = []
        for lv in zip(*per):
            if lv[0] is None:
                out.append(None)
            else:
                out.append((lv[0][0], torch.cat([x[1] for x in lv], -1), lv[0][2], lv[0][3]))
        return out

    def buffer_items(self):
        per = [g.buffer_items() for g in self.groups]
        return per[0][0], torch.cat([p[1] for p in per], -1), per[0][2]

    def reference_state_bytes(self, elem: int, include_feature_map: bool = False) -> int:
        return self.groups[0].reference_state_bytes(elem, include_feature_map, value_dim=self.dv)

    def state_dict(self) -> Dict[str, object]:
        return {"format": 2, "value_dim": self.dv, "column_groups": [g.state_dict() for g in self.groups]}

    def load_state_dict(self, sd: Dict[str, object]) -> None:
        if sd.get("format") != 2 or sd.get("value_dim") != self.dv or \
                len(sd.get("column_groups", ())) != len(self.groups):
            raise ValueError("decode state does not match this object's value column groups")
        for g, gsd in zip(self.groups, sd["column_groups"]):
            g.load_state_dict(gsd)

    def device_bytes(self) -> int:
        return sum(g.device_bytes() for g in self.groups)


def decode_state(streams: int, dim: int, value_dim: int, **kw):
    """A DecodeState, or ColumnGroups of them when value_dim exceeds the kernels' max_dv."""
    if value_dim > _native.limits()["max_dv"]:
        return ColumnGroups(streams, dim, value_dim, **kw)
    return DecodeState(streams, dim, value_dim, **kw)
