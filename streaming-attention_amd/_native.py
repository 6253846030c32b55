"""ctypes binding of libstreamattn.so (the C ABI declared in include/streamattn.h).

The shared library is built in-tree next to this file (see ``build_native.py``).  There is no CPU
fallback anywhere in this package: if the library or a ROCm device is missing, ``lib()`` raises.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
from typing import Optional

import torch

_HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = _HERE / "libstreamattn.so"

STA_OK = 0
STA_ERR_SHAPE = 1
STA_ERR_UNSUPPORTED = 2
STA_ERR_DTYPE = 3
STA_ERR_HIP = 4
STA_ERR_ARG = 5
STA_ERR_SCRATCH = 6

DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
STA_F64 = 3  # sta_compress_nodes' float64 scoring
PRODUCTS_FP32 = 0
PRODUCTS_SPLIT_BF16 = 1

_c_p = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# name -> (restype, argtypes); must mirror include/streamattn.h
_SIGNATURES = {
    "sta_version": (_i32, []),
    "sta_status_string": (ctypes.c_char_p, [_i32]),
    "sta_last_hip_error": (_i32, []),
    "sta_limits": (_i32, [ctypes.POINTER(_i32)] * 4),
    "sta_tile_rows": (_i32, []),
    "sta_moment_chunk": (_i32, [_i32]),
    "sta_moments": (
        _i32,
        [_c_p, _c_p, _c_p, _i32, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _i32, _i32, _i32,
         _i32, _i32, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p],  # ... d ld_qk dv ldv ... quads coef windows num den stream
    ),
    "sta_moments_ws": (
        _i32,
        [_c_p, _c_p, _c_p, _i32, _i64, _i64, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _i32, _i32, _i32, _i32,
         _c_p, _c_p, _c_p, _c_p, _c_p, _c_p],
    ),
    "sta_moments_ws_seg": (
        _i32,
        [_c_p, _c_p, _c_p, _i32, _i64, _i64, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _i32, _i32, _i32, _i32,
         _c_p, _c_p, _c_p, _c_p, _c_p, _i32, _i32, _c_p, _c_p],
    ),
    "sta_moments_ws_seg_bytes": (_i64, [_i64, _i32, _i32, _i32, _i32, _i32]),
    "sta_moments_ws_ok": (_i32, [_i32, _i32, _i32, _i32, _i32]),
    "sta_moments_ws_handoff_bytes": (_i64, [_i64, _i32, _i32, _i32, _i32]),
    "sta_moment_columns_ok": (_i32, [_i32, _i32, _i32, _i32, _i32]),
    "sta_moment_mixed_ok": (_i32, [_i32, _i32, _i32]),
    "sta_moment_wave_tiles": (_i32, [_i32, _i32, _i32]),
    "sta_moment_occupancy": (_i32, [_i32, _i32]),
    "sta_moment_occupancy_degree": (_i32, [_i32, _i32, _i32]),
    "sta_moment_partials_layout": (_i32, [_i64, _i32, ctypes.POINTER(_i64), ctypes.POINTER(_i32), ctypes.POINTER(_i32)]),
    "sta_compress_nodes": (
        _i32,
        [_c_p, _i32, _i64, _i64, _i32, _c_p, _i32, _c_p, _i32, _i32, _c_p, _c_p, _c_p, _i32, _i32, _c_p, _c_p,
         _c_p, _c_p, _i32, _c_p, _c_p],  # ... node_src node_w node_level anc anc_levels level_scores stream
    ),
    "sta_compress_merges": (
        _i32,
        [_c_p, _i32, _i64, _i64, _i32, _c_p, _i32, _i32, _i32, _i32, _c_p, _i32, _i32, _c_p, _c_p, _c_p, _i32,
         _i32, _c_p, _c_p, _c_p, _i32, _c_p, _c_p],  # k .. table n_groups steps groups group_threads desc ...
    ),
    "sta_segment_mean": (_i32, [_c_p, _c_p, _i32, _i64, _i64, _i32, _i32, _i32, _i32, _i64, _c_p, _c_p, _c_p]),
    "sta_block_attention": (
        _i32,
        [
            _c_p, _c_p, _c_p, _i32, _i64, _i64, _i32, _i32, _i32, _i32,  # q k v dtype bh n d dv ld_qk ld_v
            _i32, _f32, _f32, _i32, _i32, _i32, _i32, _i32, _i32,  # degree scale eps mode block chunk shift clamp products
            _c_p, _c_p, _i32,  # low_num low_den fsplit
            _c_p, _c_p, _i32, _c_p, _i32, _i32,  # tile_ptr tile_nodes n_tiles node_meta n_nodes cap
            _c_p, _c_p, _c_p, _c_p, _i32, _i32, _i64,  # node_src node_w rep_k rep_v ld_rep_k ld_rep_v n_rep
            _c_p, _i32, _c_p, _c_p,  # out out_dtype out_den stream
        ],
    ),
    "sta_flash_attention": (
        _i32, [_c_p, _c_p, _c_p, _i32, _i64, _i64, _i32, _i32, _i32, _i32, _f32, _c_p, _i32, _c_p],
    ),
    "sta_moment_accumulate_block": (
        _i32,
        [_c_p, _c_p, _i32, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _c_p, _c_p, _c_p, _i32, _c_p,
         _c_p, _c_p],  # k v dtype bh n head_rows d dv ldv degree fsplit wave_tiles column_tiles quads coef rows ...
    ),
    "sta_moment_accumulate_ws": (
        _i32,
        [_c_p, _c_p, _i32, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,  # ... fs nts mixed ct
         _c_p, _c_p, _c_p, _i32, _c_p, _c_p, _c_p],  # quads coef rows n_feat num den stream
    ),
    "sta_moment_accumulate": (
        _i32,
        [_c_p, _c_p, _i32, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32,  # k v dt bh n rows d ld dv ldv deg fs nt
         _c_p, _c_p, _c_p, _c_p, _i32, _i32, _c_p, _c_p, _c_p],  # quads coef rows windows n_feat products num den stream
    ),
    "sta_decode_layout": (_i32, [_i32, _i32, ctypes.POINTER(_i32), ctypes.POINTER(_i32)]),
    "sta_decode_moments": (
        _i32, [_c_p, _i32, _i64, _i32, _i32, _f32, _c_p, _c_p, _i32, _c_p, _i32, _i32, _c_p, _c_p, _c_p],
    ),
    "sta_decode_tail": (
        _i32,
        [
            _c_p, _c_p, _c_p, _i32, _i64, _i32, _i32, _i32, _f32, _f32, _i32,  # q k v dtype S d dv deg scale eps flags
            _c_p, _c_p, _i32, _i32,  # buf_k buf_v block buf_len
            _c_p, _c_p, _c_p, _i32, _i32, ctypes.c_uint64,  # lev_k lev_v lev_w n_levels level_size mask
            _c_p, _c_p, _i32, _c_p, _i32, _c_p, _c_p,  # part_num part_den splits out out_dtype stats stream
        ],
    ),
    "sta_decode_compress": (
        _i32,
        [
            _i64, _i32, _i32, _c_p, _c_p, _i32, _i32,  # S d dv buf_k buf_v block pos0
            _c_p, _c_p, _c_p, _c_p, _i32, _i32,  # lev_k lev_v lev_w lev_pos n_levels level_size
            _i32, _c_p, _c_p, _c_p, _c_p, _i32,  # n_calls methods dirs unif perms max_in
            _i32, _c_p, _c_p, _c_p,  # score_f64 buf_k64 lev_k64 stream
        ],
    ),
    "sta_static_scratch_bytes": (_i64, []),
    "sta_decode_step_static": (
        _i32,
        [
            _c_p, _c_p, _c_p, _i32, _i64, _i32, _i32, _i32, _f32, _f32, _i32,  # q k v dtype S d dv deg scale eps flags
            _c_p, _c_p, _i32, _c_p, _i32, _i32,  # state_num state_den n_feat feat_index index_width splits
            _c_p, _c_p, _i32, _i32,  # buf_k buf_v block buf_len
            _c_p, _c_p, _c_p, _i32, _i32, ctypes.c_uint64,  # lev_k lev_v lev_w n_levels level_size mask
            _c_p, _i32, _c_p, _c_p,  # out out_dtype stats stream
        ],
    ),
    "sta_selftest_mfma": (_i32, [_c_p, _c_p, _c_p]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lib: Optional[ctypes.CDLL] = None


class NativeError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


def load_library(path: Optional[os.PathLike] = None) -> ctypes.CDLL:
    """Load the shared library and attach the argument types (no device is touched)."""
    p = pathlib.Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise ImportError(
            f"libstreamattn.so not found at {p}; build it with `python -c 'import __graft_entry__ as g; g.build()'`"
        )
    handle = ctypes.CDLL(str(p))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    return handle


def lib() -> ctypes.CDLL:
    """The loaded library (cached)."""
    global _lib
    if _lib is None:
        _lib = load_library()
    return _lib


DRAWS_LIB_PATH = _HERE / "libstadraws.so"
COMPRESSOR_CODES = {"none": 0, "random": 1, "sorted_pair": 2}
_draws_lib: Optional[ctypes.CDLL] = None


def draws_library() -> ctypes.CDLL:
    """libstadraws.so: the compressor's seed-derived draws replayed on torch's CPU generator
    (csrc/host_draws.cpp; host only, loaded after torch so that its torch libraries resolve)."""
    global _draws_lib
    if _draws_lib is None:
        if not DRAWS_LIB_PATH.exists():
            raise ImportError(f"libstadraws.so not found at {DRAWS_LIB_PATH}; build it with "
                              f"`python -c 'import __graft_entry__ as g; g.build()'`")
        h = ctypes.CDLL(str(DRAWS_LIB_PATH))
        p, i = ctypes.c_void_p, ctypes.c_int
        for name, res, args in (("sta_draws_open", p, [p, i]),
                                ("sta_draws_close", None, [p]),
                                ("sta_draws_next", i, [p, p, i, i, i, i, p, p, p]),
                                ("sta_draws_next_typed", i, [p, p, i, i, i, i, i, p, p, p]),
                                ("sta_host_draws_typed", i, [p, i, p, i, i, i, i, i, p, p, p]),
                                ("sta_draws_state_bytes", ctypes.c_int64, []),
                                ("sta_draws_get_state", i, [p, p]),
                                ("sta_draws_set_state", i, [p, p]),
                                ("sta_host_draws", i, [p, i, p, i, i, i, i, p, p, p]),
                                ("sta_host_select", i, [p, i, ctypes.c_int64, ctypes.c_int64, i, i, p, i, i, p, p,
                                                        p, i, i, i, p, p]),
                                ("sta_draws_error", ctypes.c_char_p, [])):
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _draws_lib = h
    return _draws_lib


def _draws_fail(h) -> None:
    raise NativeError(h.sta_draws_error().decode())


# element types of the draws (stadraws.h STA_DRAW_*): the keys' dtype
DRAW_TYPES = {torch.float32: 0, torch.float64: 1, torch.bfloat16: 2, torch.float16: 3}


def draw_type(f64: bool = False, dtype: Optional[torch.dtype] = None) -> int:
    """The STA_DRAW_* code of draws in `dtype` (float32, float64, bfloat16, float16), or of float64 /
    float32 draws by the f64 flag when dtype is None."""
    if dtype is None:
        return 1 if f64 else 0
    if dtype not in DRAW_TYPES:
        raise ValueError(f"no draws in {dtype}")
    return DRAW_TYPES[dtype]


def _draw_tables(n_seq: int, call_sizes, d: int, compressor: str, max_in: int, dt: int = 0):
    import numpy as np

    if compressor not in COMPRESSOR_CODES:
        raise ValueError("compressor must be one of {'sorted_pair', 'random', 'none'}")
    cc = max(len(call_sizes), 1)
    sz = np.ascontiguousarray(np.asarray(call_sizes, dtype=np.int32))
    ft = np.float64 if dt == 1 else np.float32
    return (sz, np.zeros((n_seq, cc, d), dtype=ft), np.zeros((n_seq, cc, max_in // 2), dtype=ft),
            np.zeros((n_seq, cc, max_in), dtype=np.int32))


def host_draws(seeds, call_sizes, d: int, compressor: str, max_in: int, f64: bool = False,
               dtype: Optional[torch.dtype] = None):
    """Draw tables (dirs [S, C, d], unif [S, C, max_in // 2], perms int32 [S, C, max_in]; C = at least 1)
    of len(seeds) sequences, each on a fresh generator seeded seeds[s], over the compress calls of
    call_sizes, in call order.  The directions and uniforms are drawn in `dtype` (the keys' dtype, as the
    reference draws them; float64 tables for float64, float32 tables holding the values otherwise), or
    as float64 / float32 by the f64 flag when dtype is None."""
    import numpy as np

    dt = draw_type(f64, dtype)
    sz, dirs, unif, perms = _draw_tables(len(seeds), call_sizes, d, compressor, max_in, dt)
    sd = np.ascontiguousarray(np.asarray(seeds, dtype=np.int64))
    h = draws_library()
    if h.sta_host_draws_typed(sd.ctypes.data, len(seeds), sz.ctypes.data, len(call_sizes), d,
                              COMPRESSOR_CODES[compressor], max_in, dt, dirs.ctypes.data, unif.ctypes.data,
                              perms.ctypes.data) != 0:
        _draws_fail(h)
    return dirs, unif, perms


def host_select(keys: torch.Tensor, levels: bool, desc, n_nodes: int, cap: int, dirs, unif, perms,
                threads: int = 0):
    """Reference-order selections (sta_host_select): every compress call of a node plan run on the host
    with torch's CPU `keys @ direction` and argsort in the keys' dtype.  keys: contiguous CPU [S, N, d]
    (float32 / float64 / bfloat16 / float16; laid out as the caller's tensor); desc: int32 [n_nodes, 8]
    with methods filled; dirs / unif / perms: the draw tables of host_draws in the keys' dtype.
    Returns (node_src int32 [S, n_nodes, cap], node_w float32 [S, n_nodes, cap]) as numpy arrays."""
    import numpy as np

    if keys.device.type != "cpu" or not keys.is_contiguous() or keys.dim() != 3 or keys.dtype not in DRAW_TYPES:
        raise ValueError("host_select needs contiguous CPU [S, N, d] keys of a float dtype")
    s_, n, d = keys.shape
    dt = DRAW_TYPES[keys.dtype]
    want = np.float64 if dt == 1 else np.float32
    desc = np.ascontiguousarray(desc, dtype=np.int32)
    dirs, unif = np.ascontiguousarray(dirs), np.ascontiguousarray(unif)
    perms = np.ascontiguousarray(perms, dtype=np.int32)
    if dirs.dtype != want or unif.dtype != want:
        raise ValueError("draw tables must be float64 for float64 keys and float32 otherwise")
    if dirs.ndim != 3 or dirs.shape[0] != s_ or dirs.shape[2] != d or unif.shape[:2] != dirs.shape[:2] or \
            perms.shape[:2] != dirs.shape[:2] or unif.shape[2] * 2 > perms.shape[2] or desc.shape != (n_nodes, 8):
        raise ValueError("draw tables or node plan do not match the keys")
    n_calls, max_in = int(dirs.shape[1]), int(perms.shape[2])
    node_src = np.zeros((s_, n_nodes, cap), dtype=np.int32)
    node_w = np.zeros((s_, n_nodes, cap), dtype=np.float32)
    h = draws_library()
    if h.sta_host_select(keys.data_ptr(), dt, s_, n, d, int(bool(levels)), desc.ctypes.data, n_nodes, cap,
                         dirs.ctypes.data, unif.ctypes.data, perms.ctypes.data, n_calls, max_in, int(threads),
                         node_src.ctypes.data, node_w.ctypes.data) != 0:
        _draws_fail(h)
    return node_src, node_w


class DrawSet:
    """Persistent per-stream CPU generators (stream s seeded seeds[s]) that successive compress calls
    continue; states read and written in torch.Generator.get_state()'s layout."""

    def __init__(self, seeds) -> None:
        import numpy as np

        self._h = draws_library()
        sd = np.ascontiguousarray(np.asarray(seeds, dtype=np.int64))
        self.n = int(sd.shape[0])
        self._ptr = self._h.sta_draws_open(sd.ctypes.data, self.n)
        if not self._ptr:
            _draws_fail(self._h)

    def __del__(self) -> None:
        if getattr(self, "_ptr", None):
            self._h.sta_draws_close(self._ptr)
            self._ptr = None

    def next(self, call_sizes, d: int, compressor: str, max_in: int, f64: bool = False,
             dtype: Optional[torch.dtype] = None):
        """Tables as host_draws, continuing every stream's generator."""
        dt = draw_type(f64, dtype)
        sz, dirs, unif, perms = _draw_tables(self.n, call_sizes, d, compressor, max_in, dt)
        if self._h.sta_draws_next_typed(self._ptr, sz.ctypes.data, len(call_sizes), d, COMPRESSOR_CODES[compressor],
                                        max_in, dt, dirs.ctypes.data, unif.ctypes.data,
                                        perms.ctypes.data) != 0:
            _draws_fail(self._h)
        return dirs, unif, perms

    def get_state(self) -> torch.Tensor:
        """uint8 [n, state bytes]: row s is stream s's torch.Generator.get_state()."""
        out = torch.empty((self.n, int(self._h.sta_draws_state_bytes())), dtype=torch.uint8)
        if self._h.sta_draws_get_state(self._ptr, out.data_ptr()) != 0:
            _draws_fail(self._h)
        return out

    def set_state(self, states: torch.Tensor) -> None:
        nb = int(self._h.sta_draws_state_bytes())
        st = states.to(torch.uint8).contiguous()
        if tuple(st.shape) != (self.n, nb):
            raise ValueError(f"generator states must be uint8 [{self.n}, {nb}], got {tuple(st.shape)}")
        if self._h.sta_draws_set_state(self._ptr, st.data_ptr()) != 0:
            _draws_fail(self._h)


def check(status: int, what: str) -> None:
    if status == STA_OK:
        return
    l = lib()
    msg = l.sta_status_string(status).decode()
    if status == STA_ERR_HIP:
        msg += f" (hipError {l.sta_last_hip_error()})"
    raise NativeError(f"{what} failed: {msg}")


def require_device(t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise ValueError("the HIP kernels require tensors on a ROCm GPU device")


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_wave_tile_options: dict = {}


def moment_wave_tile_options(d: int, degree: int) -> tuple:
    """((per-wave tile count, workgroups resident per compute unit), ...) the moment kernel is built
    for at (staged width d, degree)."""
    key = (d, degree)
    if key not in _wave_tile_options:
        l = lib()
        opts = set()
        for want in range(1, 65):
            nt = l.sta_moment_wave_tiles(d, degree, want)
            if nt > 0:
                opts.add((nt, l.sta_moment_occupancy_degree(d, degree, nt)))
        _wave_tile_options[key] = tuple(sorted(opts))
    return _wave_tile_options[key]


def moment_mixed_tiles(d: int, degree: int) -> tuple:
    """Per-wave tile counts the moment kernel also runs with mixed tile counts at (d, degree)."""
    l = lib()
    return tuple(nt for nt, _ in moment_wave_tile_options(d, degree) if l.sta_moment_mixed_ok(d, degree, nt))


def moment_partials_layout(n: int, dv: int) -> tuple:
    """(rows, ld, row_offset) of the moment kernel's partial outputs."""
    rows, ld, off = _i64(), _i32(), _i32()
    check(lib().sta_moment_partials_layout(n, dv, ctypes.byref(rows), ctypes.byref(ld), ctypes.byref(off)),
          "sta_moment_partials_layout")
    return rows.value, ld.value, off.value


def decode_layout(d: int, dv: int) -> tuple:
    """(dk, ldv): row lengths of the decode buffers for keys and values (zero-padded columns)."""
    dk, ldv = _i32(), _i32()
    check(lib().sta_decode_layout(d, dv, ctypes.byref(dk), ctypes.byref(ldv)), "sta_decode_layout")
    return dk.value, ldv.value


DEC_APPEND, DEC_CURRENT, DEC_QUERY = 1, 2, 4


def limits() -> dict:
    vals = [_i32() for _ in range(4)]
    lib().sta_limits(*[ctypes.byref(x) for x in vals])
    return {"max_d": vals[0].value, "max_dv": vals[1].value, "max_degree": vals[2].value, "max_compress_in": vals[3].value}


def moment_wide_tiles(d: int, degree: int, dv: int, products: int) -> tuple:
    """Per-wave tile counts the 64-column moment kernels run for (d, degree, dv, products)."""
    lib_ = lib()
    return tuple(nt for nt in (5,) if lib_.sta_moment_columns_ok(d, degree, dv, nt, products))


WS_SLOT_TILES = (2, 3, 4, 5)  # candidates the planner offers sta_moments_ws_ok


def moment_ws_slot_tiles(d: int, degree: int, column_tiles: int, dv: int) -> tuple:
    """Tiles per slot the wave-specialised moment kernel runs for (d, degree, column_tiles, dv)."""
    lib_ = lib()
    return tuple(nt for nt in WS_SLOT_TILES if lib_.sta_moments_ws_ok(d, degree, nt, column_tiles, dv))
