"""libstadraws.so (no GPU): the natively replayed compressor draws equal torch's Python generator
calls draw for draw, one-shot and continued across calls, and generator states round-trip in
torch.Generator's layout."""

import pathlib
import re

import numpy as np
import pytest
import torch

import _native
import _plan

ROOT = pathlib.Path(__file__).resolve().parents[1]


def test_library_exports_header_symbols():
    text = (ROOT / "include" / "stadraws.h").read_text()
    syms = set(re.findall(r"^\s*(?:int64_t|int|void\*|void|const char\*)\s+(sta_\w+)\s*\(", text, flags=re.M))
    assert len(syms) == 11
    lib = _native.draws_library()
    for s in syms:
        assert hasattr(lib, s), s


CASES = [
    # (seeds, call sizes, d, compressor)
    (tuple(range(32)), _plan.levels_plan(65536, 256, "sorted_pair").call_sizes[:40], 64, "sorted_pair"),
    ((7, 8, 9), _plan.levels_plan(16384, 128, "sorted_pair").call_sizes[:30], 16, "sorted_pair"),
    ((0, 3), [17, 2, 9, 1, 0, 33, 2, 64], 6, "sorted_pair"),  # d below the 16-wide normal fill
    ((5,), [31, 16, 3, 2], 5, "sorted_pair"),
    ((1, 2, 3, 4), [256, 128, 2, 1, 7], 64, "random"),
    ((11,), [64, 32], 24, "none"),
    ((2 ** 40 + 3, 12345), [100, 51, 50], 33, "sorted_pair"),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("seeds,sizes,d,comp", CASES)
def test_native_draws_equal_python_replay(seeds, sizes, d, comp, dtype):
    """The native replay equals torch's own calls, for float32 draws, the float64 draws of a float64
    caller (which consume the generator differently: different values, not a rounding) and the 16-bit
    draws of a 16-bit caller (their values held exactly in float32 tables)."""
    f64 = dtype == torch.float64
    nat, m_nat = _plan._collect_draws(list(seeds), list(sizes), d, comp, dtype=dtype)
    py, m_py = _plan._collect_draws_py(list(seeds), list(sizes), d, comp, dtype=dtype)
    assert m_nat == m_py
    for a, b in ((nat.dirs, py.dirs), (nat.unif, py.unif), (nat.perms, py.perms)):
        assert a.shape == b.shape and a.dtype == b.dtype
        assert np.array_equal(a, b)
    assert (nat.n_calls, nat.max_in) == (py.n_calls, py.max_in)
    if f64 and comp == "sorted_pair":
        assert nat.dirs.dtype == np.float64
        f32, _ = _plan._collect_draws(list(seeds), list(sizes), d, comp, False)
        drawn = np.abs(f32.dirs).sum(-1) > 0
        assert not np.allclose(nat.dirs[drawn], f32.dirs[drawn].astype(np.float64), atol=1e-6)


def test_draw_set_continues_and_round_trips_state():
    seeds = [4, 5, 6]
    sizes = [256, 256, 256, 2, 255]
    d, max_in = 32, 256
    one = _native.host_draws(seeds, sizes, d, "sorted_pair", max_in)
    ds = _native.DrawSet(seeds)
    first = ds.next(sizes[:2], d, "sorted_pair", max_in)
    state = ds.get_state()
    rest = ds.next(sizes[2:], d, "sorted_pair", max_in)
    for full, a, b in zip(one, first, rest):
        assert np.array_equal(full[:, :2], a) and np.array_equal(full[:, 2:], b)
    # the state after two calls is torch.Generator's after the same two calls
    for s, seed in enumerate(seeds):
        g = torch.Generator(device="cpu")
        g.manual_seed(seed)
        for n_in in sizes[:2]:
            _plan._draw_one_call(g, n_in, d, "sorted_pair")
        assert torch.equal(state[s], g.get_state())
    # restoring the state replays the rest
    other = _native.DrawSet([0, 0, 0])
    other.set_state(state)
    again = other.next(sizes[2:], d, "sorted_pair", max_in)
    for a, b in zip(rest, again):
        assert np.array_equal(a, b)
    with pytest.raises(ValueError):
        other.set_state(state[:2])


def test_bad_arguments_raise():
    with pytest.raises(ValueError):
        _native.host_draws([0], [8], 4, "bogus", 8)
    with pytest.raises(_native.NativeError, match="max_in"):
        _native.host_draws([0], [16], 4, "sorted_pair", 8)
