"""Device choice, timing and byte formatting shared by the command-line benchmarks of the three API
modules."""

from __future__ import annotations

import math
import statistics
import time
from typing import Callable, Optional, Tuple, Union

import torch

_UNITS = ("B", "KiB", "MiB", "GiB", "TiB")


def pick_device(spec: Optional[Union[str, torch.device]]) -> torch.device:
    """None or "auto": the first ROCm GPU when one is visible, else the CPU; anything else as given."""
    if spec is None or str(spec) == "auto":
        return torch.device("cuda" if torch.cuda.is_available() else "cpu")
    return torch.device(spec)


def settle(device: torch.device) -> None:
    """Wait for the work queued on a GPU device (no-op on the CPU)."""
    if device.type == "cuda":
        torch.cuda.synchronize(device)


def fmt_bytes(n: float) -> str:
    """n bytes in the largest binary unit (up to TiB) whose value stays below 1024, two decimals."""
    x = float(n)
    e = 0 if x == 0 else min(max(int(math.log2(abs(x))) // 10, 0), len(_UNITS) - 1)
    return f"{x / 1024.0 ** e:.2f} {_UNITS[e]}"


def wall_ms(fn: Callable[[], object], repeats: int, device: torch.device) -> Tuple[float, float]:
    """(median, min) host wall time in ms of `repeats` calls, each waited for, after one untimed call."""
    samples = []
    for i in range(repeats + 1):
        t0 = time.perf_counter()
        fn()
        settle(device)
        if i:
            samples.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(samples), min(samples)


def event_ms(fn: Callable[[], object], repeats: int, warmup: int = 3) -> float:
    """Median device time in ms of `repeats` calls, each between two HIP events on the current stream,
    after `warmup` untimed calls; the events are read after one final synchronisation."""
    for _ in range(warmup):
        fn()
    marks = []
    for _ in range(repeats):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        marks.append((a, b))
    torch.cuda.synchronize()
    return statistics.median(float(a.elapsed_time(b)) for a, b in marks)
