"""bench.py's host side without a GPU: the measured-traffic lines it reads from the committed
rocprofv3 summaries, the host CPU description of its CPU baseline, and the refusal of several GPUs."""

import pathlib
import subprocess
import sys

import bench

ROOT = pathlib.Path(__file__).resolve().parents[1]


def test_measured_traffic_reads_the_committed_profiles():
    for workload, kernel in (("prefill_levels_c3", "moments_ws_kernel"), ("prefill_levels_c4", "moments_ws_kernel"),
                             ("decode_levels_c5", "decode_moments_kernel"), ("flash_c3", "flash_attn_kernel")):
        t = bench.measured_traffic(workload, kernel)
        assert t is not None and t > 1e8, (workload, kernel)
    assert bench.measured_traffic("prefill_levels_c3", "no_such_kernel") is None
    assert bench.measured_traffic("no_such_workload", "moments_ws_kernel") is None


def test_host_cpus_describes_the_host():
    info, usable = bench.host_cpus()
    assert usable >= 1 and info["os_cpu_count"] >= 1 and info["cpus_allowed"] >= usable
    assert "cpu_model" in info


def test_several_gpus_are_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 2 and "one GPU" in r.stderr
