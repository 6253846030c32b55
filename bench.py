"""Headline benchmark: streaming Taylor + merge-and-reduce coreset causal attention prefill on one
MI355X.

Workload (default): batch 1 x 32 heads, N = 65536, d = dv = 64, Taylor degree 2 (2145 monomial
features), article block 256, scale 1/sqrt(64), sorted_pair compressor with log2(N/256) merge levels,
fp32; q and k uniform in the radius-1 ball, v ~ N(0, 1), seed 0 (synthetic, generated on the host in
the reference's draw order and copied to HBM before timing).

One step = one full forward through the public API path (moment scan K1, level-tree compressor K3,
fused residual + normalisation K2/K4).  Prints one JSON line:
  value = head-tokens/s (B*H*N / step time), roofline of the dominant kernel (the moment scan; its
  split-bf16 matrix-core products bound fp32-equivalent flops at a third of the bf16 peak) from HIP
  events recorded around its launches inside the timed region, and the CPU baseline: the reference
  CPU fast path (oracle restatement, flat sorted_pair coreset, stream moments) timed on
  a bounded sample of one head on this host's cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

`--workload decode_levels_c5` measures streaming decode instead: 64 x 32 = 2048 streams, each holding the
state after a 32768-token prefix (moments plus merge-and-reduce levels, block 256), d = dv = 64,
degree 2, scale 1/8, bf16 inputs q, k, v ~ N(0,1)/8 (generated on the GPU); one step = update(k, v) +
query(q) for every stream, block completions (compress + merges) included.  value = stream-tokens/s;
roofline of the moment-state read (HBM); CPU baseline = the reference's per-token streaming object
restated in oracle/, one stream with the same state sizes.

`--workload prefill_flat_c2` (8 x 16 heads, N = 4096, d = dv = 64, degree 2, block 256, scale 1/8, bf16
inputs ~ N(0, 1), the drop-in fast path with the flat sorted_pair coreset) and `--workload
prefill_levels_c4` (4 x 32 heads, N = 16384, d = 16, dv = 64, degree 3 (969 features), block 128, scale 1,
fp32, q and k in the radius-1.5 ball, levels) are the same measurement on the other prefill
configurations.

`--workload flash_c3` measures the exact causal softmax baseline (triton_flash_causal_attention) on the
default workload's inputs (1 x 32 heads, N = 65536, d = dv = 64, scale 1/8, fp32): value =
head-tokens/s, roofline of the flash kernel against the fp32 MFMA peak (algorithmic (d + dv) N (N + 1)
flop per head); CPU baseline = torch's fp32 softmax attention on the host over a bounded row sample.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for p in (str(ROOT / "streaming-attention_amd"),):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402

WORKLOAD = dict(workload="prefill_levels_c3", batch=1, heads=32, seq_len=65536, d=64, dv=64, degree=2, block=256,
                scale=0.125, compressor="sorted_pair", semantics="merge-and-reduce levels", data="unit_ball r=1",
                dtype="fp32", seed=0)

DECODE = dict(workload="decode_levels_c5", batch=64, heads=32, prefix=32768, d=64, dv=64, degree=2, block=256,
              scale=0.125, compressor="sorted_pair", data="N(0,1)/8", dtype="bf16", seed=0)

# the other prefill configurations, as secondary bench lines (`--workload`): the batched bf16 prefill
# through the drop-in fast path (flat coreset) and the degree-3 long-sequence prefill (levels)
PREFILL_C2 = dict(workload="prefill_flat_c2", batch=8, heads=16, seq_len=4096, d=64, dv=64, degree=2, block=256,
                  scale=0.125, compressor="sorted_pair", semantics="flat (fast_article_causal_attention)",
                  data="N(0,1)", dtype="bf16", seed=0)
PREFILL_C4 = dict(workload="prefill_levels_c4", batch=4, heads=32, seq_len=16384, d=16, dv=64, degree=3, block=128,
                  scale=1.0, compressor="sorted_pair", semantics="merge-and-reduce levels", data="unit_ball r=1.5",
                  dtype="fp32", seed=0)
PREFILL = {w["workload"]: w for w in (WORKLOAD, PREFILL_C2, PREFILL_C4)}

FLASH = dict(WORKLOAD, workload="flash_c3", semantics="exact causal softmax attention")
for _k in ("degree", "block", "compressor"):
    del FLASH[_k]

MFMA_FP32_PEAK_TFLOPS = 157.3
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense
# split-bf16 products: each fp32 product is three bf16 matrix-core products, so the matrix-core bound on
# fp32-equivalent flops is a third of the bf16 peak
SPLIT_BF16_PEAK_TFLOPS = MFMA_BF16_PEAK_TFLOPS / 3.0
HBM_PEAK_GBS = 8000.0


def make_inputs(batch, heads, n, d, dv, seed, radius=1.0, ball=True):
    """randn q, k, v then ball radii radius * rand^(1/d) for q then k (the reference's draw order,
    fast_article_attention.py:738-750); ball=False: q, k, v ~ N(0, 1)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    q = torch.randn(batch, heads, n, d, generator=g)
    k = torch.randn(batch, heads, n, d, generator=g)
    v = torch.randn(batch, heads, n, dv, generator=g)
    if not ball:
        return q, k, v
    qn = torch.clamp(torch.linalg.vector_norm(q, dim=-1, keepdim=True), min=1e-12)
    kn = torch.clamp(torch.linalg.vector_norm(k, dim=-1, keepdim=True), min=1e-12)
    rq = torch.rand(batch, heads, n, 1, generator=g).pow(1.0 / d) * radius
    rk = torch.rand(batch, heads, n, 1, generator=g).pow(1.0 / d) * radius
    return q / qn * rq, k / kn * rk, v


def measured_traffic(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary of
    this workload (calibrated against a copy of known size), or None when there is none."""
    path = ROOT / "profiles" / f"{workload}_hbm_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith(f"{kernel} traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def host_cpus():
    """The host the CPU baseline runs on: os.cpu_count(), the CPUs this process may use (its affinity
    mask, capped by a cgroup v2 cpu.max quota: threads beyond the share only contend) and the CPU model
    name (the one lscpu prints, read from /proc/cpuinfo).  Returns (info dict, usable thread count)."""
    allowed = len(os.sched_getaffinity(0))
    quota = None
    try:
        q_, p_ = pathlib.Path("/sys/fs/cgroup/cpu.max").read_text().split()
        if q_ != "max":
            quota = int(q_) / int(p_)
    except (OSError, ValueError):
        pass
    usable = max(1, min(allowed, int(quota) if quota else allowed))
    model = None
    try:
        for line in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"os_cpu_count": os.cpu_count(), "cpus_allowed": allowed, "cgroup_cpu_quota": quota,
            "cpu_model": model}, usable


def warm_median(fn, runs=3):
    """One untimed warm-up call of fn (returning a dict with "total_s"), then the median of `runs` calls
    (the reference's own timer discipline, fast_article_attention.py:761-770).  Returns (median
    result, every timed total)."""
    fn()
    res = sorted((fn() for _ in range(runs)), key=lambda r: r["total_s"])
    return res[len(res) // 2], [float(f"{r['total_s']:.4g}") for r in res]


def levels_cpu_sample(oracle, w, positions=8):
    """Seconds per head of the reference's level semantics on the host (article_causal_attention:
    ArticleStreamingAttention.update + query per token, streaming_taylor_coreset_attention.py:641-687),
    sampled: `block` consecutive steps (so exactly one block completion with its compress and merges)
    from each of `positions` evenly spaced prefixes, with the state sizes of that prefix; the mean
    per-step cost is scaled by N."""
    n, blk = w["seq_len"], w["block"]
    starts = [(j * n // positions) // blk * blk + blk // 2 for j in range(positions)]
    tot = 0.0
    for p in starts:
        t = oracle.time_decode_sample(dim=w["d"], value_dim=w["dv"], degree=w["degree"], block=blk,
                                      scale=w["scale"], prefix=p, steps=blk, seed=w["seed"])
        tot += t["s_per_step"]
    return {"total_s": tot / positions * n, "s_per_step": tot / positions, "prefixes": starts}


def cpu_baseline(q, k, v, w):
    """Reference CPU fast path on one head (bounded sample), via the oracle: one warm-up, then the
    median of 3 runs, with every usable host thread and with 1 thread; plus the reference's level
    semantics (the per-token streaming object, which is what the GPU computes) sampled the same way."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import reference_cpu as oracle

    info, threads = host_cpus()
    threads = int(os.environ.get("STA_CPU_THREADS", "0")) or threads
    rows = int(os.environ.get("STA_CPU_SAMPLE_ROWS", "4096"))
    rows1 = int(os.environ.get("STA_CPU_SAMPLE_ROWS_1T", "2048"))
    # 16-bit inputs: the oracle runs on their values upcast to fp32 (the GPU computes in fp32 too)
    qh, kh, vh = (x[0, 0].float().contiguous() for x in (q, k, v))

    def sample(r):
        return lambda: oracle.time_fast_path_sample(qh, kh, vh, degree=w["degree"], block=w["block"],
                                                    scale=w["scale"], seed=w["seed"], rows=r)

    n = w["seq_len"]
    torch.set_num_threads(threads)
    t, totals = warm_median(sample(rows))
    torch.set_num_threads(1)
    t1, totals1 = warm_median(sample(rows1))
    torch.set_num_threads(threads)
    lev, lev_totals = (warm_median(lambda: levels_cpu_sample(oracle, w))
                       if w["semantics"].startswith("merge") else (None, None))
    rows, rows1 = min(rows, n), min(rows1, n)
    general = " with the general feature map (the reference fast path raises for degree 3)" if w["degree"] > 2 else ""
    out = {
        "value": n / t["total_s"],
        "unit": "head-tokens/s",
        "cores": threads,
        "kind": "port",
        "extrapolated": True,
        "torch_threads": threads,
        **info,
        "one_thread_value": n / t1["total_s"],
        "runs_s_per_head": totals,
        "one_thread_runs_s_per_head": totals1,
        "sample": (f"reference CPU fast path restated in oracle/{general} (stream moments, flat sorted_pair coreset, "
                   f"query chunks of 2048), 1 head of the workload (N={n}); token loop, q x reps residual and "
                   f"in-block residual timed over the first {rows} rows ({rows1} at 1 thread) and scaled by "
                   f"N/rows, reps built for all N; 1 warm-up then the median of 3 runs; heads are independent "
                   f"and serial in the reference, so head-tokens/s holds for B*H heads; median per-part "
                   f"seconds/head {json.dumps({k2: round(v2, 3) for k2, v2 in t.items()})}"),
    }
    if lev is not None:
        out["levels_semantics"] = {
            "value": n / lev["total_s"],
            "unit": "head-tokens/s",
            "runs_s_per_head": lev_totals,
            "sample": (f"the reference's level semantics (per-token update + query of the streaming object, "
                       f"restated in oracle/), {w['block']} steps from each of the prefixes {lev['prefixes']} "
                       f"(one block completion each), mean {lev['s_per_step'] * 1e3:.3f} ms/step scaled by N; "
                       f"1 warm-up then the median of 3"),
        }
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default: prefill >= 10 steps and >= 0.3 s of GPU time; decode 256; flash 3)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps first (default: prefill >= 0.2 s of GPU time; decode 8; flash 1)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seq-len", type=int, default=None, help="override the prefill workload's N")
    ap.add_argument("--heads", type=int, default=None, help="override the prefill workload's heads")
    ap.add_argument("--workload", default=WORKLOAD["workload"],
                    choices=list(PREFILL) + [DECODE["workload"], FLASH["workload"]])
    ap.add_argument("--streams", type=int, default=DECODE["batch"] * DECODE["heads"], help="decode streams")
    ap.add_argument("--prefix", type=int, default=DECODE["prefix"], help="decode prefix tokens")
    ap.add_argument("--flash-dtype", default="fp32", choices=["fp32", "bf16", "fp16"],
                    help="input dtype of the flash workload (16-bit inputs run on the 16-bit matrix cores)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only copy a MIB-MiB fp32 tensor 3 times (calibration kernel for the HBM byte counters)")
    args = ap.parse_args()
    decode = args.workload == DECODE["workload"]
    flash = args.workload == FLASH["workload"]
    # prefill without --steps / --warmup: sized from a measured step (warm-up >= 0.2 s of GPU time, the
    # timed region >= 0.3 s and at least 10 steps), so a small workload is timed at steady clocks
    args.auto_steps = args.steps is None and not (decode or flash)
    args.auto_warmup = args.warmup is None and not (decode or flash)
    if args.steps is None:
        args.steps = 256 if decode else (3 if flash else 10)
    if args.warmup is None:
        args.warmup = 8 if decode else (1 if flash else 2)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the heads shard with no "
              f"communication across GPUs: one process per GPU runs its share of the heads)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2

    if args.copy_probe:
        src = torch.ones(args.copy_probe * (1 << 18), device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_each_way": src.numel() * 4, "copies": 3}))
        return 0

    if decode:
        return run_decode(args)
    if flash:
        return run_flash(args)

    import _engine
    import _plan
    import streaming_taylor_coreset_attention as stc

    import fast_article_attention as faa

    w = dict(PREFILL[args.workload])
    if args.seq_len is not None:
        w["seq_len"] = args.seq_len
    if args.heads is not None:
        w["heads"] = args.heads
    bh, n, d, dv = w["batch"] * w["heads"], w["seq_len"], w["d"], w["dv"]
    flat = w["semantics"].startswith("flat")
    ball = w["data"].startswith("unit_ball")
    in_dtype = {"fp32": torch.float32, "bf16": torch.bfloat16}[w["dtype"]]
    print(f"[bench] generating inputs {w['batch']}x{w['heads']}x{n}x{d}", file=sys.stderr, flush=True)
    q, k, v = make_inputs(w["batch"], w["heads"], n, d, dv, w["seed"],
                          radius=float(w["data"].split("r=")[1]) if ball else 1.0, ball=ball)
    q, k, v = q.to(in_dtype), k.to(in_dtype), v.to(in_dtype)  # bf16 inputs: generated in fp32, then cast
    dev = torch.device("cuda:0")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    q3, k3, v3 = qd.reshape(bh, n, d), kd.reshape(bh, n, d), vd.reshape(bh, n, dv)

    t_plan = time.perf_counter()
    plan = (_plan.flat_plan if flat else _plan.levels_plan)(n, w["block"], w["compressor"])
    _plan.draws_for(plan, _plan.sequence_seeds(w["seed"], bh), d, w["compressor"])
    t_plan = time.perf_counter() - t_plan

    def step(timer=None):
        return _engine.prefill(q3, k3, v3, degree=w["degree"], block=w["block"], scale=w["scale"],
                               semantics="flat" if flat else "levels", compressor=w["compressor"], seed=w["seed"],
                               out_dtype=in_dtype, timer=timer)

    # the public API path once, checked against the engine call the timing uses
    api = faa.fast_article_causal_attention if flat else stc.article_causal_attention
    api_out = api(qd, kd, vd, degree=w["degree"], block_size=w["block"], scale=w["scale"],
                  compressor=w["compressor"], seed=w["seed"])
    res = step()
    if args.auto_steps or args.auto_warmup:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(2):
            step()
        e1.record()
        torch.cuda.synchronize()
        est_s = max(e0.elapsed_time(e1) / 2e3, 1e-6)
        if args.auto_warmup:
            args.warmup = max(args.warmup, 3 + math.ceil(0.2 / est_s))
        if args.auto_steps:
            args.steps = min(2000, max(args.steps, math.ceil(0.3 / est_s)))
        done = 3
    else:
        done = 1
    for _ in range(args.warmup - done):
        step()
    torch.cuda.synchronize()
    assert torch.equal(res.out.reshape(api_out.shape), api_out)
    print(f"[bench] warmup done", file=sys.stderr, flush=True)

    # timed region: HIP events around the moment scan only (the roofline kernel); events around every
    # launch would add their own GPU time to the step
    timer = _engine.KernelTimer(only=("moments",))
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        step(timer)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = start.elapsed_time(end) / args.steps
    mom_tot, mom_launches = timer.totals_ms()["moments"]

    # per-kernel breakdown: 3 more steps with events around every launch
    brk = _engine.KernelTimer()
    b0 = torch.cuda.Event(enable_timing=True)
    b1 = torch.cuda.Event(enable_timing=True)
    b0.record()
    for _ in range(3):
        step(brk)
    b1.record()
    torch.cuda.synchronize()
    per_kernel = {name: {"ms_total": round(tot, 4), "launches": cnt, "ms_per_step": round(tot / 3, 4)}
                  for name, (tot, cnt) in brk.totals_ms().items()}
    per_kernel_step_ms = b0.elapsed_time(b1) / 3

    # the compressor alone: the same steps with its launches on the main stream, not overlapping the scan
    overlap = _engine.OVERLAP_COMPRESS
    _engine.OVERLAP_COMPRESS = False
    serial = _engine.KernelTimer()
    for _ in range(3):
        step(serial)
    torch.cuda.synchronize()
    _engine.OVERLAP_COMPRESS = overlap
    ser = serial.totals_ms()
    compress_alone = ({"ms_per_step": round(ser["compress"][0] / 3, 4), "launches_per_step": ser["compress"][1] // 3}
                      if "compress" in ser else None)

    # cold calls through the public API, each at a seed no earlier call used: host draw replay, their
    # upload and the kernels (and, the second time, the plan of a shape seen for the first time)
    def cold_call(fresh_seed, clear_plans):
        if clear_plans:
            _plan._cache.clear()
            _engine._dev_cache.clear()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        api(qd, kd, vd, degree=w["degree"], block_size=w["block"], scale=w["scale"], compressor=w["compressor"],
            seed=fresh_seed)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3

    cold_ms = [cold_call(w["seed"] + 7919 * (i + 1), False) for i in range(3)]
    cold_plan_ms = cold_call(w["seed"] + 7919 * 4, True)

    # reference_scores=True: every compress call on the host in torch's CPU `keys @ direction` order (key
    # copy to the host, host draw replay and selection, node-table upload, then the GPU kernels); the
    # first call at a fresh seed, then the best of two more at that seed (draws cached)
    def ref_call(seed_):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        api(qd, kd, vd, degree=w["degree"], block_size=w["block"], scale=w["scale"], compressor=w["compressor"],
            seed=seed_, reference_scores=True)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3

    ref_cold_ms = ref_call(w["seed"] + 7919 * 6)
    ref_warm_ms = min(ref_call(w["seed"] + 7919 * 6) for _ in range(2))
    t0 = time.perf_counter()
    _plan.draws_for(plan, _plan.sequence_seeds(w["seed"] + 7919 * 5, bh), d, w["compressor"])
    draws_ms = (time.perf_counter() - t0) * 1e3

    f = _plan.num_features(d, w["degree"])
    mom_flops = 4.0 * f * (dv + 1) * bh * n  # algorithmic: update + query, 2*F*(dv+1) each per head-token
    mom_ms = mom_tot / mom_launches
    achieved = mom_flops / (mom_ms * 1e-3) / 1e12
    value = bh * n / (ms_step * 1e-3)
    split = _engine.MOMENT_PRODUCTS == _engine._native.PRODUCTS_SPLIT_BF16
    peak = SPLIT_BF16_PEAK_TFLOPS if split else MFMA_FP32_PEAK_TFLOPS

    line = {
        "metric": "head-tokens/sec, N=64K d=64 deg-2; % of HBM/MFMA roofline",
        "value": value,
        "unit": "head-tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "steps_rule": ("sized from a measured step: warm-up >= 0.2 s, timed region >= 0.3 s of GPU time and >= 10 "
                       "steps" if args.auto_steps else "as given"),
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": w,
        "roofline": {
            "kernel": f"{res.moment_kernel} (K1, exact Taylor moment scan)",
            "bound": "mfma",
            "achieved": achieved,
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": achieved / peak,
            "products": "split-bf16" if split else "fp32",
            "peak_basis": ("fp32-equivalent flops of split-bf16 products: bf16 dense peak / 3 (three bf16 "
                           "matrix-core products per fp32 product)" if split else "fp32 matrix-core peak"),
            "traffic": measured_traffic(w["workload"], res.moment_kernel),
            # the same fp32-equivalent rate against the bound fp32 matrix-core products would have
            "achieved_vs_fp32_mfma_peak": achieved / MFMA_FP32_PEAK_TFLOPS,
            "algorithmic_flops_per_launch": mom_flops,
            "avg_launch_ms": mom_ms,
        },
        "kernels": per_kernel,
        "kernels_note": ("3 steps after the timed region with HIP events around every launch (they take "
                         f"{per_kernel_step_ms:.4f} ms per step); "
                         + ("compress runs on a second stream overlapping moments; its HIP-event interval "
                            "includes the wait for compute units" if _engine.OVERLAP_COMPRESS else "")),
        "compress_alone": compress_alone,
        "host_plan_and_draws_s": round(t_plan, 3),
        "cold_call_ms": round(sorted(cold_ms)[1], 3),
        "cold_call_note": ("public API call at a seed no earlier call used (host draw replay for every sequence, "
                           "its upload, kernels; synchronised), median of 3; the warm ms_per_step reuses the "
                           "seed's cached draws"),
        "cold_call_new_shape_ms": round(cold_plan_ms, 3),
        "host_draws_fresh_seed_ms": round(draws_ms, 3),
        "reference_scores_ms": {"cold": round(ref_cold_ms, 3), "warm": round(ref_warm_ms, 3),
                                "note": ("public API call with reference_scores=True (compress calls run on the "
                                         "host in the order of torch's CPU keys @ direction; keys copied to "
                                         "the host); cold: a fresh seed; warm: the same seed again")},
        "host_threads": torch.get_num_threads(),
        "wall_s_timed_region": round(wall, 4),
    }
    if not args.no_cpu_baseline:
        print(f"[bench] timing CPU baseline", file=sys.stderr, flush=True)
        cb = cpu_baseline(q, k, v, w)
        line["cpu_baseline"] = cb
        line["speedup_vs_cpu_baseline"] = value / cb["value"]
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line))
    return 0


def run_flash(args) -> int:
    """Exact causal softmax attention throughput (see the module docstring)."""
    import _engine
    import triton_article_attention as taa

    in_dtype = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}[args.flash_dtype]
    w = dict(FLASH, dtype=args.flash_dtype)
    if args.seq_len is not None:
        w["seq_len"] = args.seq_len
    if args.heads is not None:
        w["heads"] = args.heads
    if args.flash_dtype != "fp32":
        w["workload"] = f"flash_c3_{args.flash_dtype}"
    bh, n, d, dv = w["batch"] * w["heads"], w["seq_len"], w["d"], w["dv"]
    print(f"[bench] flash: generating inputs {w['batch']}x{w['heads']}x{n}x{d}", file=sys.stderr, flush=True)
    q, k, v = (x.to(in_dtype) for x in make_inputs(w["batch"], w["heads"], n, d, dv, w["seed"]))
    dev = torch.device("cuda:0")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    q3, k3, v3 = qd.reshape(bh, n, d), kd.reshape(bh, n, d), vd.reshape(bh, n, dv)

    def step(timer=None):
        return _engine.flash(q3, k3, v3, scale=w["scale"], timer=timer)

    api_out = taa.triton_flash_causal_attention(qd, kd, vd, scale=w["scale"])
    out = step()
    for _ in range(args.warmup - 1):
        step()
    torch.cuda.synchronize()
    assert torch.equal(out.reshape(api_out.shape), api_out)
    print(f"[bench] flash: warmup done", file=sys.stderr, flush=True)

    timer = _engine.KernelTimer()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        step(timer)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = start.elapsed_time(end) / args.steps
    tot, cnt = timer.totals_ms()["flash"]
    k_ms = tot / cnt
    flops = float(d + dv) * n * (n + 1) * bh  # QK^T and PV over the n (n + 1) / 2 causal pairs
    achieved = flops / (k_ms * 1e-3) / 1e12
    value = bh * n / (ms_step * 1e-3)
    peak = MFMA_FP32_PEAK_TFLOPS if args.flash_dtype == "fp32" else MFMA_BF16_PEAK_TFLOPS
    line = {
        "metric": "head-tokens/sec, exact causal softmax attention, N=64K d=64; % of MFMA roofline",
        "value": value,
        "unit": "head-tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.flash_dtype,
        "data": "synthetic",
        "config": w,
        "roofline": {
            "kernel": ("flash_attn_kernel (online-softmax exact attention, fp32 matrix cores)" if args.flash_dtype == "fp32"
                       else "flash_attn16_kernel (online-softmax exact attention, 16-bit matrix cores: one product "
                            "for QK^T, two (P as hi + lo) for PV)"),
            "bound": "mfma",
            "achieved": achieved,
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": achieved / peak,
            "traffic": measured_traffic(w["workload"], "flash_attn_kernel"),
            "algorithmic_flops_per_launch": flops,
            "avg_launch_ms": k_ms,
        },
        "kernels": {"flash": {"ms_total": round(tot, 4), "launches": cnt}},
        "wall_s_timed_region": round(wall, 4),
    }
    if not args.no_cpu_baseline:
        print(f"[bench] flash: timing CPU baseline", file=sys.stderr, flush=True)
        info, threads = host_cpus()
        threads = int(os.environ.get("STA_CPU_THREADS", "0")) or threads
        chunk = 2048  # query rows per host product (the whole N x N logits of a head would be 17 GB)
        qh, kh, vh = q[0, 0].float(), k[0, 0].float(), v[0, 0].float()
        kt = kh.T.contiguous()
        los = list(range(0, n, chunk))
        # a chunk's cost grows with its prefix (its end row): time every eighth chunk and scale by the
        # ratio of the summed prefix lengths
        pick = los[len(los) % 8 // 2::8] if len(los) >= 8 else los
        cost = lambda lo: min(lo + chunk, n)  # noqa: E731

        def sample():
            t0 = time.perf_counter()
            for lo in pick:
                hi = min(lo + chunk, n)
                logits = (qh[lo:hi] @ kt[:, :hi]) * w["scale"]
                mask = torch.arange(hi)[None, :] > torch.arange(lo, hi)[:, None]
                o = torch.softmax(logits.masked_fill(mask, float("-inf")), dim=-1) @ vh[:hi]
                assert bool(torch.isfinite(o).all())
            return {"total_s": (time.perf_counter() - t0) * sum(map(cost, los)) / sum(map(cost, pick))}

        torch.set_num_threads(threads)
        t, totals = warm_median(sample)
        torch.set_num_threads(1)
        t1, _ = warm_median(sample, runs=1)
        torch.set_num_threads(threads)
        line["cpu_baseline"] = {
            "value": n / t["total_s"],
            "unit": "head-tokens/s",
            "cores": threads,
            "kind": "port",
            "extrapolated": True,
            "torch_threads": threads,
            **info,
            "one_thread_value": n / t1["total_s"],
            "runs_s_per_head": totals,
            "sample": (f"torch fp32 causal softmax attention on the host (the reference's "
                       f"torch_classical_causal_attention, triton_article_attention.py:123-143) over one head "
                       f"(N={n}) in blocks of {chunk} query rows against their prefix: {len(pick)} of the "
                       f"{len(los)} blocks timed and scaled by their share of the summed prefix lengths; 1 "
                       f"warm-up then the median of 3 (1 thread: one run after a warm-up)"),
        }
        line["speedup_vs_cpu_baseline"] = value / line["cpu_baseline"]["value"]
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line))
    return 0


def run_decode(args) -> int:
    """Streaming decode throughput (see the module docstring)."""
    import _engine
    import _plan
    import streaming_taylor_coreset_attention as stc

    w = dict(DECODE, prefix=args.prefix)
    s_total, d, dv = args.streams, w["d"], w["dv"]
    w["streams"] = s_total
    dev = torch.device("cuda:0")
    st = stc.ArticleStreamingAttention(d, dv, degree=w["degree"], block_size=w["block"], scale=w["scale"],
                                       compressor=w["compressor"], device=dev, dtype=torch.bfloat16, seed=w["seed"],
                                       streams=s_total)
    gen = torch.Generator(device=dev)
    gen.manual_seed(w["seed"])

    def draw(*shape):
        return (torch.randn(*shape, generator=gen, device=dev) * 0.125).to(torch.bfloat16)

    print(f"[bench] decode: building the state of {s_total} streams after {w['prefix']} tokens", file=sys.stderr,
          flush=True)
    t0 = time.perf_counter()
    chunk = 4096
    ext_timer = _engine.KernelTimer(only=("moment_accumulate",))  # the state accumulation of each chunk
    st._st.timer = ext_timer
    for lo in range(0, w["prefix"], chunk):
        n = min(chunk, w["prefix"] - lo)
        st.extend(draw(s_total, n, d), draw(s_total, n, dv))
    torch.cuda.synchronize()
    st._st.timer = None
    t_prefix = time.perf_counter() - t0
    ext_ms = [s_.elapsed_time(e_) for s_, e_ in ext_timer.events.get("moment_accumulate", [])]
    total = args.warmup + args.steps
    xs = draw(total + args.steps, 3, s_total, d)  # warm-up, timed steps, breakdown steps
    t0 = time.perf_counter()
    st._st.reserve_draws(total + args.steps)
    t_draws = time.perf_counter() - t0
    print(f"[bench] decode: prefix {t_prefix:.1f}s, draws {t_draws:.1f}s; warmup", file=sys.stderr, flush=True)
    for i in range(args.warmup):
        st.step(xs[i, 0], xs[i, 1], xs[i, 2])
    torch.cuda.synchronize()
    # timed region: HIP events around the moment-state read only (the roofline kernel)
    timer = _engine.KernelTimer(only=("decode_moments",))
    st._st.timer = timer
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    start.record()
    for i in range(args.warmup, total):
        st.step(xs[i, 0], xs[i, 1], xs[i, 2])
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = start.elapsed_time(end) / args.steps
    mom_tot, mom_launches = timer.totals_ms()["decode_moments"]
    # per-kernel breakdown: as many steps again, with events around every launch
    brk = _engine.KernelTimer()
    st._st.timer = brk
    for i in range(total, total + args.steps):
        st.step(xs[i, 0], xs[i, 1], xs[i, 2])
    torch.cuda.synchronize()
    st._st.timer = None
    per_kernel = {name: {"ms_total": round(tot, 4), "launches": cnt, "ms_per_launch": round(tot / cnt, 5)}
                  for name, (tot, cnt) in brk.totals_ms().items()}
    f = _plan.num_features(d, w["degree"])
    state_bytes = s_total * f * (dv + 1) * 4  # algorithmic: the moment state is read once per step
    mom_ms = mom_tot / mom_launches
    achieved = state_bytes / (mom_ms * 1e-3) / 1e9
    value = s_total / (ms_step * 1e-3)  # every stream advances one token per step
    line = {
        "metric": "decode stream-tokens/sec (update + query per stream), prefix 32K, d=64 deg-2; % of HBM roofline",
        "value": value,
        "unit": "stream-tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 inputs, fp32 state",
        "data": "synthetic",
        "config": w,
        "roofline": {
            "kernel": "decode_moments_kernel (moment-state read of every stream)",
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": measured_traffic(w["workload"], "decode_moments_kernel"),
            "algorithmic_bytes_per_launch": state_bytes,
            "avg_launch_ms": mom_ms,
        },
        "kernels": per_kernel,
        "kernels_note": "the steps after the timed region, with HIP events around every launch",
        "block_completions_timed": (w["prefix"] + total) // w["block"] - (w["prefix"] + args.warmup) // w["block"],
        "block_completions_breakdown": ((w["prefix"] + total + args.steps) // w["block"]
                                        - (w["prefix"] + total) // w["block"]),
        "host_prefix_build_s": round(t_prefix, 3),
        "extend_accumulate_ms": [round(x, 3) for x in ext_ms],
        "extend_accumulate_note": (f"state accumulation of each extend() chunk of up to {chunk} tokens of every "
                                   "stream while the prefix is built (HIP events)"),
        "host_draws_s": round(t_draws, 3),
        "wall_s_timed_region": round(wall, 4),
    }
    if not args.no_cpu_baseline:
        sys.path.insert(0, str(ROOT / "oracle"))
        import reference_cpu as oracle

        info, threads = host_cpus()
        threads = int(os.environ.get("STA_CPU_THREADS", "0")) or threads
        torch.set_num_threads(threads)
        steps = int(os.environ.get("STA_CPU_DECODE_STEPS", "256"))
        print(f"[bench] timing CPU baseline ({steps} steps of one stream)", file=sys.stderr, flush=True)

        def sample():
            t = oracle.time_decode_sample(dim=d, value_dim=dv, degree=w["degree"], block=w["block"],
                                          scale=w["scale"], prefix=w["prefix"], steps=steps, seed=w["seed"])
            return dict(t, total_s=t["s_per_step"])

        t, totals = warm_median(sample)
        torch.set_num_threads(1)
        t1, _ = warm_median(sample)
        torch.set_num_threads(threads)
        cb = {"value": 1.0 / t["s_per_step"], "unit": "stream-tokens/s", "cores": threads, "kind": "port",
              "extrapolated": True, "torch_threads": threads, **info, "one_thread_value": 1.0 / t1["s_per_step"],
              "runs_s_per_step": totals,
              "sample": (f"reference ArticleStreamingAttention update+query restated in oracle/ (per-token torch "
                         f"ops), one stream with the state sizes after a {w['prefix']}-token prefix, {steps} steps "
                         f"(block completions included), 1 warm-up then the median of 3; the reference runs "
                         f"streams one after another, so stream-tokens/s holds for every stream count")}
        line["cpu_baseline"] = cb
        line["speedup_vs_cpu_baseline"] = value / cb["value"]
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
