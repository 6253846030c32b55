"""Build libstreamattn.so in-tree for gfx950 with hipcc.

    python streaming-attention_amd/build_native.py

The library is 99 objects compiled in parallel and linked into one shared object: api.hip (entry
points, compressor and decode kernels), launch_moments_ws.hip (the wave-specialised moment scan, per
element size and column-tile count), launch_moments.hip (fp32 and split-bf16 products, 32 or 64
columns), launch_accumulate.hip, and
launch_block.hip and launch_flash.hip once per residual / flash kernel configuration (padded key
width, value-column tiles, element size).  Objects go to streaming-attention_amd/_build/.

Packed-fp32 VALU instructions are disabled (-packed-fp32-ops): the kernels are written for the
scalar fp32 and MFMA paths.

libstadraws.so (csrc/host_draws.cpp, host only) is built beside it with g++ against torch's CPU
libraries: the replay of the compressor's seed-derived draws on torch's CPU generator.
"""

from __future__ import annotations

import os
import pathlib
import shutil
import subprocess
import sys
import time

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
# (source, object stem, defines), slowest first
UNITS = tuple(("launch_moments_ws.hip", f"launch_moments_ws_{es}_{ct}", (f"-DSTA_WS_ES={es}", f"-DSTA_WS_CT={ct}"))
              for es in (4, 2) for ct in (4, 2)) + (
    ("launch_moments.hip", "launch_moments_split", ("-DSTA_MOM_SPLIT=1",)),
    ("launch_moments.hip", "launch_moments_split64", ("-DSTA_MOM_SPLIT=1", "-DSTA_MOM_CG=64")),
    ("launch_moments.hip", "launch_moments", ("-DSTA_MOM_SPLIT=0",)),
    ("launch_accumulate.hip", "launch_accumulate", ()),
) + tuple(("launch_block.hip", f"launch_block_{dp}_{dvt}_{es}",
           (f"-DSTA_BLOCK_DP={dp}", f"-DSTA_BLOCK_DVT={dvt}", f"-DSTA_BLOCK_ES={es}"))
          for dp in (256, 128, 64, 32, 16) for dvt in (4, 2, 8, 1, 16) for es in (4, 2)) + tuple(
    ("launch_flash.hip", f"launch_flash_{dp}_{dvt}_{es}",
     (f"-DSTA_FLASH_DP={dp}", f"-DSTA_FLASH_DVT={dvt}", f"-DSTA_FLASH_ES={es}"))
    for dp in (128, 64, 32, 16) for dvt in (4, 2, 8, 1, 16) for es in (4, 2)) + (
    ("api.hip", "api", ()),
)
OBJDIR = HERE / "_build"
OUT = HERE / "libstreamattn.so"
DRAWS_OUT = HERE / "libstadraws.so"
ARCH = os.environ.get("STA_OFFLOAD_ARCH", "gfx950")
NOISE = "'-packed-fp32-ops' is not a recognized feature for this target"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def _flags() -> list[str]:
    return [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-Wall", "-Wno-unused-function"]


def _messages(res_out: str) -> list[str]:
    return [ln for ln in res_out.splitlines() if NOISE not in ln]


def _draws_cmd(out: pathlib.Path) -> list[str]:
    import torch.utils.cpp_extension as ext
    import torch

    inc = ext.include_paths()
    libs = ext.library_paths()
    return ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
            f"-D_GLIBCXX_USE_CXX11_ABI={int(torch.compiled_with_cxx11_abi())}",
            *[f"-I{d}" for d in inc], str(CSRC / "host_draws.cpp"), "-o", str(out),
            *[f"-L{d}" for d in libs], "-lc10", "-ltorch_cpu", *[f"-Wl,-rpath,{d}" for d in libs]]


def build(verbose: bool = False, only: str = "") -> pathlib.Path:
    """Compile every unit (or, with `only`, the units whose object stem starts with it, reusing the
    other objects from an earlier build) and link the library; libstadraws.so is rebuilt alongside
    unless `only` names HIP units."""
    OBJDIR.mkdir(exist_ok=True)
    with_host = not only or only == "host"
    hip_only = "\0" if only == "host" else only  # "\0": no HIP unit matches
    cc = hipcc()
    jobs = max(1, min(len(UNITS), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    pending = [u for u in UNITS if u[1].startswith(hip_only)]
    running, failed = [], []
    objs = [str(OBJDIR / f"{stem}.o") for _, stem, _ in UNITS if not stem.startswith(hip_only)]
    # every check that can refuse the build runs before any compiler process is started
    missing = [o for o in objs if not pathlib.Path(o).exists()]
    if missing:
        raise RuntimeError(f"objects of an earlier build are missing: {missing[:3]}; build without `only`")
    draws = None
    if with_host:
        tmp_d = DRAWS_OUT.with_suffix(".so.tmp")
        cmd = _draws_cmd(tmp_d)
        if verbose:
            print(" ".join(cmd), flush=True)
        dlog = open(OBJDIR / "host_draws.log", "w+")
        draws = (dlog, tmp_d, subprocess.Popen(cmd, stdout=dlog, stderr=subprocess.STDOUT))
    t0 = time.time()
    while pending or running:
        while pending and len(running) < jobs:
            src, stem, defs = pending.pop(0)
            obj = OBJDIR / f"{stem}.o"
            cmd = [cc, *_flags(), *defs, "-c", str(CSRC / src), "-o", str(obj)]
            if verbose:
                print(" ".join(cmd), flush=True)
            log = open(OBJDIR / f"{stem}.log", "w+")  # a file, not a pipe: long diagnostics cannot block
            running.append((stem, log, subprocess.Popen(cmd, stdout=log, stderr=subprocess.STDOUT)))
            objs.append(str(obj))
        time.sleep(0.2)
        for item in [r for r in running if r[2].poll() is not None]:
            running.remove(item)
            stem, log, p = item
            log.seek(0)
            msgs = _messages(log.read())
            log.close()
            if p.returncode != 0:
                failed.append(f"{stem}:\n" + "\n".join(msgs))
            elif verbose and msgs:
                print("\n".join(msgs))
            if verbose:
                print(f"  {stem}: done at {time.time() - t0:.0f} s", flush=True)
    if draws is not None:
        dlog, tmp_d, p = draws
        p.wait()
        dlog.seek(0)
        msg = dlog.read()
        dlog.close()
        if p.returncode != 0:
            failed.append("host_draws.cpp:\n" + msg)
        else:
            os.replace(tmp_d, DRAWS_OUT)
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n".join(failed))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    msgs = _messages(res.stdout + res.stderr)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + "\n".join(msgs))
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True, only=sys.argv[1] if len(sys.argv) > 1 else ""))
    sys.exit(0)
