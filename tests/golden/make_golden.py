"""Write the golden vectors under tests/golden/ from the reference implementation.

Run in the development container only (the reference tree is not available on the GPU machines):

    python tests/golden/make_golden.py [/path/to/reference] [case ...]

With case names, only those cases are written (the selection cases below: selection_dtypes,
selection_near_ties); without, every case.

The reference's public functions are called on fixed synthetic inputs.  While they run, the torch
RNG calls (randn / rand / randperm) and argsort are wrapped so that the draws the reference consumed,
the projection scores it sorted and the order it obtained are recorded exactly.  Kept coreset items
are mapped back to token indices by exact row match.  Only data (inputs, draws, selected indices,
outputs) is written; no reference code is stored.
"""

from __future__ import annotations

import importlib
import json
import pathlib
import sys

import numpy as np
import torch

OUT = pathlib.Path(__file__).resolve().parent
REF = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
ONLY = set(sys.argv[2:])


class Recorder:
    """Wraps torch.randn/rand/randperm/argsort while active and logs their results."""

    def __init__(self):
        self.log = []
        self._orig = {}

    def __enter__(self):
        for name in ("randn", "rand", "randperm", "argsort"):
            orig = getattr(torch, name)
            self._orig[name] = orig

            def wrapped(*args, _orig=orig, _name=name, **kwargs):
                out = _orig(*args, **kwargs)
                if _name == "argsort":
                    self.log.append(("argsort", args[0].detach().clone(), out.detach().clone()))
                elif kwargs.get("generator") is not None:
                    self.log.append((_name, None, out.detach().clone()))
                return out

            setattr(torch, name, wrapped)
        return self

    def __exit__(self, *exc):
        for name, orig in self._orig.items():
            setattr(torch, name, orig)


def token_index(k: torch.Tensor, rows: torch.Tensor) -> np.ndarray:
    """Map each row of `rows` to the unique index of the identical row of k."""
    eq = (rows[:, None, :] == k[None, :, :]).all(-1)
    assert bool((eq.sum(-1) == 1).all()), "coreset rows must match exactly one key row"
    return eq.float().argmax(-1).numpy().astype(np.int64)


def calls_from_log(log, kind_of_call):
    """Group the RNG/argsort log into compress calls."""
    calls = []
    i = 0
    while i < len(log):
        name, inp, out = log[i]
        if name == "randn":
            _, _, u = log[i + 2] if log[i + 1][0] == "argsort" else (None, None, None)
            rec = {"method": "sorted_pair", "direction_raw": out.numpy()}
            assert log[i + 1][0] == "argsort" and log[i + 2][0] == "rand"
            rec["scores"] = log[i + 1][1].numpy()
            rec["order"] = log[i + 1][2].numpy()
            rec["uniforms"] = log[i + 2][2].numpy()
            calls.append(rec)
            i += 3
        elif name == "randperm":
            calls.append({"method": "perm", "perm": out.numpy()})
            i += 1
        else:
            raise AssertionError(f"unexpected RNG call {name}")
    return calls


def save(name: str, arrays: dict, meta: dict) -> None:
    arrays = {k: np.asarray(v) for k, v in arrays.items()}
    arrays["meta_json"] = np.frombuffer(json.dumps(meta, sort_keys=True).encode(), dtype=np.uint8)
    np.savez_compressed(OUT / f"{name}.npz", **arrays)
    print(f"wrote {name}.npz ({sum(a.nbytes for a in arrays.values())} raw bytes)")


def cpu_model() -> str:
    for line in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
        if line.startswith("model name"):
            return line.split(":", 1)[1].strip()
    return "unknown"


def spied_levels(stc, k, run):
    """Runs `run()` with MergeReduceCoreset._compress wrapped; returns every call's (src_in, w_in, src_out,
    w_out) as token indices into k and weights (float64 for the 16-bit and float64 runs)."""
    compressed = []
    orig = stc.MergeReduceCoreset._compress

    def spy(self, block):
        out = orig(self, block)
        compressed.append((token_index(k, block.keys), block.weights.double().numpy().copy(),
                           token_index(k, out.keys), out.weights.double().numpy().copy()))
        return out

    stc.MergeReduceCoreset._compress = spy
    try:
        result = run()
    finally:
        stc.MergeReduceCoreset._compress = orig
    return result, compressed


def selection_cases(faa, stc, base_meta) -> None:
    """Coreset selections of the reference in each input dtype (its draws and pair rule run in the keys'
    dtype), and on keys whose projections nearly tie (rows repeated with one coordinate moved by one
    ulp), where the order of torch's CPU `keys @ direction` decides which token is kept.  The host's
    CPU model goes into the metadata: the near-tie orders belong to its BLAS code path."""
    cpu = torch.device("cpu")
    if not ONLY or "selection_dtypes" in ONLY:
        arrays, meta = {}, dict(base_meta, cpu_model=cpu_model(), cases=[])
        for tag, dtype in (("f64", torch.float64), ("bf16", torch.bfloat16), ("f16", torch.float16)):
            n, d, dv, B, seed = 320, 16, 8, 32, 13
            q, k, v = faa._make_data(n, d, dv, radius=1.0, data="unit_ball", device=cpu, dtype=dtype, seed=seed)
            out, calls = spied_levels(stc, k, lambda: stc.article_causal_attention(
                q, k, v, degree=2, block_size=B, scale=1.0, compressor="sorted_pair", seed=seed))
            arrays[f"{tag}_k"] = k.double().numpy()
            arrays[f"{tag}_levels_ncalls"] = np.array(len(calls))
            for ci, (si, wi, so, wo) in enumerate(calls):
                arrays[f"{tag}_levels_call{ci}_src_out"] = so
                arrays[f"{tag}_levels_call{ci}_w_out"] = wo
            reps = faa._build_completed_block_reps(k, v, block_size=B, compressor="sorted_pair", seed=seed)
            arrays[f"{tag}_flat_rep_idx"] = token_index(k, reps.keys)
            arrays[f"{tag}_flat_rep_w"] = reps.weights.double().numpy()
            meta["cases"].append(dict(tag=tag, n=n, d=d, dv=dv, block=B, seed=seed))
        save("selection_dtypes", arrays, meta)
    if not ONLY or "selection_near_ties" in ONLY:
        n_base, copies, d, dv, B, seed = 48, 8, 16, 8, 32, 21
        g = torch.Generator().manual_seed(seed)
        base = torch.randn(n_base, d, generator=g) * 0.5
        k = base.repeat_interleave(copies, 0)
        for r in range(k.shape[0]):
            j = r % copies
            if j:
                c = j - 1
                k[r, c] = torch.nextafter(k[r, c], torch.tensor(float("inf")))
        perm = torch.randperm(k.shape[0], generator=g)
        k = k[perm].contiguous()
        n = k.shape[0]
        q = torch.randn(n, d, generator=g) * 0.5
        v = torch.randn(n, dv, generator=g)
        _, calls = spied_levels(stc, k, lambda: stc.article_causal_attention(
            q, k, v, degree=2, block_size=B, scale=1.0, compressor="sorted_pair", seed=seed))
        arrays = {"q": q.numpy(), "k": k.numpy(), "v": v.numpy(), "levels_ncalls": np.array(len(calls))}
        for ci, (si, wi, so, wo) in enumerate(calls):
            arrays[f"levels_call{ci}_src_out"] = so
            arrays[f"levels_call{ci}_w_out"] = wo.astype(np.float32)
        reps = faa._build_completed_block_reps(k, v, block_size=B, compressor="sorted_pair", seed=seed)
        arrays["flat_rep_idx"] = token_index(k, reps.keys)
        arrays["flat_rep_w"] = reps.weights.numpy()
        save("selection_near_ties", arrays, dict(base_meta, cpu_model=cpu_model(), n=n, d=d, dv=dv, block=B,
                                                 seed=seed))


def main() -> None:
    sys.path.insert(0, str(REF))
    faa = importlib.import_module("fast_article_attention")
    stc = importlib.import_module("streaming_taylor_coreset_attention")
    taa = importlib.import_module("triton_article_attention")
    torch.set_num_threads(1)
    base_meta = {"torch": torch.__version__, "generator": "cpu"}
    if ONLY:
        selection_cases(faa, stc, base_meta)
        return

    # ---- flat fast path (config c1 shape) ----
    n, d, dv, B = 1024, 32, 32, 128
    q, k, v = faa._make_data(n, d, dv, radius=1.0, data="unit_ball", device=torch.device("cpu"),
                             dtype=torch.float32, seed=0)
    arrays = {"q": q.numpy(), "k": k.numpy(), "v": v.numpy()}
    arrays["out_none"] = faa.fast_article_causal_attention(q, k, v, degree=2, block_size=B, scale=1.0,
                                                           compressor="none", low_mode="stream").numpy()
    arrays["exact"] = faa.classical_causal_attention(q, k, v, scale=1.0).numpy()
    for comp in ("sorted_pair", "random"):
        with Recorder() as rec:
            reps = faa._build_completed_block_reps(k, v, block_size=B, compressor=comp, seed=0)
        calls = calls_from_log(rec.log, comp)
        arrays[f"{comp}_rep_idx"] = token_index(k, reps.keys)
        arrays[f"{comp}_rep_w"] = reps.weights.numpy()
        arrays[f"{comp}_rep_active"] = reps.active_from.numpy()
        arrays[f"{comp}_out"] = faa.fast_article_causal_attention(
            q, k, v, degree=2, block_size=B, scale=1.0, compressor=comp, seed=0, low_mode="stream").numpy()
        for ci, c in enumerate(calls):
            for key, val in c.items():
                if key != "method":
                    arrays[f"{comp}_call{ci}_{key}"] = val
        arrays[f"{comp}_ncalls"] = np.array(len(calls))
    low_num, low_den, f = faa.low_degree_taylor_causal_sums(q, k, v, degree=2, scale=1.0, mode="stream")
    arrays["low_num"] = low_num.numpy()
    arrays["low_den"] = low_den.numpy()
    save("flat_c1", arrays, dict(base_meta, n=n, d=d, dv=dv, block=B, scale=1.0, degree=2, seed=0,
                                 data="unit_ball", radius=1.0, features=f))

    # ---- [B,H,N,D] flat with per-sequence seeds (seed + b*H + h) ----
    bsz, heads, n2, d2, dv2, B2 = 2, 3, 200, 16, 8, 32
    g = torch.Generator().manual_seed(5)
    q4 = torch.randn(bsz, heads, n2, d2, generator=g) * 0.3
    k4 = torch.randn(bsz, heads, n2, d2, generator=g) * 0.3
    v4 = torch.randn(bsz, heads, n2, dv2, generator=g)
    out4, st4 = faa.fast_article_causal_attention(q4, k4, v4, degree=2, block_size=B2, scale=None,
                                                  compressor="sorted_pair", seed=7, low_mode="stream",
                                                  return_stats=True)
    save("flat_bh", {"q": q4.numpy(), "k": k4.numpy(), "v": v4.numpy(), "out": out4.numpy(),
                     "stats": np.array([st4.degree, st4.block_size, st4.feature_count, st4.coreset_items,
                                        st4.approx_streaming_state_bytes, st4.scratch_low_prefix_bytes,
                                        st4.scratch_residual_matrix_bytes])},
         dict(base_meta, block=B2, seed=7, degree=2, scale=None))

    # ---- merge-and-reduce levels (streaming prototype semantics) ----
    def level_case(name, n, d, dv, B, degree, comp, radius, scale, seed):
        q, k, v = faa._make_data(n, d, dv, radius=radius, data="unit_ball", device=torch.device("cpu"),
                                 dtype=torch.float32, seed=seed)
        compressed = []
        orig = stc.MergeReduceCoreset._compress

        def spy(self, block):
            out = orig(self, block)
            compressed.append((token_index(k, block.keys), block.weights.numpy().copy(),
                               token_index(k, out.keys), out.weights.numpy().copy()))
            return out

        stc.MergeReduceCoreset._compress = spy
        try:
            with Recorder() as rec:
                out = stc.article_causal_attention(q, k, v, degree=degree, block_size=B, scale=scale,
                                                   compressor=comp, seed=seed)
        finally:
            stc.MergeReduceCoreset._compress = orig
        calls = calls_from_log(rec.log, comp)
        arrays = {"q": q.numpy(), "k": k.numpy(), "v": v.numpy(), "out": out.numpy(),
                  "exact": stc.classical_causal_attention(q, k, v, scale=scale).numpy(),
                  "ncalls": np.array(len(compressed))}
        for ci, (si, wi, so, wo) in enumerate(compressed):
            arrays[f"call{ci}_src_in"] = si
            arrays[f"call{ci}_w_in"] = wi
            arrays[f"call{ci}_src_out"] = so
            arrays[f"call{ci}_w_out"] = wo
        assert len(calls) == len([c for c in compressed if c[0].shape[0] > 1]) or comp == "none"
        for ci, c in enumerate(calls):
            for key, val in c.items():
                if key != "method":
                    arrays[f"call{ci}_{key}"] = val
        save(name, arrays, dict(base_meta, n=n, d=d, dv=dv, block=B, degree=degree, compressor=comp,
                                radius=radius, scale=scale, seed=seed))

    level_case("levels_c1", 1024, 32, 32, 64, 2, "sorted_pair", 1.0, 1.0, 0)
    level_case("levels_random", 256, 16, 8, 32, 2, "random", 1.0, 1.0, 3)
    level_case("levels_deg3", 256, 8, 8, 32, 3, "sorted_pair", 1.5, 1.0, 1)
    level_case("levels_oddblock", 300, 12, 5, 33, 2, "sorted_pair", 1.0, None, 2)
    level_case("levels_block2", 16, 4, 3, 2, 2, "sorted_pair", 1.0, 1.0, 4)

    # ---- flat with an odd block size (odd tail keeps weight 1) ----
    n, d, dv, B = 200, 12, 5, 33
    q, k, v = faa._make_data(n, d, dv, radius=1.0, data="unit_ball", device=torch.device("cpu"),
                             dtype=torch.float32, seed=9)
    with Recorder() as rec:
        reps = faa._build_completed_block_reps(k, v, block_size=B, compressor="sorted_pair", seed=9)
    calls = calls_from_log(rec.log, "sorted_pair")
    arrays = {"q": q.numpy(), "k": k.numpy(), "v": v.numpy(), "rep_idx": token_index(k, reps.keys),
              "rep_w": reps.weights.numpy(), "rep_active": reps.active_from.numpy(),
              "out": faa.fast_article_causal_attention(q, k, v, degree=2, block_size=B, scale=1.0,
                                                       compressor="sorted_pair", seed=9, low_mode="stream").numpy(),
              "ncalls": np.array(len(calls))}
    for ci, c in enumerate(calls):
        for key, val in c.items():
            if key != "method":
                arrays[f"call{ci}_{key}"] = val
    save("flat_oddblock", arrays, dict(base_meta, n=n, d=d, dv=dv, block=B, seed=9, scale=1.0, degree=2))

    # ---- Triton path's segment-mean coreset (CPU-runnable part) ----
    g = torch.Generator().manual_seed(11)
    k3 = torch.randn(2, 17, 4, generator=g)
    v3 = torch.randn(2, 17, 5, generator=g)
    rk, rv, rpb = taa.build_segment_mean_coreset(k3, v3, block_size=8, compress_stride=2)
    save("segment_mean", {"k": k3.numpy(), "v": v3.numpy(), "rep_k": rk.numpy(), "rep_v": rv.numpy(),
                          "reps_per_block": np.array(rpb)}, dict(base_meta, block=8, stride=2))

    # ---- feature map and exp_taylor values ----
    x = torch.linspace(-1.5, 1.5, 7 * 5).reshape(7, 5)
    save("features", {"x": x.numpy(),
                      "key2": faa._taylor_features_degree012(x, 2, key_side=True).numpy(),
                      "query2": faa._taylor_features_degree012(x, 2, key_side=False).numpy(),
                      "taylor3": faa.exp_taylor(x, 3).numpy()}, base_meta)
    selection_cases(faa, stc, base_meta)


if __name__ == "__main__":
    main()
