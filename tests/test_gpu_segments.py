"""The segmented moment scan (sta_moments_ws_seg: few heads, each head's sequence cut into segments of
whole query blocks, a scan over the segment totals, then a query pass against each segment's starting
state) on the GPU: outputs within fp32 rounding of the whole-sequence scan and within the parity
tolerance of the oracle, coreset selections unchanged."""

import pytest
import torch

import _engine
import _native
import _plan
import reference_cpu as orc

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def rel(a, b):
    return orc.rel_l2(torch.as_tensor(a).float().cpu(), torch.as_tensor(b).float().cpu())


CASES = [
    # semantics, heads, n, d, dv, degree, block, dtype
    ("levels", 1, 16384, 64, 64, 2, 256, torch.float32),
    ("flat", 2, 8192, 64, 64, 2, 256, torch.bfloat16),
    ("levels", 1, 8192, 16, 64, 3, 128, torch.float32),
    ("levels", 3, 6000, 32, 40, 2, 64, torch.float32),
]


@pytest.mark.parametrize("semantics,heads,n,d,dv,degree,block,dtype", CASES)
def test_segmented_scan_matches_whole_scan_and_oracle(monkeypatch, semantics, heads, n, d, dv, degree, block, dtype):
    print(f"segments: {semantics} heads={heads} n={n} d={d} dv={dv} degree={degree} block={block} {dtype}",
          flush=True)
    ft = _plan.feature_tiles(_engine._unit_width(d, torch.tensor([], dtype=dtype).element_size()), degree)
    ct = 4 if (-(-dv // 32)) % 2 == 0 else 2
    opts = _native.moment_ws_slot_tiles(ft.d, degree, ct, dv)
    shift = 1 if semantics == "levels" else 0
    nseg, _ = _plan.ws_segments(n, shift, block, heads, ft, dv, opts, ct)
    assert nseg > 1
    q, k, v = orc.make_data((heads,), n, d, dv, radius=1.0, data="unit_ball", seed=11)
    q, k, v = (x.to(dtype) for x in (q, k, v))
    kw = dict(degree=degree, block=block, scale=1.0, semantics=semantics, compressor="sorted_pair", seed=3,
              out_dtype=torch.float32)
    seg = _engine.prefill(q.to(DEV), k.to(DEV), v.to(DEV), **kw)
    monkeypatch.setattr(_engine, "WS_SEGMENTS", False)
    whole = _engine.prefill(q.to(DEV), k.to(DEV), v.to(DEV), **kw)
    torch.cuda.synchronize()
    assert seg.moment_kernel == whole.moment_kernel == "moments_ws_kernel"
    assert torch.equal(seg.node_src, whole.node_src) and torch.equal(seg.node_w, whole.node_w)
    assert rel(seg.out, whole.out) < 2e-6
    tol = 1e-4 if dtype == torch.float32 else 5e-3
    fwd = orc.levels_forward if semantics == "levels" else orc.fast_path_forward
    for h in sorted({0, heads - 1}):
        ref = fwd(q[h].float(), k[h].float(), v[h].float(), degree=degree, block=block, scale=1.0,
                  compressor="sorted_pair", seed=3 + h)
        assert rel(seg.out[h], ref) < tol
