"""bf16 inputs take instantiations that leave out the split products with the zero lo planes of exact
bf16 keys and values (the moment scan's update and the residual kernel).  With the same values given
as fp32 the kernels run the full three-product form, whose extra products are then exactly zero: the
outputs must be equal bit for bit."""

import pytest
import torch

import _engine
import reference_cpu as orc

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")

CASES = [
    # semantics, heads, n, d, dv, degree, block
    ("flat", 4, 4096, 64, 64, 2, 256),
    ("levels", 3, 5000, 64, 64, 2, 256),
    ("levels", 2, 3000, 16, 64, 3, 128),
    ("flat", 2, 700, 32, 40, 2, 64),
    ("levels", 1, 20000, 64, 64, 2, 256),  # segmented scan
]


@pytest.mark.parametrize("semantics,heads,n,d,dv,degree,block", CASES)
def test_bf16_inputs_equal_their_fp32_upcast(semantics, heads, n, d, dv, degree, block):
    print(f"bf16 exact: {semantics} heads={heads} n={n} d={d} dv={dv} degree={degree} block={block}", flush=True)
    q, k, v = orc.make_data((heads,), n, d, dv, radius=1.0, data="unit_ball", seed=21)
    q, k, v = (x.to(torch.bfloat16).to(DEV) for x in (q, k, v))
    kw = dict(degree=degree, block=block, scale=0.125, semantics=semantics, compressor="sorted_pair", seed=5,
              out_dtype=torch.float32)
    low = _engine.prefill(q, k, v, **kw)
    full = _engine.prefill(q.float(), k.float(), v.float(), **kw)
    torch.cuda.synchronize()
    assert torch.equal(low.node_src, full.node_src) and torch.equal(low.node_w, full.node_w)
    assert torch.equal(low.out, full.out)
