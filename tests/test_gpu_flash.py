"""GPU parity of the exact causal flash baseline (sta_flash_attention behind
triton_flash_causal_attention, triton_article_attention.py:580-637) against the oracle: float64 causal
softmax attention on the same (upcast) inputs, and the oracle's blocked online-softmax recursion.

The kernel's products are exact fp32 products of the inputs and its sums fp32, so every input dtype is
held to rel-L2 <= 2e-5 against float64 (the reference holds its tf32 Triton kernel to 2e-2,
test_triton_article_attention.py:69); 16-bit outputs to their rounding."""

import pytest
import torch

import reference_cpu as orc
import triton_article_attention as taa

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 2e-5


def rel(a, b):
    return orc.rel_l2(torch.as_tensor(a).cpu(), torch.as_tensor(b).cpu())


def classical(q, k, v, scale):
    """float64 reference per [.., N, D] sequence."""
    return orc.classical_attention(q.float(), k.float(), v.float(), scale)


@pytest.mark.parametrize("lead,n,d,dv,dtype", [
    ((), 1, 16, 16, torch.float32),
    ((), 77, 8, 5, torch.float32),
    ((), 300, 20, 24, torch.float32),
    ((2, 3), 257, 64, 64, torch.float32),
    ((), 1000, 128, 256, torch.float32),
    ((), 513, 100, 130, torch.float32),
    ((1, 2), 129, 6, 3, torch.float32),
    ((2, 2), 400, 64, 64, torch.bfloat16),
    ((), 333, 32, 48, torch.float16),
    ((3, 1), 200, 128, 64, torch.bfloat16),
])
def test_flash_matches_softmax_attention(lead, n, d, dv, dtype):
    print(f"flash lead={lead} n={n} d={d} dv={dv} {dtype}", flush=True)
    g = torch.Generator().manual_seed(n * 7 + d)
    q = torch.randn(*lead, n, d, generator=g).to(dtype)
    k = torch.randn(*lead, n, d, generator=g).to(dtype)
    v = torch.randn(*lead, n, dv, generator=g).to(dtype)
    out = taa.triton_flash_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    assert out.shape == (*lead, n, dv) and out.dtype == torch.float32
    assert rel(out, classical(q, k, v, d ** -0.5)) < TOL


def test_flash_large_logits_use_the_running_maximum():
    # logits in the hundreds: exp without the running maximum would overflow fp32
    g = torch.Generator().manual_seed(5)
    q = torch.randn(600, 32, generator=g)
    k = torch.randn(600, 32, generator=g)
    v = torch.randn(600, 16, generator=g)
    out = taa.triton_flash_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV), scale=4.0)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert rel(out, classical(q, k, v, 4.0)) < 1e-4
    assert rel(out, orc.flash_attention_blocked(q, k, v, 4.0, 64)) < 1e-4


@pytest.mark.parametrize("out_dtype,tol", [(torch.bfloat16, 8e-3), (torch.float16, 1e-3)])
def test_flash_output_dtypes(out_dtype, tol):
    g = torch.Generator().manual_seed(9)
    q, k, v = (torch.randn(2, 2, 190, 48, generator=g) for _ in range(3))
    out = taa.triton_flash_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV), scale=0.2, output_dtype=out_dtype)
    torch.cuda.synchronize()
    assert out.dtype == out_dtype
    assert rel(out.float(), classical(q, k, v, 0.2)) < tol


def test_flash_long_sequence_two_heads():
    g = torch.Generator().manual_seed(11)
    q, k = (torch.randn(2, 4096, 64, generator=g) * 0.5 for _ in range(2))
    v = torch.randn(2, 4096, 64, generator=g)
    out = taa.triton_flash_causal_attention(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV), scale=0.125)
    torch.cuda.synchronize()
    assert rel(out[0], classical(q, k, v, 0.125)) < TOL


def test_flash_strided_inputs_and_default_scale():
    g = torch.Generator().manual_seed(13)
    big = torch.randn(300, 80, generator=g)
    q, k, v = big[:, :24], big[:, 24:48], big[:, 48:78]  # column slices of one tensor
    out = taa.triton_flash_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    assert rel(out, classical(q, k, v, 24 ** -0.5)) < TOL


def test_reference_triton_numerics_case():
    # test_triton_article_attention.py:48-69: fp16 inputs, flash and the stride-1 article path vs exact
    torch.manual_seed(0)
    n, d, dv = 64, 16, 16
    q = (torch.randn(n, d, dtype=torch.float16) / d ** 0.5).to(DEV)
    k = (torch.randn(n, d, dtype=torch.float16) / d ** 0.5).to(DEV)
    v = torch.randn(n, dv, dtype=torch.float16).to(DEV)
    exact = taa.torch_classical_causal_attention(q.float(), k.float(), v.float(), scale=1.0)
    flash = taa.triton_flash_causal_attention(q, k, v, scale=1.0, output_dtype=torch.float32)
    article = taa.triton_article_causal_attention(q, k, v, degree=2, block_size=16, compress_stride=1, scale=1.0,
                                                  output_dtype=torch.float32)
    torch.cuda.synchronize()
    assert taa.safe_relative_l2(flash, exact) < 2e-2
    assert taa.safe_relative_l2(article, exact) < 2e-2
    assert rel(flash, classical(q.cpu(), k.cpu(), v.cpu(), 1.0)) < TOL


def test_flash_argument_errors():
    q = torch.randn(8, 129, device=DEV)
    with pytest.raises(ValueError):
        taa.triton_flash_causal_attention(q, q, torch.randn(8, 4, device=DEV))
    q = torch.randn(8, 16, device=DEV)
    with pytest.raises(ValueError):
        taa.triton_flash_causal_attention(q, q, torch.randn(8, 257, device=DEV))
    with pytest.raises(ValueError):
        taa.triton_flash_causal_attention(q, q[:4], torch.randn(8, 4, device=DEV))
