"""RMSNorm against the reference's op sequence (needle/layers/norm.py:14-17).

The module normalises with torch's fused RMS normalisation and multiplies by the weight as
its own op; the reference runs x.float().pow(2).mean, rsqrt, the fp32 product, the cast and
the weight product one op at a time.  With weights other than one (so that the reference's
two roundings are exercised), in each model dtype: the same bits on the CPU; on the GPU the
fused kernel's fp32 statistic and reciprocal square root can differ from the separate
kernels' in their last bits, which moves a 16-bit element by an ulp now and then (at most 1
in 1000 of them, none by more than two ulps) and a float32 row by a few float32 ulps (the
bound: 8, i.e. a relative 2^-20, where a wrong eps, statistic or rounding is off by orders
of magnitude more).
"""
import pytest
import torch

from needle_amd.layers.norm import RMSNorm


def _reference(x, weight, eps):
    variance = x.float().pow(2).mean(-1, keepdim=True)       # norm.py:15
    y = x * torch.rsqrt(variance + eps)                      # norm.py:16
    return weight * y.to(weight.dtype)                       # norm.py:17


_MANTISSA = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}


def _check(device, dtype, rows, hidden, eps, exact=True):
    g = torch.Generator().manual_seed(rows + hidden)
    x = (torch.randn(rows, hidden, generator=g) * 3).to(dtype).to(device)
    norm = RMSNorm(hidden, eps).to(device=device, dtype=dtype)
    with torch.no_grad():
        norm.weight.copy_((torch.randn(hidden, generator=g) * 0.2 + 1).to(dtype))
        got = norm(x)
        want = _reference(x, norm.weight, eps)
    assert got.dtype == dtype and got.shape == x.shape
    got, want = got.cpu(), want.cpu()
    if exact:
        assert torch.equal(got, want)
        return
    d = (got.double() - want.double()).abs()
    ulp = want.double().abs() * 2.0 ** -_MANTISSA[dtype]
    if dtype == torch.float32:
        assert (d <= 8 * ulp).all(), f"max relative diff {(d / want.double().abs()).max():.3g}"
        return
    assert (d <= 2 * ulp).all(), f"max |diff| {d.max().item():.3g}"
    assert (got == want).double().mean().item() >= 0.999


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,hidden", [(1, 896), (37, 896), (8, 3584), (64, 4096)])
def test_rmsnorm_matches_reference_ops_cpu(dtype, rows, hidden):
    _check("cpu", dtype, rows, hidden, 1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,hidden", [(1, 896), (48, 896), (256, 896), (64, 4096)])
def test_rmsnorm_matches_reference_ops_gpu(dtype, rows, hidden):
    _check("cuda:0", dtype, rows, hidden, 1e-6, exact=False)
