"""The decoder layer's elementwise ops against the reference's op sequences.

RMSNorm (needle/layers/norm.py:14-17) and the residual add before it (needle/model/qwen2.py:58,
:63): x.float().pow(2).mean, rsqrt, the fp32 product, the cast and the weight product, one op
at a time, after `residual + x` in the model dtype.  On the CPU the module runs torch ops:
the same bits.  On the GPU it is one HIP kernel (ndl_rms_norm): the residual sum is the
same bits (one rounding of an exact fp32 sum); the normalised output can differ from the
separate kernels' in its last bits, since the fp32 sum of squares is added in another order
(16-bit formats: at most 1 in 1000 elements differ, none by more than two ulps; float32:
within 8 ulps, i.e. a relative 2^-20, where a wrong eps, statistic or rounding is off by
orders of magnitude more).  Weights other than one exercise the reference's two roundings.

SiLU(gate) * up (needle/model/llama.py:37): on the GPU one HIP kernel (ndl_silu_mul) against
torch's F.silu(gate) * up on the same GPU, and against the fp64 closed form
g / (1 + exp(-g)) rounded to the dtype, times up, rounded again.  The SiLU's fp32 exponential
may differ from torch's (or from fp64) in its last bit, which reaches the rounded SiLU
rarely; a SiLU one ulp off moves the product by up to two ulps of the format after its own
rounding (16-bit formats: at most 1 in 1000 elements differ, none by more than two ulps;
float32: within 4 ulps).
"""
import pytest
import torch
import torch.nn.functional as F

from needle_amd.layers.norm import RMSNorm

DTYPES = [torch.bfloat16, torch.float16, torch.float32]
_MANTISSA = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}


def _reference(x, weight, eps):
    variance = x.float().pow(2).mean(-1, keepdim=True)       # norm.py:15
    y = x * torch.rsqrt(variance + eps)                      # norm.py:16
    return weight * y.to(weight.dtype)                       # norm.py:17


def _inputs(device, dtype, rows, hidden, eps):
    g = torch.Generator().manual_seed(rows + hidden)
    x = (torch.randn(rows, hidden, generator=g) * 3).to(dtype).to(device)
    res = (torch.randn(rows, hidden, generator=g) * 2).to(dtype).to(device)
    norm = RMSNorm(hidden, eps).to(device=device, dtype=dtype)
    with torch.no_grad():
        norm.weight.copy_((torch.randn(hidden, generator=g) * 0.2 + 1).to(dtype))
    return x, res, norm


def _ulp(want, dtype):
    """The spacing of the format at each value of want (subnormal spacing near zero)."""
    fi = torch.finfo(dtype)
    tiny = fi.smallest_normal * fi.eps
    _, e = torch.frexp(want.abs())
    ulp = torch.clamp(torch.ldexp(torch.ones_like(want), e - 1 - _MANTISSA[dtype]), min=tiny)
    return torch.where(want == 0, torch.full_like(want, tiny), ulp)


def _close(got, want, dtype, max_ulps16=2, max_ulps32=8, min_equal=0.999):
    assert got.dtype == want.dtype and got.shape == want.shape
    got, want = got.cpu().double(), want.cpu().double()
    d = (got - want).abs()
    ulps = d / _ulp(want, dtype)
    equal = (got == want).double().mean().item()
    if dtype == torch.float32:
        assert ulps.max() <= max_ulps32, f"{ulps.max():.3g} ulps (equal {equal:.5f})"
        return
    assert ulps.max() <= max_ulps16, f"{ulps.max():.3g} ulps (equal {equal:.5f})"
    assert equal >= min_equal, f"only {equal:.5f} of the elements are equal"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,hidden", [(1, 896), (37, 896), (8, 3584), (64, 4096)])
def test_rmsnorm_matches_reference_ops_cpu(dtype, rows, hidden):
    x, res, norm = _inputs("cpu", dtype, rows, hidden, 1e-6)
    with torch.no_grad():
        assert torch.equal(norm(x), _reference(x, norm.weight, 1e-6))
        got, h = norm(x, res)
        want_h = res + x                                      # qwen2.py:58
        assert torch.equal(h, want_h)
        assert torch.equal(got, _reference(want_h, norm.weight, 1e-6))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,hidden", [(1, 896), (48, 896), (256, 896), (64, 4096),
                                         (5, 3584), (3, 8192), (17, 64)])
def test_rmsnorm_matches_reference_ops_gpu(dtype, rows, hidden):
    x, res, norm = _inputs("cuda:0", dtype, rows, hidden, 1e-6)
    with torch.no_grad():
        _close(norm(x), _reference(x, norm.weight, 1e-6), dtype)
        got, h = norm(x, res)
        want_h = res + x
        assert torch.equal(h, want_h), "the residual sum is one rounding of an exact sum"
        _close(got, _reference(want_h, norm.weight, 1e-6), dtype)
        # the inputs are left as they were
        x2, res2, _ = _inputs("cuda:0", dtype, rows, hidden, 1e-6)
        assert torch.equal(x, x2) and torch.equal(res, res2)


@pytest.mark.gpu
def test_rmsnorm_strided_rows_and_shapes_gpu():
    """Rows with a stride (a column slice of a wider tensor), 3-D activations, zero rows."""
    x, res, norm = _inputs("cuda:0", torch.bfloat16, 12, 896, 1e-6)
    wide = torch.zeros(12, 896 + 64, dtype=torch.bfloat16, device="cuda:0")
    wide[:, 32:32 + 896] = x
    with torch.no_grad():
        assert torch.equal(norm(wide[:, 32:32 + 896]), norm(x))
        assert torch.equal(norm(x.view(3, 4, 896)), norm(x).view(3, 4, 896))
        empty = x[:0]
        assert norm(empty).shape == (0, 896)
        got, h = norm(empty, res[:0])
        assert got.shape == (0, 896) and h.shape == (0, 896)


@pytest.mark.gpu
def test_rmsnorm_rejects_unsupported_shapes_gpu():
    from needle_amd._lib import NeedleAmdError
    norm = RMSNorm(900).to(device="cuda:0", dtype=torch.bfloat16)   # hidden % 8 != 0
    with pytest.raises((ValueError, NeedleAmdError)):
        norm(torch.ones(2, 900, dtype=torch.bfloat16, device="cuda:0"))
    norm = RMSNorm(8200).to(device="cuda:0", dtype=torch.bfloat16)  # above 8192
    with pytest.raises(NeedleAmdError):
        norm(torch.ones(2, 8200, dtype=torch.bfloat16, device="cuda:0"))


def _silu_closed_form(gate, up, dtype):
    """g / (1 + exp(-g)) in fp64 rounded to the dtype, times up in fp64, rounded again."""
    g = gate.cpu().double()
    s = (g / (1 + torch.exp(-g))).to(dtype).double()
    return (s * up.cpu().double()).to(dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,inter", [(1, 4864), (48, 4864), (300, 4864), (7, 18944),
                                        (9, 8)])
def test_silu_mul_matches_torch_gpu(dtype, rows, inter):
    from needle_amd import ops
    g = torch.Generator().manual_seed(rows * 31 + inter)
    # one fused gate/up projection output: gate and up are its two halves
    gu = (torch.randn(rows, 2 * inter, generator=g) * 4).to(dtype).to("cuda:0")
    gate, up = gu[:, :inter], gu[:, inter:]
    got = ops.silu_mul(gate, up)
    _close(got, F.silu(gate) * up, dtype, max_ulps16=2, max_ulps32=4)
    _close(got, _silu_closed_form(gate, up, dtype), dtype, max_ulps16=2, max_ulps32=4)
    # separate, contiguous operands give the same bits
    assert torch.equal(ops.silu_mul(gate.contiguous(), up.contiguous()), got)


@pytest.mark.gpu
def test_silu_mul_extremes_gpu():
    from needle_amd import ops
    vals = torch.tensor([0.0, -0.0, 1.0, -1.0, 20.0, -20.0, 80.0, -80.0, 1e4, -1e4,
                         float("inf"), float("-inf"), 3e-3, -3e-3, 0.5, -0.5])
    gate = vals.repeat(4, 1).to(torch.bfloat16).to("cuda:0")
    up = torch.full_like(gate, 1.5)
    got = ops.silu_mul(gate, up)
    want = F.silu(gate) * up
    assert torch.equal(got.isnan(), want.isnan())
    assert torch.equal(got.nan_to_num(), want.nan_to_num())
