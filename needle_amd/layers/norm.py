"""RMSNorm (reference needle/layers/norm.py:8-17).

The reference computes, in torch ops,
    y = (x * rsqrt(mean(x.float()^2) + eps)).to(dtype)     fp32 statistic and product
    out = weight * y                                      rounded in the model dtype
which is five elementwise kernels and a reduction before the weight product.  Here the
first line is torch's fused RMS normalisation without a weight (the same fp32 statistic and
product, one rounding to x's dtype, in one kernel) and the weight product stays its own op,
so the output keeps the reference's two roundings.  Against the reference's op sequence
(tests/test_norm.py): the same bits on the CPU; on the GPU the fused statistic and
reciprocal square root can differ in their last bit, which moves an element by an ulp of
the format now and then.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F


class RMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = F.rms_norm(x, (x.shape[-1],), None, self.eps)
        return self.weight * y.to(self.weight.dtype)
