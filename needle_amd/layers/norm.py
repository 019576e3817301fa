"""RMSNorm (reference needle/layers/norm.py:8-17), with the residual add before it.

The reference computes, in torch ops,
    y = (x * rsqrt(mean(x.float()^2) + eps)).to(dtype)     fp32 statistic and product
    out = weight * y                                      rounded in the model dtype
and its decoder layer adds the residual before each norm (needle/model/qwen2.py:58, :63).
On the GPU, forward(x, residual) is one HIP kernel (ndl_rms_norm: the add, the statistic,
the two products, with the same roundings); only the order of the fp32 sum of squares
differs from torch's reduction, which moves an element by an ulp of its format now and
then (tests/test_layer_ops.py).  On the CPU (the oracle runner of the tests and the CPU
baseline) it is torch's fused RMS normalisation without a weight followed by the weight
product: the same bits as the reference's op sequence.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import ops


class RMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        """norm(x), or with residual: (norm(x + residual), x + residual)."""
        if x.is_cuda:
            shape = x.shape
            x2 = x.reshape(-1, shape[-1])
            if residual is None:
                return ops.rms_norm(x2, self.weight, self.eps).view(shape)
            out, h = ops.rms_norm(x2, self.weight, self.eps, residual.reshape(-1, shape[-1]))
            return out.view(shape), h.view(shape)
        if residual is not None:
            h = x + residual
            return self._torch(h), h
        return self._torch(x)

    def _torch(self, x: torch.Tensor) -> torch.Tensor:
        y = F.rms_norm(x, (x.shape[-1],), None, self.eps)
        return self.weight * y.to(self.weight.dtype)
