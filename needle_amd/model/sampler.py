"""Next-token sampling (reference needle/model/sampler.py:16-46), greedy only.

Greedy rows (temperature 0) take the argmax of the logits (sampler.py:27-28), computed for
the whole batch on the device (ndl_greedy_argmax, torch's argmax order) and copied to the
host once; on the CPU, torch's argmax.  Temperature, top-k and top-p sampling are outside
the paged-KV path this package rebuilds; a request that asks for them is refused
(LLMEngine.add_request raises before it is queued, and this function raises too).
"""
from __future__ import annotations

from typing import List

import torch

from .. import ops
from ..backend.request import SamplingParams


def check_greedy(params: SamplingParams) -> None:
    if not params.greedy:
        raise NotImplementedError(
            f"temperature {params.temperature}: only greedy sampling (temperature 0) is built")


@torch.no_grad()
def sample(logits: torch.Tensor, params: List[SamplingParams]) -> List[int]:
    if logits.shape[0] != len(params):
        raise ValueError(f"{logits.shape[0]} logit rows for {len(params)} sequences")
    for p in params:
        check_greedy(p)
    if logits.is_cuda:
        return ops.greedy_argmax(logits).tolist()  # the whole batch, one host copy
    return logits.argmax(dim=-1).tolist()
