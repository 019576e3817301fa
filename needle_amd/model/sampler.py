"""Next-token sampling (reference needle/model/sampler.py:16-46).

Greedy rows (temperature 0) take argmax of the logits, computed for the whole
batch on the device and copied to the host once.  Other rows follow the
reference per row: temperature scaling, top-k (keep values >= the k-th
largest), top-p (drop a sorted token once the probability mass before it
exceeds top_p), then one multinomial draw.
"""
from __future__ import annotations

from typing import List, Optional

import torch
import torch.nn.functional as F

from ..backend.request import SamplingParams


@torch.no_grad()
def sample(logits: torch.Tensor, params: List[SamplingParams],
           generator: Optional[torch.Generator] = None) -> List[int]:
    assert logits.shape[0] == len(params)
    greedy = logits.argmax(dim=-1).tolist()          # one host copy for the batch
    out = list(greedy)
    for i, p in enumerate(params):
        if p.temperature == 0.0:
            continue
        logit = logits[i].float() / p.temperature
        if p.top_k > 0:
            k = min(p.top_k, logit.size(-1))
            kth = logit.topk(k).values[-1]
            logit = logit.masked_fill(logit < kth, float("-inf"))
        if p.top_p < 1.0:
            sorted_logits, idx = logit.sort(descending=True)
            probs = sorted_logits.softmax(dim=-1)
            remove = probs.cumsum(dim=-1) - probs > p.top_p
            sorted_logits[remove] = float("-inf")
            logit = logit.scatter(0, idx, sorted_logits)
        out[i] = int(torch.multinomial(F.softmax(logit, dim=-1), 1, generator=generator))
    return out
