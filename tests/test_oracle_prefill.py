"""Pins the oracle's varlen causal prefill (attention.py:120-134) on the CPU.

* fp32 oracle vs an fp64 causal closed form (tight), bf16 oracle within the
  bf16 parity tolerance;
* reading K/V back through block_table after write_kv equals the fresh
  tensors (context 0), so the paged closed form equals the dense one;
* first token of a sequence attends only itself; sequences do not leak
  into each other.
"""
import numpy as np
import torch

from oracle import closed_form, paged_ref
from needle_amd import workloads as wl


def _max_excess(a, b, atol, rtol):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float((np.abs(a - b) - (atol + rtol * np.abs(b))).max())


def test_fp32_oracle_matches_dense_closed_form():
    shape = wl.QWEN2_7B
    case = wl.prefill_case(shape, [1, 17, 40, 5], seed=31, dtype=torch.float32)
    got = paged_ref.prefill_pytorch(case.q, case.k, case.v, case.cu_seqlens, shape.num_heads,
                                    shape.num_kv_heads)
    want = closed_form.dense_causal_fp64(case.q, case.k, case.v, case.cu_seqlens, shape.scale,
                                         shape.num_heads, shape.num_kv_heads)
    assert _max_excess(got, want, 1e-5, 1e-5) <= 0


def test_bf16_oracle_within_tolerance():
    shape = wl.QWEN2_05B
    case = wl.prefill_case(shape, [64, 3, 130], seed=32)
    got = paged_ref.prefill_pytorch(case.q, case.k, case.v, case.cu_seqlens, shape.num_heads,
                                    shape.num_kv_heads)
    want = closed_form.dense_causal_fp64(case.q, case.k, case.v, case.cu_seqlens, shape.scale,
                                         shape.num_heads, shape.num_kv_heads)
    assert _max_excess(got.float(), want, 2e-2, 1e-2) <= 0


def test_paged_readback_equals_fresh_kv():
    shape = wl.LLAMA3_8B
    case = wl.prefill_case(shape, [20, 33, 16], seed=33, dtype=torch.float32)
    pool = case.kv_cache.clone()
    paged_ref.write_kv(case.k, case.v, pool, case.block_table, case.cu_seqlens, case.context_lens)
    paged = closed_form.prefill_fp64(case.q, pool, case.block_table, case.cu_seqlens,
                                     case.context_lens, shape.scale, shape.num_heads,
                                     shape.num_kv_heads)
    dense = closed_form.dense_causal_fp64(case.q, case.k, case.v, case.cu_seqlens, shape.scale,
                                          shape.num_heads, shape.num_kv_heads)
    assert np.array_equal(paged, dense)


def test_first_token_attends_itself_and_no_cross_talk():
    shape = wl.QWEN2_7B
    case = wl.prefill_case(shape, [4, 9], seed=34, dtype=torch.float32)
    out = paged_ref.prefill_pytorch(case.q, case.k, case.v, case.cu_seqlens, shape.num_heads,
                                    shape.num_kv_heads)
    g = shape.group
    for start in (0, 4):
        for h in range(shape.num_heads):
            assert torch.allclose(out[start, h], case.v[start, h // g], atol=1e-6)
    k2, v2 = case.k.clone(), case.v.clone()
    k2[4:] = torch.randn_like(k2[4:])
    v2[4:] = torch.randn_like(v2[4:])
    out2 = paged_ref.prefill_pytorch(case.q, k2, v2, case.cu_seqlens, shape.num_heads,
                                     shape.num_kv_heads)
    assert torch.equal(out[:4], out2[:4])
