"""Recomputes, on the CPU, the oracle's own logits spread that the GPU engine test's bounds
are derived from (tests/logits_spread.py): the real Qwen2-0.5B on 8 benchmark requests with
the reference attention in bf16 against the same attention in fp32.  The recorded spread
must be what the computation gives (within 5%: CPU GEMM blocking can change with the
thread count), and it must be large against the attention tolerance's scale, which is why
the logits bound is not the attention tolerance."""
import logits_spread as ls


def test_recorded_spread_is_the_computed_one():
    worst, rel, forwards = ls.logits_spread()
    print(f"oracle bf16 vs fp32-attention logits: max |diff| {worst:.5g}, relative L2 "
          f"{rel:.5g} over {forwards} forwards")
    assert forwards >= 8
    assert abs(worst - ls.SPREAD_MAX_DIFF) <= 0.05 * ls.SPREAD_MAX_DIFF, worst
    assert abs(rel - ls.SPREAD_REL_L2) <= 0.05 * ls.SPREAD_REL_L2, rel
    assert worst > 2e-2
