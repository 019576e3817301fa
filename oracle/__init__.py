"""CPU oracle of Needle's paged-KV hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this package, and only as the reference results are compared against (or as the
timed CPU baseline).  The product path (needle_amd) never imports it.

Contents (each function cites the reference file:line it restates):
  paged_ref.slot_of_tokens   integer slot rule      attention.py:141-146, 217-237
  paged_ref.decode_append    decode append          attention.py:141-154
  paged_ref.write_kv         varlen append          attention.py:204-246
  paged_ref.decode_pytorch   paged decode           attention.py:291-310
  paged_ref.prefill_pytorch  varlen causal prefill  attention.py:120-134
  closed_form.*              fp64 textbook forms and brute-force loops that pin
                             the functions above (see tests/test_oracle_*.py)

Pinning status: every function above is checked against an independent
closed form, a brute-force loop or a library routine in tests/; the reference
ships no golden vectors for this path (its only numeric test,
tests/unit/test_paged_attention.py:44-68, is reused as a known-answer case).
"""
