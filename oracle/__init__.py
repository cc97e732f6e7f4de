"""CPU oracle for the V1 query-indexing hot path -- TEST INFRASTRUCTURE ONLY.

Plain numpy restatements of the reference algorithms, each citing the
reference file:line it follows.  Only tests/, the smoke check and the CPU
baseline leg of bench.py may import this package, and only as the checker:
no product code path calls it.

Pinning (what checks each function beyond its own text):
  fp8 decode          every code vs torch.float8_e4m3fn (tests/test_oracle_fp8.py)
  route               reference example known answer + brute force on small rows
  topk_select         brute-force sort, tie/ -inf / ±0 special cases, L <= T rule
  fused_topk          reference example (mask, mapping, both direct_fine settings)
  transform_topk      closed form on identity / random tables
  mask_fine/output_ids  equal to fused_topk's mask / epilogue on the same data
  sort_f32 / sort_i64 reference KAT values (test_fused_grouping_small.py:88-115)
  page manager        reference lifecycle KAT (test_page_management_and_tail_small.py:14-57),
                      fingerprint KAT [3141875, 26276919], word-wise identity
  stage_tail_shared   reference KAT (test_page_management_and_tail_small.py:59-88)
  query_metadata      closed form + tail-share KAT owners [0,0,2,2]
  gather              reference KAT (test_gather_slots_small.py:26-64)
  score               fp32/fp64 dequantised formula; relu/weights/scale order checked
                      against hand-computed single-key cases
"""
