"""CPU oracle for the V1 query-indexing hot path -- TEST INFRASTRUCTURE ONLY.

Plain numpy restatements of the reference algorithms, each citing the
reference file:line it follows.  Only tests/, the smoke check and the CPU
baseline leg of bench.py may import this package, and only to check results
or time the host baseline: no product code path calls it.

Pinning (what checks each function beyond its own text):
  fp8 decode          every code vs torch.float8_e4m3fn (tests/test_oracle.py)
  route               reference example known answer + brute force on small rows;
                      fine table over every rank < take (take > take_stride)
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
                      against hand-computed single-key cases; the page/slot/scale
                      addressing through per-row and shared block tables by one-hot
                      keys with per-token scales, worked by hand and by lookup
  index build         reference KATs of _dots / _anchor (test_fused_grouping_small.py:57-86),
                      the four-partial reduction order, unit vectors, RNE e4m3 vs torch,
                      hierarchical clusters split exactly, float64 bisection where decided
                      (tests/test_oracle_build.py)
  shared tail union   the reference's 64K/4K answers (tail_union_lab README.md:54-63), the
                      candidate-set rule, union = per-row staging byte for byte, one
                      canonical order from shared / per-row / split scoring
                      (tests/test_oracle_union.py)
  expand_logical      hand KAT, int32 wrap, equal to fused_topk's expansion
  decode_attention    closed forms: mean, one-hot, single key, key order, linearity, shift
                      (tests/test_oracle_attention.py)
"""
