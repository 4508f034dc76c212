"""CPU oracle for the routed relation path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithm (Ahmet2001/relation-lm) in numpy
so that the HIP kernels can be checked against it.  It is imported only by
``tests/``, by ``__graft_entry__.smoke()`` (as the checker) and by the
``cpu_baseline`` leg of ``bench.py``.  The product path never imports it and
has no CPU fallback: it fails loudly when the HIP library is missing.

Modules
  select   -- relation_select_packed / anchor_select / partner_topk (decode and
              sequence forms), block scoring, block picks
  reduce   -- factorization, expanded cache, relation hidden (+cache update),
              norm-reduce, packed projection, linear
  router   -- DistilledBlockRouter.block_statistics / _scores restated
  dense    -- RelationLexLM.relation_context and MultiAnchorRelationBlock
              selection restated (dense O(T^2) forms used as special cases)
  dense_block -- the reference's MultiAnchorRelationBlock module structure in
              dense torch (float64), the independent check of the routed block
  multi_block -- the multi-anchor block after selection (relation MLP, slot
              reduce, stack) restated in numpy
  eager    -- the whole path in eager fp32 torch (the CPU baseline of bench.py)

Numerics contract shared with the kernels (the reference computes in fp32 with
Triton's reduction order, which no CPU code can reproduce bit for bit):
  * every dot product is accumulated in float64 from the exact float64 value
    of each input element, then rounded ONCE to float32;
  * block scores (softplus, per-head terms, pairwise log-sum-exp) are evaluated
    in float64 and rounded once to float32;
  * every comparison and tie-break happens on those float32 values.
Products of bf16/fp32 inputs are exact in float64, so the float32 results do
not depend on summation order except when the float64 sum lies within a few
float64 ulps of a float32 rounding boundary.

Parity status of each function (what pins it) is listed in each module's
docstring.
"""
