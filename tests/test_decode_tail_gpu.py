"""GPU parity of relation_hidden_linear_norm_reduce_output: the decode step's relation
tail -- relation_hidden_cached (kernels/relation_reduce.py:149-183), the second linear
and relation_norm_reduce (relation_reduce.py:420-450) with the output-head preparation
(relation_lm.py:203-206) -- in one launch.

The kernel rounds the hidden to bf16 for the second linear (as the two-op form's 16-bit
linear does) and adds the per-slice partial products in a fixed order of its own, so
it is checked
  * against the two ops it replaces (relation_hidden_cached(_ring) then
    relation_linear_norm_reduce_output): context within 2e-4 absolute -- a hidden value
    whose fp32 sum rounds to the other side of a bf16 boundary moves a raw element by
    about one bf16 ulp of the hidden times a weight;
  * against the float64 oracle chain (relation_hidden_cached, bf16 rounding of the
    hidden, linear, relation_norm_reduce, output_prep) at the north-star tolerance:
    2e-2 absolute, and 5e-3 asserted beside it (the final row, stored in the query's
    dtype, one ulp of that dtype on top; and within one ulp of output_prep applied to
    the returned context);
  * for the decode shapes it does not take, bit for bit against the two ops (it runs
    them).
The workgroups meet through counters that the last arrival resets: repeated calls with
different inputs, and replays of a captured graph with inputs changed between them,
must each match the eager two-op result.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reduce as ored
from relation_lm.kernels.relation_reduce import (relation_hidden_cached,
                                                 relation_hidden_linear_norm_reduce_output,
                                                 relation_linear_norm_reduce_output)
from relation_lm.kernels.ring import relation_hidden_cached_ring

pytestmark = pytest.mark.gpu

CONTEXT_TWO_OPS = 2e-4
CONTEXT_ABS = 2e-2
CONTEXT_TIGHT = 5e-3


def host(t):
    return t.detach().float().cpu().numpy()


def make_case(batch, k_out, relation_dim, hidden_dim, d, seed, device, *, cache_rows=512,
              position=300, ring=False, query_dtype=torch.bfloat16, cache_dtype=torch.bfloat16,
              bad_indices=True):
    g = torch.Generator().manual_seed(seed)
    t_lim = cache_rows if not ring else position + 1
    anchor = torch.randint(0, t_lim, (batch,), generator=g)
    partner = torch.randint(0, t_lim, (batch, k_out), generator=g)
    if ring:  # ring caches: absolute positions, row index mod T
        partner[:, 0] = position
    elif bad_indices and k_out > 2:
        partner[0, 1] = -1                    # outside the cache: a zero row
        partner[-1, 2] = cache_rows + 5
    scores = torch.randn(batch, k_out, generator=g)
    if k_out > 1:
        scores[:, -1] = -torch.inf
    c = {
        "expanded_cache": torch.randn(batch, cache_rows, 2 * hidden_dim, generator=g).mul(0.5)
        .to(device, cache_dtype),
        "operand_cache": torch.randn(batch, cache_rows, relation_dim, generator=g)
        .to(device, cache_dtype),
        "anchor_index": anchor.to(device),
        "partner_index": partner.to(device),
        "product_weight": (torch.randn(hidden_dim, relation_dim, generator=g)
                           * relation_dim ** -0.5).to(device, cache_dtype),
        "second_weight": (torch.randn(d, hidden_dim, generator=g)
                          * hidden_dim ** -0.5).to(device, cache_dtype),
        "second_bias": (0.1 * torch.randn(d, generator=g)).to(device),
        "partner_scores": scores.to(device),
        "norm_weight": (1 + 0.1 * torch.randn(d, generator=g)).to(device),
        "norm_bias": (0.1 * torch.randn(d, generator=g)).to(device),
        "position": torch.tensor(position, device=device),
        "query": torch.randn(batch, d, generator=g).to(device, query_dtype),
        "mix_logit": torch.tensor(-0.7, device=device),
        "output_weight": (1 + 0.1 * torch.randn(d, generator=g)).to(device, query_dtype),
        "output_bias": (0.1 * torch.randn(d, generator=g)).to(device),
        "ring": ring,
    }
    return c


TAIL_ARGS = ("second_weight", "second_bias", "partner_scores", "norm_weight", "norm_bias",
             "position")
HEAD_ARGS = ("query", "mix_logit", "output_weight", "output_bias")


def run_fused(c):
    return relation_hidden_linear_norm_reduce_output(
        c["expanded_cache"], c["operand_cache"], c["anchor_index"], c["partner_index"],
        c["product_weight"], *(c[k] for k in TAIL_ARGS), 1e-5, *(c[k] for k in HEAD_ARGS), 1e-5,
        ring=c["ring"])


def run_two_ops(c):
    cached = relation_hidden_cached_ring if c["ring"] else relation_hidden_cached
    hidden = cached(c["expanded_cache"], c["operand_cache"], c["anchor_index"],
                    c["partner_index"], c["product_weight"])
    return relation_linear_norm_reduce_output(hidden, *(c[k] for k in TAIL_ARGS), 1e-5,
                                              *(c[k] for k in HEAD_ARGS), 1e-5)


def oracle_chain(c):
    """float64: hidden, rounded to bf16 as the linear sees it, linear, norm-reduce, head."""
    cached = ored.relation_hidden_cached_ring if c["ring"] else ored.relation_hidden_cached
    hidden = cached(host(c["expanded_cache"]), host(c["operand_cache"]),
                    c["anchor_index"].cpu().numpy(), c["partner_index"].cpu().numpy(),
                    host(c["product_weight"]))
    hidden = ored.round_to(hidden, "bf16")
    raw = ored.linear(hidden, host(c["second_weight"]), host(c["second_bias"]))
    context = ored.relation_norm_reduce(raw, host(c["partner_scores"]), host(c["norm_weight"]),
                                        host(c["norm_bias"]), c["position"].cpu().numpy(), 1e-5)
    final = ored.output_prep(host(c["query"]), context, -0.7, host(c["output_weight"]),
                             host(c["output_bias"]), 1e-5)
    return context, final


def check(c, ctx, final, tag):
    ctx2, final2 = run_two_ops(c)
    torch.cuda.synchronize()
    assert ctx.shape == ctx2.shape and ctx.dtype == torch.float32, tag
    assert final.shape == final2.shape and final.dtype == c["query"].dtype, tag
    got = host(ctx)
    np.testing.assert_allclose(got, host(ctx2), rtol=0, atol=CONTEXT_TWO_OPS, err_msg=str(tag))
    ref_ctx, ref_final = oracle_chain(c)
    err = np.abs(got - ref_ctx).max()
    assert err <= CONTEXT_ABS and err <= CONTEXT_TIGHT, (tag, err)
    # The final row is stored in the query's dtype: one ulp of it on top of the bounds.
    fin = host(final)
    if c["query"].dtype == torch.bfloat16:
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref_final), 1e-30))) - 7)
    else:
        ulp = np.zeros_like(ref_final)
    own = ored.output_prep(host(c["query"]), got, -0.7, host(c["output_weight"]),
                           host(c["output_bias"]), 1e-5)
    assert (np.abs(fin - own) <= ulp + 2e-5).all(), tag
    ferr = (np.abs(fin - ref_final) - ulp).max()
    assert ferr <= CONTEXT_ABS and ferr <= CONTEXT_TIGHT, (tag, ferr)


# A workgroup holds floor(16 / K) queries: batch 3 and 8 leave the last group short
# for some K (K = 8: 2 + 1; K = 5: 3 + 3 + 2; K = 3: 5 + 3), batch 1 uses one row group.
@pytest.mark.parametrize("batch", [1, 3, 8])
@pytest.mark.parametrize("k_out,relation_dim,hidden_dim,d", [
    (8, 128, 2304, 576),   # cfg3
    (5, 64, 1024, 512),
    (8, 128, 3072, 768),   # the largest hidden dim and d_model taken
    (1, 128, 64, 128),     # one slice, one group
    (3, 64, 192, 100),     # three slices of one group each
])
@pytest.mark.parametrize("ring", [False, True])
def test_matches_two_ops_and_oracle(device, batch, k_out, relation_dim, hidden_dim, d, ring):
    tag = (batch, k_out, relation_dim, hidden_dim, d, ring)
    print("case", tag, flush=True)
    c = make_case(batch, k_out, relation_dim, hidden_dim, d, batch * 97 + hidden_dim + d,
                  device, ring=ring, position=4095 if ring else 300)
    ctx, final = run_fused(c)
    check(c, ctx, final, tag)


@pytest.mark.parametrize("position", [0, 3, 511])
def test_partner_limit_by_position(device, position):
    # k_limit(t): the first tokens see fewer partners (kernels/relation_reduce.py:400-401).
    c = make_case(2, 8, 128, 2304, 576, 11 + position, device, position=position)
    ctx, final = run_fused(c)
    check(c, ctx, final, position)


def test_repeated_calls_reset_counters(device):
    # Each call leaves the counters at zero for the next: different inputs every call.
    for i in range(4):
        c = make_case(8 if i % 2 else 1, 8, 128, 2304, 576, 100 + i, device, ring=bool(i % 2),
                      position=4095 if i % 2 else 200 + i)
        ctx, final = run_fused(c)
        check(c, ctx, final, i)


def test_same_inputs_same_bits(device):
    # The partial products are summed in slice and group order, whatever the arrival order.
    c = make_case(8, 8, 128, 2304, 576, 5, device)
    a = run_fused(c)
    b = run_fused(c)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_graph_replays(device):
    c = make_case(8, 8, 128, 2304, 576, 21, device)
    run_fused(c)  # eager first: the counters of this stream exist before capture
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        run_fused(c)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ctx, final = run_fused(c)
    g = torch.Generator().manual_seed(77)
    for replay in range(3):
        # The program's own eager work between replays: new scores, queries, position.
        c["partner_scores"].copy_(torch.randn(c["partner_scores"].shape, generator=g))
        c["query"].copy_(torch.randn(c["query"].shape, generator=g))
        c["position"].fill_(250 + replay)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ctx_e, final_e = run_fused(c)
        torch.cuda.synchronize()
        assert torch.equal(ctx, ctx_e), replay
        assert torch.equal(final, final_e), replay
        check(c, ctx, final, ("replay", replay))


@pytest.mark.parametrize("k_out,d,cache_dtype", [(16, 576, torch.bfloat16),
                                                 (8, 1024, torch.bfloat16),
                                                 (8, 576, torch.float32)])
def test_other_shapes_run_the_two_ops(device, k_out, d, cache_dtype):
    c = make_case(2, k_out, 128, 1024, d, k_out + d, device, cache_dtype=cache_dtype)
    ctx, final = run_fused(c)
    ctx2, final2 = run_two_ops(c)
    torch.cuda.synchronize()
    assert torch.equal(ctx, ctx2) and torch.equal(final, final2)
