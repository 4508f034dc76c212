"""GPU parity of relation_linear_norm_reduce_output: the decode step's second linear
(benchmarks/benchmark_relation_reduce.py:80-81) folded into the norm-reduce with the output-head preparation
(relation_lm.py:203-206).

The fused form splits the hidden dim, writes fp32 partial products and lets the
per-query norm kernel add them in split order, so its raw rows differ from the
one-launch linear's by fp32 summation order only.  Checked against
  * the oracle in float64 (linear of the bf16 operands, norm-reduce, output prep):
    context within 1e-4 absolute, the final vector against output_prep of the
    returned context (fp32 within 2e-5, bf16 within one ulp);
  * the two ops it replaces, relation_linear then relation_norm_reduce_output:
    context within 1e-4, and bit-identical where the op falls back to them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reduce as ored
from relation_lm.kernels.relation_reduce import (relation_linear,
                                                 relation_linear_norm_reduce_output,
                                                 relation_norm_reduce_output)

pytestmark = pytest.mark.gpu


def host(t):
    return t.detach().float().cpu().numpy()


def check_final(got, expected, dtype):
    if dtype == torch.float32:
        np.testing.assert_allclose(got, expected, rtol=0, atol=2e-5)
    else:
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(expected), 1e-30))) - 7)
        assert (np.abs(got - expected) <= ulp + 1e-5).all()


def make_case(batch, k_out, hidden_dim, d, weight_dtype, query_dtype, seed, device,
              position=300, masked=1):
    g = torch.Generator().manual_seed(seed)
    hidden = torch.randn(batch, k_out, hidden_dim, generator=g).to(device, weight_dtype)
    w2 = (torch.randn(d, hidden_dim, generator=g) * hidden_dim ** -0.5).to(device, weight_dtype)
    b2 = (0.1 * torch.randn(d, generator=g)).to(device)
    scores = torch.randn(batch, k_out, generator=g)
    if masked:
        scores[:, -masked:] = -torch.inf
    case = {
        "hidden": hidden, "second_weight": w2, "second_bias": b2,
        "partner_scores": scores.to(device),
        "norm_weight": (1 + 0.1 * torch.randn(d, generator=g)).to(device),
        "norm_bias": (0.1 * torch.randn(d, generator=g)).to(device),
        "position": torch.tensor(position, device=device),
        "query": torch.randn(batch, d, generator=g).to(device, query_dtype),
        "mix_logit": torch.tensor(-0.7, device=device),
        "output_weight": (1 + 0.1 * torch.randn(d, generator=g)).to(device, query_dtype),
        "output_bias": (0.1 * torch.randn(d, generator=g)).to(device),
    }
    return case


def run_fused(c):
    return relation_linear_norm_reduce_output(
        c["hidden"], c["second_weight"], c["second_bias"], c["partner_scores"], c["norm_weight"],
        c["norm_bias"], c["position"], 1e-5, c["query"], c["mix_logit"], c["output_weight"],
        c["output_bias"], 1e-5)


def run_two_ops(c):
    raw = relation_linear(c["hidden"], c["second_weight"], c["second_bias"],
                          out_dtype=torch.float32)
    return relation_norm_reduce_output(
        raw, c["partner_scores"], c["norm_weight"], c["norm_bias"], c["position"], 1e-5,
        c["query"], c["mix_logit"], c["output_weight"], c["output_bias"], 1e-5)


def expected_context(c):
    raw = ored.linear(host(c["hidden"]), host(c["second_weight"]), host(c["second_bias"]))
    return ored.relation_norm_reduce(raw, host(c["partner_scores"]), host(c["norm_weight"]),
                                     host(c["norm_bias"]), c["position"].cpu().numpy(), 1e-5)


@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("k_out,hidden_dim,d", [(8, 2048, 512), (8, 1024, 576), (6, 2304, 512),
                                                (5, 1000, 100), (8, 4096, 1024), (1, 256, 64)])
@pytest.mark.parametrize("query_dtype", [torch.float32, torch.bfloat16])
def test_matches_oracle_and_two_ops(device, batch, k_out, hidden_dim, d, query_dtype):
    c = make_case(batch, k_out, hidden_dim, d, torch.bfloat16, query_dtype,
                  batch * 1000 + k_out * 100 + d, device, masked=1 if k_out > 1 else 0)
    ctx, final = run_fused(c)
    ctx2, final2 = run_two_ops(c)
    torch.cuda.synchronize()
    tag = (batch, k_out, hidden_dim, d, query_dtype)
    assert ctx.shape == (batch, d) and ctx.dtype == torch.float32, tag
    assert final.shape == (batch, d) and final.dtype == query_dtype, tag
    np.testing.assert_allclose(host(ctx), expected_context(c), rtol=0, atol=1e-4, err_msg=str(tag))
    np.testing.assert_allclose(host(ctx), host(ctx2), rtol=0, atol=1e-4, err_msg=str(tag))
    expected = ored.output_prep(host(c["query"]), host(ctx), -0.7, host(c["output_weight"]),
                                host(c["output_bias"]), 1e-5)
    check_final(host(final), expected, query_dtype)


@pytest.mark.parametrize("position", [0, 3, 7, 511, 100000])
def test_partner_limit_by_position(device, position):
    # k_limit(t): the first tokens see fewer partners (kernels/relation_reduce.py:400-401).
    c = make_case(2, 8, 2048, 512, torch.bfloat16, torch.bfloat16, 17 + position, device,
                  position=position, masked=0)
    ctx, _ = run_fused(c)
    torch.cuda.synchronize()
    np.testing.assert_allclose(host(ctx), expected_context(c), rtol=0, atol=1e-4)


@pytest.mark.parametrize("batch,k_out,weight_dtype", [(16, 8, torch.bfloat16),
                                                      (2, 8, torch.float32),
                                                      (300, 1, torch.bfloat16)])
def test_fallback_is_the_two_ops(device, batch, k_out, weight_dtype):
    # More than 64 hidden rows, fp32 weights: the op runs relation_linear then
    # relation_norm_reduce_output and must return exactly their result.
    c = make_case(batch, k_out, 1024, 512, weight_dtype, torch.bfloat16, batch + k_out, device,
                  masked=0)
    ctx, final = run_fused(c)
    ctx2, final2 = run_two_ops(c)
    torch.cuda.synchronize()
    assert torch.equal(ctx, ctx2)
    assert torch.equal(final, final2)


def test_same_result_twice(device):
    # Deterministic: no atomics, fixed split order.
    c = make_case(8, 8, 2048, 512, torch.bfloat16, torch.bfloat16, 3, device)
    a = run_fused(c)
    b = run_fused(c)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
