"""GPU parity of the norm-reduce with the last-token output preparation fused as
its epilogue (relation_lm::relation_norm_reduce_output[_seq]; the reference's
roadmap item README.md:150-151, computing RelationLexLM.forward's
output_norm(query + sigmoid(relation_mix_logit) * context), relation_lm.py:203-206).

The context output must be bit-identical to relation_norm_reduce's (same
kernel, same arithmetic); the final vector is checked against oracle
output_prep in float64: fp32 within 2e-5, bf16 within one bf16 ulp.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reduce as ored
from relation_lm.kernels.relation_reduce import (relation_norm_reduce, relation_norm_reduce_output,
                                                 relation_norm_reduce_output_seq,
                                                 relation_norm_reduce_seq)

pytestmark = pytest.mark.gpu


def host(t):
    return t.detach().float().cpu().numpy()


def check_final(got, expected, dtype):
    if dtype == torch.float32:
        np.testing.assert_allclose(got, expected, rtol=0, atol=2e-5)
    else:
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(expected), 1e-30))) - 7)
        assert (np.abs(got - expected) <= ulp + 1e-5).all()


@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("k_out,d", [(8, 576), (6, 512), (5, 100), (8, 2048), (7, 7)])
@pytest.mark.parametrize("query_dtype", [torch.float32, torch.bfloat16])
def test_decode_output_prep(device, batch, k_out, d, query_dtype):
    g = torch.Generator().manual_seed(batch * 100 + k_out * 10 + d)
    raw = torch.randn(batch, k_out, d, generator=g).to(device)
    scores = torch.randn(batch, k_out, generator=g)
    scores[:, -1] = -torch.inf
    scores = scores.to(device)
    w = (1 + 0.1 * torch.randn(d, generator=g)).to(device)
    b = (0.1 * torch.randn(d, generator=g)).to(device)
    query = torch.randn(batch, d, generator=g).to(device=device, dtype=query_dtype)
    mix = torch.tensor(-0.4, device=device)
    ow = (1 + 0.1 * torch.randn(d, generator=g)).to(device)
    ob = (0.1 * torch.randn(d, generator=g)).to(device)
    position = torch.tensor(300, device=device)
    ctx, final = relation_norm_reduce_output(raw, scores, w, b, position, 1e-5, query, mix, ow,
                                             ob, 1e-5)
    plain = relation_norm_reduce(raw, scores, w, b, position, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(ctx, plain)
    assert final.dtype == query_dtype and final.shape == (batch, d)
    expected = ored.output_prep(host(query), host(ctx), -0.4, host(ow), host(ob), 1e-5)
    check_final(host(final), expected, query_dtype)


@pytest.mark.parametrize("query_dtype", [torch.float32, torch.bfloat16])
def test_sequence_output_prep(device, query_dtype):
    g = torch.Generator().manual_seed(5)
    bsz, tq, k, d = 2, 33, 8, 512
    raw = torch.randn(bsz, tq, k, d, generator=g).to(device)
    scores = torch.randn(bsz, tq, k, generator=g).to(device)
    w = (1 + 0.1 * torch.randn(d, generator=g)).to(device)
    b = (0.1 * torch.randn(d, generator=g)).to(device)
    query = torch.randn(bsz, tq, d, generator=g).to(device=device, dtype=query_dtype)
    mix = torch.tensor(1.3, dtype=torch.bfloat16, device=device)
    ow = (1 + 0.1 * torch.randn(d, generator=g)).to(device=device, dtype=torch.bfloat16)
    ob = (0.1 * torch.randn(d, generator=g)).to(device)
    positions = torch.arange(tq, device=device)
    ctx, final = relation_norm_reduce_output_seq(raw, scores, w, b, positions, 1e-5, query, mix,
                                                 ow, ob, 1e-6)
    plain = relation_norm_reduce_seq(raw, scores, w, b, positions, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(ctx, plain)
    expected = ored.output_prep(host(query), host(ctx), float(mix.float()), host(ow), host(ob),
                                1e-6)
    check_final(host(final), expected, query_dtype)


def test_rejects_mismatched_query(device):
    raw = torch.randn(2, 4, 64, device=device)
    scores = torch.randn(2, 4, device=device)
    w = torch.ones(64, device=device)
    with pytest.raises(RuntimeError, match="query"):
        relation_norm_reduce_output(raw, scores, w, w, torch.tensor(5, device=device), 1e-5,
                                    torch.randn(2, 32, device=device), torch.tensor(0.0, device=device),
                                    w, w, 1e-5)
