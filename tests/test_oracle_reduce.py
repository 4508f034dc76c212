"""Pins of the reduce/projection oracle (oracle/reduce.py) against closed forms in torch."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import reduce as ored


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).double()


@pytest.mark.parametrize("batch,k_out", [(1, 5), (3, 8)])
def test_hidden_equals_unfactorized_first_layer(batch, k_out):
    """GELU(W1 [a,p,a*p,a-p] + b1) (tests/test_relation_reduce_gpu.py:80-101)."""
    rng = np.random.default_rng(20260818 + batch)
    context, relation_dim, hidden_dim = 64, 16, 48
    operand = rng.standard_normal((batch, context, relation_dim)).astype(np.float32)
    first_weight = (rng.standard_normal((hidden_dim, 4 * relation_dim)) * 0.2).astype(np.float32)
    first_bias = (rng.standard_normal(hidden_dim) * 0.1).astype(np.float32)
    factors = ored.factor_relation_first_layer(first_weight, first_bias, relation_dim)
    expanded = ored.linear(operand, factors["expanded_weight"], factors["expanded_bias"])
    anchor = rng.integers(0, context, batch)
    partner = rng.integers(0, context, (batch, k_out))
    got = ored.relation_hidden_cached(expanded, operand, anchor, partner,
                                      factors["product_weight"])
    b = torch.arange(batch)
    a_op = _t(operand)[b, torch.from_numpy(anchor)]
    p_op = _t(operand)[b[:, None], torch.from_numpy(partner)]
    a_exp = a_op[:, None].expand(-1, k_out, -1)
    product = (a_exp.float() * p_op.float()).double()   # the reference's fp32 product
    features = torch.cat((a_exp, p_op, product, a_exp - p_op), dim=-1)
    expected = F.gelu(F.linear(features, _t(first_weight), _t(first_bias)))
    assert torch.allclose(torch.from_numpy(got).double(), expected, rtol=2e-6, atol=1e-6)


def test_hidden_guarded_gather_reads_zero_rows():
    rng = np.random.default_rng(1)
    operand = rng.standard_normal((1, 8, 4)).astype(np.float32)
    expanded = rng.standard_normal((1, 8, 6)).astype(np.float32)
    wm = rng.standard_normal((3, 4)).astype(np.float32)
    got = ored.relation_hidden_cached(expanded, operand, np.array([2]), np.array([[-3, 9]]), wm)
    expected = ored.gelu_erf(expanded[0, 2, :3].astype(np.float64))
    assert np.allclose(got[0, 0], expected, atol=1e-7)
    assert np.allclose(got[0, 1], expected, atol=1e-7)


def test_cache_update_row_and_hidden():
    """relation_reduce.py:215-279: fresh row written, hidden equals the cached op on it."""
    rng = np.random.default_rng(7)
    batch, context, relation_dim, hidden_dim, k = 2, 32, 8, 24, 4
    operand = rng.standard_normal((batch, context, relation_dim)).astype(np.float32)
    first_weight = (rng.standard_normal((hidden_dim, 4 * relation_dim)) * 0.3).astype(np.float32)
    first_bias = (rng.standard_normal(hidden_dim) * 0.1).astype(np.float32)
    f = ored.factor_relation_first_layer(first_weight, first_bias, relation_dim)
    expanded = ored.linear(operand, f["expanded_weight"], f["expanded_bias"]).astype(np.float32)
    t = 31
    stale = expanded.copy()
    stale[:, t] = 0.0
    anchor = np.array([t, 3])
    partner = np.array([[t, 1, 2, 3], [4, t, 6, 7]])
    hidden, updated = ored.relation_hidden_cache_update(
        stale, operand, anchor, partner, f["anchor_weight"], f["partner_weight"],
        f["product_weight"], f["first_bias"], t)
    assert np.allclose(updated[:, t], expanded[:, t], rtol=1e-6, atol=1e-6)
    cached = ored.relation_hidden_cached(expanded, operand, anchor, partner, f["product_weight"])
    assert np.allclose(hidden, cached, rtol=1e-6, atol=1e-6)


def _reference_context(raw, scores, weight, bias, position, eps):
    """tests/test_relation_reduce_gpu.py:21-43 in float64."""
    relations = F.layer_norm(raw, (raw.size(-1),), weight, bias, eps)
    limit = int(math.ceil(math.log2(float(position) + 2.0)))
    limit = max(1, min(limit, scores.size(1)))
    ranks = torch.arange(scores.size(1))[None]
    active = torch.isfinite(scores) & ranks.lt(limit)
    safe = scores.masked_fill(~active, -1.0e4)
    weights = safe.softmax(-1) * active
    weights = weights / weights.sum(-1, keepdim=True).clamp_min(1.0e-9)
    return (weights.unsqueeze(-1) * relations).sum(1)


@pytest.mark.parametrize("k_out", [5, 6, 7, 8])
@pytest.mark.parametrize("position", [0, 1, 2, 6, 511])
def test_norm_reduce_matches_layer_norm_softmax(k_out, position):
    rng = np.random.default_rng(20260830 + k_out)
    raw = rng.standard_normal((3, k_out, 576)).astype(np.float32)
    scores = rng.standard_normal((3, k_out)).astype(np.float32)
    scores[:, -1] = -np.inf
    weight = (rng.standard_normal(576) * 0.05 + 1.0).astype(np.float32)
    bias = (rng.standard_normal(576) * 0.01).astype(np.float32)
    got = ored.relation_norm_reduce(raw, scores, weight, bias, position, 1e-5)
    expected = _reference_context(_t(raw), _t(scores), _t(weight), _t(bias), position, 1e-5)
    assert np.allclose(got, expected.numpy(), rtol=1e-6, atol=1e-6)


def test_norm_reduce_all_inactive_is_zero():
    raw = np.ones((1, 4, 8), np.float32)
    scores = np.full((1, 4), -np.inf, np.float32)
    got = ored.relation_norm_reduce(raw, scores, np.ones(8), np.zeros(8), 100, 1e-5)
    assert np.all(got == 0.0)


def test_k_limit_matches_float_ceil_log2():
    t = np.arange(0, 1 << 20)
    expected = np.clip(np.ceil(np.log2(t.astype(np.float64) + 2.0)).astype(np.int64), 1, 64)
    assert np.array_equal(ored.k_limit(t, 64), expected)


@pytest.mark.parametrize("batch", [1, 8])
def test_packed_projection_equals_separate_linears(batch):
    """tests/test_packed_cache_projection.py:10-25."""
    rng = np.random.default_rng(20260822 + batch)
    memory = rng.standard_normal((batch, 576)).astype(np.float32)
    widths = (64, 64, 128, 128, 64, 64)
    weights = [(rng.standard_normal((w, 576)) * 0.02).astype(np.float32) for w in widths]
    packed = ored.packed_sparse_cache_projection(memory, np.concatenate(weights, axis=0))
    parts = np.split(packed, np.cumsum(widths)[:-1], axis=1)
    for w, part in zip(weights, parts):
        assert np.allclose(part, F.linear(_t(memory), _t(w)).numpy(), rtol=1e-12, atol=1e-12)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(100000) * 10.0 ** rng.integers(-5, 5, 100000)).astype(np.float32)
    expected = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ored.round_to(x, "bfloat16").astype(np.float32), expected)


def test_output_prep_matches_torch_layer_norm():
    rng = np.random.default_rng(31)
    query, context = rng.normal(size=(3, 40)), rng.normal(size=(3, 40))
    w, b = rng.normal(1.0, 0.1, 40), rng.normal(0.0, 0.1, 40)
    got = ored.output_prep(query, context, 0.35, w, b, 1e-5)
    tq = torch.from_numpy(query) + torch.sigmoid(torch.tensor(0.35, dtype=torch.float64)) * torch.from_numpy(context)
    ref = torch.nn.functional.layer_norm(tq, (40,), torch.from_numpy(w), torch.from_numpy(b), 1e-5)
    np.testing.assert_allclose(got, ref.numpy(), rtol=0, atol=1e-12)
    # A mix logit of -inf gates the context out: the LayerNorm of the query alone.
    only_query = ored.output_prep(query, 1e3 * context, -np.inf, w, b, 1e-5)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(query), (40,), torch.from_numpy(w),
                                         torch.from_numpy(b), 1e-5)
    np.testing.assert_allclose(only_query, ref.numpy(), rtol=0, atol=1e-12)
