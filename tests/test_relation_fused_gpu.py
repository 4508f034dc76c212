"""GPU parity of the fused relation reduce (hidden -> second linear -> norm-reduce).

The fused op has no reference counterpart; the reference runs the three ops in
sequence (benchmarks/benchmark_relation_reduce.py:55-64).  It is checked
  * against the float64 oracle chain with the hidden rounded to bf16 before the
    second linear (what the bf16 linear of the unfused path sees), and
  * against this library's own unfused three-op chain on the same inputs.
Tolerance: bf16 inputs, absolute error <= 2e-2 (north_star).  A 5e-3 bound is
asserted too so that a dropped or mis-indexed term cannot hide under the loose
one; what remains is the rare hidden value that lands on the other side of a
bf16 rounding boundary (different fp32 summation order), worth ~1e-3 at most.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reduce as ored
from relation_lm.kernels.relation_reduce import (
    mfma_fragments,
    relation_hidden_cached_seq,
    relation_linear,
    relation_norm_reduce_seq,
    relation_reduce_fused_seq,
)
from relation_lm.workloads import CONFIGS, RelationConfig, causal_partner_indices, reduce_inputs

pytestmark = pytest.mark.gpu

BF16_ABS = 2e-2
TIGHT_ABS = 5e-3


def host(t):
    return t.detach().float().cpu().numpy() if t.dtype.is_floating_point else t.cpu().numpy()


def abs_err(got, expected):
    return float(np.abs(np.asarray(got, np.float64) - np.asarray(expected, np.float64)).max())


def indices_and_scores(batch, queries, context, k, seed, *, sentinels=True):
    """Anchor/partner indices over the causal history plus partner scores.

    Query tq sits at position tq (the sequence form of cfg2); partner slots past
    the available history carry the select op's sentinel (t-LOCAL+1, -inf).
    """
    g = torch.Generator().manual_seed(seed)
    pos = torch.arange(queries)
    anchor = (torch.rand(batch, queries, generator=g) * (pos + 1)).long()
    partner = (torch.rand(batch, queries, k, generator=g) * (pos[None, :, None] + 1)).long()
    scores = torch.randn(batch, queries, k, generator=g)
    if sentinels:
        few = pos < k  # fewer than k candidates: trailing slots are sentinels
        for t in range(min(queries, k)):
            partner[:, t, t:] = t - 64 + 1
            scores[:, t, t:] = -torch.inf
        assert few.any()
    return anchor.int(), partner.int(), scores, pos


def oracle_chain(red, expanded, anchor, partner, scores, positions, rows=slice(None)):
    """float64 chain on the device's bf16 expanded cache, hidden rounded to bf16."""
    expanded = host(expanded)
    hidden = ored.relation_hidden_cached_seq(expanded[rows], host(red["operand_cache"])[rows],
                                             anchor[rows], partner[rows],
                                             host(red["product_weight"]))
    hidden = ored.round_to(hidden, "bfloat16")
    raw = ored.linear(hidden, host(red["second_weight"]), host(red["second_bias"]))
    return ored.relation_norm_reduce_seq(raw, scores[rows], host(red["norm_weight"]),
                                         host(red["norm_bias"]), positions, 1e-5)


def run_fused(red, expanded, anchor, partner, scores, positions, device):
    return relation_reduce_fused_seq(expanded, red["operand_cache"], anchor.to(device),
                                     partner.to(device), red["product_weight"],
                                     red["second_weight"], red["second_bias"], scores.to(device),
                                     red["norm_weight"], red["norm_bias"], positions.to(device),
                                     1e-5)


def run_unfused(red, expanded, anchor, partner, scores, positions, device):
    hidden = relation_hidden_cached_seq(expanded, red["operand_cache"], anchor.to(device),
                                        partner.to(device), red["product_weight"])
    raw = relation_linear(hidden, red["second_weight"], red["second_bias"],
                          out_dtype=torch.float32)
    return relation_norm_reduce_seq(raw, scores.to(device), red["norm_weight"],
                                    red["norm_bias"], positions.to(device), 1e-5)


def test_cfg2_fused_matches_unfused_and_oracle(device):
    cfg = CONFIGS["cfg2"]
    red = reduce_inputs(cfg, device=device)
    expanded = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])
    anchor, partner, scores, pos = indices_and_scores(cfg.batch, cfg.context, cfg.context,
                                                      cfg.k_out, seed=31)
    fused = run_fused(red, expanded, anchor, partner, scores, pos, device)
    unfused = run_unfused(red, expanded, anchor, partner, scores, pos, device)
    torch.cuda.synchronize()
    assert fused.shape == (cfg.batch, cfg.context, cfg.d_model)
    assert torch.isfinite(fused).all()
    assert abs_err(host(fused), host(unfused)) <= TIGHT_ABS
    # oracle on batch row 0, the first 96 queries (covers the sentinel slots)
    rows = slice(0, 1)
    expected = oracle_chain(red, expanded, host(anchor)[:, :96], host(partner)[:, :96],
                            host(scores)[:, :96], np.arange(96), rows)
    got = host(fused)[0:1, :96]
    assert abs_err(got, expected) <= BF16_ABS
    assert abs_err(got, expected) <= TIGHT_ABS


@pytest.mark.parametrize("k_out", [1, 2, 3, 4, 5, 6, 7, 8, 12, 16])
@pytest.mark.parametrize("d_model", [128, 256, 384])
def test_fused_partner_counts_and_widths(device, k_out, d_model):
    cfg = RelationConfig("fused", 2, 96, d_model, 32, 64, 2, k_out, torch.bfloat16,
                         relation_dim=64, hidden_dim=256, seed=777 + k_out)
    red = reduce_inputs(cfg, device=device)
    expanded = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])
    anchor, partner, scores, pos = indices_and_scores(2, 96, 96, k_out, seed=5 + k_out)
    fused = run_fused(red, expanded, anchor, partner, scores, pos, device)
    unfused = run_unfused(red, expanded, anchor, partner, scores, pos, device)
    torch.cuda.synchronize()
    assert abs_err(host(fused), host(unfused)) <= TIGHT_ABS
    expected = oracle_chain(red, expanded, host(anchor), host(partner), host(scores),
                            np.arange(96))
    assert abs_err(host(fused), expected) <= TIGHT_ABS


def test_fused_batched_positions_and_ragged_rows(device):
    """[B,Tq] positions, Tq not a multiple of the workgroup's 16 queries."""
    cfg = RelationConfig("fused", 3, 80, 512, 16, 32, 2, 8, torch.bfloat16,
                         relation_dim=128, hidden_dim=384, seed=4321)
    red = reduce_inputs(cfg, device=device)
    expanded = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])
    anchor, partner, scores, _ = indices_and_scores(3, 37, 80, 8, seed=9, sentinels=False)
    positions = torch.stack([torch.arange(37) + 40, torch.arange(37) + 3, torch.arange(37)])
    fused = run_fused(red, expanded, anchor, partner, scores, positions, device)
    unfused = run_unfused(red, expanded, anchor, partner, scores, positions, device)
    torch.cuda.synchronize()
    assert fused.shape == (3, 37, 512)
    assert abs_err(host(fused), host(unfused)) <= TIGHT_ABS


@pytest.mark.parametrize("d_model,relation_dim,k_out", [(512, 128, 8), (384, 64, 5),
                                                        (256, 32, 16), (128, 128, 1)])
def test_fragment_order_second_weight_same_bits(device, d_model, relation_dim, k_out):
    """second_weight in MFMA fragment order (mfma_fragments) reads the same fragments from
    contiguous memory: the output equals the [D, H] weight's bit for bit."""
    cfg = RelationConfig("frag", 2, 96, d_model, 32, 64, 2, k_out, torch.bfloat16,
                         relation_dim=relation_dim, hidden_dim=256, seed=99 + d_model)
    red = reduce_inputs(cfg, device=device)
    expanded = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])
    anchor, partner, scores, pos = indices_and_scores(2, 96, 96, k_out, seed=17)
    plain = run_fused(red, expanded, anchor, partner, scores, pos, device)
    frag = relation_reduce_fused_seq(expanded, red["operand_cache"], anchor.to(device),
                                     partner.to(device), red["product_weight"],
                                     mfma_fragments(red["second_weight"]), red["second_bias"],
                                     scores.to(device), red["norm_weight"], red["norm_bias"],
                                     pos.to(device), 1e-5)
    torch.cuda.synchronize()
    assert frag.shape == plain.shape
    assert torch.equal(frag, plain)


def test_fragment_order_outside_the_kernel_raises(device):
    # d_model 576: the three-op chain needs the [D, H] weight.
    cfg = RelationConfig("frag", 1, 64, 576, 32, 64, 2, 4, torch.bfloat16, relation_dim=128,
                         hidden_dim=256, seed=5)
    red = reduce_inputs(cfg, device=device)
    expanded = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])
    anchor, partner, scores, pos = indices_and_scores(1, 64, 64, 4, seed=2)
    with pytest.raises(RuntimeError, match="fragment order needs the fused kernel"):
        relation_reduce_fused_seq(expanded, red["operand_cache"], anchor.to(device),
                                  partner.to(device), red["product_weight"],
                                  mfma_fragments(red["second_weight"]), red["second_bias"],
                                  scores.to(device), red["norm_weight"], red["norm_bias"],
                                  pos.to(device), 1e-5)


def test_fused_op_runs_the_chain_outside_the_kernel_bf16(device):
    """cfg3's d_model 576 is outside the fused kernel's register budget: the op
    runs the unfused three-op chain and still matches the oracle chain."""
    cfg = RelationConfig(**{**CONFIGS["cfg3"].__dict__, "batch": 2})
    red = reduce_inputs(cfg, device=device)
    expanded = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])
    anchor, partner, scores, pos = indices_and_scores(2, 40, cfg.context, cfg.k_out, seed=13)
    fused = run_fused(red, expanded, anchor, partner, scores, pos, device)
    unfused = run_unfused(red, expanded, anchor, partner, scores, pos, device)
    torch.cuda.synchronize()
    assert fused.shape == (2, 40, 576)
    assert torch.equal(fused, unfused)
    expected = oracle_chain(red, expanded, host(anchor), host(partner), host(scores),
                            np.arange(40))
    assert abs_err(host(fused), expected) <= TIGHT_ABS


def rel_err(got, expected):
    got = np.asarray(got, np.float64)
    expected = np.asarray(expected, np.float64)
    return float(np.abs(got - expected).max() / max(np.abs(expected).max(), 1e-30))


@pytest.mark.parametrize("k_out", [5, 6, 7])
def test_fused_op_reference_shapes_fp32(device, k_out):
    """The reference's fp32 d_model 576 / hidden 2304 reduce with K = 5, 6, 7
    (tests/test_relation_reduce_gpu.py:163-200 of the reference) through
    relation_reduce_fused_seq: fp32 operands run the three-op chain on HIP;
    float64 oracle chain (no bf16 rounding) at 1e-5 relative."""
    g = torch.Generator().manual_seed(20261130 + k_out)
    batch, context, queries, rdim, hdim, dmodel = 2, 64, 24, 128, 2304, 576
    operand = torch.randn(batch, context, rdim, generator=g)
    expanded = torch.randn(batch, context, 2 * hdim, generator=g) * 0.5
    product_weight = torch.randn(hdim, rdim, generator=g) * 0.05
    second_weight = torch.randn(dmodel, hdim, generator=g) * 0.02
    second_bias = torch.randn(dmodel, generator=g) * 0.01
    norm_weight = torch.randn(dmodel, generator=g) * 0.05 + 1.0
    norm_bias = torch.randn(dmodel, generator=g) * 0.01
    anchor, partner, scores, pos = indices_and_scores(batch, queries, context, k_out,
                                                      seed=70 + k_out)
    got = relation_reduce_fused_seq(expanded.to(device), operand.to(device), anchor.to(device),
                                    partner.to(device), product_weight.to(device),
                                    second_weight.to(device), second_bias.to(device),
                                    scores.to(device), norm_weight.to(device),
                                    norm_bias.to(device), pos.to(device), 1e-5)
    torch.cuda.synchronize()
    assert got.shape == (batch, queries, dmodel) and got.dtype == torch.float32
    hidden = ored.relation_hidden_cached_seq(host(expanded), host(operand), host(anchor),
                                             host(partner), host(product_weight))
    raw = ored.linear(hidden, host(second_weight), host(second_bias))
    expected = ored.relation_norm_reduce_seq(raw, host(scores), host(norm_weight),
                                             host(norm_bias), host(pos), 1e-5)
    assert rel_err(host(got), expected) <= 1e-5


def test_cfg4_fused_reduce(device):
    """Config 4 shape: B=8, T=2048, d_model 512, hidden 1024, K=8 -- the full run
    against the unfused chain, a sample of queries against the float64 oracle."""
    cfg = CONFIGS["cfg4"]
    red = reduce_inputs(cfg, device=device)
    expanded = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])
    anchor, partner, scores, pos = causal_partner_indices(cfg, seed=41)
    assert bool((partner[:, 1:] != anchor[:, 1:, None]).all())
    assert bool(((partner[:, 1:] >= 0) & (partner[:, 1:] <= pos[None, 1:, None])).all())
    fused = run_fused(red, expanded, anchor, partner, scores, pos, device)
    unfused = run_unfused(red, expanded, anchor, partner, scores, pos, device)
    torch.cuda.synchronize()
    assert fused.shape == (cfg.batch, cfg.context, cfg.d_model)
    assert bool(torch.isfinite(fused).all())
    assert abs_err(host(fused), host(unfused)) <= TIGHT_ABS
    sample = np.array([0, 1, 2, 7, 8, 63, 64, 511, 1024, 1500, 2046, 2047])
    for b in (0, cfg.batch - 1):
        rows = slice(b, b + 1)
        expected = oracle_chain(red, expanded, host(anchor)[:, sample], host(partner)[:, sample],
                                host(scores)[:, sample], sample, rows)
        got = host(fused)[b:b + 1, sample]
        assert abs_err(got, expected) <= TIGHT_ABS, b
