"""GPU parity of relation_select_packed_expand_row: the decode-form selection
and the token's expanded-cache row in one launch.

The selection must equal relation_select_packed / relation_select_packed_ring
bit for bit (those are checked against the float64 oracle in
test_relation_select_gpu.py and test_ring_gpu.py).  The written row must be
F.linear(operand_cache[:, r], expanded_weight, expanded_bias) -- fp32 sums of
exact bf16 products rounded once to bf16, so within one bf16 rounding of an
fp32 CPU product -- with r the position (ring: position mod T), and every other
cache row untouched.  The cached hidden over the updated cache must then equal
the reference decode's B == 1 update form (relation_hidden_cache_update) to
fp32 rounding.  Covered: cfg3 at B=1 and B=8, a linear cache at its last and a
middle row, a ring cache at a wrapped position, bias absent or fp32, the
stand-alone row launch (2 router heads: the decode kernel does not apply), and
argument errors.
"""
from __future__ import annotations

import pytest
import torch

from relation_lm.kernels.relation_reduce import relation_hidden_cache_update, relation_hidden_cached
from relation_lm.kernels.relation_select import (
    relation_select_packed,
    relation_select_packed_expand_row,
)
from relation_lm.kernels.ring import relation_select_packed_ring
from relation_lm.workloads import CONFIGS, RelationConfig, reduce_inputs, select_args, selection_inputs

pytestmark = pytest.mark.gpu


def cfg3(batch, **kw):
    return RelationConfig(**{**CONFIGS["cfg3"].__dict__, "batch": batch, **kw})


def expected_row(red, weight, bias, r):
    op = red["operand_cache"][:, r].float().cpu()
    out = op @ weight.float().cpu().t()
    if bias is not None:
        out = out + bias.float().cpu()
    return out


def run_case(device, cfg, position, ring, bias_kind="model"):
    sel = selection_inputs(cfg, queries=1, device=device)
    red = reduce_inputs(cfg, device=device)
    sel["position"] = torch.tensor(position, dtype=torch.int64, device=device)
    args = select_args(sel, cfg)
    weight = red["expanded_weight"]
    bias = {"model": red["expanded_bias"], "none": None,
            "f32": red["expanded_bias"].float()}[bias_kind]
    g = torch.Generator().manual_seed(position + 17)
    cache = torch.randn(cfg.batch, cfg.context, weight.shape[0], generator=g).to(device,
                                                                                 torch.bfloat16)
    before = cache.clone()
    got = relation_select_packed_expand_row(*args, red["operand_cache"], weight, bias, cache,
                                            ring)
    ref = (relation_select_packed_ring if ring else relation_select_packed)(*args)
    torch.cuda.synchronize()
    for name, a, b in zip(("anchor", "anchor_score", "partner", "partner_score"), got, ref):
        assert torch.equal(a, b), f"{name} differs from the selection alone"
    r = position % cfg.context if ring else position
    rows = torch.ones(cfg.context, dtype=torch.bool, device=device)
    rows[r] = False
    assert torch.equal(cache[:, rows], before[:, rows]), "rows other than the token's changed"
    torch.testing.assert_close(cache[:, r].float().cpu(), expected_row(red, weight, bias, r),
                               rtol=8e-3, atol=1e-6)
    return sel, red, got, cache, r


@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("position,ring", [(511, False), (300, False), (4095, True), (1000, True)])
def test_cfg3_rows_and_selection(device, batch, position, ring):
    print(f"expand_row B={batch} t={position} ring={ring}", flush=True)
    run_case(device, cfg3(batch), position, ring)


@pytest.mark.parametrize("bias_kind", ["none", "f32"])
def test_bias_forms(device, bias_kind):
    print(f"expand_row bias={bias_kind}", flush=True)
    run_case(device, cfg3(2, seed=501), 400, False, bias_kind)


def test_standalone_row_launch(device):
    # Two router heads of 32: not the decode kernel's shape, so the selection
    # runs on select_kernel and the row on its own launch.
    cfg = cfg3(3, heads=2, head_dim=32, seed=502)
    print("expand_row stand-alone launch", flush=True)
    run_case(device, cfg, 450, False)


def test_cached_hidden_matches_update_form(device):
    # The reference decode's B == 1 path: relation_hidden_cache_update computes
    # the token's row itself.  After the folded row write, the cached form must
    # give the same hidden rows (to fp32 rounding: the row's sums differ in order).
    cfg = cfg3(1, seed=503)
    sel, red, got, cache, r = run_case(device, cfg, 511, False)
    anchor, _, partner, _ = got
    hid_cached = relation_hidden_cached(cache, red["operand_cache"], anchor, partner,
                                        red["product_weight"])
    fresh = cache.clone()
    hid_update = relation_hidden_cache_update(fresh, red["operand_cache"], anchor, partner,
                                              red["anchor_weight"], red["partner_weight"],
                                              red["product_weight"], red["first_bias"],
                                              sel["position"])
    torch.cuda.synchronize()
    torch.testing.assert_close(hid_cached, hid_update, rtol=2e-2, atol=2e-2)


def test_argument_errors(device):
    cfg = cfg3(1, seed=504)
    sel = selection_inputs(cfg, queries=1, device=device)
    red = reduce_inputs(cfg, device=device)
    args = select_args(sel, cfg)
    cache = torch.zeros(cfg.batch, cfg.context, red["expanded_weight"].shape[0],
                        dtype=torch.float32, device=device)
    with pytest.raises(RuntimeError, match="expanded_cache"):
        relation_select_packed_expand_row(*args, red["operand_cache"], red["expanded_weight"],
                                          red["expanded_bias"], cache)
    with pytest.raises(RuntimeError, match="expanded_weight"):
        relation_select_packed_expand_row(*args, red["operand_cache"],
                                          red["expanded_weight"][:-8].contiguous(),
                                          red["expanded_bias"][:-8].contiguous(),
                                          cache.bfloat16()[..., :-8].contiguous())
