"""The eager fp32 torch restatement (oracle/eager.py, the CPU baseline bench.py
times) against the float64 oracle on seeded inputs: selected indices equal
(fp32 accumulation can only move a near-tie within an fp32 ulp, which these
seeds do not contain) and contexts within 1e-4 absolute."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import eager
from oracle import reduce as ored
from oracle import select as osel
from relation_lm.workloads import CONFIGS, RelationConfig, SELECT_ORDER, reduce_inputs, selection_inputs


def f32(d):
    return {k: (v.float() if v.dtype.is_floating_point else v) for k, v in d.items()}


def np64(d):
    return {k: v.numpy() for k, v in d.items()}


@pytest.mark.parametrize("cfg", [CONFIGS["cfg1"],
                                 RelationConfig("small", 2, 256, 256, 32, 64, 4, 8, torch.float32,
                                                hidden_dim=256, seed=77),
                                 RelationConfig("strict", 1, 192, 256, 16, 48, 3, 5, torch.float32,
                                                hidden_dim=256, strict_valid=True, seed=78)])
def test_eager_chain_matches_oracle(cfg):
    sel = f32(selection_inputs(cfg))
    red = f32(reduce_inputs(cfg))
    a, p, ctx = eager.relation_chain_seq(sel, red, cfg)
    hs, hr = np64(sel), np64(red)
    oa, _, op, ops = osel.relation_select_packed_seq(*[hs[k] for k in SELECT_ORDER],
                                                     hs["positions"], cfg.local_window,
                                                     cfg.top_blocks, cfg.k_out, cfg.strict_valid)
    np.testing.assert_array_equal(a.numpy(), oa)
    np.testing.assert_array_equal(p.numpy(), op)
    expanded = ored.linear(hr["operand_cache"], hr["expanded_weight"], hr["expanded_bias"])
    hidden = ored.relation_hidden_cached_seq(expanded, hr["operand_cache"], oa, op,
                                             hr["product_weight"])
    raw = ored.linear(hidden, hr["second_weight"], hr["second_bias"])
    octx = ored.relation_norm_reduce_seq(raw, ops, hr["norm_weight"], hr["norm_bias"],
                                         hs["positions"], 1e-5)
    np.testing.assert_allclose(ctx.numpy(), octx, atol=1e-4, rtol=0)


def test_eager_decode_step_matches_oracle():
    cfg = RelationConfig(**{**CONFIGS["cfg3"].__dict__, "batch": 2, "dtype": torch.float32,
                            "hidden_dim": 256})
    sel = f32(selection_inputs(cfg, queries=1))
    red = f32(reduce_inputs(cfg))
    memory = torch.randn(2, cfg.d_model, generator=torch.Generator().manual_seed(5))
    weight = torch.randn(512, cfg.d_model, generator=torch.Generator().manual_seed(6)) * 0.04
    projected, a, p, ctx = eager.relation_decode_step(sel, red, eager.expanded_cache(red), memory,
                                                      weight, cfg)
    hs, hr = np64(sel), np64(red)
    oa, _, op, ops = osel.relation_select_packed(*[hs[k] for k in SELECT_ORDER], hs["position"],
                                                 cfg.local_window, cfg.top_blocks, cfg.k_out,
                                                 cfg.strict_valid)
    np.testing.assert_array_equal(a.numpy(), oa)
    np.testing.assert_array_equal(p.numpy(), op)
    np.testing.assert_allclose(projected.numpy(),
                               ored.packed_sparse_cache_projection(memory.numpy(), weight.numpy()),
                               atol=1e-4, rtol=0)
    expanded = ored.linear(hr["operand_cache"], hr["expanded_weight"], hr["expanded_bias"])
    hidden = ored.relation_hidden_cached(expanded, hr["operand_cache"], oa, op, hr["product_weight"])
    raw = ored.linear(hidden, hr["second_weight"], hr["second_bias"])
    octx = ored.relation_norm_reduce(raw, ops, hr["norm_weight"], hr["norm_bias"], hs["position"],
                                     1e-5)
    np.testing.assert_allclose(ctx.numpy(), octx, atol=1e-4, rtol=0)
