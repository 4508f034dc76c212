"""Pins oracle/multi_block.py: the multi-anchor block after selection.

(1) Against a dense torch forward written with the reference module's structure
(src/relation_lm/models/multi_relation_blocks.py:21-207: nn.Linear / nn.LayerNorm
/ nn.GELU modules, the iterative distinct-anchor argmax with F.one_hot masks,
torch.topk over the all-anchor-masked partner scores, softmax / masked
renormalisations), in float64 on tiny shapes: the oracle, fed that forward's
own selection, must reproduce its output, and the stack with its final norm.
(2) Invariants of the mixing rules, on random inputs.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from oracle import multi_block as omb
from oracle.dense_block import DenseBlock


def params_of(block: DenseBlock) -> dict:
    n = lambda t: t.detach().numpy()
    return {"operand": n(block.operand.weight),
            "mlp_w1": n(block.relation_mlp[0].weight), "mlp_b1": n(block.relation_mlp[0].bias),
            "mlp_w2": n(block.relation_mlp[2].weight), "mlp_b2": n(block.relation_mlp[2].bias),
            "mlp_ln_w": n(block.relation_mlp[3].weight), "mlp_ln_b": n(block.relation_mlp[3].bias),
            "slot_mix_logits": n(block.slot_mix_logits), "residual_gate": float(block.residual_gate.detach())}


def make_block(seed, d=16, g=8, r=6, slots=3, k=4):
    torch.manual_seed(seed)
    block = DenseBlock(d, g, r, slots, k).double()
    with torch.no_grad():
        block.input_norm.weight.normal_(1.0, 0.1)
        block.input_norm.bias.normal_(0.0, 0.1)
        block.relation_mlp[3].weight.normal_(1.0, 0.1)
        block.relation_mlp[3].bias.normal_(0.0, 0.1)
    return block


@pytest.mark.parametrize("seed,t", [(0, 5), (1, 9), (2, 12)])
def test_post_selection_matches_dense_forward(seed, t):
    block = make_block(seed)
    g = torch.Generator().manual_seed(100 + seed)
    hidden = torch.randn(2, t, 16, generator=g, dtype=torch.float64)
    memory = torch.randn(2, t, 16, generator=g, dtype=torch.float64)
    with torch.no_grad():
        out, diag = block(hidden, memory)
    got, context = omb.block_post_selection(hidden.numpy(), memory.numpy(),
                                            diag["anchor_index"].numpy(),
                                            diag["partner_index"].numpy(), diag["top"].numpy(),
                                            params_of(block))
    np.testing.assert_allclose(got, out.numpy(), rtol=0, atol=1e-12)
    np.testing.assert_allclose(context, diag["context"].numpy(), rtol=0, atol=1e-12)


def test_stack_with_final_norm():
    blocks = [make_block(10 + i) for i in range(3)]
    final = nn.LayerNorm(16).double()
    with torch.no_grad():
        final.weight.normal_(1.0, 0.1)
        final.bias.normal_(0.0, 0.1)
    g = torch.Generator().manual_seed(7)
    hidden = torch.randn(1, 10, 16, generator=g, dtype=torch.float64)
    memory = torch.randn(1, 10, 16, generator=g, dtype=torch.float64)
    x, y = hidden, hidden.numpy()
    with torch.no_grad():
        for block in blocks:
            x, diag = block(x, memory)
            y, _ = omb.block_post_selection(y, memory.numpy(), diag["anchor_index"].numpy(),
                                            diag["partner_index"].numpy(), diag["top"].numpy(),
                                            params_of(block))
        ref = final(x)
    got = omb.layer_norm(y, final.weight.detach().numpy(), final.bias.detach().numpy(), 1e-5)
    np.testing.assert_allclose(got, ref.numpy(), rtol=0, atol=1e-11)


def random_reduce_case(seed, b=2, tq=7, s=3, k=5, d=12):
    rng = np.random.default_rng(seed)
    raw = rng.normal(size=(b, tq, s, k, d))
    scores = rng.normal(size=(b, tq, s, k)).astype(np.float32)
    scores[rng.random(scores.shape) < 0.3] = -np.inf
    return dict(raw=raw, partner_scores=scores, norm_weight=rng.normal(1, 0.1, d),
                norm_bias=rng.normal(0, 0.1, d), slot_mix_logits=rng.normal(size=s),
                residual_gate=0.4, hidden=rng.normal(size=(b, tq, d)),
                positions=np.arange(tq), norm_eps=1e-5)


def test_gate_to_minus_infinity_returns_input():
    case = random_reduce_case(1)
    case["residual_gate"] = -np.inf
    out, _ = omb.multi_relation_reduce_seq(**case)
    np.testing.assert_array_equal(out, case["hidden"])


def test_partner_order_does_not_matter():
    case = random_reduce_case(2)
    out, ctx = omb.multi_relation_reduce_seq(**case)
    perm = np.random.default_rng(3).permutation(case["raw"].shape[3])
    case["raw"] = case["raw"][:, :, :, perm]
    case["partner_scores"] = case["partner_scores"][:, :, :, perm]
    out2, ctx2 = omb.multi_relation_reduce_seq(**case)
    np.testing.assert_allclose(out2, out, rtol=0, atol=1e-12)


def test_slot_weights_sum_to_one_over_active_slots():
    active = omb.slot_activity(np.arange(6), 4)
    w = omb.slot_weights(np.array([0.3, -1.0, 2.0, 0.0]), active)
    np.testing.assert_allclose(w.sum(axis=1), 1.0, rtol=0, atol=1e-15)
    assert (w[~active] == 0).all()


def test_all_inactive_slot_adds_nothing():
    case = random_reduce_case(4)
    case["partner_scores"][:, :, 1] = -np.inf
    out, ctx = omb.multi_relation_reduce_seq(**case)
    case["raw"][:, :, 1] = 1.0e3 * np.random.default_rng(5).normal(size=case["raw"][:, :, 1].shape)
    out2, ctx2 = omb.multi_relation_reduce_seq(**case)
    np.testing.assert_array_equal(ctx2, ctx)


def test_block_statistics_against_torch():
    keys = np.random.default_rng(6).normal(size=(2, 24, 5))
    mean, std = omb.block_statistics(keys, 8)
    grouped = torch.from_numpy(keys).view(2, 3, 8, 5)
    np.testing.assert_allclose(mean, grouped.mean(2).numpy(), rtol=0, atol=1e-14)
    np.testing.assert_allclose(std, grouped.std(2, unbiased=False).numpy(), rtol=0, atol=1e-14)
