"""The headline step end to end against the float64 oracle, every query.

bench.py's cfg2 step is expanded projection -> relation_select_packed_seq ->
relation_reduce_fused_seq.  Here the same three launches run on the device and
the oracle recomputes the whole chain from the same seeded inputs on the CPU:
its own expanded projection (float64, stored as bf16 as the device stores it),
its own selection (reference semantics, relation_select.py:9-308), the hidden
(relation_reduce.py:87-146) rounded to bf16 as the fused kernel hands it to
the bf16 second linear, the second linear and the LayerNorm / active-K softmax
/ partner sum (relation_reduce.py:374-417).
  * indices: bit-exact for all 4096 queries (anchor and every partner slot);
  * scores: equal to the oracle's float32 values;
  * context: absolute error <= 2e-2 (north_star, bf16) and <= 5e-3 (tight bound
    that a dropped or mis-indexed term cannot hide under).
The cfg4 fused reduce is checked the same way on all 16384 queries.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reduce as ored
from oracle import select as osel
from relation_lm.kernels.relation_reduce import (mfma_fragments, relation_linear,
                                                 relation_reduce_fused_seq)
from relation_lm.kernels.relation_select import relation_select_packed_seq
from relation_lm.workloads import (
    CONFIGS,
    SELECT_ORDER,
    causal_partner_indices,
    reduce_inputs,
    select_args,
    selection_inputs,
)

pytestmark = pytest.mark.gpu

BF16_ABS = 2e-2
TIGHT_ABS = 5e-3


def host(t):
    return t.detach().float().cpu().numpy() if t.dtype.is_floating_point else t.cpu().numpy()


def oracle_reduce_chain(expanded, red, anchor, partner, scores, positions, chunk=256):
    """float64 hidden (rounded to bf16) -> second linear -> norm-reduce, chunked over queries.

    expanded [B,T,2H] float64 values, anchor [B,Q], partner [B,Q,K], scores [B,Q,K],
    positions [Q].  Returns ctx [B,Q,D] float32.
    """
    operand = host(red["operand_cache"])
    wm, w2, b2 = host(red["product_weight"]), host(red["second_weight"]), host(red["second_bias"])
    gamma, beta = host(red["norm_weight"]), host(red["norm_bias"])
    batch, queries = anchor.shape
    out = np.zeros((batch, queries, w2.shape[0]), np.float32)
    for b in range(batch):
        for lo in range(0, queries, chunk):
            sl = slice(lo, min(queries, lo + chunk))
            hidden = ored.relation_hidden_cached_seq(expanded[b:b + 1], operand[b:b + 1],
                                                     anchor[b:b + 1, sl], partner[b:b + 1, sl], wm)
            raw = ored.linear(ored.round_to(hidden, "bfloat16"), w2, b2)
            out[b, sl] = ored.relation_norm_reduce_seq(raw, scores[b:b + 1, sl], gamma, beta,
                                                       positions[sl], 1e-5)[0]
    return out


def assert_context(got, expected):
    err = float(np.abs(got.astype(np.float64) - expected.astype(np.float64)).max())
    assert np.isfinite(got).all()
    assert err <= BF16_ABS, err
    assert err <= TIGHT_ABS, err


def test_cfg2_headline_step_every_query(device):
    cfg = CONFIGS["cfg2"]
    sel = selection_inputs(cfg, device=device)
    red = reduce_inputs(cfg, device=device)
    positions = sel["positions"]
    print(f"cfg2 headline step: B={cfg.batch} T={cfg.context}", flush=True)

    # The device step, launch for launch as bench.py runs it.
    expanded = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])
    a, s, p, ps = relation_select_packed_seq(*select_args(sel, cfg))
    ctx = relation_reduce_fused_seq(expanded, red["operand_cache"], a, p, red["product_weight"],
                                    mfma_fragments(red["second_weight"]), red["second_bias"], ps,
                                    red["norm_weight"], red["norm_bias"], positions, 1e-5)
    torch.cuda.synchronize()

    # The oracle chain from the same host inputs.
    hs = {k: host(sel[k]) for k in SELECT_ORDER}
    ea, es, ep, eps_ = osel.relation_select_packed_seq(
        *[hs[k] for k in SELECT_ORDER], host(positions), cfg.local_window, cfg.top_blocks,
        cfg.k_out, cfg.strict_valid)
    assert np.array_equal(host(a), ea)
    assert np.array_equal(host(p), ep)
    assert np.array_equal(host(s), es)
    assert np.array_equal(host(ps), eps_)
    e_expanded = ored.round_to(ored.linear(host(red["operand_cache"]), host(red["expanded_weight"]),
                                           host(red["expanded_bias"])), "bfloat16")
    # The device's expanded cache equals the oracle's up to one bf16 rounding step.
    d_expanded = host(expanded).astype(np.float64)
    assert np.abs(d_expanded - e_expanded).max() <= 2.0 ** -7 * np.abs(e_expanded).max()
    expected = oracle_reduce_chain(e_expanded, red, ea, ep, eps_, host(positions))
    assert_context(host(ctx), expected)


def test_cfg4_fused_reduce_every_query(device):
    cfg = CONFIGS["cfg4"]
    red = reduce_inputs(cfg, device=device)
    anchor, partner, scores, pos = causal_partner_indices(cfg, seed=41)
    print(f"cfg4 fused reduce: B={cfg.batch} T={cfg.context}", flush=True)
    expanded = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])
    ctx = relation_reduce_fused_seq(expanded, red["operand_cache"], anchor.to(device),
                                    partner.to(device), red["product_weight"],
                                    mfma_fragments(red["second_weight"]), red["second_bias"],
                                    scores.to(device),
                                    red["norm_weight"], red["norm_bias"], pos.to(device), 1e-5)
    torch.cuda.synchronize()
    expected = oracle_reduce_chain(host(expanded).astype(np.float64), red, host(anchor),
                                   host(partner), host(scores), host(pos), chunk=512)
    assert_context(host(ctx), expected)
