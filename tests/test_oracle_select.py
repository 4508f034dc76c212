"""Pins of the routed-selection oracle (oracle/select.py) against independent formulations.

Each test compares the lane-based oracle with something it does not share code
with: the dense causal argmax/top-k of relation_context (torch), the router's
logsumexp block scores, a per-query brute force over Python sets, or answers
fixed by construction (duplicate keys, sentinels).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import dense, router
from oracle import select as osel


def _inputs(rng, batch, context, blocks, *, exact_dim=64, heads=4, head_dim=16, rel_buckets=16,
            queries=None, bf16=False):
    """Seeded inputs in the layout of tests/test_relation_select_gpu.py:16-31."""
    q = context if queries is None else queries

    def randn(*shape):
        x = rng.standard_normal(shape).astype(np.float32)
        if bf16:
            x = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
        return x

    return {
        "anchor_query": randn(batch, q, exact_dim),
        "anchor_keys": randn(batch, context, exact_dim),
        "anchor_router_query": randn(batch, q, heads * head_dim),
        "anchor_block_mean": randn(batch, blocks, heads, head_dim),
        "anchor_block_std": np.abs(randn(batch, blocks, heads, head_dim)),
        "anchor_gamma": randn(heads),
        "anchor_bias": randn(heads, rel_buckets),
        "partner_base": randn(batch, q, 2 * exact_dim),
        "partner_anchor_cache": randn(batch, context, 2 * exact_dim),
        "partner_keys": randn(batch, context, exact_dim),
        "partner_block_mean": randn(batch, blocks, heads, head_dim),
        "partner_block_std": np.abs(randn(batch, blocks, heads, head_dim)),
        "partner_gamma": randn(heads),
        "partner_bias": randn(heads, rel_buckets),
    }


def _seq(inp, positions, local, top, k, strict):
    return osel.relation_select_packed_seq(
        inp["anchor_query"], inp["anchor_keys"], inp["anchor_router_query"],
        inp["anchor_block_mean"], inp["anchor_block_std"], inp["anchor_gamma"],
        inp["anchor_bias"], inp["partner_base"], inp["partner_anchor_cache"],
        inp["partner_keys"], inp["partner_block_mean"], inp["partner_block_std"],
        inp["partner_gamma"], inp["partner_bias"], positions, local, top, k, strict)


def test_floor_log2_matches_float_log2():
    n = np.arange(1, 1 << 16)
    expected = np.floor(np.log2(n.astype(np.float64))).astype(np.int64)
    assert np.array_equal(osel.floor_log2(n), expected)


@pytest.mark.parametrize("strict", [False, True])
def test_block_scores_match_router_logsumexp(strict):
    """Pairwise LSE over heads == router logsumexp - log H (block_router.py:96-101)."""
    rng = np.random.default_rng(11)
    batch, length, block_size, heads, head_dim = 2, 96, 8, 4, 16
    blocks = length // block_size
    keys = rng.standard_normal((batch, length, heads * head_dim))
    query = rng.standard_normal((batch, length, heads * head_dim)).astype(np.float32)
    mean, std = router.block_statistics(keys, block_size, heads, head_dim)
    mean, std = mean.astype(np.float32), std.astype(np.float32)
    gamma = rng.standard_normal(heads).astype(np.float32)
    bias = rng.standard_normal((heads, 16)).astype(np.float32)
    expected = router.router_scores(query, mean, std, gamma, bias, block_size) + math.log(heads)
    batch_of = np.repeat(np.arange(batch), length)
    t = np.tile(np.arange(length), batch)
    got = osel.block_scores(query.reshape(batch * length, -1), mean, std, gamma, bias, batch_of,
                            t, block_size=block_size, local_window=16, strict_valid=strict)
    got = got.reshape(batch, length, blocks)
    eligible, _, _ = osel.block_geometry(t, blocks, block_size, 16, strict, 16)
    eligible = eligible.reshape(batch, length, blocks)
    assert np.all(np.isneginf(got[~eligible]))
    finite = eligible
    assert np.allclose(got[finite], expected[finite], rtol=2e-7, atol=2e-6)
    if not strict:
        assert np.array_equal(np.isfinite(got), np.isfinite(expected))


def test_one_shot_and_pairwise_head_logsumexp_agree():
    """The reference kernel's pairwise fold == one-shot logsumexp, to float64 ulps."""
    rng = np.random.default_rng(17)
    per_head = rng.standard_normal((20000, 4)) * rng.choice([0.01, 1.0, 30.0], (20000, 1))
    one = osel.logsumexp_heads(per_head)
    pair = osel.logsumexp_heads_pairwise(per_head)
    assert np.max(np.abs(one - pair) / np.maximum(np.abs(pair), 1.0)) < 1e-14
    # and both round to the same float32 on this sample
    assert np.array_equal(one.astype(np.float32), pair.astype(np.float32))
    # exact special cases: equal heads give s + log(H); one dominant head gives s
    assert osel.logsumexp_heads(np.full((1, 4), 2.5))[0] == 2.5 + np.log(4.0)
    assert osel.logsumexp_heads(np.array([[800.0, 0.0, 0.0, 0.0]]))[0] == 800.0


def test_block_statistics_match_torch():
    rng = np.random.default_rng(5)
    keys = rng.standard_normal((2, 40, 64))
    mean, std = router.block_statistics(keys, 8, 4, 16)
    grouped = torch.from_numpy(keys).view(2, 5, 8, 4, 16)
    assert np.allclose(mean, grouped.mean(2).numpy(), atol=1e-12)
    assert np.allclose(std, grouped.std(2, unbiased=False).numpy(), atol=1e-12)


def _dense_check(inp, local, top, k, strict, context):
    a, s, p, ps = _seq(inp, np.arange(context), local, top, k, strict)
    t_inp = {key: torch.from_numpy(np.ascontiguousarray(v)) for key, v in inp.items()}
    da, ds, dp, dps = dense.relation_context_selection(
        t_inp["anchor_query"], t_inp["anchor_keys"], t_inp["partner_base"],
        t_inp["partner_anchor_cache"], t_inp["partner_keys"], k)
    assert np.array_equal(a, da.numpy().astype(np.int32))
    assert np.array_equal(s, ds.numpy())
    finite = np.isfinite(dps.numpy())
    assert np.array_equal(np.isfinite(ps), finite)
    assert np.array_equal(p[finite], dp.numpy()[finite].astype(np.int32))
    assert np.array_equal(ps[finite], dps.numpy()[finite])
    # slots past the available candidates repeat lane 0 (position t-LOCAL+1, -inf)
    t = np.broadcast_to(np.arange(context)[None, :, None], p.shape)
    assert np.array_equal(p[~finite], (t - local + 1)[~finite])
    return a, s, p, ps


@pytest.mark.parametrize("bf16", [False, True])
def test_short_context_equals_dense_selection(bf16):
    """T <= LOCAL: local window covers [0, t], no remote block is ever eligible."""
    rng = np.random.default_rng(29)
    inp = _inputs(rng, batch=3, context=32, blocks=4, bf16=bf16)
    _dense_check(inp, local=32, top=2, k=8, strict=False, context=32)


def test_all_blocks_picked_equals_dense_selection():
    """Compat mode, TOP >= blocks, LOCAL >= BS: candidates are exactly [0, t]."""
    rng = np.random.default_rng(31)
    inp = _inputs(rng, batch=2, context=64, blocks=8)
    _dense_check(inp, local=8, top=8, k=8, strict=False, context=64)


def _brute_force(inp, b, t, local, top, k, strict):
    """Per-query set construction from the router's logsumexp block ranking."""
    context = inp["anchor_keys"].shape[1]
    blocks = inp["anchor_block_mean"].shape[1]
    block_size = context // blocks
    local_start = max(t - local + 1, 0)

    def ranked_blocks(side, q_router):
        queries = np.zeros((1, t + 1, q_router.shape[-1]), dtype=np.float32)
        queries[0, t] = q_router
        scores = router.router_scores(
            queries, inp[f"{side}_block_mean"][b:b + 1], inp[f"{side}_block_std"][b:b + 1],
            inp[f"{side}_gamma"], inp[f"{side}_bias"], block_size)[0, t]
        ok = [j for j in range(blocks)
              if (j + 1) * block_size - 1 <= t
              and (not strict or (j + 1) * block_size - 1 < local_start)]
        return sorted(ok, key=lambda j: (-np.float32(scores[j] + math.log(4)), j))[:top]

    def lanes(chosen):
        out = [p for p in range(t - local + 1, t + 1) if p >= 0]
        for j in chosen:
            out += [p for p in range(j * block_size, (j + 1) * block_size) if p < local_start]
        return out

    def score(keys, pos, query):
        return np.float32(np.dot(keys[b, pos].astype(np.float64), query.astype(np.float64))
                          / math.sqrt(keys.shape[-1]))

    aq = inp["anchor_query"][b, t]
    cand = lanes(ranked_blocks("anchor", inp["anchor_router_query"][b, t]))
    anchor = min(cand, key=lambda p: (-score(inp["anchor_keys"], p, aq), p))
    contribution = inp["partner_anchor_cache"][b, anchor]
    base = inp["partner_base"][b, t]
    pq = (base[:64] + contribution[:64]).astype(np.float32)
    prq = (base[64:] + contribution[64:]).astype(np.float32)
    cand = [p for p in lanes(ranked_blocks("partner", prq)) if p != anchor]
    order = sorted(range(len(cand)), key=lambda i: (-score(inp["partner_keys"], cand[i], pq), i))
    partners = [cand[i] for i in order[:k]]
    partners += [t - local + 1] * (k - len(partners))
    return anchor, partners


@pytest.mark.parametrize("strict", [False, True])
def test_brute_force_routed_selection(strict):
    rng = np.random.default_rng(41 + strict)
    context, blocks, local, top, k = 64, 8, 8, 2, 6
    inp = _inputs(rng, batch=2, context=context, blocks=blocks)
    a, _, p, _ = _seq(inp, np.arange(context), local, top, k, strict)
    for b in range(2):
        for t in range(context):
            anchor, partners = _brute_force(inp, b, t, local, top, k, strict)
            assert a[b, t] == anchor, (b, t)
            assert list(p[b, t]) == partners, (b, t)


def test_anchor_ties_go_to_lowest_position():
    rng = np.random.default_rng(3)
    context, blocks, local = 64, 8, 8
    inp = _inputs(rng, batch=1, context=context, blocks=blocks, queries=1)
    t = 63
    aq = inp["anchor_query"][0, 0]
    # make position 5 (remote block 0) and 60 (local) exact duplicates that dominate
    strong = (aq * 10.0).astype(np.float32)
    inp["anchor_keys"][0, 5] = strong
    inp["anchor_keys"][0, 60] = strong
    inp["anchor_block_mean"][0, 0] = 50.0   # block 0 wins the anchor routing
    a, s, _, _ = _seq(inp, np.array([t]), local, 2, 4, False)
    assert a[0, 0] == 5
    inp["anchor_block_mean"][0, 0] = -50.0  # block 0 not routed: only the local copy is seen
    a, _, _, _ = _seq(inp, np.array([t]), local, 2, 4, False)
    assert a[0, 0] == 60


def test_partner_ties_go_to_lowest_lane_not_position():
    """Local lanes precede remote lanes (relation_select.py:246-300)."""
    rng = np.random.default_rng(4)
    context, blocks, local = 64, 8, 8
    inp = _inputs(rng, batch=1, context=context, blocks=blocks, queries=1)
    t = 63
    inp["anchor_keys"][0] = 0.0
    inp["anchor_keys"][0, 62] = inp["anchor_query"][0, 0] * 4.0   # anchor = 62
    contribution = inp["partner_anchor_cache"][0, 62]
    pq = (inp["partner_base"][0, 0, :64] + contribution[:64]).astype(np.float32)
    strong = (pq * 8.0).astype(np.float32)
    inp["partner_keys"][0, 9] = strong      # remote (block 1)
    inp["partner_keys"][0, 57] = strong     # local
    inp["partner_block_mean"][0, 1] = 80.0  # block 1 routed first
    a, _, p, ps = _seq(inp, np.array([t]), local, 2, 4, False)
    assert a[0, 0] == 62
    assert list(p[0, 0, :2]) == [57, 9]
    assert ps[0, 0, 0] == ps[0, 0, 1]


def test_sentinel_for_missing_partners():
    rng = np.random.default_rng(8)
    inp = _inputs(rng, batch=2, context=64, blocks=8)
    local, k = 16, 8
    _, _, p, ps = _seq(inp, np.arange(64), local, 2, k, True)
    for t in range(5):
        available = t  # t+1 causal positions minus the anchor
        assert np.all(np.isfinite(ps[:, t, :available]))
        assert np.all(np.isneginf(ps[:, t, available:]))
        assert np.all(p[:, t, available:] == t - local + 1)


def test_invariants_at_cfg2_shape():
    """Anchor <= t; partners distinct, != anchor, <= t; scores non-increasing; rescoring."""
    rng = np.random.default_rng(20261203)
    context, blocks, local, top, k = 512, 16, 64, 4, 8
    inp = _inputs(rng, batch=2, context=context, blocks=blocks, bf16=True)
    for strict in (False, True):
        a, s, p, ps = _seq(inp, np.arange(context), local, top, k, strict)
        t = np.arange(context)[None, :]
        assert np.all((a >= 0) & (a <= t))
        finite = np.isfinite(ps)
        assert np.all(np.diff(ps, axis=-1)[np.isfinite(ps[..., 1:])] <= 0)
        for b in range(2):
            for tt in range(0, context, 37):
                valid = p[b, tt][finite[b, tt]]
                assert len(set(valid.tolist())) == len(valid)
                assert a[b, tt] not in valid and np.all(valid <= tt) and np.all(valid >= 0)
                if strict:
                    local_start = max(tt - local + 1, 0)
                    remote = valid[valid < local_start]
                    assert np.all(((remote // 32) + 1) * 32 - 1 < local_start)
                rescored = np.float32(np.dot(inp["anchor_keys"][b, a[b, tt]].astype(np.float64),
                                             inp["anchor_query"][b, tt].astype(np.float64)) / 8.0)
                assert rescored == s[b, tt]


def test_packed_equals_two_op_composition():
    """Packed op == anchor_select followed by partner_topk (tests/test_relation_select_gpu.py:33-87)."""
    rng = np.random.default_rng(29)
    inp = _inputs(rng, batch=4, context=512, blocks=64, queries=1)
    dec = {k: (v[:, 0] if v.ndim == 3 and v.shape[1] == 1 else v) for k, v in inp.items()}
    position = 511
    packed = osel.relation_select_packed(
        dec["anchor_query"], dec["anchor_keys"], dec["anchor_router_query"],
        dec["anchor_block_mean"], dec["anchor_block_std"], dec["anchor_gamma"],
        dec["anchor_bias"], dec["partner_base"], dec["partner_anchor_cache"],
        dec["partner_keys"], dec["partner_block_mean"], dec["partner_block_std"],
        dec["partner_gamma"], dec["partner_bias"], position, 16, 2, 8, False)
    anchor, anchor_score = osel.anchor_select(
        dec["anchor_query"], dec["anchor_keys"], dec["anchor_router_query"],
        dec["anchor_block_mean"], dec["anchor_block_std"], dec["anchor_gamma"],
        dec["anchor_bias"], position, 16, 2, False)
    contribution = dec["partner_anchor_cache"][np.arange(4), anchor]
    partner, partner_score = osel.partner_topk(
        dec["partner_base"][:, :64] + contribution[:, :64], dec["partner_keys"],
        dec["partner_base"][:, 64:] + contribution[:, 64:], dec["partner_block_mean"],
        dec["partner_block_std"], dec["partner_gamma"], dec["partner_bias"], position, anchor,
        16, 2, 8, False)
    assert np.array_equal(packed[0], anchor) and np.array_equal(packed[2], partner)
    assert np.array_equal(packed[1], anchor_score) and np.array_equal(packed[3], partner_score)
