"""Pins of the routed multi-anchor selection oracle (oracle/select.py).

The routed multi-anchor op has no reference kernel; its semantics are those of
MultiAnchorRelationBlock (multi_relation_blocks.py:69-147) with the dense
causal candidate set replaced by the routed one.  The oracle is pinned by:
  * one slot: exactly the single-anchor packed selection (a separate code path);
  * every causal position a candidate (T <= LOCAL, or compat mode with all
    blocks picked): exactly the dense multi-anchor selection restated with
    torch on full score matrices (oracle/dense.py);
  * strict mode: a per-query brute force over Python sets;
  * invariants: distinct active anchors, all-anchor partner exclusion,
    inactive-slot conventions.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import dense, router
from oracle import select as osel


def multi_inputs(rng, batch, context, blocks, slots, *, exact_dim=64, heads=4, head_dim=16,
                 rel_buckets=16, queries=None, bf16=False):
    q = context if queries is None else queries

    def randn(*shape):
        x = rng.standard_normal(shape).astype(np.float32)
        if bf16:
            x = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
        return x

    rd = heads * head_dim
    return {
        "anchor_query": randn(batch, q, slots, exact_dim),
        "anchor_keys": randn(batch, context, slots, exact_dim),
        "anchor_router_query": randn(batch, q, rd),
        "anchor_block_mean": randn(batch, blocks, heads, head_dim),
        "anchor_block_std": np.abs(randn(batch, blocks, heads, head_dim)),
        "anchor_gamma": randn(heads),
        "anchor_bias": randn(heads, rel_buckets),
        "partner_base": randn(batch, q, slots, exact_dim + rd),
        "partner_anchor_cache": randn(batch, context, slots, exact_dim + rd),
        "partner_keys": randn(batch, context, slots, exact_dim),
        "partner_block_mean": randn(batch, blocks, heads, head_dim),
        "partner_block_std": np.abs(randn(batch, blocks, heads, head_dim)),
        "partner_gamma": randn(heads),
        "partner_bias": randn(heads, rel_buckets),
    }


ORDER = ("anchor_query", "anchor_keys", "anchor_router_query", "anchor_block_mean",
         "anchor_block_std", "anchor_gamma", "anchor_bias", "partner_base",
         "partner_anchor_cache", "partner_keys", "partner_block_mean", "partner_block_std",
         "partner_gamma", "partner_bias")


def run_multi(inp, positions, local, top, k, strict):
    return osel.multi_relation_select_seq(*[inp[n] for n in ORDER], positions, local, top, k,
                                          strict)


def test_one_slot_equals_single_anchor_selection():
    rng = np.random.default_rng(101)
    for strict in (False, True):
        inp = multi_inputs(rng, batch=2, context=128, blocks=8, slots=1)
        single = {n: (v[:, :, 0] if v.ndim == 4 and n not in ("anchor_block_mean",
                                                              "anchor_block_std",
                                                              "partner_block_mean",
                                                              "partner_block_std") else v)
                  for n, v in inp.items()}
        pos = np.arange(128)
        a, s, p, ps = run_multi(inp, pos, 16, 3, 6, strict)
        sa, ss, sp, sps = osel.relation_select_packed_seq(*[single[n] for n in ORDER], pos, 16,
                                                          3, 6, strict)
        np.testing.assert_array_equal(a[:, :, 0], sa)
        np.testing.assert_array_equal(s[:, :, 0], ss)
        np.testing.assert_array_equal(p[:, :, 0], sp)
        np.testing.assert_array_equal(ps[:, :, 0], sps)


def _dense_check(inp, local, top, k, strict, context):
    slots = inp["anchor_query"].shape[2]
    a, s, p, ps = run_multi(inp, np.arange(context), local, top, k, strict)
    t_inp = {n: torch.from_numpy(np.ascontiguousarray(v)) for n, v in inp.items()}
    da, ds, active, dp, dps = dense.multi_anchor_selection(
        t_inp["anchor_query"], t_inp["anchor_keys"], t_inp["partner_base"],
        t_inp["partner_anchor_cache"], t_inp["partner_keys"], k)
    act = np.broadcast_to(active.numpy()[None], a.shape)
    np.testing.assert_array_equal(a, da.numpy().astype(np.int32))  # inactive slots are 0 in both
    np.testing.assert_array_equal(s, ds.numpy())
    assert np.array_equal(np.isfinite(s), act)
    finite = np.isfinite(dps.numpy())
    assert np.array_equal(np.isfinite(ps), finite)
    np.testing.assert_array_equal(p[finite], dp.numpy()[finite].astype(np.int32))
    np.testing.assert_array_equal(ps[finite], dps.numpy()[finite])
    t = np.broadcast_to(np.arange(context)[None, :, None, None], p.shape)
    np.testing.assert_array_equal(p[~finite], (t - local + 1)[~finite])
    assert slots == a.shape[2]
    return a, s, p, ps


@pytest.mark.parametrize("bf16", [False, True])
def test_short_context_equals_dense_multi_anchor(bf16):
    """T <= LOCAL: every causal position is a local candidate."""
    rng = np.random.default_rng(103 + bf16)
    inp = multi_inputs(rng, batch=2, context=48, blocks=4, slots=4, bf16=bf16)
    _dense_check(inp, local=48, top=2, k=6, strict=False, context=48)


def test_all_blocks_picked_equals_dense_multi_anchor():
    """Compat mode, TOP >= blocks, LOCAL >= BS: candidates are exactly [0, t]."""
    rng = np.random.default_rng(107)
    inp = multi_inputs(rng, batch=2, context=64, blocks=8, slots=3)
    _dense_check(inp, local=8, top=8, k=5, strict=False, context=64)


def _brute_force(inp, b, t, local, top, k, strict):
    """Per-query, per-slot set construction from the router's logsumexp ranking."""
    context = inp["anchor_keys"].shape[1]
    blocks = inp["anchor_block_mean"].shape[1]
    slots = inp["anchor_query"].shape[2]
    exact_dim = inp["anchor_query"].shape[3]
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
        return np.float32(np.dot(keys.astype(np.float64)[b, pos], query.astype(np.float64))
                          / math.sqrt(exact_dim))

    cand = lanes(ranked_blocks("anchor", inp["anchor_router_query"][b, t]))
    anchors = []
    for s in range(min(slots, t + 1)):
        left = [p for p in cand if p not in anchors]
        aq = inp["anchor_query"][b, t, s]
        anchors.append(min(left, key=lambda p: (-score(inp["anchor_keys"][:, :, s], p, aq), p)))
    partners = []
    for s in range(slots):
        if s >= len(anchors):
            partners.append([t - local + 1] * k)
            continue
        contribution = inp["partner_anchor_cache"][b, anchors[s], s]
        base = inp["partner_base"][b, t, s]
        pq = (base[:exact_dim] + contribution[:exact_dim]).astype(np.float32)
        prq = (base[exact_dim:] + contribution[exact_dim:]).astype(np.float32)
        cand_p = [p for p in lanes(ranked_blocks("partner", prq)) if p not in anchors]
        keys = inp["partner_keys"][:, :, s]
        order = sorted(range(len(cand_p)), key=lambda i: (-score(keys, cand_p[i], pq), i))
        got = [cand_p[i] for i in order[:k]]
        partners.append(got + [t - local + 1] * (k - len(got)))
    return anchors + [0] * (slots - len(anchors)), partners


@pytest.mark.parametrize("strict", [False, True])
def test_brute_force_routed_multi_anchor(strict):
    rng = np.random.default_rng(109 + strict)
    context, blocks, local, top, k, slots = 64, 8, 8, 2, 4, 3
    inp = multi_inputs(rng, batch=2, context=context, blocks=blocks, slots=slots)
    a, _, p, _ = run_multi(inp, np.arange(context), local, top, k, strict)
    for b in range(2):
        for t in range(context):
            anchors, partners = _brute_force(inp, b, t, local, top, k, strict)
            assert list(a[b, t]) == anchors, (b, t)
            assert [list(x) for x in p[b, t]] == partners, (b, t)


def test_invariants_at_cfg5_like_shape():
    """Distinct active anchors, all-anchor exclusion, causal partners, inactive slots."""
    rng = np.random.default_rng(113)
    context, blocks, slots, k, local, top = 512, 8, 4, 6, 128, 2
    queries = np.array([0, 1, 2, 3, 63, 64, 200, 511])
    inp = multi_inputs(rng, batch=1, context=context, blocks=blocks, slots=slots,
                       queries=len(queries), bf16=True)
    a, s, p, ps = run_multi(inp, queries, local, top, k, True)
    for qi, t in enumerate(queries):
        active = [h for h in range(slots) if h <= t]
        chosen = [int(a[0, qi, h]) for h in active]
        assert len(set(chosen)) == len(chosen)
        assert all(0 <= x <= t for x in chosen)
        for h in range(slots):
            if h not in active:
                assert a[0, qi, h] == 0 and s[0, qi, h] == -np.inf
                assert np.all(ps[0, qi, h] == -np.inf)
                assert np.all(p[0, qi, h] == t - local + 1)
                continue
            fin = np.isfinite(ps[0, qi, h])
            got = p[0, qi, h][fin]
            assert not set(got.tolist()) & set(chosen)
            assert np.all(got <= t) and np.all(got >= 0)
            assert len(set(got.tolist())) == len(got)
            assert np.all(np.diff(ps[0, qi, h][fin]) <= 0)
            # as many partners as causal non-anchor candidates allow
            assert fin.sum() == min(k, t + 1 - len(chosen)) or t >= local
