"""Pins of the ring-buffer oracles (oracle/select.py, router.py, reduce.py: *_ring).

A ring cache of C rows holds the last C positions (row p mod C; statistics slot
j holds the newest absolute block = j mod NB).  Pinned by:
  * selection, t < C: equals the linear decode oracle on the same buffers;
  * selection, t >= C: the ring form over ring storage equals the linear oracle
    over the rebased window [t0, t0 + C) of the same long sequence, t0 = first
    position of the oldest fully resident block, with positions shifted back by
    t0 (positions, distances and tie orders are all shift-invariant);
  * slot -> absolute block mapping by brute force;
  * router update: a 3C-token replay from empty caches equals the linear
    update over a 3C-row cache (outputs, statistics slots, last C rows);
  * hidden update: a 2C-step replay with resident indices equals the linear
    update over a 2C-row cache; non-resident indices read zeros.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import select as osel

ORDER = ("anchor_query", "anchor_keys", "anchor_router_query", "anchor_block_mean",
         "anchor_block_std", "anchor_gamma", "anchor_bias", "partner_base",
         "partner_anchor_cache", "partner_keys", "partner_block_mean", "partner_block_std",
         "partner_gamma", "partner_bias")


def long_sequence(rng, batch, length, block_size, e=64, heads=4, head_dim=16, buckets=16,
                  bf16=False):
    def randn(*shape):
        x = rng.standard_normal(shape).astype(np.float32)
        if bf16:
            x = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
        return x

    rd = heads * head_dim
    seq = {"anchor_keys": randn(batch, length, e), "partner_keys": randn(batch, length, e),
           "partner_anchor_cache": randn(batch, length, 2 * e)}
    for side in ("anchor", "partner"):
        blocks = length // block_size
        seq[f"{side}_block_mean"] = randn(batch, blocks, heads, head_dim)
        seq[f"{side}_block_std"] = np.abs(randn(batch, blocks, heads, head_dim))
        seq[f"{side}_gamma"] = randn(heads)
        seq[f"{side}_bias"] = randn(heads, buckets)
    query = {"anchor_query": randn(batch, e), "anchor_router_query": randn(batch, rd),
             "partner_base": randn(batch, 2 * e)}
    return seq, query


def ring_view(seq, t, capacity, block_size):
    """Ring storage at position t: row r holds the newest position <= t that is r mod C."""
    out = {}
    rows = np.arange(capacity)
    pos = t - np.mod(t - rows, capacity)
    for name in ("anchor_keys", "partner_keys", "partner_anchor_cache"):
        x = seq[name]
        out[name] = np.where((pos >= 0)[None, :, None], x[:, np.maximum(pos, 0)], 0.0)
    blocks = capacity // block_size
    jb = osel.ring_blocks(np.array([t]), blocks, block_size)[0]
    for side in ("anchor", "partner"):
        for stat in ("mean", "std"):
            x = seq[f"{side}_block_{stat}"]
            out[f"{side}_block_{stat}"] = np.where((jb >= 0)[None, :, None, None],
                                                   x[:, np.maximum(jb, 0)], 0.0)
        out[f"{side}_gamma"] = seq[f"{side}_gamma"]
        out[f"{side}_bias"] = seq[f"{side}_bias"]
    return out


def linear_window(seq, t0, capacity, block_size):
    out = {}
    for name in ("anchor_keys", "partner_keys", "partner_anchor_cache"):
        out[name] = seq[name][:, t0:t0 + capacity]
    j0 = t0 // block_size
    for side in ("anchor", "partner"):
        for stat in ("mean", "std"):
            out[f"{side}_block_{stat}"] = seq[f"{side}_block_{stat}"][:, j0:j0 + capacity // block_size]
        out[f"{side}_gamma"] = seq[f"{side}_gamma"]
        out[f"{side}_bias"] = seq[f"{side}_bias"]
    return out


def test_ring_blocks_brute_force():
    for blocks, bs in ((8, 16), (4, 32)):
        cap = blocks * bs
        for t in range(0, 5 * cap, 7):
            got = osel.ring_blocks(np.array([t]), blocks, bs)[0]
            for j in range(blocks):
                cands = [jb for jb in range(-blocks, t // bs + 1) if jb % blocks == j]
                assert got[j] == max(cands)


@pytest.mark.parametrize("strict", [False, True])
def test_ring_before_wrap_equals_linear(strict):
    rng = np.random.default_rng(211 + strict)
    cap, bs = 256, 32
    seq, query = long_sequence(rng, 2, cap, bs)
    for t in (0, 5, 31, 32, 100, 255):
        inp = {**seq, **query}
        lin = osel.relation_select_packed(*[inp[n] for n in ORDER], t, 48, 3, 6, strict)
        ring = osel.relation_select_packed_ring(*[inp[n] for n in ORDER], t, 48, 3, 6, strict)
        for a, b in zip(lin, ring):
            np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("strict", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
def test_ring_after_wrap_equals_rebased_linear(strict, bf16):
    rng = np.random.default_rng(223 + 2 * strict + bf16)
    cap, bs, local, top, k = 256, 32, 64, 3, 6
    length = 4 * cap
    seq, query = long_sequence(rng, 2, length, bs, bf16=bf16)
    for t in (cap, cap + 1, cap + bs - 1, cap + bs, 2 * cap + 77, length - 1):
        t0 = -(-(t - cap + 1) // bs) * bs  # first position of the oldest whole resident block
        ring = osel.relation_select_packed_ring(
            *[{**ring_view(seq, t, cap, bs), **query}[n] for n in ORDER], t, local, top, k,
            strict)
        lin = osel.relation_select_packed(
            *[{**linear_window(seq, t0, cap, bs), **query}[n] for n in ORDER], t - t0, local,
            top, k, strict)
        np.testing.assert_array_equal(ring[0], lin[0] + t0)
        np.testing.assert_array_equal(ring[1], lin[1])
        np.testing.assert_array_equal(ring[2], lin[2] + t0)
        np.testing.assert_array_equal(ring[3], lin[3])
        assert np.all(ring[0] > t - cap) and np.all(ring[2] > t - cap)


def test_router_ring_replay_equals_linear_long_cache():
    """3C tokens from empty caches: the ring state is the last C rows / NB blocks of the
    linear state over a 3C-row cache, and the conv outputs agree at every step."""
    from oracle import router

    rng = np.random.default_rng(227)
    batch, dim, cap, bs = 2, 16, 32, 8
    length = 3 * cap
    w = {s: (rng.standard_normal((dim, 3)) * 0.3).astype(np.float32) for s in ("a", "p")}

    def empty(rows, blocks):
        z = np.zeros((batch, rows, dim), np.float32)
        st = np.zeros((batch, blocks, 4, dim // 4), np.float32)
        return [z.copy(), z.copy(), z.copy(), z.copy(), st.copy(), st.copy(), st.copy(), st.copy()]

    names = ("anchor_raw_cache", "partner_raw_cache", "anchor_conv_cache", "partner_conv_cache",
             "anchor_mean", "anchor_std", "partner_mean", "partner_std")
    lin = dict(zip(names, empty(length, length // bs)))
    ring = dict(zip(names, empty(cap, cap // bs)))
    for t in range(length):
        xa = rng.standard_normal((batch, dim)).astype(np.float32)
        xp = rng.standard_normal((batch, dim)).astype(np.float32)
        out_l, lin = router.router_cache_update(xa, xp, *[lin[n] for n in names], w["a"], w["p"],
                                                t, bs)
        out_r, ring = router.router_cache_update_ring(xa, xp, *[ring[n] for n in names], w["a"],
                                                      w["p"], t, bs)
        np.testing.assert_array_equal(out_r, out_l)
        j = t // bs
        for n in ("anchor_mean", "anchor_std", "partner_mean", "partner_std"):
            np.testing.assert_array_equal(ring[n][:, j % (cap // bs)], lin[n][:, j])
    for n in names[:4]:
        rows = np.arange(cap)
        pos = (length - 1) - np.mod(length - 1 - rows, cap)
        np.testing.assert_array_equal(ring[n], lin[n][:, pos])


def test_hidden_update_ring_replay_equals_linear_long_cache():
    """2C decode steps with resident indices: ring update == linear update on a 2C-row
    cache (same absolute indices), and the ring rows track the linear rows."""
    from oracle import reduce as ored

    rng = np.random.default_rng(229)
    batch, cap, r, h, k = 2, 16, 8, 12, 3
    length = 2 * cap
    op_long = rng.standard_normal((batch, length, r)).astype(np.float32)
    wa, wp = (rng.standard_normal((h, r)).astype(np.float32) for _ in range(2))
    wm = rng.standard_normal((h, r)).astype(np.float32)
    b1 = rng.standard_normal(h).astype(np.float32)
    lin = np.zeros((batch, length, 2 * h))
    ring = np.zeros((batch, cap, 2 * h))
    op_ring = np.zeros((batch, cap, r), np.float32)
    for t in range(length):
        op_ring[:, t % cap] = op_long[:, t]
        lo = max(0, t - cap + 1)
        a = rng.integers(lo, t + 1, size=batch)
        p = rng.integers(lo, t + 1, size=(batch, k))
        p[:, 0] = t  # the fresh row in use
        h_l, lin = ored.relation_hidden_cache_update(lin, op_long, a, p, wa, wp, wm, b1, t)
        h_r, ring = ored.relation_hidden_cache_update_ring(ring, op_ring, a, p, wa, wp, wm, b1, t)
        np.testing.assert_array_equal(h_r, h_l)
        resident = np.arange(lo, t + 1)
        np.testing.assert_array_equal(ring[:, resident % cap], lin[:, resident])
    # indices outside the resident range read zeros
    stale = np.full(batch, length - 1 - cap)
    got, _ = ored.relation_hidden_cache_update_ring(ring, op_ring, stale, p, wa, wp, wm, b1,
                                                    length - 1)
    zero_a, _ = ored.relation_hidden_cache_update_ring(ring, op_ring, np.full(batch, -1), p, wa,
                                                       wp, wm, b1, length - 1)
    np.testing.assert_array_equal(got, zero_a)
