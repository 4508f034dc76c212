"""Pins of the router oracle (CPU): causal conv and the decode-time cache update.

``router_cache_update`` (router_cache.py:9-197) is the token-by-token form of
``DistilledBlockRouter``'s causal conv and block statistics
(block_router.py:50-68).  Replaying it from empty caches over a whole sequence
must therefore reproduce ``causal_conv`` of the raw sequence and, at every
step, ``block_statistics`` of the conv sequence so far (zero-padded: the
cache rows past the token are still zero).  ``causal_conv`` itself is pinned
against torch's depthwise conv1d.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import router


def test_causal_conv_matches_torch_conv1d():
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, 37, 24, generator=g, dtype=torch.float64)
    w = torch.randn(24, 1, 3, generator=g, dtype=torch.float64)
    expected = F.conv1d(x.transpose(1, 2), w, padding=2, groups=24)[..., :37].transpose(1, 2)
    got = router.causal_conv(x.numpy(), w.numpy())
    np.testing.assert_allclose(got, expected.numpy(), rtol=1e-12, atol=1e-12)


def _empty_state(batch, length, dim, blocks, dtype=np.float32):
    z = np.zeros((batch, length, dim), dtype=dtype)
    s = np.zeros((batch, blocks, 4, dim // 4), dtype=dtype)
    return {"anchor_raw_cache": z.copy(), "partner_raw_cache": z.copy(),
            "anchor_conv_cache": z.copy(), "partner_conv_cache": z.copy(),
            "anchor_mean": s.copy(), "anchor_std": s.copy(),
            "partner_mean": s.copy(), "partner_std": s.copy()}


def _step(state, anchor_raw, partner_raw, wa, wp, t, block_size):
    return router.router_cache_update(
        anchor_raw, partner_raw, state["anchor_raw_cache"], state["partner_raw_cache"],
        state["anchor_conv_cache"], state["partner_conv_cache"], state["anchor_mean"],
        state["anchor_std"], state["partner_mean"], state["partner_std"], wa, wp, t, block_size)


@pytest.mark.parametrize("block_size", [8, 16])
def test_replay_equals_causal_conv_and_block_statistics(block_size):
    rng = np.random.default_rng(7 + block_size)
    batch, length, dim = 2, 48, 64
    blocks = length // block_size
    raw = {s: rng.standard_normal((batch, length, dim)).astype(np.float32)
           for s in ("anchor", "partner")}
    w = {s: (rng.standard_normal((dim, 3)) * 0.3).astype(np.float32) for s in ("anchor", "partner")}
    conv_full = {s: router.causal_conv(raw[s], w[s][:, None, :]) for s in raw}
    state = _empty_state(batch, length, dim, blocks)
    for t in range(length):
        out, state = _step(state, raw["anchor"][:, t], raw["partner"][:, t], w["anchor"],
                           w["partner"], t, block_size)
        j = t // block_size
        for k, s in enumerate(("anchor", "partner")):
            np.testing.assert_allclose(out[:, k], conv_full[s][:, t], rtol=1e-6, atol=1e-6)
            # statistics of the conv sequence so far, last block zero-padded
            mean, std = router.block_statistics(
                conv_full[s][:, :t + 1].astype(np.float32), block_size, 4, dim // 4)
            np.testing.assert_allclose(state[f"{s}_mean"][:, j], mean[:, j], rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(state[f"{s}_std"][:, j], std[:, j], rtol=1e-5, atol=1e-6)
    for s in ("anchor", "partner"):
        np.testing.assert_array_equal(state[f"{s}_raw_cache"], raw[s])
        np.testing.assert_allclose(state[f"{s}_conv_cache"], conv_full[s], rtol=1e-6, atol=1e-6)


def test_first_positions_ignore_stale_rows():
    """At t = 0 and t = 1 the missing previous rows contribute nothing, whatever the cache holds."""
    rng = np.random.default_rng(3)
    batch, length, dim = 1, 16, 8
    state = _empty_state(batch, length, dim, 2)
    state["anchor_raw_cache"][:] = 1.0e3  # stale contents must not leak in
    state["partner_raw_cache"][:] = -1.0e3
    w = rng.standard_normal((dim, 3)).astype(np.float32)
    x0 = rng.standard_normal((batch, dim)).astype(np.float32)
    out, s1 = _step(state, x0, x0, w, w, 0, 8)
    np.testing.assert_allclose(out[:, 0], x0 * w[:, 2], rtol=1e-7)
    x1 = rng.standard_normal((batch, dim)).astype(np.float32)
    out, _ = _step(s1, x1, x1, w, w, 1, 8)
    np.testing.assert_allclose(out[:, 0], x1 * w[:, 2] + x0 * w[:, 1], rtol=1e-6)


def test_position_outside_cache_changes_nothing():
    state = _empty_state(1, 16, 8, 2)
    x = np.ones((1, 8), dtype=np.float32)
    w = np.ones((8, 3), dtype=np.float32)
    for t in (-1, 16):
        out, new = _step(state, x, x, w, w, t, 8)
        assert not out.any()
        for k in state:
            np.testing.assert_array_equal(new[k], state[k])
