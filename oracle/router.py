"""Block-router oracle -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates ``DistilledBlockRouter`` (src/relation_lm/routing/block_router.py):
  * ``block_statistics``  :54-68  per-block mean and biased std
  * ``_causal_conv``      :50-52  depthwise causal conv (kernel 3)
  * ``_scores``           :70-101 batched block scores for every query position
and its decode-time form, ``router_cache_update``
(src/relation_lm/kernels/router_cache.py:9-197): one token's causal conv from
the two previous raw rows, the raw/conv cache writes, and the statistics of
the block that holds the token.

This is the reference's only batched (all-queries) definition of block
scoring.  It produces the block statistics consumed by relation_select and,
through ``router_scores``, an independent formulation (logsumexp over heads,
minus log H) of the per-query block scores that oracle/select.py evaluates by
pairwise log-sum-exp: the two agree up to the constant log H
(tests/test_oracle_select.py).

Parity pins: block_statistics is checked against torch's mean/std(unbiased=False)
on the grouped view; causal_conv against torch's depthwise conv1d;
router_scores is the pin of oracle.select.block_scores.  router_cache_update is
pinned by replaying it token by token from empty caches: the conv cache must
equal causal_conv of the raw sequence and every completed block's statistics
must equal block_statistics (tests/test_oracle_router.py), plus the t = 0 / 1
edges and the zero rows a partly filled block averages over.
"""
from __future__ import annotations

import math

import numpy as np


def _f64(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float64)


def causal_conv(x, weight) -> np.ndarray:
    """Depthwise causal conv, kernel 3, left padding 2 (block_router.py:50-52).

    x [B,T,C], weight [C,1,3]; y[t,c] = sum_j w[c,0,j] * x[t-2+j, c].
    """
    x = _f64(x)
    w = _f64(weight)
    padded = np.concatenate([np.zeros_like(x[:, :2]), x], axis=1)
    t = x.shape[1]
    return sum(padded[:, j:j + t] * w[None, None, :, 0, j] for j in range(3))


def block_statistics(key, block_size: int, heads: int, head_dim: int):
    """(mean, biased std) per block and head: [B,NB,H,HD] each (block_router.py:54-68).

    The last block is zero-padded when T is not a multiple of the block size.
    """
    key = _f64(key)
    batch, length, _ = key.shape
    blocks = (length + block_size - 1) // block_size
    padding = blocks * block_size - length
    if padding:
        key = np.concatenate([key, np.zeros((batch, padding, key.shape[2]))], axis=1)
    grouped = key.reshape(batch, blocks, block_size, heads, head_dim)
    mean = grouped.mean(axis=2)
    std = np.sqrt(((grouped - mean[:, :, None]) ** 2).mean(axis=2))
    return mean, std


def router_scores(query, mean, std, gamma, bias, block_size: int) -> np.ndarray:
    """Scores [B,T,NB] of block_router.py:78-101 given block stats (conv already applied).

    softplus is torch's thresholded form (beta=1, threshold=20) as F.softplus.
    """
    q = _f64(query)
    batch, length, _ = q.shape
    heads, head_dim = mean.shape[2], mean.shape[3]
    blocks = mean.shape[1]
    q = q.reshape(batch, length, heads, head_dim)
    content = np.einsum("bthd,bnhd->bthn", q, _f64(mean))
    uncertainty = np.einsum("bthd,bnhd->bthn", np.abs(q), _f64(std))
    g = _f64(gamma)
    sp = np.where(g > 20.0, g, np.log1p(np.exp(np.minimum(g, 20.0))))
    uncertainty = uncertainty * sp[None, None, :, None]
    position = np.arange(length)[:, None]
    block_end = (np.arange(blocks) + 1) * block_size - 1
    distance = np.maximum(position - block_end[None], 0)
    bucket = np.minimum(np.floor(np.log2(distance + 1.0)).astype(np.int64), bias.shape[1] - 1)
    relative = np.transpose(_f64(bias)[:, bucket], (1, 0, 2))[None]   # [1,T,H,NB]
    per_head = (content + uncertainty) * head_dim ** -0.5 + relative
    mx = per_head.max(axis=2, keepdims=True)
    lse = mx[:, :, 0] + np.log(np.exp(per_head - mx).sum(axis=2))
    scores = lse - math.log(heads)
    complete = block_end[None] <= np.arange(length)[:, None]
    return np.where(complete[None], scores, -np.inf)


def router_cache_update(anchor_raw, partner_raw, anchor_raw_cache, partner_raw_cache,
                        anchor_conv_cache, partner_conv_cache, anchor_mean, anchor_std,
                        partner_mean, partner_std, anchor_conv_weight, partner_conv_weight,
                        position: int, block_size: int):
    """One decode step of both router streams (router_cache.py:36-197), in float64.

    anchor_raw / partner_raw [B,D]; raw and conv caches [B,T,D]; mean / std
    [B,NB,...] with D values per block; conv weights [D,3] (column 2 multiplies
    the current row, 1 the previous, 0 the one before, as causal_conv).
    Returns (output [B,2,D], dict of the eight updated buffers); the inputs are
    not modified.  For position t:
      conv   = raw*w2 + raw_cache[t-1]*w1*[t>=1] + raw_cache[t-2]*w0*[t>=2]  (:81-90)
      raw_cache[t] = raw, conv_cache[t] = conv                               (:92-96)
      block j = t // block_size: mean and biased std over ALL block_size rows
      of conv_cache (rows past t hold whatever the cache holds), with row t
      replaced by the fresh conv                                            (:98-128)
    Rows past the cache end read as zero and a position outside [0, T) leaves
    every buffer unchanged and returns zeros (the reference reads and writes
    out of bounds there); a block index past NB updates no statistics.
    """
    raw = {"anchor": _f64(anchor_raw), "partner": _f64(partner_raw)}
    bufs = {"anchor_raw_cache": anchor_raw_cache, "partner_raw_cache": partner_raw_cache,
            "anchor_conv_cache": anchor_conv_cache, "partner_conv_cache": partner_conv_cache,
            "anchor_mean": anchor_mean, "anchor_std": anchor_std,
            "partner_mean": partner_mean, "partner_std": partner_std}
    out_bufs = {k: np.array(v, copy=True) for k, v in bufs.items()}
    weights = {"anchor": _f64(anchor_conv_weight), "partner": _f64(partner_conv_weight)}
    b, t_max, d = np.shape(anchor_raw_cache)
    output = np.zeros((b, 2, d), dtype=np.float64)
    t = int(position)
    if not 0 <= t < t_max:
        return output, out_bufs
    nb = np.shape(anchor_mean)[1]
    j = t // block_size
    for side_index, side in enumerate(("anchor", "partner")):
        cache = _f64(bufs[f"{side}_raw_cache"])
        w = weights[side]
        conv = raw[side] * w[:, 2]
        if t >= 1:
            conv = conv + cache[:, t - 1] * w[:, 1]
        if t >= 2:
            conv = conv + cache[:, t - 2] * w[:, 0]
        output[:, side_index] = conv
        out_bufs[f"{side}_raw_cache"][:, t] = raw[side]
        out_bufs[f"{side}_conv_cache"][:, t] = conv
        if j < nb:
            rows = np.zeros((b, block_size, d), dtype=np.float64)
            stop = min(j * block_size + block_size, t_max)
            rows[:, :stop - j * block_size] = _f64(out_bufs[f"{side}_conv_cache"])[:, j * block_size:stop]
            mean = rows.mean(axis=1)
            std = np.sqrt(((rows - mean[:, None]) ** 2).mean(axis=1))
            shape = out_bufs[f"{side}_mean"].shape
            out_bufs[f"{side}_mean"].reshape(b, nb, -1)[:, j] = mean
            out_bufs[f"{side}_std"].reshape(b, nb, -1)[:, j] = std
            assert out_bufs[f"{side}_mean"].shape == shape
    return output, out_bufs


def router_cache_update_ring(anchor_raw, partner_raw, anchor_raw_cache, partner_raw_cache,
                             anchor_conv_cache, partner_conv_cache, anchor_mean, anchor_std,
                             partner_mean, partner_std, anchor_conv_weight, partner_conv_weight,
                             position: int, block_size: int):
    """router_cache_update over ring-buffer caches of C rows (no reference op).

    Position p lives in row p mod C; block j's statistics in slot j mod NB
    (NB * block_size == C).  The conv reads rows t-1 and t-2 mod C; the block
    statistics use the block's rows up to t and count the rows past t as zero
    (those ring rows still hold positions from C earlier).  t < 0 changes
    nothing and returns zeros.  Same return convention as router_cache_update.
    """
    raw = {"anchor": _f64(anchor_raw), "partner": _f64(partner_raw)}
    bufs = {"anchor_raw_cache": anchor_raw_cache, "partner_raw_cache": partner_raw_cache,
            "anchor_conv_cache": anchor_conv_cache, "partner_conv_cache": partner_conv_cache,
            "anchor_mean": anchor_mean, "anchor_std": anchor_std,
            "partner_mean": partner_mean, "partner_std": partner_std}
    out_bufs = {k: np.array(v, copy=True) for k, v in bufs.items()}
    weights = {"anchor": _f64(anchor_conv_weight), "partner": _f64(partner_conv_weight)}
    b, cap, d = np.shape(anchor_raw_cache)
    output = np.zeros((b, 2, d), dtype=np.float64)
    t = int(position)
    if t < 0:
        return output, out_bufs
    nb = np.shape(anchor_mean)[1]
    assert nb * block_size == cap, "ring caches hold whole blocks"
    j = t // block_size
    for side_index, side in enumerate(("anchor", "partner")):
        cache = _f64(bufs[f"{side}_raw_cache"])
        w = weights[side]
        conv = raw[side] * w[:, 2]
        if t >= 1:
            conv = conv + cache[:, (t - 1) % cap] * w[:, 1]
        if t >= 2:
            conv = conv + cache[:, (t - 2) % cap] * w[:, 0]
        output[:, side_index] = conv
        out_bufs[f"{side}_raw_cache"][:, t % cap] = raw[side]
        out_bufs[f"{side}_conv_cache"][:, t % cap] = conv
        rows = np.zeros((b, block_size, d), dtype=np.float64)
        first = j * block_size
        for p in range(first, t + 1):
            rows[:, p - first] = _f64(out_bufs[f"{side}_conv_cache"])[:, p % cap]
        mean = rows.mean(axis=1)
        std = np.sqrt(((rows - mean[:, None]) ** 2).mean(axis=1))
        out_bufs[f"{side}_mean"].reshape(b, nb, -1)[:, j % nb] = mean
        out_bufs[f"{side}_std"].reshape(b, nb, -1)[:, j % nb] = std
    return output, out_bufs
