"""Block-router oracle -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates ``DistilledBlockRouter`` (src/relation_lm/routing/block_router.py):
  * ``block_statistics``  :54-68  per-block mean and biased std
  * ``_causal_conv``      :50-52  depthwise causal conv (kernel 3)
  * ``_scores``           :70-101 batched block scores for every query position

This is the reference's only batched (all-queries) definition of block
scoring.  It produces the block statistics consumed by relation_select and,
through ``router_scores``, an independent formulation (logsumexp over heads,
minus log H) of the per-query block scores that oracle/select.py evaluates by
pairwise log-sum-exp: the two agree up to the constant log H
(tests/test_oracle_select.py).

Parity pins: block_statistics is checked against torch's mean/std(unbiased=False)
on the grouped view; router_scores is the pin of oracle.select.block_scores.
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
