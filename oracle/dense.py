"""Dense O(T^2) selection oracle -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates, with torch on the CPU, the dense selection of
  * ``RelationLexLM.relation_context``   src/relation_lm/models/relation_lm.py:143-177
  * ``MultiAnchorRelationBlock``         src/relation_lm/models/multi_relation_blocks.py:69-168
over the full causal score matrix.  When every causal position is a candidate
of the routed path (T <= LOCAL, or compat mode with all complete blocks picked
and LOCAL >= BS) the routed selection must reduce to this one, which pins
oracle/select.py with an independent formulation (full matrix + argmax/topk).

Scores follow the oracle's numerics contract: float64 dot, one rounding to
float32, comparisons in float32.  Queries are given already projected: the
partner query of a query at t with anchor a is partner_base[t] +
partner_anchor_cache[a] -- the split form of partner_query(cat(query, anchor))
that relation_select.py:165-175 relies on.
"""
from __future__ import annotations

import math

import torch


def causal_scores(query: torch.Tensor, key: torch.Tensor) -> torch.Tensor:
    """fp32(q . k * E^-0.5) with future positions at -inf (relation_lm.py:142-149)."""
    q = query.to(torch.float64)
    k = key.to(torch.float64)
    score = torch.einsum("btd,bsd->bts", q, k) * (1.0 / math.sqrt(query.size(-1)))
    score = score.to(torch.float32)
    length_q, length_k = query.size(1), key.size(1)
    future = torch.ones(length_q, length_k, dtype=torch.bool).triu(1)
    return score.masked_fill(future[None], -torch.inf)


def relation_context_selection(anchor_query, anchor_keys, partner_base, partner_anchor_cache,
                               partner_keys, k: int):
    """Anchor argmax, partner top-k with the anchor excluded (relation_lm.py:158-167).

    All tensors [B,T,*]; queries at positions 0..T-1.  Returns
    (anchor [B,T], anchor_score [B,T], partner [B,T,k], partner_score [B,T,k]).
    """
    exact_dim = anchor_keys.size(-1)
    anchor_scores = causal_scores(anchor_query, anchor_keys)
    anchor_idx = anchor_scores.argmax(-1)
    anchor_score = anchor_scores.gather(-1, anchor_idx[..., None])[..., 0]
    batch = torch.arange(anchor_keys.size(0))[:, None]
    contribution = partner_anchor_cache.to(torch.float32)[batch, anchor_idx]
    base = partner_base.to(torch.float32)
    partner_query = base[..., :exact_dim] + contribution[..., :exact_dim]
    partner_scores = causal_scores(partner_query, partner_keys)
    partner_scores = partner_scores.scatter(2, anchor_idx[..., None], -torch.inf)
    top_scores, partner_idx = partner_scores.topk(k, dim=-1)
    return anchor_idx, anchor_score, partner_idx, top_scores


def relation_context_weights(top_scores: torch.Tensor, k: int) -> torch.Tensor:
    """Active-K softmax weights (relation_lm.py:169-177)."""
    length = top_scores.size(1)
    position = torch.arange(length)
    k_limit = torch.ceil(torch.log2(position.double() + 2)).long().clamp(1, k)
    ranks = torch.arange(k)[None, None]
    active = torch.isfinite(top_scores) & ranks.lt(k_limit[None, :, None])
    safe = top_scores.double().masked_fill(~active, -1e4)
    weights = safe.softmax(-1) * active
    return weights / weights.sum(-1, keepdim=True).clamp_min(1e-9)


def distinct_anchors(scores: torch.Tensor, anchors: int):
    """Distinct anchors by iterative argmax with a used mask (multi_relation_blocks.py:69-99).

    scores [B,H,T,T] already causal-masked; returns (index [B,T,H], active [T,H]).
    """
    batch, heads, length, _ = scores.shape
    time = torch.arange(length)
    slot = torch.arange(anchors)
    active = slot[None, :] <= time[:, None]
    selected = []
    for slot_index in range(anchors):
        slot_score = scores[:, slot_index]
        if selected:
            used = torch.stack(selected, dim=-1)
            used_mask = torch.nn.functional.one_hot(used, num_classes=length).any(dim=-2)
            slot_score = slot_score.masked_fill(used_mask, -torch.inf)
        index = slot_score.argmax(dim=-1)
        index = torch.where(active[:, slot_index][None].expand(batch, -1), index,
                            torch.zeros_like(index))
        selected.append(index)
    return torch.stack(selected, dim=-1), active


def multi_anchor_selection(anchor_query, anchor_keys, partner_base, partner_anchor_cache,
                           partner_keys, k: int):
    """MultiAnchorRelationBlock selection over full score matrices
    (multi_relation_blocks.py:69-147).

    Tensors [B,T,S,*] (S anchor slots), queries at positions 0..T-1.  Per slot:
    causal anchor scores, distinct anchors by iterative argmax (:69-99), the
    split partner query partner_base[s] + partner_anchor_cache[anchor, s] (the
    anchor vector of an inactive slot is zero, :98), partner scores with every
    active anchor and every inactive slot masked (:133-142), top-k (:144).
    Returns (anchor [B,T,S], anchor_score [B,T,S], active [T,S],
    partner [B,T,S,k], partner_score [B,T,S,k]).
    """
    batch, length, slots, exact_dim = anchor_query.shape
    scores = torch.stack([causal_scores(anchor_query[:, :, s], anchor_keys[:, :, s])
                          for s in range(slots)], dim=1)  # [B,S,T,T]
    index, active = distinct_anchors(scores, slots)
    anchor_score = scores.permute(0, 2, 1, 3).gather(-1, index[..., None])[..., 0]
    anchor_active = active[None].expand(batch, -1, -1)
    anchor_score = anchor_score.masked_fill(~anchor_active, -torch.inf)
    one_hot = torch.nn.functional.one_hot(index, num_classes=length).bool()
    all_anchor = (one_hot & anchor_active[..., None]).any(dim=-2)  # [B,T,T]
    rows = torch.arange(batch)[:, None]
    cache = partner_anchor_cache.to(torch.float32)
    partner, partner_score = [], []
    for s in range(slots):
        contribution = cache[rows, index[:, :, s], s] * anchor_active[:, :, s, None]
        query = partner_base[:, :, s].to(torch.float32)[..., :exact_dim] + contribution[..., :exact_dim]
        ps = causal_scores(query, partner_keys[:, :, s])
        ps = ps.masked_fill(all_anchor, -torch.inf)
        ps = ps.masked_fill(~anchor_active[:, :, s, None], -torch.inf)
        top, idx = ps.topk(k, dim=-1)
        partner.append(idx)
        partner_score.append(top)
    return (index, anchor_score, active, torch.stack(partner, dim=2),
            torch.stack(partner_score, dim=2))
