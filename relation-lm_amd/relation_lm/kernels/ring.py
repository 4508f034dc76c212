"""Ring-buffer forms of the decode-path ops: contexts beyond the cache length.

No reference counterpart: the reference lists "persistent ring-buffer state
and contexts beyond 512" on its roadmap (README.md:150, docs/roadmap.md:8)
and its decode ops reject positions past the cache end.  Each op here takes
exactly the arguments of its linear form:

  relation_select_packed_ring        <- relation_select_packed
  relation_hidden_cached_ring        <- relation_hidden_cached
  relation_hidden_cache_update_ring  <- relation_hidden_cache_update
  router_cache_update_ring           <- router_cache_update

Positions stay absolute in every input and output and may exceed the cache
length T (a power of two).  Position p lives in cache row p mod T; block
statistics slot j holds the newest absolute block jb <= t // BS with
jb = j (mod NB), NB * BS == T.  At position t the resident positions are
[t-T+1, t]; routing considers only whole resident blocks, and block picks tie
to the lowest absolute block.  For t < T every op equals its linear form.
The caller writes the token's key/cache rows at row t mod T.
"""
from __future__ import annotations

import torch
from torch import Tensor

from relation_lm import _native  # noqa: F401  (registers torch.ops.relation_lm)


def ring_row(position: int, capacity: int) -> int:
    """Cache row of an absolute position in a ring cache of `capacity` rows."""
    return position % capacity


def relation_select_packed_ring(anchor_query: Tensor, anchor_keys: Tensor,
                                anchor_router_query: Tensor, anchor_block_mean: Tensor,
                                anchor_block_std: Tensor, anchor_gamma: Tensor,
                                anchor_bias: Tensor, partner_base: Tensor,
                                partner_anchor_cache: Tensor, partner_keys: Tensor,
                                partner_block_mean: Tensor, partner_block_std: Tensor,
                                partner_gamma: Tensor, partner_bias: Tensor, position: Tensor,
                                local_window: int, top_blocks: int, k_out: int,
                                strict_valid: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Decode-form selection over ring caches; returns absolute positions."""
    return torch.ops.relation_lm.relation_select_packed_ring(
        anchor_query, anchor_keys, anchor_router_query, anchor_block_mean, anchor_block_std,
        anchor_gamma, anchor_bias, partner_base, partner_anchor_cache, partner_keys,
        partner_block_mean, partner_block_std, partner_gamma, partner_bias, position,
        local_window, top_blocks, k_out, strict_valid)


def relation_hidden_cached_ring(expanded_cache: Tensor, operand_cache: Tensor,
                                anchor_index: Tensor, partner_index: Tensor,
                                product_weight: Tensor) -> Tensor:
    """relation_hidden_cached with absolute indices read from rows index mod T."""
    return torch.ops.relation_lm.relation_hidden_cached_ring(
        expanded_cache, operand_cache, anchor_index, partner_index, product_weight)


def relation_hidden_cache_update_ring(expanded_cache: Tensor, operand_cache: Tensor,
                                      anchor_index: Tensor, partner_index: Tensor,
                                      anchor_weight: Tensor, partner_weight: Tensor,
                                      product_weight: Tensor, first_bias: Tensor,
                                      position: Tensor) -> Tensor:
    """Writes the expanded row of `position` at row position mod T; f32 [B,K,H]."""
    return torch.ops.relation_lm.relation_hidden_cache_update_ring(
        expanded_cache, operand_cache, anchor_index, partner_index, anchor_weight,
        partner_weight, product_weight, first_bias, position)


def router_cache_update_ring(anchor_raw: Tensor, partner_raw: Tensor, anchor_raw_cache: Tensor,
                             partner_raw_cache: Tensor, anchor_conv_cache: Tensor,
                             partner_conv_cache: Tensor, anchor_mean: Tensor, anchor_std: Tensor,
                             partner_mean: Tensor, partner_std: Tensor,
                             anchor_conv_weight: Tensor, partner_conv_weight: Tensor,
                             position: Tensor, block_size: int) -> Tensor:
    """Router update over ring caches; rows of the token's block past it count as zero."""
    return torch.ops.relation_lm.router_cache_update_ring(
        anchor_raw, partner_raw, anchor_raw_cache, partner_raw_cache, anchor_conv_cache,
        partner_conv_cache, anchor_mean, anchor_std, partner_mean, partner_std,
        anchor_conv_weight, partner_conv_weight, position, int(block_size))
