"""Packed relation selection on gfx950.

``relation_select_packed`` keeps the signature and semantics of the reference
op ``relation_lm::relation_select_packed``
(src/relation_lm/kernels/relation_select.py:311-382): anchor block scoring,
exact top-1 anchor (ties to the lowest position), factorized partner query,
partner block routing and exact top-k partners (ties to the lowest candidate
lane) with anchor exclusion and strict/compat remote-block validity.

``relation_select_packed_seq`` is the sequence (prefill) form: query-side
tensors carry a query axis and ``positions`` holds one position per query.
"""
from __future__ import annotations

from torch import Tensor

from relation_lm import _native  # noqa: F401  (registers torch.ops.relation_lm)
import torch


def relation_select_packed(
    anchor_query: Tensor,
    anchor_keys: Tensor,
    anchor_router_query: Tensor,
    anchor_block_mean: Tensor,
    anchor_block_std: Tensor,
    anchor_gamma: Tensor,
    anchor_bias: Tensor,
    partner_base: Tensor,
    partner_anchor_cache: Tensor,
    partner_keys: Tensor,
    partner_block_mean: Tensor,
    partner_block_std: Tensor,
    partner_gamma: Tensor,
    partner_bias: Tensor,
    position: Tensor,
    local_window: int,
    top_blocks: int,
    k_out: int,
    strict_valid: bool,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Returns (anchor int32 [B], anchor_score f32 [B], partner int32 [B,K], partner_score f32 [B,K])."""
    return torch.ops.relation_lm.relation_select_packed(
        anchor_query, anchor_keys, anchor_router_query, anchor_block_mean, anchor_block_std,
        anchor_gamma, anchor_bias, partner_base, partner_anchor_cache, partner_keys,
        partner_block_mean, partner_block_std, partner_gamma, partner_bias, position,
        local_window, top_blocks, k_out, strict_valid)


def relation_select_packed_seq(
    anchor_query: Tensor,
    anchor_keys: Tensor,
    anchor_router_query: Tensor,
    anchor_block_mean: Tensor,
    anchor_block_std: Tensor,
    anchor_gamma: Tensor,
    anchor_bias: Tensor,
    partner_base: Tensor,
    partner_anchor_cache: Tensor,
    partner_keys: Tensor,
    partner_block_mean: Tensor,
    partner_block_std: Tensor,
    partner_gamma: Tensor,
    partner_bias: Tensor,
    positions: Tensor,
    local_window: int,
    top_blocks: int,
    k_out: int,
    strict_valid: bool,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Sequence form: anchor_query [B,Tq,E] ..., positions [Tq] or [B,Tq].

    Returns (anchor [B,Tq], anchor_score [B,Tq], partner [B,Tq,K], partner_score [B,Tq,K]).
    """
    return torch.ops.relation_lm.relation_select_packed_seq(
        anchor_query, anchor_keys, anchor_router_query, anchor_block_mean, anchor_block_std,
        anchor_gamma, anchor_bias, partner_base, partner_anchor_cache, partner_keys,
        partner_block_mean, partner_block_std, partner_gamma, partner_bias, positions,
        local_window, top_blocks, k_out, strict_valid)


def multi_relation_select_seq(
    anchor_query: Tensor,
    anchor_keys: Tensor,
    anchor_router_query: Tensor,
    anchor_block_mean: Tensor,
    anchor_block_std: Tensor,
    anchor_gamma: Tensor,
    anchor_bias: Tensor,
    partner_base: Tensor,
    partner_anchor_cache: Tensor,
    partner_keys: Tensor,
    partner_block_mean: Tensor,
    partner_block_std: Tensor,
    partner_gamma: Tensor,
    partner_bias: Tensor,
    positions: Tensor,
    local_window: int,
    top_blocks: int,
    k_out: int,
    strict_valid: bool,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Routed multi-anchor selection (no reference kernel; the dense semantics are
    MultiAnchorRelationBlock's, multi_relation_blocks.py:69-147).

    anchor_query [B,Tq,S,E], anchor_keys [B,T,S,E], anchor_router_query [B,Tq,RD],
    partner_base [B,Tq,S,E+RD], partner_anchor_cache [B,T,S,E+RD],
    partner_keys [B,T,S,E]; block statistics, gamma and bias as the single-anchor
    op (the partner statistics are shared by the S slots); positions [Tq] or [B,Tq].
    Slot s is active iff s <= t.  Returns (anchor int32 [B,Tq,S], anchor_score f32
    [B,Tq,S], partner int32 [B,Tq,S,K], partner_score f32 [B,Tq,S,K]); the partner
    mask of the dense block is isfinite(partner_score).
    """
    return torch.ops.relation_lm.multi_relation_select_seq(
        anchor_query, anchor_keys, anchor_router_query, anchor_block_mean, anchor_block_std,
        anchor_gamma, anchor_bias, partner_base, partner_anchor_cache, partner_keys,
        partner_block_mean, partner_block_std, partner_gamma, partner_bias, positions,
        local_window, top_blocks, k_out, strict_valid)


def relation_select_packed_expand_row(
    anchor_query: Tensor,
    anchor_keys: Tensor,
    anchor_router_query: Tensor,
    anchor_block_mean: Tensor,
    anchor_block_std: Tensor,
    anchor_gamma: Tensor,
    anchor_bias: Tensor,
    partner_base: Tensor,
    partner_anchor_cache: Tensor,
    partner_keys: Tensor,
    partner_block_mean: Tensor,
    partner_block_std: Tensor,
    partner_gamma: Tensor,
    partner_bias: Tensor,
    position: Tensor,
    local_window: int,
    top_blocks: int,
    k_out: int,
    strict_valid: bool,
    operand_cache: Tensor,
    expanded_weight: Tensor,
    expanded_bias: Tensor | None,
    expanded_cache: Tensor,
    ring: bool = False,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Decode-form ``relation_select_packed`` (``ring``: ``relation_select_packed_ring``)
    that also writes the token's expanded-cache row in place:
    ``expanded_cache[:, r] = F.linear(operand_cache[:, r], expanded_weight, expanded_bias)``
    with r the position (ring: position mod T), read on the device.

    The reference decode builds that row with a separate BLAS projection for B > 1
    (docs/benchmarks.md:80-81) or inside ``relation_hidden_cache_update`` for B == 1
    (relation_reduce.py:215-251); afterwards ``relation_hidden_cached`` serves both.
    The selection launch runs one workgroup per batch row on a few CUs, so the row
    is projected by extra workgroups of the same launch on CUs that would idle.
    bf16 caches and weights, relation dim 32..128, width a multiple of 16.
    """
    return torch.ops.relation_lm.relation_select_packed_expand_row(
        anchor_query, anchor_keys, anchor_router_query, anchor_block_mean, anchor_block_std,
        anchor_gamma, anchor_bias, partner_base, partner_anchor_cache, partner_keys,
        partner_block_mean, partner_block_std, partner_gamma, partner_bias, position,
        local_window, top_blocks, k_out, strict_valid, operand_cache, expanded_weight,
        expanded_bias, expanded_cache, ring)



def relation_select_packed_seq_expand(
    anchor_query: Tensor,
    anchor_keys: Tensor,
    anchor_router_query: Tensor,
    anchor_block_mean: Tensor,
    anchor_block_std: Tensor,
    anchor_gamma: Tensor,
    anchor_bias: Tensor,
    partner_base: Tensor,
    partner_anchor_cache: Tensor,
    partner_keys: Tensor,
    partner_block_mean: Tensor,
    partner_block_std: Tensor,
    partner_gamma: Tensor,
    partner_bias: Tensor,
    positions: Tensor,
    local_window: int,
    top_blocks: int,
    k_out: int,
    strict_valid: bool,
    operand_cache: Tensor,
    expanded_weight: Tensor,
    expanded_bias: Tensor | None,
    expanded_cache: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Sequence-form ``relation_select_packed_seq`` that also writes the whole
    expanded cache in place:
    ``expanded_cache = F.linear(operand_cache, expanded_weight, expanded_bias)`` in
    bf16 with fp32 sums, the same bits as ``relation_linear`` on those operands.

    The reference projects the expanded cache with its own linear call
    (tests/test_relation_reduce_gpu.py:64-68) and selects separately.  Here the
    selection's workgroups project 128 x 128 cache tiles while their own loads are
    in flight, so the prefill step needs one launch less; shapes the selection's
    matrix-core kernel does not take (or N % 128 != 0, or T < max(4 R, 272)) run the
    projection as a launch of its own after the selection.  bf16 caches and
    weights, relation dim 32..128, width a multiple of 16.
    """
    return torch.ops.relation_lm.relation_select_packed_seq_expand(
        anchor_query, anchor_keys, anchor_router_query, anchor_block_mean, anchor_block_std,
        anchor_gamma, anchor_bias, partner_base, partner_anchor_cache, partner_keys,
        partner_block_mean, partner_block_std, partner_gamma, partner_bias, positions,
        local_window, top_blocks, k_out, strict_valid, operand_cache, expanded_weight,
        expanded_bias, expanded_cache)
