"""Two-op form of the routed selection (anchor, then partners) on gfx950.

The module keeps the reference's name (src/relation_lm/kernels/triton_select.py)
so imports keep working; the ops are HIP kernels registered under the
reference's ``relationlex`` namespace:
  * ``anchor_select``  -- triton_select.py:255-295
  * ``partner_topk``   -- triton_select.py:298-346 (partner/router queries and the
    anchor index are supplied by the caller)
"""
from __future__ import annotations

import torch
from torch import Tensor

from relation_lm import _native  # noqa: F401  (registers torch.ops.relationlex)


def anchor_select(
    anchor_query: Tensor,
    anchor_keys: Tensor,
    router_query: Tensor,
    block_mean: Tensor,
    block_std: Tensor,
    gamma: Tensor,
    bias: Tensor,
    position: Tensor,
    local_window: int,
    top_blocks: int,
    strict_valid: bool,
) -> tuple[Tensor, Tensor]:
    """Returns (anchor int32 [B], anchor_score f32 [B])."""
    return torch.ops.relationlex.anchor_select(
        anchor_query, anchor_keys, router_query, block_mean, block_std, gamma, bias, position,
        local_window, top_blocks, strict_valid)


def partner_topk(
    partner_query: Tensor,
    partner_keys: Tensor,
    router_query: Tensor,
    block_mean: Tensor,
    block_std: Tensor,
    gamma: Tensor,
    bias: Tensor,
    position: Tensor,
    anchor_index: Tensor,
    local_window: int,
    top_blocks: int,
    k_out: int,
    strict_valid: bool,
) -> tuple[Tensor, Tensor]:
    """Returns (partner int32 [B,K], partner_score f32 [B,K])."""
    return torch.ops.relationlex.partner_topk(
        partner_query, partner_keys, router_query, block_mean, block_std, gamma, bias, position,
        anchor_index, local_window, top_blocks, k_out, strict_valid)
