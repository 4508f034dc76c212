"""Router cache update on gfx950.

Mirrors src/relation_lm/kernels/router_cache.py: ``router_cache_update``
(:181-241) behind the same ``torch.ops.relation_lm.router_cache_update`` schema
(the eight cache/statistics buffers are mutated in place), backed by the HIP
kernel of relation-lm_amd/csrc/rlm_router.hip.
"""
from __future__ import annotations

import torch
from torch import Tensor

from relation_lm import _native  # noqa: F401  (registers torch.ops.relation_lm)


def router_cache_update(
    anchor_raw: Tensor,
    partner_raw: Tensor,
    anchor_raw_cache: Tensor,
    partner_raw_cache: Tensor,
    anchor_conv_cache: Tensor,
    partner_conv_cache: Tensor,
    anchor_mean: Tensor,
    anchor_std: Tensor,
    partner_mean: Tensor,
    partner_std: Tensor,
    anchor_conv_weight: Tensor,
    partner_conv_weight: Tensor,
    position: Tensor,
    block_size: int,
) -> Tensor:
    """Update both router streams, causal conv state, and current-block stats.

    ``anchor_raw`` and ``partner_raw`` may be row-strided views of a larger
    packed projection (unit column stride).  Returns ``[B, 2, D]`` fp32: the
    anchor and partner conv rows of the current token.
    """
    return torch.ops.relation_lm.router_cache_update(
        anchor_raw, partner_raw, anchor_raw_cache, partner_raw_cache, anchor_conv_cache,
        partner_conv_cache, anchor_mean, anchor_std, partner_mean, partner_std,
        anchor_conv_weight, partner_conv_weight, position, int(block_size))
