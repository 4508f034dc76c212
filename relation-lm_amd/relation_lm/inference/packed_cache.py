"""Packed sparse-cache projection (reference: src/relation_lm/inference/packed_cache.py).

One ``[576 -> 512]`` projection produces the six token-local decode caches in
the order ``SPARSE_CACHE_NAMES``.  The dataclass, its properties, validation
errors and the packing helper keep the reference contract (:10-94); the GEMM
behind ``project`` is the gfx950 MFMA kernel registered as
``relation_lm::packed_sparse_cache_projection`` (the reference calls
``F.linear``; the op has no name there).  CPU tensors take the op's CPU
implementation, ``at::linear``, so ``project`` runs on any device as the
reference's does.
"""
from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch
from torch import Tensor

from relation_lm import _native  # noqa: F401  (registers torch.ops.relation_lm)

SPARSE_CACHE_NAMES = (
    "anchor_key",
    "partner_key",
    "operand",
    "partner_anchor",
    "anchor_router_key",
    "partner_router_key",
)


@dataclass(frozen=True)
class PackedSparseCacheProjection:
    """One linear projection that produces all sparse-decode cache features."""

    weight: Tensor
    split_sizes: tuple[int, ...]
    names: tuple[str, ...] = SPARSE_CACHE_NAMES

    def __post_init__(self) -> None:
        if self.weight.ndim != 2:
            raise ValueError("weight must be a 2D tensor")
        if len(self.split_sizes) != len(self.names):
            raise ValueError("split_sizes and names must have the same length")
        if any(size <= 0 for size in self.split_sizes):
            raise ValueError("split sizes must be positive")
        if sum(self.split_sizes) != self.weight.size(0):
            raise ValueError("split sizes must sum to the packed output width")

    @property
    def input_width(self) -> int:
        return int(self.weight.size(1))

    @property
    def output_width(self) -> int:
        return int(self.weight.size(0))

    def project(self, memory: Tensor) -> tuple[Tensor, ...]:
        """Project ``memory`` and return views in ``names`` order."""
        if memory.size(-1) != self.input_width:
            raise ValueError("memory width does not match packed projection input")
        packed = torch.ops.relation_lm.packed_sparse_cache_projection(memory, self.weight)
        return packed.split(self.split_sizes, dim=-1)

    def project_into(self, memory: Tensor, anchor_keys: Tensor, partner_keys: Tensor,
                     operand_cache: Tensor, partner_anchor_cache: Tensor, position: Tensor,
                     *, ring: bool = False) -> tuple[Tensor, ...]:
        """``project`` plus the decode-time cache writes in one kernel (no reference
        counterpart).

        The first four segments (anchor_key, partner_key, operand, partner_anchor)
        are also written to row ``position`` of the four caches ``[B, T, width]``
        (row ``position % T`` when ``ring``; T a power of two), as
        ``cache[:, position] = segment`` would.  ``memory`` is ``[B, input_width]``
        with B <= 64.  Returns the same views as ``project``.
        """
        if memory.size(-1) != self.input_width:
            raise ValueError("memory width does not match packed projection input")
        caches = (anchor_keys, partner_keys, operand_cache, partner_anchor_cache)
        if tuple(int(c.size(-1)) for c in caches) != tuple(self.split_sizes[:4]):
            raise ValueError("cache widths must equal the first four split sizes")
        packed = torch.ops.relation_lm.packed_projection_to_caches(
            memory, self.weight, *caches, position, ring)
        return packed.split(self.split_sizes, dim=-1)

    def project_into_routed(self, memory: Tensor, anchor_keys: Tensor, partner_keys: Tensor,
                            operand_cache: Tensor, partner_anchor_cache: Tensor,
                            position: Tensor, anchor_raw_cache: Tensor,
                            partner_raw_cache: Tensor, anchor_conv_cache: Tensor,
                            partner_conv_cache: Tensor, anchor_block_mean: Tensor,
                            anchor_block_std: Tensor, partner_block_mean: Tensor,
                            partner_block_std: Tensor, anchor_conv_weight: Tensor,
                            partner_conv_weight: Tensor, block_size: int, *,
                            ring: bool = False) -> tuple[tuple[Tensor, ...], Tensor]:
        """``project_into`` with the router cache update of the last two segments
        (anchor_router_key, partner_router_key) folded in -- the reference's roadmap
        item "fold the router cache update into the packed projection"
        (README.md:148-149); no reference counterpart.

        Same results as ``project_into(...)`` followed by
        ``router_cache_update(parts[4], parts[5], <router tensors>, position,
        block_size)`` (``router_cache_update_ring`` when ``ring``), in one launch for
        decode shapes.  Returns (the ``project`` views, the router's conv rows
        [B, 2, D] fp32)."""
        if memory.size(-1) != self.input_width:
            raise ValueError("memory width does not match packed projection input")
        caches = (anchor_keys, partner_keys, operand_cache, partner_anchor_cache)
        if tuple(int(c.size(-1)) for c in caches) != tuple(self.split_sizes[:4]):
            raise ValueError("cache widths must equal the first four split sizes")
        packed, router_out = torch.ops.relation_lm.packed_projection_router_update(
            memory, self.weight, *caches, position, ring, anchor_raw_cache, partner_raw_cache,
            anchor_conv_cache, partner_conv_cache, anchor_block_mean, anchor_block_std,
            partner_block_mean, partner_block_std, anchor_conv_weight, partner_conv_weight,
            block_size)
        return packed.split(self.split_sizes, dim=-1), router_out

    def project_dict(self, memory: Tensor) -> dict[str, Tensor]:
        """Project ``memory`` and return a name-to-tensor mapping."""
        return dict(zip(self.names, self.project(memory), strict=True))


def pack_sparse_cache_projection_weights(
    weights: Sequence[Tensor],
    *,
    names: Sequence[str] = SPARSE_CACHE_NAMES,
) -> PackedSparseCacheProjection:
    """Concatenate token-local sparse cache projection weights in ``names`` order."""
    tensors = tuple(weights)
    output_names = tuple(names)
    if not tensors:
        raise ValueError("at least one weight is required")
    if len(tensors) != len(output_names):
        raise ValueError("weights and names must have the same length")
    if any(weight.ndim != 2 for weight in tensors):
        raise ValueError("every weight must be a 2D tensor")
    input_width = tensors[0].size(1)
    if any(weight.size(1) != input_width for weight in tensors):
        raise ValueError("all weights must have the same input width")
    device = tensors[0].device
    dtype = tensors[0].dtype
    if any(weight.device != device or weight.dtype != dtype for weight in tensors):
        raise ValueError("all weights must share device and dtype")
    return PackedSparseCacheProjection(
        weight=torch.cat(tensors, dim=0).contiguous(),
        split_sizes=tuple(int(weight.size(0)) for weight in tensors),
        names=output_names,
    )
