"""CPU behaviour of the packed sparse-cache projection.

Mirrors the reference's CPU tests (tests/test_packed_cache_projection.py:10-33 of
Ahmet2001/relation-lm): on CPU tensors ``project`` is ``F.linear`` and must equal
the six separate linears at fp32 within 2e-5, and mismatched widths raise
``ValueError``.  Device tensors go to the HIP kernel (tests/test_relation_reduce_gpu.py).
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from relation_lm.inference import (
    SPARSE_CACHE_NAMES,
    PackedSparseCacheProjection,
    pack_sparse_cache_projection_weights,
)

WIDTHS = (64, 64, 128, 128, 64, 64)


@pytest.mark.parametrize("batch", [1, 8])
def test_cpu_project_equals_six_linears(batch):
    gen = torch.Generator().manual_seed(20260822 + batch)
    memory = torch.randn(batch, 576, generator=gen)
    weights = [torch.randn(w, 576, generator=gen) * 0.02 for w in WIDTHS]
    packed = pack_sparse_cache_projection_weights(weights)
    assert packed.input_width == 576 and packed.output_width == sum(WIDTHS)
    parts = packed.project(memory)
    assert len(parts) == len(WIDTHS)
    for w, got in zip(weights, parts):
        assert got.shape == (batch, w.shape[0])
        torch.testing.assert_close(got, F.linear(memory, w), atol=2e-5, rtol=2e-5)
    named = packed.project_dict(memory)
    assert tuple(named) == SPARSE_CACHE_NAMES


def test_cpu_project_leading_dims_and_dtype():
    gen = torch.Generator().manual_seed(7)
    memory = torch.randn(2, 3, 576, generator=gen, dtype=torch.float64)
    weights = [torch.randn(w, 576, generator=gen, dtype=torch.float64) for w in WIDTHS]
    parts = pack_sparse_cache_projection_weights(weights).project(memory)
    for w, got in zip(weights, parts):
        assert got.dtype == torch.float64
        torch.testing.assert_close(got, memory @ w.T)


def test_mismatched_input_widths_raise():
    with pytest.raises(ValueError):
        pack_sparse_cache_projection_weights((torch.randn(4, 8), torch.randn(4, 9)),
                                             names=("a", "b"))


def test_dataclass_validation_errors():
    with pytest.raises(ValueError, match="2D"):
        PackedSparseCacheProjection(torch.randn(4), (4,), ("a",))
    with pytest.raises(ValueError, match="same length"):
        PackedSparseCacheProjection(torch.randn(4, 3), (2, 2), ("a",))
    with pytest.raises(ValueError, match="positive"):
        PackedSparseCacheProjection(torch.randn(4, 3), (4, 0), ("a", "b"))
    with pytest.raises(ValueError, match="sum"):
        PackedSparseCacheProjection(torch.randn(4, 3), (2, 1), ("a", "b"))
    packed = PackedSparseCacheProjection(torch.randn(4, 3), (2, 2), ("a", "b"))
    with pytest.raises(ValueError, match="width"):
        packed.project(torch.randn(1, 5))
