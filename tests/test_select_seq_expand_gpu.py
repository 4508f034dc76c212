"""GPU parity of relation_select_packed_seq_expand: the sequence-form selection
plus the whole expanded cache in one call.

Reference: the selection is relation_select_packed (relation_select.py:9-308)
per query, as relation_select_packed_seq; the expanded cache is the reference's
own projection expanded = F.linear(operand_cache, W_e, b_e)
(tests/test_relation_reduce_gpu.py:64-68), which this library serves with
relation_linear.  The op must return exactly relation_select_packed_seq's
outputs and write exactly relation_linear's bf16 cache (the projection takes
the same k-steps on the matrix cores, so the bits agree), on the path where
the selection's workgroups project the cache tiles (cfg2: one 128 x 128 tile
per workgroup; wider caches: several; narrower: fewer tiles than workgroups;
relation dim 64) and on the two-launch fallbacks (width not a multiple of 128,
cache too short for the staged tiles).  The selection itself is pinned to
the float64 oracle by test_select_tile_gpu.py / test_relation_select_gpu.py.
"""
from __future__ import annotations

import pytest
import torch

from relation_lm import _native  # noqa: F401  (registers torch.ops.relation_lm)
from relation_lm.kernels.relation_reduce import relation_linear
from relation_lm.kernels.relation_select import (relation_select_packed_seq,
                                                 relation_select_packed_seq_expand)
from relation_lm.workloads import CONFIGS, RelationConfig, select_args, selection_inputs

pytestmark = pytest.mark.gpu


def run_case(device, cfg, width, rdim, with_bias=True, seed=0):
    sel = selection_inputs(cfg, device=device)
    sargs = select_args(sel, cfg)
    g = torch.Generator().manual_seed(1000 + width + rdim + seed)
    operand = torch.randn(cfg.batch, cfg.context, rdim, generator=g).to(torch.bfloat16).to(device)
    weight = (torch.randn(width, rdim, generator=g) * rdim ** -0.5).to(torch.bfloat16).to(device)
    bias = (0.1 * torch.randn(width, generator=g)).to(torch.bfloat16).to(device) if with_bias \
        else None
    print(f"select_seq_expand B={cfg.batch} T={cfg.context} N={width} R={rdim} "
          f"bias={with_bias}", flush=True)
    cache = torch.full((cfg.batch, cfg.context, width), float("nan"), dtype=torch.bfloat16,
                       device=device)
    got = relation_select_packed_seq_expand(*sargs, operand, weight, bias, cache)
    want = relation_select_packed_seq(*sargs)
    expanded = relation_linear(operand, weight, bias)
    torch.cuda.synchronize()
    for name, a, b in zip(("anchor", "anchor_score", "partner", "partner_score"), got, want):
        assert torch.equal(a, b), name
    assert expanded.dtype == torch.bfloat16
    assert torch.equal(cache, expanded), (cache.float() - expanded.float()).abs().max().item()


def test_cfg2_one_tile_per_workgroup(device):
    run_case(device, CONFIGS["cfg2"], 1024, 128)


@pytest.mark.parametrize("width,rdim,with_bias", [
    (2048, 128, True),   # two cache tiles per workgroup
    (256, 128, False),   # fewer tiles than workgroups, no bias
    (1024, 64, True),    # relation dim 64
    (1024, 32, True),    # relation dim 32: the output staging is larger than the two tiles
    (1008, 128, True),   # width not a multiple of 128: the GEMM launch after the selection
])
def test_cfg2_shapes(device, width, rdim, with_bias):
    run_case(device, CONFIGS["cfg2"], width, rdim, with_bias)


def test_short_cache_falls_back(device):
    # T = 256 < 4 R: the two staged tiles exceed the key rows' LDS.
    cfg = RelationConfig(name="short", batch=3, context=256, d_model=256, block_size=32,
                         local_window=64, top_blocks=4, k_out=8, dtype=torch.bfloat16,
                         seed=4242)
    run_case(device, cfg, 1024, 128)


def test_partial_last_row_tile(device):
    # B*T = 3 * 448 rows: the last 128-row cache tile is partial.
    cfg = RelationConfig(name="rows", batch=3, context=448, d_model=256, block_size=32,
                         local_window=64, top_blocks=4, k_out=8, dtype=torch.bfloat16,
                         seed=4243)
    run_case(device, cfg, 512, 96)


def test_repeat_identical(device):
    cfg = CONFIGS["cfg2"]
    sel = selection_inputs(cfg, device=device)
    sargs = select_args(sel, cfg)
    g = torch.Generator().manual_seed(77)
    operand = torch.randn(cfg.batch, cfg.context, 128, generator=g).to(torch.bfloat16).to(device)
    weight = (torch.randn(1024, 128, generator=g) / 11.3).to(torch.bfloat16).to(device)
    caches = [torch.empty(cfg.batch, cfg.context, 1024, dtype=torch.bfloat16, device=device)
              for _ in range(2)]
    outs = [relation_select_packed_seq_expand(*sargs, operand, weight, None, c) for c in caches]
    torch.cuda.synchronize()
    assert torch.equal(caches[0], caches[1])
    for a, b in zip(*outs):
        assert torch.equal(a, b)
