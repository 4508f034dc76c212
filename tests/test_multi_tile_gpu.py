"""GPU parity of the routed multi-anchor selection's matrix-core-filtered kernel.

multi_relation_select_seq with bf16 activations, 64-wide exact/router vectors,
whole blocks of >= 16 rows, <= 64 blocks and <= 1024 candidates runs
rlm_multi_tile.hip: the 16 queries of a workgroup share the scoring of every
candidate key tile on the matrix cores, and each query verifies the candidates
that can reach its top-k in float64 (multi_relation_blocks.py:69-147 in the
routed form).  Every case must equal the float64 oracle bit for bit -- anchors,
partners, scores and the inactive/exhausted sentinels -- including the shapes
that stress its bookkeeping: block sizes 16..64 and 4..64 blocks, up to 1024
candidates per routing, 1/2/8 router heads, 1..8 slots, k up to 16, strict
validity, bf16 statistics, arbitrary positions and query counts that are not a
multiple of 16, and exact ties (duplicate keys) that put more candidates
within the filter's margin than one 64-entry window holds.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from oracle import select as osel
from relation_lm.kernels.relation_select import multi_relation_select_seq
from relation_lm.workloads import (MULTI_CONFIGS, SELECT_ORDER, multi_select_args,
                                   multi_selection_inputs)

pytestmark = pytest.mark.gpu

CFG5 = MULTI_CONFIGS["cfg5"]


def cfg_of(**kw):
    base = dict(batch=2, context=512, block_size=32, local_window=64, top_blocks=4, k_out=6,
                dtype=torch.bfloat16)
    base.update(kw)
    return dataclasses.replace(CFG5, **base)


def np32(t):
    return t.detach().float().cpu().numpy() if t.dtype.is_floating_point else t.cpu().numpy()


def check(inp, cfg, device, what):
    dev = {k: v.to(device) for k, v in inp.items()}
    got = multi_relation_select_seq(*multi_select_args(dev, cfg))
    torch.cuda.synchronize()
    host = {k: np32(v) for k, v in inp.items()}
    expected = osel.multi_relation_select_seq(*[host[k] for k in SELECT_ORDER], host["positions"],
                                              cfg.local_window, cfg.top_blocks, cfg.k_out,
                                              cfg.strict_valid)
    names = ("anchor", "anchor_score", "partner", "partner_score")
    for name, g, e in zip(names, got, expected):
        g = g.cpu().numpy()
        assert g.shape == e.shape, (what, name, g.shape, e.shape)
        bad = np.argwhere(g != e)
        if len(bad):
            i = tuple(bad[0])
            raise AssertionError(f"{what} {name}: {len(bad)} mismatches, first {bad[:4].tolist()}: "
                                 f"got {g[i]} expected {e[i]}")


@pytest.mark.parametrize("context,block", [(256, 16), (512, 32), (1024, 64), (256, 64), (1024, 16)])
def test_block_sizes_and_counts(device, context, block):
    cfg = cfg_of(context=context, block_size=block, local_window=max(16, block), top_blocks=3)
    check(multi_selection_inputs(cfg, seed=context + block), cfg, device, f"T={context} BS={block}")


@pytest.mark.parametrize("local,top,k", [(16, 1, 1), (64, 15, 16), (200, 2, 3), (256, 12, 6),
                                         (8, 0, 4), (37, 3, 6), (255, 1, 5)])
def test_routing_parameters(device, local, top, k):
    # (64, 15) and (256, 12) at block 64 are the 1024-candidate limit; top 0 routes the
    # local window only; (37, 3) and (255, 1) end the candidate list inside a quad.
    cfg = cfg_of(context=1024, block_size=64, local_window=local, top_blocks=top, k_out=k,
                 slots=min(4, local))
    check(multi_selection_inputs(cfg, seed=local * 100 + top), cfg, device,
          f"local={local} top={top} k={k}")


@pytest.mark.parametrize("heads", [1, 2, 8])
def test_router_heads(device, heads):
    cfg = cfg_of(heads=heads, head_dim=64 // heads)
    check(multi_selection_inputs(cfg, seed=40 + heads), cfg, device, f"heads={heads}")


@pytest.mark.parametrize("slots", [1, 2, 5, 8])
def test_slot_counts(device, slots):
    cfg = cfg_of(slots=slots, local_window=max(32, slots), k_out=5)
    check(multi_selection_inputs(cfg, seed=60 + slots), cfg, device, f"S={slots}")


@pytest.mark.parametrize("strict", [False, True])
@pytest.mark.parametrize("stat_dtype", [torch.float32, torch.bfloat16])
def test_strict_and_statistics_dtype(device, strict, stat_dtype):
    cfg = cfg_of(strict_valid=strict)
    inp = multi_selection_inputs(cfg, seed=70 + strict)
    for side in ("anchor", "partner"):
        for kind in ("mean", "std"):
            inp[f"{side}_block_{kind}"] = inp[f"{side}_block_{kind}"].to(stat_dtype)
    check(inp, cfg, device, f"strict={strict} stats={stat_dtype}")


def test_arbitrary_positions_and_ragged_query_count(device):
    cfg = cfg_of()
    rng = np.random.default_rng(11)
    positions = torch.from_numpy(np.stack([rng.permutation(512)[:45] for _ in range(2)]))
    check(multi_selection_inputs(cfg, positions=positions, seed=80), cfg, device, "ragged")
    early = torch.tensor([0, 1, 2, 3, 4, 5, 6, 7, 31, 32, 33])  # inactive slots, short windows
    check(multi_selection_inputs(cfg, positions=early, seed=81), cfg, device, "early")


def test_duplicate_keys_many_ties(device):
    # Every key vector of slot 0 in blocks 0..5 and of every slot of the partner
    # keys in rows 100..299 identical: hundreds of exact ties inside the filter's
    # margin, past one 64-member window; ties go to the lowest position
    # (anchors) and the lowest candidate lane (partners).
    cfg = cfg_of(local_window=128, top_blocks=8, k_out=16)
    inp = multi_selection_inputs(cfg, seed=90)
    inp["anchor_keys"][:, : 6 * 32, 0] = inp["anchor_keys"][:, :1, 0]
    inp["partner_keys"][:, 100:300] = inp["partner_keys"][:, 99:100]
    check(inp, cfg, device, "ties")


def test_magnitudes_spanning_decades(device):
    cfg = cfg_of()
    inp = multi_selection_inputs(cfg, seed=95)
    scale = torch.logspace(-3, 3, cfg.context).to(torch.bfloat16)
    for name in ("anchor_keys", "partner_keys"):
        inp[name] = (inp[name].float() * scale[None, :, None, None].float()).to(torch.bfloat16)
    check(inp, cfg, device, "decades")
