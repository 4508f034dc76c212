"""GPU parity of the sequence-form selection's matrix-core-filtered kernel.

relation_select_packed_seq with bf16 activations, 64-wide exact/router vectors
and caches of at most 512 rows runs rlm_select_tile.hip: candidate scores on
the matrix cores, float64 verification of the candidates that can reach the
top-k (relation_select.py:9-308 semantics).  Every case here takes that path
and must equal the float64 oracle bit for bit -- indices, scores and the
invalid-slot sentinels -- including shapes that stress its bookkeeping: exact
ties across many candidates (more members than one 64-entry window), 1/2/8
router heads, 4..64 blocks, unusual local windows / picks / k, arbitrary
per-query positions, query counts that are not a multiple of 16, bf16
statistics, and inputs whose magnitudes span six decades.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import select as osel
from relation_lm.kernels.relation_select import relation_select_packed_seq
from relation_lm.workloads import CONFIGS, SELECT_ORDER, RelationConfig, select_args, selection_inputs

pytestmark = pytest.mark.gpu

QUERY_SIDE = ("anchor_query", "anchor_router_query", "partner_base")


def np32(t):
    return t.detach().float().cpu().numpy() if t.dtype.is_floating_point else t.cpu().numpy()


def oracle(inp, cfg):
    host = {k: np32(v) for k, v in inp.items()}
    return osel.relation_select_packed_seq(*[host[k] for k in SELECT_ORDER], host["positions"],
                                           cfg.local_window, cfg.top_blocks, cfg.k_out,
                                           cfg.strict_valid)


def check(inp, cfg, what):
    got = relation_select_packed_seq(*select_args(inp, cfg))
    torch.cuda.synchronize()
    expected = oracle(inp, cfg)
    names = ("anchor", "anchor_score", "partner", "partner_score")
    for name, g, e in zip(names, got, expected):
        g = g.cpu().numpy()
        assert g.shape == e.shape, (what, name, g.shape, e.shape)
        bad = np.argwhere(g != e)
        if len(bad):
            i = tuple(bad[0])
            raise AssertionError(f"{what} {name}: {len(bad)} mismatches, first {bad[:4].tolist()}: "
                                 f"got {g[i]} expected {e[i]}")
    return expected


def small(**kw):
    base = dict(name="tile", batch=2, context=256, d_model=256, block_size=32, local_window=64,
                top_blocks=4, k_out=8, dtype=torch.bfloat16, seed=9001)
    base.update(kw)
    return RelationConfig(**base)


@pytest.mark.parametrize("strict", [False, True])
@pytest.mark.parametrize("stat_dtype", [torch.float32, torch.bfloat16])
def test_cfg2_strict_and_statistics_dtype(device, strict, stat_dtype):
    cfg = RelationConfig(**{**CONFIGS["cfg2"].__dict__, "strict_valid": strict})
    inp = selection_inputs(cfg, device=device)
    for k in ("anchor_block_mean", "anchor_block_std", "partner_block_mean", "partner_block_std"):
        inp[k] = inp[k].to(stat_dtype)
    print(f"tile cfg2 strict={strict} stats={stat_dtype}", flush=True)
    check(inp, cfg, f"cfg2 strict={strict} stats={stat_dtype}")


@pytest.mark.parametrize("heads", [1, 2, 8])
def test_router_heads(device, heads):
    cfg = small(heads=heads, head_dim=64 // heads, seed=9100 + heads)
    inp = selection_inputs(cfg, device=device)
    check(inp, cfg, f"heads={heads}")


@pytest.mark.parametrize("context,block,local,top", [(256, 64, 64, 2), (256, 16, 32, 4),
                                                     (256, 4, 16, 8), (512, 16, 48, 3)])
def test_block_counts(device, context, block, local, top):
    # 4, 16, 64 and 32 blocks: one, one, four and two blocks per lane.
    cfg = small(context=context, block_size=block, local_window=local, top_blocks=top,
                seed=9200 + block)
    inp = selection_inputs(cfg, device=device)
    check(inp, cfg, f"T={context} block={block}")


@pytest.mark.parametrize("local,top,k", [(16, 1, 8), (32, 2, 16), (64, 4, 1), (48, 3, 5),
                                         (8, 0, 8), (1, 6, 3), (64, 6, 16)])
def test_routing_parameters(device, local, top, k):
    cfg = small(local_window=local, top_blocks=top, k_out=k, seed=9300 + local + top + k)
    inp = selection_inputs(cfg, device=device)
    check(inp, cfg, f"L={local} top={top} k={k}")


def test_arbitrary_positions_and_ragged_query_count(device):
    cfg = small(batch=3, seed=9400)
    inp = selection_inputs(cfg, device=device)
    tq = 37
    for k in QUERY_SIDE:
        inp[k] = inp[k][:, :tq].contiguous()
    g = torch.Generator().manual_seed(17)
    pos = torch.randint(0, cfg.context, (cfg.batch, tq), generator=g)
    pos[0, :5] = torch.tensor([0, 1, 2, cfg.context - 1, 63])
    inp["positions"] = pos.to(torch.int32).to(device)
    check(inp, cfg, "positions [B,Tq] int32, Tq=37")
    inp["positions"] = pos[1].to(device)  # [Tq] int64, shared by the batch
    check(inp, cfg, "positions [Tq] int64")


def test_exact_ties_span_several_windows(device):
    """Identical keys tie every candidate: more than 64 members per query, and the
    tie rules (anchor -> lowest position, partners -> lowest lane) decide."""
    cfg = small(batch=2, seed=9500)
    inp = selection_inputs(cfg, device="cpu")
    inp["anchor_keys"][:] = inp["anchor_keys"][:, :1]
    inp["partner_keys"][0] = inp["partner_keys"][0, 7:8]
    inp["partner_keys"][1, ::2] = inp["partner_keys"][1, 3:4]
    dev = {k: v.to(device) for k, v in inp.items()}
    expected = check(dev, cfg, "identical keys")
    # Every valid anchor candidate ties, so each anchor is its candidate set's
    # lowest position: never above the local window's start.
    t = np.arange(cfg.context)
    assert (expected[0] <= np.maximum(t - cfg.local_window + 1, 0)[None, :]).all()


def test_magnitudes_spanning_decades(device):
    cfg = small(batch=2, seed=9600)
    inp = selection_inputs(cfg, device="cpu")
    g = torch.Generator().manual_seed(3)
    for k in ("anchor_keys", "partner_keys", "partner_anchor_cache"):
        scale = 10.0 ** (torch.rand(inp[k].shape[:-1] + (1,), generator=g) * 6 - 3)
        inp[k] = (inp[k].float() * scale).to(torch.bfloat16)
    for k in QUERY_SIDE:
        scale = 10.0 ** (torch.rand(inp[k].shape[:-1] + (1,), generator=g) * 4 - 2)
        inp[k] = (inp[k].float() * scale).to(torch.bfloat16)
    dev = {k: v.to(device) for k, v in inp.items()}
    check(dev, cfg, "magnitudes 1e-3..1e3")


def test_near_ties_below_bf16_resolution(device):
    """Keys that differ only in their last bf16 bit: approximate scores sit within
    the error bound of each other, so the float64 verification decides."""
    cfg = small(batch=2, seed=9700)
    inp = selection_inputs(cfg, device="cpu")
    for k in ("anchor_keys", "partner_keys"):
        base = inp[k][:, :1].float()
        bits = base.to(torch.bfloat16).view(torch.int16).expand(inp[k].shape).clone()
        g = torch.Generator().manual_seed(11)
        bits += torch.randint(-1, 2, bits.shape, generator=g, dtype=torch.int16)
        inp[k] = bits.view(torch.bfloat16)
    dev = {k: v.to(device) for k, v in inp.items()}
    check(dev, cfg, "last-bit near ties")
