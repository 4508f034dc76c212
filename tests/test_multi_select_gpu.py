"""GPU parity of the routed multi-anchor selection against the CPU oracle.

relation_lm::multi_relation_select_seq has no reference kernel; the oracle
(oracle/select.py: multi_relation_select_seq) restates the dense
MultiAnchorRelationBlock selection (multi_relation_blocks.py:69-147) over the
routed candidate set and is pinned on the CPU (tests/test_oracle_multi_select.py).
Indices and scores must be bit-exact, as for the single-anchor op: both sides
accumulate every dot in float64 and round once to float32.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from oracle import select as osel
from relation_lm.kernels.relation_select import (multi_relation_select_seq,
                                                 relation_select_packed_seq)
from relation_lm.workloads import (MULTI_CONFIGS, SELECT_ORDER, multi_select_args,
                                   multi_selection_inputs)

pytestmark = pytest.mark.gpu

CFG5 = MULTI_CONFIGS["cfg5"]


def small(**kw):
    base = dict(batch=2, context=256, block_size=32, local_window=32, top_blocks=3, k_out=6)
    base.update(kw)
    return dataclasses.replace(CFG5, **base)


def np32(t):
    return t.detach().float().cpu().numpy() if t.dtype.is_floating_point else t.cpu().numpy()


def run_oracle(inp, cfg):
    host = {k: np32(v) for k, v in inp.items()}
    return osel.multi_relation_select_seq(*[host[k] for k in SELECT_ORDER], host["positions"],
                                          cfg.local_window, cfg.top_blocks, cfg.k_out,
                                          cfg.strict_valid)


def assert_equal(got, expected, what=""):
    names = ("anchor", "anchor_score", "partner", "partner_score")
    for name, g, e in zip(names, got, expected):
        g = g.cpu().numpy()
        assert g.shape == e.shape, (what, name, g.shape, e.shape)
        if not np.array_equal(g, e):
            bad = np.argwhere(g != e)
            raise AssertionError(f"{what} {name}: {len(bad)} mismatches, first "
                                 f"{bad[:5].tolist()}: got {g[tuple(bad[0])]} expected "
                                 f"{e[tuple(bad[0])]}")


def run_gpu(inp, cfg, device):
    dev = {k: v.to(device) for k, v in inp.items()}
    out = multi_relation_select_seq(*multi_select_args(dev, cfg))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("strict", [False, True])
def test_multi_select_matches_oracle(device, dtype, strict):
    cfg = small(dtype=dtype, strict_valid=strict)
    inp = multi_selection_inputs(cfg, seed=501 + strict)
    assert_equal(run_gpu(inp, cfg, device), run_oracle(inp, cfg), f"{dtype} strict={strict}")


@pytest.mark.parametrize("slots", [1, 2, 3, 8])
def test_slot_counts(device, slots):
    cfg = small(slots=slots, local_window=max(16, slots), k_out=5)
    inp = multi_selection_inputs(cfg, seed=600 + slots)
    assert_equal(run_gpu(inp, cfg, device), run_oracle(inp, cfg), f"S={slots}")


def test_ragged_positions_per_row(device):
    """[B,Tq] positions in arbitrary order, Tq not a multiple of the workgroup's 8 queries."""
    cfg = small()
    rng = np.random.default_rng(7)
    positions = torch.from_numpy(np.stack([rng.permutation(256)[:37] for _ in range(2)]))
    inp = multi_selection_inputs(cfg, positions=positions, seed=700)
    assert_equal(run_gpu(inp, cfg, device), run_oracle(inp, cfg), "ragged")


def test_one_slot_equals_single_anchor_op(device):
    cfg = small(slots=1, dtype=torch.bfloat16)
    inp = multi_selection_inputs(cfg, seed=800)
    dev = {k: v.to(device) for k, v in inp.items()}
    multi = multi_relation_select_seq(*multi_select_args(dev, cfg))
    single_in = {k: (v[:, :, 0].contiguous() if v.dim() == 4 and "block" not in k else v)
                 for k, v in dev.items()}
    single = relation_select_packed_seq(*[single_in[k] for k in SELECT_ORDER],
                                        single_in["positions"], cfg.local_window,
                                        cfg.top_blocks, cfg.k_out, cfg.strict_valid)
    torch.cuda.synchronize()
    for m, s in zip(multi, single):
        assert torch.equal(m[:, :, 0], s)


def test_cfg5_sample_matches_oracle_and_full_run(device):
    """Full cfg5 shape: a sample of positions against the oracle, and the same
    rows of the full-sequence run against the sample run."""
    cfg = CFG5
    sample = torch.tensor([0, 1, 2, 3, 5, 63, 64, 127, 128, 129, 1000, 2047, 2048, 3000, 4095])
    full = multi_selection_inputs(cfg, device=device)
    inp = dict(full)
    for k in ("anchor_query", "anchor_router_query", "partner_base"):
        inp[k] = full[k][:, sample].contiguous()
    inp["positions"] = sample.to(device)
    got = multi_relation_select_seq(*multi_select_args(inp, cfg))
    torch.cuda.synchronize()
    assert_equal(got, run_oracle(inp, cfg), "cfg5 sample")
    whole = multi_relation_select_seq(*multi_select_args(full, cfg))
    torch.cuda.synchronize()
    for w, g in zip(whole, got):
        assert torch.equal(w[:, sample.to(device)], g)


def test_cfg5_invariants(device):
    """Size-independent properties over every query of the cfg5 shape."""
    cfg = CFG5
    inp = multi_selection_inputs(cfg, device=device)
    a, s, p, ps = multi_relation_select_seq(*multi_select_args(inp, cfg))
    torch.cuda.synchronize()
    t = torch.arange(cfg.context, device=device)[None, :, None]
    slot = torch.arange(cfg.slots, device=device)[None, None, :]
    active = slot <= t
    assert torch.equal(torch.isfinite(s), active.expand_as(s))
    assert bool((a[~active.expand_as(a)] == 0).all())
    assert bool(((a >= 0) & (a <= t)).all())
    # distinct active anchors
    for i in range(cfg.slots):
        for j in range(i + 1, cfg.slots):
            both = active[..., i] & active[..., j]
            assert not bool(((a[..., i] == a[..., j]) & both).any())
    fin = torch.isfinite(ps)
    # every slot with an active anchor has its K partners once t is large enough
    assert bool(fin[:, cfg.k_out + cfg.slots:].all())
    # partners are causal, never an active anchor of the query, in descending order
    pt = t[..., None]
    assert bool(((p <= pt) & (p >= 0))[fin].all())
    hit = (p[..., None] == a[:, :, None, None, :]) & active[:, :, None, None, :]
    assert not bool((hit.any(-1) & fin).any())
    d = ps[..., 1:] - ps[..., :-1]
    both = fin[..., 1:] & fin[..., :-1]
    assert bool((d[both] <= 0).all())
    # distinct partners within a slot
    srt = torch.sort(torch.where(fin, p, -1 - torch.arange(cfg.k_out, device=device)), dim=-1)[0]
    assert not bool((srt[..., 1:] == srt[..., :-1]).any())


def test_rejects_local_window_below_slots(device):
    cfg = small(local_window=2)
    inp = multi_selection_inputs(cfg, device=device)
    with pytest.raises(RuntimeError, match="local_window"):
        multi_relation_select_seq(*multi_select_args(inp, cfg))
