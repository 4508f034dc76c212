"""GPU parity of the ring-buffer decode ops against the CPU oracle.

The ring forms have no reference op (roadmap item "persistent ring-buffer state
and contexts beyond 512", README.md:150).  Their oracle (oracle/select.py,
oracle/router.py, oracle/reduce.py: *_ring) is pinned on the CPU by
tests/test_oracle_ring.py against the linear oracles.  Bars as the linear ops:
selection bit-exact; router 1e-6 (fp32); hidden fp32 rel 1e-5, bf16 abs 2e-2.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from oracle import reduce as ored
from oracle import router as orouter
from oracle import select as osel
from relation_lm.kernels.relation_reduce import relation_linear
from relation_lm.kernels.relation_select import relation_select_packed
from relation_lm.kernels.ring import (relation_hidden_cache_update_ring,
                                      relation_hidden_cached_ring, relation_select_packed_ring,
                                      router_cache_update_ring)
from relation_lm.workloads import (CONFIGS, SELECT_ORDER, reduce_inputs, router_cache_inputs,
                                   select_args, selection_inputs)

pytestmark = pytest.mark.gpu

FP32_REL = 1e-5
BF16_ABS = 2e-2


def host(t):
    return t.detach().float().cpu().numpy() if t.dtype.is_floating_point else t.cpu().numpy()


def rel_err(got, expected):
    got = np.asarray(got, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    return float(np.abs(got - expected).max() / max(np.abs(expected).max(), 1e-30))


def ring_select_case(batch, position, dtype, strict, device, seed=0):
    cfg = dataclasses.replace(CONFIGS["cfg3"], batch=batch, dtype=dtype, strict_valid=strict)
    inp = selection_inputs(cfg, queries=1, seed=cfg.seed + seed)
    inp["position"] = torch.tensor(position, dtype=torch.int64)
    dev = {k: v.to(device) for k, v in inp.items()}
    return cfg, inp, dev


def assert_select_equal(got, expected, what):
    for name, g, e in zip(("anchor", "anchor_score", "partner", "partner_score"), got, expected):
        g = g.cpu().numpy()
        assert g.shape == e.shape, (what, name)
        if not np.array_equal(g, e):
            bad = np.argwhere(g != e)
            raise AssertionError(f"{what} {name}: {len(bad)} mismatches, first {bad[:3].tolist()}"
                                 f": got {g[tuple(bad[0])]} expected {e[tuple(bad[0])]}")


@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("strict", [False, True])
@pytest.mark.parametrize("position", [0, 31, 511, 512, 543, 544, 1000, 4095, 100000])
def test_select_ring_matches_oracle(device, batch, dtype, strict, position):
    cfg, inp, dev = ring_select_case(batch, position, dtype, strict, device, seed=position)
    got = relation_select_packed_ring(*select_args(dev, cfg))
    torch.cuda.synchronize()
    h = {k: host(v) for k, v in inp.items()}
    expected = osel.relation_select_packed_ring(*[h[k] for k in SELECT_ORDER], position,
                                                cfg.local_window, cfg.top_blocks, cfg.k_out,
                                                cfg.strict_valid)
    assert_select_equal(got, expected, f"B={batch} {dtype} strict={strict} t={position}")
    # every output is resident: (t - T, t]
    a, _, p, ps = got
    assert bool((a > position - cfg.context).all()) and bool((a <= position).all())
    fin = torch.isfinite(ps)
    assert bool(((p > position - cfg.context) & (p <= position))[fin].all())


def test_select_ring_before_wrap_equals_linear_op(device):
    cfg, inp, dev = ring_select_case(8, 300, torch.bfloat16, False, device)
    ring = relation_select_packed_ring(*select_args(dev, cfg))
    lin = relation_select_packed(*select_args(dev, cfg))
    torch.cuda.synchronize()
    for r, l in zip(ring, lin):
        assert torch.equal(r, l)


def test_select_ring_rejects_non_power_of_two_cache(device):
    cfg, inp, dev = ring_select_case(1, 10, torch.float32, False, device)
    for k in ("anchor_keys", "partner_keys", "partner_anchor_cache"):
        dev[k] = dev[k][:, :480].contiguous()
    for k in ("anchor_block_mean", "anchor_block_std", "partner_block_mean", "partner_block_std"):
        dev[k] = dev[k][:, :15].contiguous()
    with pytest.raises(RuntimeError, match="ring-buffer"):
        relation_select_packed_ring(*select_args(dev, cfg))


ROUTER_BUFFERS = ("anchor_raw_cache", "partner_raw_cache", "anchor_conv_cache",
                  "partner_conv_cache", "anchor_mean", "anchor_std", "partner_mean", "partner_std")


def router_case(batch, cap, block, seed, device, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    dim = 64
    st = {}
    for s in ("anchor", "partner"):
        st[f"{s}_raw_cache"] = torch.randn(batch, cap, dim, generator=g)
        st[f"{s}_conv_cache"] = torch.randn(batch, cap, dim, generator=g)
        st[f"{s}_mean"] = torch.randn(batch, cap // block, 4, 16, generator=g)
        st[f"{s}_std"] = torch.rand(batch, cap // block, 4, 16, generator=g)
        st[f"{s}_weight"] = torch.randn(dim, 3, generator=g) * 0.1
    packed = torch.randn(batch, 512, generator=g)
    st = {k: v.to(dtype) for k, v in st.items()}
    dev = {k: v.to(device) for k, v in st.items()}
    return st, dev, packed.to(dtype), packed.to(dtype).to(device)


def run_router_ring(dev, packed, position, block, device):
    return router_cache_update_ring(
        packed[:, 384:448], packed[:, 448:512], *[dev[k] for k in ROUTER_BUFFERS],
        dev["anchor_weight"], dev["partner_weight"],
        torch.tensor(position, device=device), block)


@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("position", [0, 1, 95, 511, 512, 513, 519, 520, 1023, 4095])
def test_router_ring_matches_oracle(device, batch, position):
    cap, block = 512, 8
    st, dev, packed, dpacked = router_case(batch, cap, block, 300 + position, device)
    out = run_router_ring(dev, dpacked, position, block, device)
    torch.cuda.synchronize()
    p = packed.numpy()
    exp_out, exp = orouter.router_cache_update_ring(
        p[:, 384:448], p[:, 448:512], *[st[k].numpy() for k in ROUTER_BUFFERS],
        st["anchor_weight"].numpy(), st["partner_weight"].numpy(), position, block)
    np.testing.assert_allclose(host(out), exp_out, atol=1e-6, rtol=1e-6)
    for k in ROUTER_BUFFERS:
        np.testing.assert_allclose(host(dev[k]), exp[k], atol=1e-6, rtol=1e-6, err_msg=k)


@pytest.mark.parametrize("block", [8, 16])
def test_router_ring_replay_three_wraps(device, block):
    """Tokens 0..3C-1 from zeroed ring caches, the ring oracle replayed alongside."""
    cap, batch = 64, 2
    st, dev, _, _ = router_case(batch, cap, block, 7, device)
    state = {}
    for k in ROUTER_BUFFERS:
        st[k].zero_()
        dev[k].zero_()
        state[k] = st[k].numpy().copy()
    g = torch.Generator().manual_seed(8)
    for t in range(3 * cap):
        packed = torch.randn(batch, 512, generator=g)
        out = run_router_ring(dev, packed.to(device), t, block, device)
        exp_out, state = orouter.router_cache_update_ring(
            packed[:, 384:448].numpy(), packed[:, 448:512].numpy(), *[state[k] for k in ROUTER_BUFFERS],
            st["anchor_weight"].numpy(), st["partner_weight"].numpy(), t, block)
        torch.cuda.synchronize()
        np.testing.assert_allclose(host(out), exp_out, atol=1e-6, rtol=1e-6)
    for k in ROUTER_BUFFERS:
        np.testing.assert_allclose(host(dev[k]), state[k], atol=1e-6, rtol=1e-5, err_msg=k)


def test_router_ring_bf16_general_block(device):
    """bf16 state (fast kernel) and a block size outside the fast set (general kernel)."""
    cap = 512
    for dtype, block in ((torch.bfloat16, 32), (torch.float32, 4)):
        st, dev, packed, dpacked = router_case(2, cap, block, 11, device, dtype=dtype)
        out = run_router_ring(dev, dpacked, 2000, block, device)
        torch.cuda.synchronize()
        p = packed.float().numpy()
        exp_out, exp = orouter.router_cache_update_ring(
            p[:, 384:448], p[:, 448:512], *[st[k].float().numpy() for k in ROUTER_BUFFERS],
            st["anchor_weight"].float().numpy(), st["partner_weight"].float().numpy(), 2000,
            block)
        tol = 1e-5 if dtype == torch.bfloat16 else 1e-6
        np.testing.assert_allclose(host(out), exp_out, atol=tol, rtol=tol)
        for k in ROUTER_BUFFERS:
            bar = 2e-2 if dtype == torch.bfloat16 else 1e-6
            np.testing.assert_allclose(host(dev[k]), exp[k], atol=bar, rtol=1e-2, err_msg=k)


@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("position", [511, 512, 700, 4095])
def test_hidden_update_ring_matches_oracle(device, batch, position):
    cfg = dataclasses.replace(CONFIGS["cfg3"], batch=batch)
    red = reduce_inputs(cfg, device=device)
    operand = red["operand_cache"][:batch].contiguous()
    cap = operand.shape[1]
    expanded = relation_linear(operand, red["expanded_weight"], red["expanded_bias"])
    g = torch.Generator().manual_seed(position + batch)
    lo = max(0, position - cap + 1)
    anchor = torch.randint(lo, position + 1, (batch,), generator=g)
    partner = torch.randint(lo, position + 1, (batch, 8), generator=g)
    anchor[0] = position
    partner[:, 1] = position
    partner[:, 2] = position - cap  # no longer resident: reads zeros
    mutable = expanded.clone()
    before = host(mutable)
    pos = torch.tensor(position, device=device)
    hidden = relation_hidden_cache_update_ring(
        mutable, operand, anchor.to(device), partner.to(device), red["anchor_weight"],
        red["partner_weight"], red["product_weight"], red["expanded_bias"][:2304], pos)
    torch.cuda.synchronize()
    exp_hidden, exp_cache = ored.relation_hidden_cache_update_ring(
        before, host(operand), anchor.numpy(), partner.numpy(), host(red["anchor_weight"]),
        host(red["partner_weight"]), host(red["product_weight"]),
        host(red["expanded_bias"][:2304]), position, cache_dtype="bfloat16")
    assert float(np.abs(host(hidden) - exp_hidden).max()) <= BF16_ABS
    assert rel_err(host(hidden), exp_hidden) <= FP32_REL
    assert float(np.abs(host(mutable) - exp_cache).max()) <= BF16_ABS
    cached = relation_hidden_cached_ring(mutable, operand, anchor.to(device),
                                         partner[:, :2].contiguous().to(device),
                                         red["product_weight"])
    torch.cuda.synchronize()
    exp_cached = ored.relation_hidden_cached_ring(host(mutable), host(operand), anchor.numpy(),
                                                  partner[:, :2].numpy(),
                                                  host(red["product_weight"]))
    assert rel_err(host(cached), exp_cached) <= FP32_REL


@pytest.mark.parametrize("local,top,block", [(32, 2, 16), (32, 4, 16), (64, 8, 32)])
@pytest.mark.parametrize("position", [40, 511, 1300])
def test_select_ring_candidate_capacities(device, local, top, block, position):
    # Capacities 64, 96 and 320: one, two and four waves per query.
    cfg = dataclasses.replace(CONFIGS["cfg3"], batch=3, local_window=local, top_blocks=top,
                              block_size=block)
    inp = selection_inputs(cfg, queries=1, seed=cfg.seed + position)
    inp["position"] = torch.tensor(position, dtype=torch.int64)
    dev = {k: v.to(device) for k, v in inp.items()}
    got = relation_select_packed_ring(*select_args(dev, cfg))
    torch.cuda.synchronize()
    h = {k: host(v) for k, v in inp.items()}
    expected = osel.relation_select_packed_ring(*[h[k] for k in SELECT_ORDER], position,
                                                cfg.local_window, cfg.top_blocks, cfg.k_out,
                                                cfg.strict_valid)
    assert_select_equal(got, expected, f"L={local} top={top} BS={block} t={position}")
