"""The measured cfg3 decode step, end to end, against the oracle chain.

bench.py times relation_lm.workloads.decode_step: the packed 576->512
projection writing the token's cache rows with the router cache update folded
in, relation_select_packed with the token's expanded-cache row, the cached
relation hidden, and the split-K second linear with the norm-reduce and the
output-head preparation.  This test runs that same function at B=1 and B=8,
over linear caches (t = 509, 510, 511 of 512) and ring-buffer caches
(t = 4093, 4094, 4095 over 512 rows), three consecutive tokens each with a new
memory row and new query-side vectors, and checks every token against an
independent float64 chain on the host, started from the same initial state:

  oracle/reduce.py    packed_sparse_cache_projection (bf16 cache rows)
  oracle/router.py    router_cache_update(_ring) on the projection's router rows
  oracle/select.py    relation_select_packed(_ring)
  oracle/reduce.py    the token's expanded row (linear, bf16), relation_hidden_cached(_ring),
                      linear (hidden rounded to bf16 as the bf16 second linear reads it),
                      relation_norm_reduce, output_prep

Indices and scores are bit-exact; the relation context within 5e-3 (and the
2e-2 bf16 bar); the final bf16 row within 2e-2 plus half an ulp; the cache rows
the step writes within one bf16 rounding and the router caches and block
statistics within fp32 accumulation of the oracle's.  Each stage's device
result, once checked, is the next oracle stage's input (a rounding flip of one
bf16 element would otherwise move every later stage).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reduce as ored
from oracle import router as orouter
from oracle import select as osel
from relation_lm.workloads import CONFIGS, RelationConfig, decode_state, decode_step

pytestmark = pytest.mark.gpu

CTX_TIGHT = 5e-3
BF16_ABS = 2e-2
ROUTER_KEYS = ("anchor_raw_cache", "partner_raw_cache", "anchor_conv_cache", "partner_conv_cache")
STAT_KEYS = ("anchor_block_mean", "anchor_block_std", "partner_block_mean", "partner_block_std")


def host(t):
    return t.detach().cpu().double().numpy() if t.dtype.is_floating_point else t.cpu().numpy()


def bf16(x):
    return ored.round_to(x, "bfloat16")


def new_token(st, cfg, step, device):
    """Fresh memory row and query-side vectors for the next token (seeded)."""
    g = torch.Generator().manual_seed(cfg.seed + 1000 + step)
    sel = st["sel"]
    st["memory"].copy_(torch.randn(st["memory"].shape, generator=g).to(cfg.dtype))
    for k in ("anchor_query", "anchor_router_query", "partner_base"):
        sel[k].copy_(torch.randn(sel[k].shape, generator=g).to(cfg.dtype))
    st["head"]["query"].copy_(torch.randn(st["head"]["query"].shape, generator=g).to(cfg.dtype))


def snapshot(st):
    """The whole decode state as float64 / int numpy arrays."""
    sel, red, rc = st["sel"], st["red"], st["router"]
    out = {k: host(v) for k, v in sel.items()}
    out.update({k: host(v) for k, v in red.items()})
    out.update({k: host(v) for k, v in rc.items()})
    out["expanded_cache"] = host(st["expanded_cache"])
    out["memory"] = host(st["memory"])
    out["projection"] = host(st["projection"].weight)
    out.update({f"head_{k}": host(v) for k, v in st["head"].items()})
    return out


def assert_within_ulp(got, exp, what):
    """|got - exp| <= one bf16 ulp of exp: the device rounds an fp32 sum, the
    oracle a float64 one, so an element may land on the other side of a
    rounding boundary."""
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(exp), 1e-30))) - 7)
    worst = float((np.abs(got - exp) - ulp).max())
    assert worst <= 1e-9, (what, worst)


def check_step(h, dev, got, cfg, t, ring, tag):
    """One decode step of the oracle chain from host state h (the state before
    the step, updated in place), checked stage by stage against the device's
    state after the step (dev) and its outputs (got).  Each stage's device
    result, once checked, is the next stage's input, so a one-ulp rounding
    difference of one stage does not move the next."""
    cap = h["anchor_keys"].shape[1]
    row = t % cap
    # 1. packed projection: the token's cache rows (bf16) and router rows.
    parts = bf16(ored.packed_sparse_cache_projection(h["memory"], h["projection"]))
    widths = np.cumsum([0, 64, 64, 128, 128, 64, 64])
    seg = [parts[:, widths[i]:widths[i + 1]] for i in range(6)]
    for name, part in zip(("anchor_keys", "partner_keys", "operand_cache",
                           "partner_anchor_cache"), seg[:4]):
        assert_within_ulp(dev[name][:, row], part, f"{tag} {name}")
        h[name][:, row] = dev[name][:, row]
    raw_rows = []
    for side, part in (("anchor", seg[4]), ("partner", seg[5])):
        assert_within_ulp(dev[f"{side}_raw_cache"][:, row], part, f"{tag} {side} router row")
        raw_rows.append(dev[f"{side}_raw_cache"][:, row])
    # 2. router cache update of both streams.
    update = orouter.router_cache_update_ring if ring else orouter.router_cache_update
    _, bufs = update(raw_rows[0], raw_rows[1], h["anchor_raw_cache"], h["partner_raw_cache"],
                     h["anchor_conv_cache"], h["partner_conv_cache"], h["anchor_block_mean"],
                     h["anchor_block_std"], h["partner_block_mean"], h["partner_block_std"],
                     h["anchor_conv_weight"], h["partner_conv_weight"], t, cfg.block_size)
    names = dict(zip(("anchor_mean", "anchor_std", "partner_mean", "partner_std"), STAT_KEYS))
    for k, v in bufs.items():
        key = names.get(k, k)
        np.testing.assert_allclose(dev[key], v.reshape(dev[key].shape), rtol=1e-5, atol=1e-5,
                                   err_msg=f"{tag} {key}")
        h[key] = dev[key]
    # 3. selection: bit-exact.
    select = osel.relation_select_packed_ring if ring else osel.relation_select_packed
    exp = select(*(h[k] for k in ("anchor_query", "anchor_keys", "anchor_router_query",
                                  "anchor_block_mean", "anchor_block_std", "anchor_gamma",
                                  "anchor_bias", "partner_base", "partner_anchor_cache",
                                  "partner_keys", "partner_block_mean", "partner_block_std",
                                  "partner_gamma", "partner_bias")),
                 t, cfg.local_window, cfg.top_blocks, cfg.k_out, cfg.strict_valid)
    for name, g_, e_ in zip(("anchor", "anchor_score", "partner", "partner_score"), got[:4], exp):
        np.testing.assert_array_equal(host(g_).astype(np.asarray(e_).dtype), e_,
                                      err_msg=f"{tag} {name}")
    a, _, p, ps = exp
    # 4. the token's expanded-cache row (written by the selection launch).
    e_row = bf16(ored.linear(h["operand_cache"][:, row], h["expanded_weight"],
                             h["expanded_bias"]))
    assert_within_ulp(dev["expanded_cache"][:, row], e_row, f"{tag} expanded row")
    h["expanded_cache"][:, row] = dev["expanded_cache"][:, row]
    # 5. hidden -> second linear (the bf16 linear reads the hidden rounded to
    #    bf16) -> norm-reduce -> output-head preparation.
    cached = ored.relation_hidden_cached_ring if ring else ored.relation_hidden_cached
    hidden = cached(h["expanded_cache"], h["operand_cache"], a, p, h["product_weight"])
    raw = ored.linear(bf16(hidden), h["second_weight"], h["second_bias"])
    ctx = ored.relation_norm_reduce(raw, ps, h["norm_weight"], h["norm_bias"], t, 1e-5)
    final = ored.output_prep(h["head_query"], ctx, h["head_mix"], h["head_weight"],
                             h["head_bias"], 1e-5)
    ctx_err = float(np.abs(host(got[4]) - ctx).max())
    assert ctx_err <= BF16_ABS and ctx_err <= CTX_TIGHT, (tag, ctx_err)
    half_ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(final), 1e-30))) - 8)
    final_err = float((np.abs(host(got[5]) - final) - half_ulp).max())
    assert final_err <= BF16_ABS, (tag, final_err)


@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("start", [509, 4093])
def test_decode_step_chain(device, batch, start):
    cfg = RelationConfig(**{**CONFIGS["cfg3"].__dict__, "batch": batch})
    st = decode_state(cfg, device=device, position=start)
    ring = start >= cfg.context
    assert st["ring"] == ring
    host_state = snapshot(st)
    for step in range(3):
        t = start + step
        print(f"decode step B={batch} t={t} ring={ring}", flush=True)
        st["sel"]["position"].fill_(t)
        new_token(st, cfg, step, device)
        fresh = snapshot(st)
        for k in ("memory", "anchor_query", "anchor_router_query", "partner_base", "head_query"):
            host_state[k] = fresh[k]
        got = decode_step(st, cfg)
        torch.cuda.synchronize()
        check_step(host_state, snapshot(st), got, cfg, t, ring, f"B={batch} t={t}")
