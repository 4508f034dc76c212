"""packed_projection_router_update: the packed projection with the router cache update
folded in (the reference's roadmap item, README.md:148-149) against the two ops it
replaces, packed_projection_to_caches then router_cache_update(_ring) on the router
segments.  Every output and every mutated cache -- the packed rows, the four token
caches, the raw / conv caches, the block statistics and the conv rows -- must be
bit-identical, for the single-launch shapes and for the fallback (B > 16, mixed router
dtypes), at positions inside and outside the cache, linear and ring.
The router update itself is pinned against the oracle by tests/test_router_cache_gpu.py
and tests/test_ring_gpu.py; the projection by tests/test_relation_reduce_gpu.py."""
from __future__ import annotations

import pytest
import torch

from relation_lm.inference import pack_sparse_cache_projection_weights
from relation_lm.kernels.ring import router_cache_update_ring
from relation_lm.kernels.router_cache import router_cache_update

pytestmark = pytest.mark.gpu

TOKEN_WIDTHS = (64, 64, 128, 128)   # anchor_key, partner_key, operand, partner_anchor
ROUTER_DIM = 64


def make_state(batch, context, block, state_dtype, seed, device, mixed=False):
    g = torch.Generator().manual_seed(seed)
    weights = [torch.randn(w, 576, generator=g) * 576 ** -0.5
               for w in TOKEN_WIDTHS + (ROUTER_DIM, ROUTER_DIM)]
    proj = pack_sparse_cache_projection_weights([w.to(device, torch.bfloat16) for w in weights])
    st = {"memory": torch.randn(batch, 576, generator=g).to(device, torch.bfloat16)}
    for name, w in zip(("anchor_keys", "partner_keys", "operand", "partner_anchor"), TOKEN_WIDTHS):
        st[name] = torch.randn(batch, context, w, generator=g).to(device, torch.bfloat16)
    blocks = context // block
    for side in ("anchor", "partner"):
        for kind in ("raw", "conv"):
            st[f"{side}_{kind}_cache"] = torch.randn(batch, context, ROUTER_DIM, generator=g)
        st[f"{side}_mean"] = torch.randn(batch, blocks, 4, 16, generator=g)
        st[f"{side}_std"] = torch.rand(batch, blocks, 4, 16, generator=g)
        st[f"{side}_weight"] = torch.randn(ROUTER_DIM, 3, generator=g) * 0.1
    for k, v in st.items():
        if k in ("memory", "anchor_keys", "partner_keys", "operand", "partner_anchor"):
            continue
        dt = state_dtype
        if mixed and k == "partner_std":
            dt = torch.float32 if state_dtype == torch.bfloat16 else torch.bfloat16
        st[k] = v.to(device, dt)
    return proj, st


ROUTER_ORDER = ("anchor_raw_cache", "partner_raw_cache", "anchor_conv_cache",
                "partner_conv_cache", "anchor_mean", "anchor_std", "partner_mean", "partner_std")


def run_both(batch, context, block, state_dtype, position, ring, device, seed=0, mixed=False):
    proj, st = make_state(batch, context, block, state_dtype, seed, device, mixed)
    a = {k: v.clone() for k, v in st.items()}
    b = {k: v.clone() for k, v in st.items()}
    pos = torch.tensor(position, dtype=torch.int64, device=device)
    parts_a, rout_a = proj.project_into_routed(
        a["memory"], a["anchor_keys"], a["partner_keys"], a["operand"], a["partner_anchor"], pos,
        *(a[k] for k in ROUTER_ORDER), a["anchor_weight"], a["partner_weight"], block, ring=ring)
    parts_b = proj.project_into(b["memory"], b["anchor_keys"], b["partner_keys"], b["operand"],
                                b["partner_anchor"], pos, ring=ring)
    update = router_cache_update_ring if ring else router_cache_update
    rout_b = update(parts_b[4], parts_b[5], *(b[k] for k in ROUTER_ORDER), b["anchor_weight"],
                    b["partner_weight"], pos, block)
    torch.cuda.synchronize()
    tag = f"B={batch} T={context} BS={block} {state_dtype} t={position} ring={ring}"
    for x, y, name in zip(parts_a, parts_b, proj.names):
        assert torch.equal(x, y), (tag, name)
    assert torch.equal(rout_a, rout_b), (tag, "router out")
    for k in st:
        assert torch.equal(a[k], b[k]), (tag, k)
    return rout_a


@pytest.mark.parametrize("batch", [1, 8, 16])
@pytest.mark.parametrize("position", [0, 1, 2, 31, 32, 33, 255, 511, 512, 900])
def test_linear_matches_two_ops(device, batch, position):
    run_both(batch, 512, 32, torch.float32, position, False, device)


@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("position", [0, 511, 512, 543, 700, 4095, 100000])
def test_ring_matches_two_ops(device, batch, position):
    run_both(batch, 512, 32, torch.float32, position, True, device)


@pytest.mark.parametrize("block", [8, 16, 32, 64])
@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
def test_block_sizes_and_state_dtypes(device, block, state_dtype):
    for position in (block - 1, block, 3 * block + 5, 511):
        run_both(4, 512, block, state_dtype, position, False, device, seed=block)
        run_both(4, 512, block, state_dtype, position + 512, True, device, seed=block + 1)


def test_fallback_shapes_match_two_ops(device):
    # More than 16 rows, a block size without a compiled form, mixed router dtypes.
    run_both(17, 512, 32, torch.float32, 300, False, device)
    run_both(2, 512, 4, torch.float32, 300, False, device)
    run_both(2, 512, 32, torch.float32, 300, False, device, mixed=True)


def test_decode_sequence_of_tokens(device):
    # A run of consecutive tokens over one state: each step's writes feed the next.
    proj, st = make_state(2, 512, 32, torch.float32, 5, device)
    a = {k: v.clone() for k, v in st.items()}
    b = {k: v.clone() for k, v in st.items()}
    for t in range(94, 100):
        pos = torch.tensor(t, device=device)
        mem = torch.randn(2, 576, generator=torch.Generator().manual_seed(t)).to(device, torch.bfloat16)
        _, ra = proj.project_into_routed(mem, a["anchor_keys"], a["partner_keys"], a["operand"],
                                         a["partner_anchor"], pos, *(a[k] for k in ROUTER_ORDER),
                                         a["anchor_weight"], a["partner_weight"], 32)
        pb = proj.project_into(mem, b["anchor_keys"], b["partner_keys"], b["operand"],
                               b["partner_anchor"], pos)
        rb = router_cache_update(pb[4], pb[5], *(b[k] for k in ROUTER_ORDER), b["anchor_weight"],
                                 b["partner_weight"], pos, 32)
        torch.cuda.synchronize()
        assert torch.equal(ra, rb), t
    for k in st:
        assert torch.equal(a[k], b[k]), k
