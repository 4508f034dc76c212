"""GPU parity of the routed selection kernels against the CPU oracle.

Indices and scores must be bit-exact: both sides accumulate every dot product
in float64 and round once to float32 (oracle/__init__.py), so equality is the
bar, including the invalid-slot sentinels (position t-LOCAL+1, score -inf).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import select as osel
from relation_lm.kernels.relation_select import relation_select_packed, relation_select_packed_seq
from relation_lm.kernels.triton_select import anchor_select, partner_topk
from relation_lm.workloads import CONFIGS, RelationConfig, select_args, selection_inputs

pytestmark = pytest.mark.gpu


def np32(t):
    return t.detach().float().cpu().numpy() if t.dtype.is_floating_point else t.cpu().numpy()


def assert_select_equal(got, expected, what=""):
    names = ("anchor", "anchor_score", "partner", "partner_score")
    for name, g, e in zip(names, got, expected):
        g = g.cpu().numpy()
        assert g.shape == e.shape, (what, name, g.shape, e.shape)
        if not np.array_equal(g, e):
            bad = np.argwhere(g != e)[:5]
            raise AssertionError(f"{what} {name}: {len(np.argwhere(g != e))} mismatches, "
                                 f"first {bad.tolist()}: got {g[tuple(bad[0])]} "
                                 f"expected {e[tuple(bad[0])]}")


def oracle_packed(inp, cfg, seq):
    host = {k: np32(v) for k, v in inp.items()}
    fn = osel.relation_select_packed_seq if seq else osel.relation_select_packed
    position = host["positions"] if seq else int(host["position"])
    return fn(*[host[k] for k in ("anchor_query", "anchor_keys", "anchor_router_query",
                                  "anchor_block_mean", "anchor_block_std", "anchor_gamma",
                                  "anchor_bias", "partner_base", "partner_anchor_cache",
                                  "partner_keys", "partner_block_mean", "partner_block_std",
                                  "partner_gamma", "partner_bias")],
              position, cfg.local_window, cfg.top_blocks, cfg.k_out, cfg.strict_valid)


def test_reference_case_packed_equals_two_op_and_oracle(device):
    """tests/test_relation_select_gpu.py:10-87 of the reference, plus oracle parity."""
    g = torch.Generator().manual_seed(29)
    batch, context, blocks = 4, 512, 64

    def rn(*s):
        return torch.randn(*s, generator=g)

    anchor_query, anchor_keys, anchor_router_query = rn(batch, 64), rn(batch, context, 64), rn(batch, 64)
    anchor_mean, anchor_std = rn(batch, blocks, 4, 16), torch.rand(batch, blocks, 4, 16, generator=g)
    anchor_gamma, anchor_bias = rn(4), rn(4, 16)
    partner_base, partner_anchor_cache = rn(batch, 128), rn(batch, context, 128)
    partner_keys = rn(batch, context, 64)
    partner_mean, partner_std = rn(batch, blocks, 4, 16), torch.rand(batch, blocks, 4, 16, generator=g)
    partner_gamma, partner_bias = rn(4), rn(4, 16)
    position = torch.tensor(context - 1, dtype=torch.long)
    cpu = [anchor_query, anchor_keys, anchor_router_query, anchor_mean, anchor_std, anchor_gamma,
           anchor_bias, partner_base, partner_anchor_cache, partner_keys, partner_mean,
           partner_std, partner_gamma, partner_bias, position]
    dev = [t.to(device) for t in cpu]
    anchor, anchor_score = anchor_select(*dev[:7], dev[14], 16, 2, False)
    batch_index = torch.arange(batch, device=device)
    contribution = dev[8][batch_index, anchor.long()]
    partner, partner_score = partner_topk(
        (dev[7][:, :64] + contribution[:, :64]).contiguous(), dev[9],
        (dev[7][:, 64:] + contribution[:, 64:]).contiguous(), dev[10], dev[11], dev[12], dev[13],
        dev[14], anchor, 16, 2, 8, False)
    fused = relation_select_packed(*dev, 16, 2, 8, False)
    torch.cuda.synchronize()
    assert torch.equal(anchor, fused[0])
    assert torch.equal(partner, fused[2])
    assert torch.allclose(anchor_score, fused[1], atol=2e-4, rtol=0)
    assert torch.allclose(partner_score, fused[3], atol=2e-4, rtol=0)
    expected = osel.relation_select_packed(*[t.numpy() for t in cpu[:14]], 511, 16, 2, 8, False)
    assert_select_equal(fused, expected, "packed")
    two_op = osel.partner_topk(
        (partner_base[:, :64] + partner_anchor_cache[torch.arange(batch), torch.from_numpy(
            expected[0]).long()][:, :64]).numpy(),
        partner_keys.numpy(),
        (partner_base[:, 64:] + partner_anchor_cache[torch.arange(batch), torch.from_numpy(
            expected[0]).long()][:, 64:]).numpy(),
        partner_mean.numpy(), partner_std.numpy(), partner_gamma.numpy(), partner_bias.numpy(),
        511, expected[0], 16, 2, 8, False)
    assert np.array_equal(partner.cpu().numpy(), two_op[0])
    assert np.array_equal(partner_score.cpu().numpy(), two_op[1])


DECODE_CASES = [
    ("cfg1", False), ("cfg1", True), ("cfg2", False), ("cfg2", True), ("cfg3", False),
]


@pytest.mark.parametrize("name,strict", DECODE_CASES)
@pytest.mark.parametrize("batch", [1, 8])
def test_decode_matches_oracle(device, name, strict, batch):
    base = CONFIGS[name]
    cfg = RelationConfig(**{**base.__dict__, "batch": batch, "strict_valid": strict})
    inp = selection_inputs(cfg, queries=1, device=device)
    got = relation_select_packed(*select_args(inp, cfg))
    torch.cuda.synchronize()
    assert_select_equal(got, oracle_packed(inp, cfg, seq=False), f"{name} strict={strict}")


@pytest.mark.parametrize("position", [0, 1, 2, 7, 31, 32, 63, 64, 65, 200, 511])
def test_decode_positions_and_sentinels(device, position):
    cfg = RelationConfig(**{**CONFIGS["cfg2"].__dict__, "batch": 3})
    inp = selection_inputs(cfg, queries=1, device=device)
    inp["position"] = torch.tensor(position, dtype=torch.int64, device=device)
    for strict in (False, True):
        cfg_s = RelationConfig(**{**cfg.__dict__, "strict_valid": strict})
        got = relation_select_packed(*select_args(inp, cfg_s))
        torch.cuda.synchronize()
        assert_select_equal(got, oracle_packed(inp, cfg_s, seq=False), f"t={position}")


@pytest.mark.parametrize("name,strict", [("cfg1", False), ("cfg2", False), ("cfg2", True)])
def test_sequence_form_matches_oracle(device, name, strict):
    cfg = RelationConfig(**{**CONFIGS[name].__dict__, "strict_valid": strict})
    inp = selection_inputs(cfg, device=device)
    got = relation_select_packed_seq(*select_args(inp, cfg))
    torch.cuda.synchronize()
    assert_select_equal(got, oracle_packed(inp, cfg, seq=True), f"{name} seq strict={strict}")


def test_sequence_form_batched_positions_int32(device):
    cfg = RelationConfig(**{**CONFIGS["cfg1"].__dict__, "batch": 2})
    inp = selection_inputs(cfg, device=device)
    g = torch.Generator().manual_seed(5)
    positions = torch.randint(0, cfg.context, (2, cfg.context), generator=g)
    inp["positions"] = positions.to(torch.int32).to(device)
    got = relation_select_packed_seq(*select_args(inp, cfg))
    torch.cuda.synchronize()
    expected = oracle_packed(inp, cfg, seq=True)
    assert_select_equal(got, expected, "batched positions")


def test_duplicate_keys_tie_rules(device):
    """Exact ties: anchor -> lowest position, partners -> lowest lane (local first)."""
    cfg = RelationConfig(**{**CONFIGS["cfg1"].__dict__, "batch": 2})
    inp = selection_inputs(cfg, queries=1, device="cpu")
    t = cfg.context - 1
    for b in range(2):
        strong = inp["anchor_query"][b] * 10.0
        inp["anchor_keys"][b, 5] = strong
        inp["anchor_keys"][b, t - 2] = strong
        inp["anchor_block_mean"][b, 0] = 50.0
    inp["partner_keys"][:, 20:30] = inp["partner_keys"][:, 20:21]
    inp["partner_keys"][:, t - 8:t] = inp["partner_keys"][:, 20:21]
    dev = {k: v.to(device) for k, v in inp.items()}
    got = relation_select_packed(*select_args(dev, cfg))
    torch.cuda.synchronize()
    expected = oracle_packed(dev, cfg, seq=False)
    assert_select_equal(got, expected, "ties")
    assert expected[0][0] == 5


@pytest.mark.parametrize("strict", [False, True])
def test_decode_duplicate_keys_tie_rules_bf16(device, strict):
    """The bf16 decode form (the staged-cache decode kernel): exact ties between
    anchor candidates (lowest position wins) and between partner lanes (local
    window first, then picks in pick order), plus all-zero key rows whose scores
    are signed zeros."""
    cfg = RelationConfig(**{**CONFIGS["cfg2"].__dict__, "batch": 3, "strict_valid": strict})
    inp = selection_inputs(cfg, queries=1, device="cpu")
    t = cfg.context - 1
    for b in range(3):
        strong = inp["anchor_query"][b] * 4.0
        inp["anchor_keys"][b, 70] = strong
        inp["anchor_keys"][b, t - 3] = strong
        inp["anchor_block_mean"][b, 2] = 20.0
    inp["partner_keys"][:, 100:140] = inp["partner_keys"][:, 100:101]
    inp["partner_keys"][:, t - 20:t] = inp["partner_keys"][:, 100:101]
    inp["partner_keys"][:, 200:232] = 0.0
    inp["partner_block_mean"][:, 6] = 15.0
    dev = {k: v.to(device) for k, v in inp.items()}
    got = relation_select_packed(*select_args(dev, cfg))
    torch.cuda.synchronize()
    assert_select_equal(got, oracle_packed(dev, cfg, seq=False), f"bf16 ties strict={strict}")


# Decode-form routing parameters inside the decode kernel's limits
# (candidates <= 256): no remote blocks, k above the candidate count, more
# picks than blocks, k = 1.
DECODE_ROUTING = [(8, 0, 8, 512), (16, 1, 40, 512), (4, 7, 16, 512), (32, 2, 1, 512),
                  (32, 6, 8, 128), (64, 4, 64, 512)]


@pytest.mark.parametrize("local,top,k,context", DECODE_ROUTING)
def test_decode_unusual_routing_parameters_bf16(device, local, top, k, context):
    cfg = RelationConfig(**{**CONFIGS["cfg2"].__dict__, "batch": 2, "local_window": local,
                            "top_blocks": top, "k_out": k, "context": context})
    inp = selection_inputs(cfg, queries=1, device=device)
    for position in (0, 5, local + 40, context - 1):
        inp["position"] = torch.tensor(position, dtype=torch.int64, device=device)
        got = relation_select_packed(*select_args(inp, cfg))
        torch.cuda.synchronize()
        assert_select_equal(got, oracle_packed(inp, cfg, seq=False),
                            f"L={local} top={top} k={k} T={context} t={position}")


@pytest.mark.parametrize("local,top,k", [(8, 0, 8), (16, 1, 40), (4, 8, 16), (32, 2, 1)])
def test_unusual_routing_parameters(device, local, top, k):
    cfg = RelationConfig(**{**CONFIGS["cfg1"].__dict__, "batch": 2, "local_window": local,
                            "top_blocks": top, "k_out": k})
    inp = selection_inputs(cfg, device=device)
    got = relation_select_packed_seq(*select_args(inp, cfg))
    torch.cuda.synchronize()
    assert_select_equal(got, oracle_packed(inp, cfg, seq=True), f"L={local} top={top} k={k}")


def test_two_op_path_matches_oracle_bf16(device):
    cfg = CONFIGS["cfg3"]
    inp = selection_inputs(cfg, queries=1, device=device)
    a, s = anchor_select(inp["anchor_query"], inp["anchor_keys"], inp["anchor_router_query"],
                         inp["anchor_block_mean"], inp["anchor_block_std"], inp["anchor_gamma"],
                         inp["anchor_bias"], inp["position"], cfg.local_window, cfg.top_blocks,
                         False)
    b = torch.arange(cfg.batch, device=device)
    contribution = inp["partner_anchor_cache"][b, a.long()]
    pq = (inp["partner_base"][:, :64] + contribution[:, :64]).contiguous()
    prq = (inp["partner_base"][:, 64:] + contribution[:, 64:]).contiguous()
    p, ps = partner_topk(pq, inp["partner_keys"], prq, inp["partner_block_mean"],
                         inp["partner_block_std"], inp["partner_gamma"], inp["partner_bias"],
                         inp["position"], a, cfg.local_window, cfg.top_blocks, cfg.k_out, False)
    torch.cuda.synchronize()
    host = {k: np32(v) for k, v in inp.items()}
    ea, es = osel.anchor_select(host["anchor_query"], host["anchor_keys"],
                                host["anchor_router_query"], host["anchor_block_mean"],
                                host["anchor_block_std"], host["anchor_gamma"],
                                host["anchor_bias"], 511, cfg.local_window, cfg.top_blocks, False)
    assert np.array_equal(a.cpu().numpy(), ea) and np.array_equal(s.cpu().numpy(), es)
    ep, eps_ = osel.partner_topk(np32(pq), host["partner_keys"], np32(prq),
                                 host["partner_block_mean"], host["partner_block_std"],
                                 host["partner_gamma"], host["partner_bias"], 511, ea,
                                 cfg.local_window, cfg.top_blocks, cfg.k_out, False)
    assert np.array_equal(p.cpu().numpy(), ep) and np.array_equal(ps.cpu().numpy(), eps_)


def test_errors_raise(device):
    cfg = CONFIGS["cfg1"]
    inp = selection_inputs(cfg, queries=1, device=device)
    args = list(select_args(inp, cfg))
    bad = list(args)
    bad[1] = inp["anchor_keys"].transpose(1, 2).contiguous().transpose(1, 2)  # non-contiguous
    with pytest.raises(RuntimeError, match="contiguous"):
        relation_select_packed(*bad)
    bad = list(args)
    bad[14] = inp["position"].cpu()
    with pytest.raises(RuntimeError, match="must be on"):
        relation_select_packed(*bad)


# Decode candidate capacities L + TOP*BS of 64, 96, 192 and 320: one, two,
# three and four waves per query (320 also takes the general top-K path).
SPLIT_CASES = [(32, 2, 16), (32, 4, 16), (64, 4, 32), (64, 8, 32)]


@pytest.mark.parametrize("local,top,block", SPLIT_CASES)
@pytest.mark.parametrize("batch", [1, 5])
def test_decode_candidate_capacities(device, local, top, block, batch):
    base = CONFIGS["cfg2"]
    cfg = RelationConfig(**{**base.__dict__, "batch": batch, "local_window": local,
                            "top_blocks": top, "block_size": block})
    inp = selection_inputs(cfg, queries=1, device=device)
    for position in (0, local + 3, cfg.context - 1):
        inp["position"] = torch.tensor(position, dtype=torch.int64, device=device)
        got = relation_select_packed(*select_args(inp, cfg))
        torch.cuda.synchronize()
        assert_select_equal(got, oracle_packed(inp, cfg, seq=False),
                            f"L={local} top={top} BS={block} t={position}")
