"""The operator boundary under torch.compile and torch.library.opcheck.

The reference runs its router update through
``torch.compile(fullgraph=True, mode="reduce-overhead")`` with
``torch.compiler.cudagraph_mark_step_begin()`` and checks the output and every
mutated buffer against eager at 1e-6 (tests/test_router_cache_update_gpu.py:217-233).
The same is done here for the router update (B = 1 and 8) and for a whole
decode step (select -> hidden -> second linear -> norm-reduce, the order of
the reference's decoder, docs/benchmarks.md:65-131): each compiled graph is
replayed as a HIP graph and must equal eager.  ``opcheck`` then exercises every
registered op's schema (declared mutations), fake kernel and
AOT-dispatch tracing with real device inputs.
"""
from __future__ import annotations

import pytest
import torch

from relation_lm.kernels.relation_reduce import (
    relation_hidden_cached,
    relation_linear,
    relation_norm_reduce,
)
from relation_lm.kernels.relation_select import relation_select_packed
from relation_lm.kernels.router_cache import router_cache_update
from relation_lm.workloads import (
    CONFIGS,
    MultiAnchorConfig,
    RelationConfig,
    SELECT_ORDER,
    multi_select_args,
    multi_selection_inputs,
    reduce_inputs,
    select_args,
    selection_inputs,
)

pytestmark = pytest.mark.gpu

ROUTER_BUFFERS = ("anchor_raw_cache", "partner_raw_cache", "anchor_conv_cache",
                  "partner_conv_cache", "anchor_mean", "anchor_std", "partner_mean",
                  "partner_std")


def router_case(batch, position, seed=0, max_context=512, block_size=8):
    g = torch.Generator().manual_seed(20260824 + batch + position + seed)
    dim, heads, head_dim = 64, 4, 16
    blocks = max_context // block_size
    case = {
        "packed": torch.randn(batch, 512, generator=g),
        "anchor_weight": torch.randn(dim, 3, generator=g) * 0.1,
        "partner_weight": torch.randn(dim, 3, generator=g) * 0.1,
        "position": torch.tensor(position, dtype=torch.long),
    }
    for side in ("anchor", "partner"):
        raw = torch.zeros(batch, max_context, dim)
        raw[:, :position] = torch.randn(batch, position, dim, generator=g)
        conv = torch.zeros(batch, max_context, dim)
        conv[:, :position] = torch.randn(batch, position, dim, generator=g)
        case[f"{side}_raw_cache"] = raw
        case[f"{side}_conv_cache"] = conv
        case[f"{side}_mean"] = torch.randn(batch, blocks, heads, head_dim, generator=g)
        case[f"{side}_std"] = torch.rand(batch, blocks, heads, head_dim, generator=g)
    return case


class RouterUpdate(torch.nn.Module):
    def __init__(self, case, device, block_size=8):
        super().__init__()
        for name in ROUTER_BUFFERS + ("anchor_weight", "partner_weight"):
            self.register_buffer(name, case[name].clone().to(device))
        self.block_size = block_size

    def forward(self, anchor_raw, partner_raw, position):
        return router_cache_update(anchor_raw, partner_raw, self.anchor_raw_cache,
                                   self.partner_raw_cache, self.anchor_conv_cache,
                                   self.partner_conv_cache, self.anchor_mean, self.anchor_std,
                                   self.partner_mean, self.partner_std, self.anchor_weight,
                                   self.partner_weight, position, self.block_size)


@pytest.mark.parametrize("batch", [1, 8])
def test_router_cache_update_fullgraph(device, batch):
    print(f"compiled router update B={batch}", flush=True)
    case = router_case(batch, 447)
    packed = case["packed"].to(device)
    position = case["position"].to(device)
    eager = RouterUpdate(case, device).eval()
    module = RouterUpdate(case, device).eval()
    compiled = torch.compile(module, fullgraph=True, mode="reduce-overhead")
    eager_out = eager(packed[:, 384:448], packed[:, 448:512], position)
    torch.compiler.cudagraph_mark_step_begin()
    compiled_out = compiled(packed[:, 384:448], packed[:, 448:512], position).clone()
    torch.cuda.synchronize()
    torch.testing.assert_close(compiled_out, eager_out, atol=1e-6, rtol=1e-6)
    compiled_buffers = dict(module.named_buffers())
    for name, buf in eager.named_buffers():
        torch.testing.assert_close(compiled_buffers[name], buf, atol=1e-6, rtol=1e-6)


class DecodeStep(torch.nn.Module):
    """One decode step over fixed caches: select -> hidden -> linear -> norm-reduce."""

    def __init__(self, sel, red, expanded, cfg):
        super().__init__()
        self.names = SELECT_ORDER
        for k in SELECT_ORDER:
            self.register_buffer(k, sel[k].clone())
        for k in ("operand_cache", "product_weight", "second_weight", "second_bias",
                  "norm_weight", "norm_bias"):
            self.register_buffer(k, red[k].clone())
        self.register_buffer("expanded", expanded.clone())
        self.cfg = cfg

    def forward(self, position):
        cfg = self.cfg
        a, s, p, ps = relation_select_packed(*[getattr(self, k) for k in self.names], position,
                                             cfg.local_window, cfg.top_blocks, cfg.k_out,
                                             cfg.strict_valid)
        hidden = relation_hidden_cached(self.expanded, self.operand_cache, a, p,
                                        self.product_weight)
        raw = relation_linear(hidden, self.second_weight, self.second_bias,
                              out_dtype=torch.float32)
        ctx = relation_norm_reduce(raw, ps, self.norm_weight, self.norm_bias, position, 1e-5)
        return a, p, ps, ctx


@pytest.mark.parametrize("batch", [1, 8])
def test_decode_step_fullgraph(device, batch):
    print(f"compiled decode step B={batch}", flush=True)
    cfg = RelationConfig(**{**CONFIGS["cfg3"].__dict__, "batch": batch})
    sel = selection_inputs(cfg, queries=1, device=device)
    red = reduce_inputs(cfg, device=device)
    expanded = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])
    module = DecodeStep(sel, red, expanded, cfg).eval()
    compiled = torch.compile(module, fullgraph=True, mode="reduce-overhead")
    for t in (511, 300, 63):  # replays of the captured graph at new positions
        position = torch.tensor(t, device=device)
        eager = module(position)
        torch.compiler.cudagraph_mark_step_begin()
        got = [x.clone() for x in compiled(position)]
        torch.cuda.synchronize()
        for x, y in zip(got[:3], eager[:3]):
            assert torch.equal(x, y), t
        torch.testing.assert_close(got[3], eager[3], atol=0.0, rtol=0.0)


# --------------------------------------------------------------------------- opcheck

SMALL = RelationConfig("opcheck", 2, 128, 256, 16, 32, 2, 8, torch.bfloat16, relation_dim=64,
                       hidden_dim=256, seed=424242)


def _small(device):
    sel_seq = selection_inputs(SMALL, device=device)
    sel_dec = selection_inputs(SMALL, queries=1, device=device)
    red = reduce_inputs(SMALL, device=device)
    expanded = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])
    return sel_seq, sel_dec, red, expanded


def op_cases(device):
    ops = torch.ops.relation_lm
    lex = torch.ops.relationlex
    sel_seq, sel_dec, red, expanded = _small(device)
    cfg = SMALL
    b, t, k = cfg.batch, cfg.context, cfg.k_out
    cases = []
    dec_args = select_args(sel_dec, cfg)
    seq_args = select_args(sel_seq, cfg)
    cases.append(("relation_select_packed", ops.relation_select_packed.default, dec_args))
    cases.append(("relation_select_packed_seq", ops.relation_select_packed_seq.default,
                  seq_args))
    xcache = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])
    cases.append(("relation_select_packed_seq_expand",
                  ops.relation_select_packed_seq_expand.default,
                  seq_args + (red["operand_cache"], red["expanded_weight"], red["expanded_bias"],
                              torch.empty_like(xcache))))
    cases.append(("relation_select_packed_expand_row",
                  ops.relation_select_packed_expand_row.default,
                  dec_args + (red["operand_cache"], red["expanded_weight"], red["expanded_bias"],
                              xcache, False)))
    ring_pos = torch.tensor(3 * t + 17, device=device)
    cases.append(("relation_select_packed_ring", ops.relation_select_packed_ring.default,
                  dec_args[:14] + (ring_pos,) + dec_args[15:]))
    e = cfg.exact_dim
    anchor, _, _, _ = ops.relation_select_packed.default(*dec_args)
    cases.append(("anchor_select", lex.anchor_select.default,
                  (sel_dec["anchor_query"], sel_dec["anchor_keys"],
                   sel_dec["anchor_router_query"], sel_dec["anchor_block_mean"],
                   sel_dec["anchor_block_std"], sel_dec["anchor_gamma"], sel_dec["anchor_bias"],
                   sel_dec["position"], cfg.local_window, cfg.top_blocks, cfg.strict_valid)))
    cases.append(("partner_topk", lex.partner_topk.default,
                  (sel_dec["partner_base"][:, :e].contiguous(), sel_dec["partner_keys"],
                   sel_dec["partner_base"][:, e:].contiguous(), sel_dec["partner_block_mean"],
                   sel_dec["partner_block_std"], sel_dec["partner_gamma"],
                   sel_dec["partner_bias"], sel_dec["position"], anchor, cfg.local_window,
                   cfg.top_blocks, cfg.k_out, cfg.strict_valid)))
    mcfg = MultiAnchorConfig("opcheck", 2, 256, 256, 32, 64, 2, 3, 4, torch.bfloat16)
    msel = multi_selection_inputs(mcfg, device=device)
    cases.append(("multi_relation_select_seq", ops.multi_relation_select_seq.default,
                  multi_select_args(msel, mcfg)))

    g = torch.Generator().manual_seed(5)
    a_dec = (torch.rand(b, generator=g) * t).int().to(device)
    p_dec = (torch.rand(b, k, generator=g) * t).int().to(device)
    a_seq = (torch.rand(b, t, generator=g) * t).int().to(device)
    p_seq = (torch.rand(b, t, k, generator=g) * t).int().to(device)
    scores_dec = torch.randn(b, k, generator=g).to(device)
    scores_seq = torch.randn(b, t, k, generator=g).to(device)
    pos = torch.tensor(t - 1, device=device)
    positions = torch.arange(t, device=device)
    wm = red["product_weight"]
    cases.append(("relation_hidden_cached", ops.relation_hidden_cached.default,
                  (expanded, red["operand_cache"], a_dec, p_dec, wm)))
    cases.append(("relation_hidden_cached_seq", ops.relation_hidden_cached_seq.default,
                  (expanded, red["operand_cache"], a_seq, p_seq, wm)))
    hid_out = torch.empty(tuple(p_seq.shape) + (wm.shape[0],), device=device,
                          dtype=torch.bfloat16)
    cases.append(("relation_hidden_cached_seq_out", ops.relation_hidden_cached_seq_out.default,
                  (expanded, red["operand_cache"], a_seq, p_seq, wm, hid_out)))
    mlp_out = torch.empty(tuple(p_seq.shape) + (red["second_weight"].shape[0],), device=device)
    cases.append(("relation_hidden_linear_seq_out", ops.relation_hidden_linear_seq_out.default,
                  (expanded, red["operand_cache"], a_seq, p_seq, ops.mfma_fragments(wm),
                   ops.mfma_fragments(red["second_weight"]), mlp_out)))
    cases.append(("mfma_fragments", ops.mfma_fragments.default, (red["second_weight"],)))
    cases.append(("relation_hidden_cached_ring", ops.relation_hidden_cached_ring.default,
                  (expanded, red["operand_cache"], a_dec + 2 * t, p_dec + 2 * t, wm)))
    update = (red["anchor_weight"], red["partner_weight"], wm, red["first_bias"])
    cases.append(("relation_hidden_cache_update", ops.relation_hidden_cache_update.default,
                  (expanded.clone(), red["operand_cache"], a_dec, p_dec) + update[:2]
                  + (wm, red["first_bias"], pos)))
    cases.append(("relation_hidden_cache_update_ring",
                  ops.relation_hidden_cache_update_ring.default,
                  (expanded.clone(), red["operand_cache"], a_dec + t, p_dec + t) + update[:2]
                  + (wm, red["first_bias"], pos + t)))
    raw_dec = torch.randn(b, k, cfg.d_model, generator=g).to(device)
    raw_seq = torch.randn(b, t, k, cfg.d_model, generator=g).to(device)
    cases.append(("relation_norm_reduce", ops.relation_norm_reduce.default,
                  (raw_dec, scores_dec, red["norm_weight"], red["norm_bias"], pos, 1e-5)))
    cases.append(("relation_norm_reduce_seq", ops.relation_norm_reduce_seq.default,
                  (raw_seq, scores_seq, red["norm_weight"], red["norm_bias"], positions, 1e-5)))
    cases.append(("relation_reduce_fused_seq", ops.relation_reduce_fused_seq.default,
                  (expanded, red["operand_cache"], a_seq, p_seq, wm, red["second_weight"],
                   red["second_bias"], scores_seq, red["norm_weight"], red["norm_bias"],
                   positions, 1e-5)))
    rc = router_case(b, 447)
    rdev = {k_: v.to(device) for k_, v in rc.items()}
    router_args = (rdev["packed"][:, 384:448], rdev["packed"][:, 448:512]) + tuple(
        rdev[n] for n in ROUTER_BUFFERS) + (rdev["anchor_weight"], rdev["partner_weight"])
    cases.append(("router_cache_update", ops.router_cache_update.default,
                  router_args + (rdev["position"], 8)))
    cases.append(("router_cache_update_ring", ops.router_cache_update_ring.default,
                  tuple(x.clone() for x in router_args) + (rdev["position"] + 512, 8)))
    memory = torch.randn(b, 576, generator=g).to(device, torch.bfloat16)
    weight = (torch.randn(512, 576, generator=g) * 0.04).to(device, torch.bfloat16)
    cases.append(("packed_sparse_cache_projection", ops.packed_sparse_cache_projection.default,
                  (memory, weight)))
    caches = tuple(torch.zeros(b, t, w, device=device, dtype=torch.bfloat16)
                   for w in (64, 64, 128, 128))
    cases.append(("packed_projection_to_caches", ops.packed_projection_to_caches.default,
                  (memory, weight) + caches + (pos, False)))
    cases.append(("packed_projection_router_update",
                  ops.packed_projection_router_update.default,
                  (memory, weight) + tuple(c.clone() for c in caches) + (rdev["position"], False)
                  + tuple(rdev[n].clone() for n in ROUTER_BUFFERS)
                  + (rdev["anchor_weight"], rdev["partner_weight"], 8)))
    cases.append(("relation_linear", ops.relation_linear.default,
                  (red["operand_cache"], red["expanded_weight"], red["expanded_bias"], None)))
    cases.append(("relation_linear_out", ops.relation_linear_out.default,
                  (red["operand_cache"][:, 3], red["expanded_weight"], red["expanded_bias"],
                   expanded.clone()[:, 3])))
    d = cfg.d_model
    query_dec = torch.randn(b, d, generator=g).to(device, torch.bfloat16)
    query_seq = torch.randn(b, t, d, generator=g).to(device, torch.bfloat16)
    head = (torch.tensor(0.2, device=device), red["norm_weight"], red["norm_bias"], 1e-5)
    cases.append(("relation_norm_reduce_output", ops.relation_norm_reduce_output.default,
                  (raw_dec, scores_dec, red["norm_weight"], red["norm_bias"], pos, 1e-5,
                   query_dec) + head))
    cases.append(("relation_norm_reduce_output_seq", ops.relation_norm_reduce_output_seq.default,
                  (raw_seq, scores_seq, red["norm_weight"], red["norm_bias"], positions, 1e-5,
                   query_seq) + head))
    hidden_dec = torch.randn(b, k, red["second_weight"].shape[1], generator=g).to(
        device, red["second_weight"].dtype)
    cases.append(("relation_linear_norm_reduce_output",
                  ops.relation_linear_norm_reduce_output.default,
                  (hidden_dec, red["second_weight"], red["second_bias"], scores_dec,
                   red["norm_weight"], red["norm_bias"], pos, 1e-5, query_dec) + head))
    cases.append(("relation_hidden_linear_norm_reduce_output",
                  ops.relation_hidden_linear_norm_reduce_output.default,
                  (expanded, red["operand_cache"], a_dec, p_dec, wm, red["second_weight"],
                   red["second_bias"], scores_dec, red["norm_weight"], red["norm_bias"], pos,
                   1e-5, query_dec) + head + (False,)))
    slots, kk = 2, 3
    raw_multi = torch.randn(b, t, slots, kk, d, generator=g).to(device)
    scores_multi = torch.randn(b, t, slots, kk, generator=g).to(device)
    cases.append(("multi_relation_reduce_seq", ops.multi_relation_reduce_seq.default,
                  (raw_multi, scores_multi, red["norm_weight"], red["norm_bias"],
                   torch.zeros(slots, device=device), torch.tensor(-1.5, device=device),
                   query_seq, positions, 1e-5)))
    cases.append(("multi_relation_reduce_seq_out", ops.multi_relation_reduce_seq_out.default,
                  (raw_multi, scores_multi, red["norm_weight"], red["norm_bias"],
                   torch.zeros(slots, device=device), torch.tensor(-1.5, device=device),
                   query_seq, positions, 1e-5, None, torch.empty_like(query_seq),
                   torch.empty(query_seq.shape, device=device, dtype=torch.float32))))
    cases.append(("layer_norm", ops.layer_norm.default,
                  (query_seq, red["norm_weight"], red["norm_bias"], 1e-5)))
    keys = torch.randn(b, t, 64, generator=g).to(device, torch.bfloat16)
    cases.append(("block_statistics", ops.block_statistics.default, (keys, cfg.block_size)))
    return cases


OP_NAMES = ("relation_select_packed", "relation_select_packed_seq",
            "relation_select_packed_seq_expand", "relation_select_packed_expand_row", "relation_select_packed_ring", "anchor_select", "partner_topk",
            "multi_relation_select_seq", "relation_hidden_cached", "relation_hidden_cached_seq",
            "relation_hidden_cached_seq_out", "relation_hidden_linear_seq_out", "mfma_fragments",
            "relation_hidden_cached_ring", "relation_hidden_cache_update",
            "relation_hidden_cache_update_ring", "relation_norm_reduce",
            "relation_norm_reduce_seq", "relation_reduce_fused_seq", "router_cache_update",
            "router_cache_update_ring", "packed_sparse_cache_projection",
            "packed_projection_to_caches", "packed_projection_router_update",
            "relation_linear", "relation_linear_out",
            "relation_norm_reduce_output", "relation_norm_reduce_output_seq",
            "relation_linear_norm_reduce_output", "relation_hidden_linear_norm_reduce_output",
            "multi_relation_reduce_seq",
            "multi_relation_reduce_seq_out", "layer_norm", "block_statistics")


def test_opcheck_every_registered_op(device):
    cases = op_cases(device)
    assert tuple(name for name, _, _ in cases) == OP_NAMES
    registered = {n.split("::")[1] for n in torch._C._dispatch_get_all_op_names()
                  if n.startswith(("relation_lm::", "relationlex::"))}
    assert registered == set(OP_NAMES)
    for name, op, args in cases:
        print(f"opcheck {name}", flush=True)
        result = torch.library.opcheck(op, args)
        assert all(v == "SUCCESS" for v in result.values()), (name, result)
