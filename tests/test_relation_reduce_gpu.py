"""GPU parity of the relation reduce kernels and the dense projections.

Tolerances (written here, checked per test):
  fp32: relative error max|x - y| / max|y| <= 1e-5
  bf16: absolute error max|x - y| <= 2e-2
The reference's own checks (tests/test_relation_reduce_gpu.py:46-200 of the
reference: atol 2e-4, rtol 2e-5 against torch closed forms) are run as well.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import reduce as ored
from oracle import select as osel
from relation_lm.kernels.relation_reduce import (
    factor_relation_first_layer,
    relation_hidden_cache_update,
    relation_hidden_cached,
    relation_hidden_cached_seq,
    relation_linear,
    relation_linear_out,
    relation_norm_reduce,
    relation_norm_reduce_seq,
)
from relation_lm.kernels.relation_select import relation_select_packed_seq
from relation_lm.inference import pack_sparse_cache_projection_weights
from relation_lm.workloads import (
    CONFIGS,
    packed_projection_inputs,
    reduce_inputs,
    select_args,
    selection_inputs,
)

pytestmark = pytest.mark.gpu

FP32_REL = 1e-5
BF16_ABS = 2e-2


def host(t):
    return t.detach().float().cpu().numpy() if t.dtype.is_floating_point else t.cpu().numpy()


def rel_err(got, expected):
    got = np.asarray(got, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    return float(np.abs(got - expected).max() / max(np.abs(expected).max(), 1e-30))


def abs_err(got, expected):
    return float(np.abs(np.asarray(got, np.float64) - np.asarray(expected, np.float64)).max())


def _reference_context(raw, scores, norm_weight, norm_bias, position, eps):
    """tests/test_relation_reduce_gpu.py:21-43 of the reference."""
    relations = F.layer_norm(raw, (raw.size(-1),), norm_weight, norm_bias, eps)
    k_limit = int(math.ceil(math.log2(float(position.item()) + 2.0)))
    k_limit = max(1, min(k_limit, scores.size(1)))
    ranks = torch.arange(scores.size(1), device=scores.device)[None]
    active = torch.isfinite(scores) & ranks.lt(k_limit)
    safe = scores.masked_fill(~active, -1.0e4)
    weights = safe.softmax(-1) * active
    weights = weights / weights.sum(-1, keepdim=True).clamp_min(1.0e-9)
    return (weights.unsqueeze(-1) * relations).sum(1)


@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("k_out", [5, 8])
def test_reference_reduce_case(device, batch, k_out):
    g = torch.Generator().manual_seed(20260818 + batch)
    context, relation_dim, hidden_dim, output_dim = 512, 128, 2304, 576
    position = torch.tensor(context - 1, device=device, dtype=torch.long)
    operand_cache = torch.randn(batch, context, relation_dim, generator=g).to(device)
    first_weight = (torch.randn(hidden_dim, 4 * relation_dim, generator=g) * 0.02).to(device)
    first_bias = (torch.randn(hidden_dim, generator=g) * 0.01).to(device)
    factors = factor_relation_first_layer(first_weight, first_bias, relation_dim)
    expanded_cache = relation_linear(operand_cache, factors.expanded_weight, factors.expanded_bias)
    torch.cuda.synchronize()
    exp_expanded = ored.linear(host(operand_cache), host(factors.expanded_weight),
                               host(factors.expanded_bias))
    assert rel_err(host(expanded_cache), exp_expanded) <= FP32_REL

    anchor_index = torch.randint(0, context, (batch,), generator=g, dtype=torch.int32).to(device)
    partner_index = torch.randint(0, context, (batch, k_out), generator=g,
                                  dtype=torch.int32).to(device)
    anchor_index[0] = position.to(torch.int32)
    partner_index[:, 0] = position.to(torch.int32)

    cached_hidden = relation_hidden_cached(expanded_cache, operand_cache, anchor_index,
                                           partner_index, factors.product_weight)
    torch.cuda.synchronize()
    expected_hidden = ored.relation_hidden_cached(host(expanded_cache), host(operand_cache),
                                                  host(anchor_index), host(partner_index),
                                                  host(factors.product_weight))
    assert rel_err(host(cached_hidden), expected_hidden) <= FP32_REL

    # the reference's closed form (torch, fp32 "highest")
    torch.backends.cuda.matmul.allow_tf32 = False
    b = torch.arange(batch, device=device)
    anchor = operand_cache[b, anchor_index.long()]
    partner = operand_cache[b[:, None], partner_index.long()]
    anchor_expanded = anchor[:, None].expand(-1, k_out, -1)
    features = torch.cat((anchor_expanded, partner, anchor_expanded * partner,
                          anchor_expanded - partner), dim=-1)
    reference_hidden = F.gelu(F.linear(features.double(), first_weight.double(),
                                       first_bias.double())).float()
    assert torch.allclose(cached_hidden, reference_hidden, atol=2.0e-4, rtol=2.0e-5)

    mutable_cache = expanded_cache.clone()
    mutable_cache[:, position.item()].zero_()
    updated_hidden = relation_hidden_cache_update(
        mutable_cache, operand_cache, anchor_index, partner_index, factors.anchor_weight,
        factors.partner_weight, factors.product_weight, factors.first_bias, position)
    torch.cuda.synchronize()
    assert rel_err(host(updated_hidden), expected_hidden) <= FP32_REL
    assert rel_err(host(mutable_cache[:, 511]), exp_expanded[:, 511]) <= FP32_REL
    untouched = torch.ones(context, dtype=torch.bool)
    untouched[511] = False
    assert torch.equal(mutable_cache[:, untouched], expanded_cache[:, untouched])

    second_weight = (torch.randn(output_dim, hidden_dim, generator=g) * 0.02).to(device)
    second_bias = (torch.randn(output_dim, generator=g) * 0.01).to(device)
    norm_weight = (torch.randn(output_dim, generator=g) * 0.05 + 1.0).to(device)
    norm_bias = (torch.randn(output_dim, generator=g) * 0.01).to(device)
    raw = relation_linear(cached_hidden, second_weight, second_bias)
    torch.cuda.synchronize()
    exp_raw = ored.linear(host(cached_hidden), host(second_weight), host(second_bias))
    assert rel_err(host(raw), exp_raw) <= FP32_REL
    scores = torch.randn(batch, k_out, generator=g).to(device)
    scores[:, -1] = -torch.inf
    context_out = relation_norm_reduce(raw, scores, norm_weight, norm_bias, position, 1e-5)
    torch.cuda.synchronize()
    expected = ored.relation_norm_reduce(host(raw), host(scores), host(norm_weight),
                                         host(norm_bias), 511, 1e-5)
    assert rel_err(host(context_out), expected) <= FP32_REL
    reference = _reference_context(raw, scores, norm_weight, norm_bias, position, 1e-5)
    assert torch.allclose(context_out, reference, atol=2.0e-4, rtol=2.0e-5)


@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("k_out", [5, 6, 7])
@pytest.mark.parametrize("position", [0, 1, 6, 511])
def test_norm_reduce_non_power_of_two_budget(device, batch, k_out, position):
    g = torch.Generator().manual_seed(20260830 + 10 * batch + k_out)
    raw = torch.randn(batch, k_out, 576, generator=g).to(device)
    scores = torch.randn(batch, k_out, generator=g).to(device)
    scores[:, -1] = -torch.inf
    norm_weight = (torch.randn(576, generator=g) * 0.05 + 1.0).to(device)
    norm_bias = (torch.randn(576, generator=g) * 0.01).to(device)
    pos = torch.tensor(position, device=device, dtype=torch.long)
    actual = relation_norm_reduce(raw, scores, norm_weight, norm_bias, pos, 1e-5)
    torch.cuda.synchronize()
    assert torch.isfinite(actual).all()
    expected = ored.relation_norm_reduce(host(raw), host(scores), host(norm_weight),
                                         host(norm_bias), position, 1e-5)
    assert rel_err(host(actual), expected) <= FP32_REL


@pytest.mark.parametrize("width", [7, 100, 256, 512, 1000, 2048])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_norm_reduce_widths(device, width, dtype):
    """Vector (width % 4 == 0) and scalar column layouts, fp32 and bf16 raw rows, K=12."""
    g = torch.Generator().manual_seed(9000 + width)
    raw = torch.randn(5, 12, width, generator=g).to(dtype)
    scores = torch.randn(5, 12, generator=g)
    scores[1, 3:] = -torch.inf
    norm_weight = torch.randn(width, generator=g) * 0.05 + 1.0
    norm_bias = torch.randn(width, generator=g) * 0.01
    pos = torch.tensor(300, device=device)
    actual = relation_norm_reduce(raw.to(device), scores.to(device), norm_weight.to(device),
                                  norm_bias.to(device), pos, 1e-5)
    torch.cuda.synchronize()
    expected = ored.relation_norm_reduce(raw.float().numpy(), scores.numpy(), norm_weight.numpy(),
                                         norm_bias.numpy(), 300, 1e-5)
    assert rel_err(host(actual), expected) <= FP32_REL


def test_hidden_guards_out_of_range_indices(device):
    """Sentinel partner indices (t-LOCAL+1 < 0) read zero rows, never out of bounds."""
    cfg = CONFIGS["cfg1"]
    red = reduce_inputs(cfg, device=device)
    expanded = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])
    anchor = torch.tensor([3], device=device, dtype=torch.int32)
    partner = torch.tensor([[2, -31, -5, 127, 128, 1 << 20, 0, 1]], device=device,
                           dtype=torch.int32)
    got = relation_hidden_cached(expanded, red["operand_cache"], anchor, partner,
                                 red["product_weight"])
    torch.cuda.synchronize()
    expected = ored.relation_hidden_cached(host(expanded), host(red["operand_cache"]),
                                           host(anchor), host(partner),
                                           host(red["product_weight"]))
    assert rel_err(host(got), expected) <= FP32_REL


@pytest.mark.parametrize("batch", [1, 8])
def test_bf16_decode_reduce(device, batch):
    cfg = CONFIGS["cfg3"]
    red = reduce_inputs(cfg, device=device)
    operand = red["operand_cache"][:batch].contiguous()
    expanded = relation_linear(operand, red["expanded_weight"], red["expanded_bias"])
    torch.cuda.synchronize()
    exp_expanded = ored.linear(host(operand), host(red["expanded_weight"]),
                               host(red["expanded_bias"]))
    assert abs_err(host(expanded), exp_expanded) <= BF16_ABS
    g = torch.Generator().manual_seed(77 + batch)
    anchor = torch.randint(0, 512, (batch,), generator=g).to(device)
    partner = torch.randint(0, 512, (batch, 8), generator=g).to(device)
    anchor[0] = 511
    partner[:, 1] = 511
    position = torch.tensor(511, device=device)
    hidden = relation_hidden_cached(expanded, operand, anchor, partner, red["product_weight"])
    torch.cuda.synchronize()
    exp_hidden = ored.relation_hidden_cached(host(expanded), host(operand), host(anchor),
                                             host(partner), host(red["product_weight"]))
    assert abs_err(host(hidden), exp_hidden) <= BF16_ABS
    # Exact bf16 products (hi/lo split on the matrix cores) with fp32 accumulation:
    # the hidden agrees with the float64 oracle to fp32 precision, not just bf16's.
    assert rel_err(host(hidden), exp_hidden) <= FP32_REL
    mutable = expanded.clone()
    mutable[:, 511] = 0
    updated = relation_hidden_cache_update(mutable, operand, anchor, partner,
                                           red["anchor_weight"], red["partner_weight"],
                                           red["product_weight"], red["expanded_bias"][:2304],
                                           position)
    torch.cuda.synchronize()
    exp_updated, exp_cache = ored.relation_hidden_cache_update(
        host(mutable), host(operand), host(anchor), host(partner), host(red["anchor_weight"]),
        host(red["partner_weight"]), host(red["product_weight"]),
        host(red["expanded_bias"][:2304]), 511, cache_dtype="bfloat16")
    assert abs_err(host(updated), exp_updated) <= BF16_ABS
    assert rel_err(host(updated), exp_updated) <= FP32_REL
    assert abs_err(host(mutable), exp_cache) <= BF16_ABS
    raw = relation_linear(hidden, red["second_weight"], red["second_bias"],
                          out_dtype=torch.float32)
    torch.cuda.synchronize()
    exp_raw = ored.linear(host(hidden), host(red["second_weight"]), host(red["second_bias"]))
    assert abs_err(host(raw), exp_raw) <= BF16_ABS
    scores = torch.randn(batch, 8, generator=g).to(device)
    ctx = relation_norm_reduce(raw, scores, red["norm_weight"], red["norm_bias"], position, 1e-5)
    torch.cuda.synchronize()
    exp_ctx = ored.relation_norm_reduce(host(raw), host(scores), host(red["norm_weight"]),
                                        host(red["norm_bias"]), 511, 1e-5)
    assert abs_err(host(ctx), exp_ctx) <= BF16_ABS


def test_sequence_chain_cfg2(device):
    """Full cfg2 prefill chain: select -> hidden -> second linear -> norm-reduce."""
    cfg = CONFIGS["cfg2"]
    sel_in = selection_inputs(cfg, device=device)
    red = reduce_inputs(cfg, device=device)
    expanded = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])
    a, s, p, ps = relation_select_packed_seq(*select_args(sel_in, cfg))
    hidden = relation_hidden_cached_seq(expanded, red["operand_cache"], a, p,
                                        red["product_weight"])
    raw = relation_linear(hidden, red["second_weight"], red["second_bias"],
                          out_dtype=torch.float32)
    ctx = relation_norm_reduce_seq(raw, ps, red["norm_weight"], red["norm_bias"],
                                   sel_in["positions"], 1e-5)
    torch.cuda.synchronize()
    hs = {k: host(v) for k, v in sel_in.items()}
    ea, es, ep, eps_ = osel.relation_select_packed_seq(
        *[hs[k] for k in ("anchor_query", "anchor_keys", "anchor_router_query",
                          "anchor_block_mean", "anchor_block_std", "anchor_gamma",
                          "anchor_bias", "partner_base", "partner_anchor_cache", "partner_keys",
                          "partner_block_mean", "partner_block_std", "partner_gamma",
                          "partner_bias")],
        hs["positions"], cfg.local_window, cfg.top_blocks, cfg.k_out, False)
    assert np.array_equal(host(a), ea) and np.array_equal(host(p), ep)
    assert np.array_equal(host(ps), eps_)
    # the reduce on the first 96 queries of row 0 (the oracle is float64 numpy)
    rows = slice(0, 1)
    exp_expanded = ored.linear(host(red["operand_cache"]), host(red["expanded_weight"]),
                               host(red["expanded_bias"]))
    assert abs_err(host(expanded), exp_expanded) <= BF16_ABS
    exp_hidden = ored.relation_hidden_cached_seq(host(expanded)[rows],
                                                 host(red["operand_cache"])[rows],
                                                 ea[rows][:, :96], ep[rows][:, :96],
                                                 host(red["product_weight"]))
    assert abs_err(host(hidden)[rows][:, :96], exp_hidden) <= BF16_ABS
    assert rel_err(host(hidden)[rows][:, :96], exp_hidden) <= FP32_REL
    exp_raw = ored.linear(host(hidden)[rows][:, :96], host(red["second_weight"]),
                          host(red["second_bias"]))
    assert abs_err(host(raw)[rows][:, :96], exp_raw) <= BF16_ABS
    exp_ctx = ored.relation_norm_reduce_seq(host(raw)[:, :96], eps_[:, :96],
                                            host(red["norm_weight"]), host(red["norm_bias"]),
                                            np.arange(96), 1e-5)
    assert abs_err(host(ctx)[:, :96], exp_ctx) <= BF16_ABS
    assert torch.isfinite(ctx).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch", [1, 8])
def test_packed_projection_matches_separate_linears(device, dtype, batch):
    """tests/test_packed_cache_projection.py:10-25 of the reference, on the MFMA kernel."""
    cfg = CONFIGS["cfg3"]
    memory, weights = packed_projection_inputs(cfg, device=device)
    memory = memory[:batch].to(dtype).contiguous()
    weights = tuple(w.to(dtype) for w in weights)
    projection = pack_sparse_cache_projection_weights(weights)
    actual = projection.project(memory)
    torch.cuda.synchronize()
    assert projection.input_width == 576 and projection.output_width == 512
    for w, got in zip(weights, actual, strict=True):
        expected = ored.linear(host(memory), host(w))
        if dtype == torch.float32:
            assert rel_err(host(got), expected) <= FP32_REL
        else:
            assert got.dtype == torch.bfloat16
            assert abs_err(host(got), expected) <= BF16_ABS
    assert tuple(projection.project_dict(memory)) == projection.names


@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("position,ring", [(0, False), (300, False), (511, False), (512, False),
                                           (-1, False), (300, True), (1000, True), (4095, True)])
def test_projection_to_caches(device, batch, position, ring):
    """project_into == project + cache[:, row] = segment (row = position, or position % T)."""
    cfg = CONFIGS["cfg3"]
    memory, weights = packed_projection_inputs(cfg, device=device)
    memory = memory[:batch].contiguous()
    projection = pack_sparse_cache_projection_weights(weights)
    g = torch.Generator().manual_seed(31 + position)
    caches = [torch.randn(batch, 512, w, generator=g).to(torch.bfloat16).to(device)
              for w in (64, 64, 128, 128)]
    expected = [c.clone() for c in caches]
    pos = torch.tensor(position, device=device)
    got = projection.project_into(memory, *caches, pos, ring=ring)
    ref = projection.project(memory)
    torch.cuda.synchronize()
    row = position % 512 if ring else position
    if 0 <= position and (ring or position < 512):
        for c, seg in zip(expected, ref[:4]):
            c[:, row] = seg
    for gp, rp in zip(got, ref):
        assert torch.equal(gp, rp)
    for c, e in zip(caches, expected):
        assert torch.equal(c, e)


def test_projection_to_caches_rejects_mismatched_widths(device):
    cfg = CONFIGS["cfg3"]
    memory, weights = packed_projection_inputs(cfg, device=device)
    projection = pack_sparse_cache_projection_weights(weights)
    caches = [torch.zeros(cfg.batch, 512, w, dtype=torch.bfloat16, device=device)
              for w in (64, 64, 128, 64)]
    with pytest.raises(ValueError, match="cache widths"):
        projection.project_into(memory, *caches, torch.tensor(3, device=device))
    caches[3] = torch.zeros(cfg.batch, 500, 128, dtype=torch.bfloat16, device=device)
    with pytest.raises(RuntimeError, match="power-of-two"):
        projection.project_into(memory, *caches, torch.tensor(3, device=device), ring=True)


@pytest.mark.parametrize("m,n,k", [(1, 512, 576), (8, 4608, 128), (100, 72, 40), (4096, 1024, 128),
                                   (8, 576, 2304), (64, 576, 2304), (65, 200, 96), (8, 24, 40),
                                   (33, 130, 72), (1000, 300, 520), (129, 40, 32), (300, 136, 64)])
def test_linear_shapes(device, m, n, k):
    g = torch.Generator().manual_seed(m * 7 + n)
    x = torch.randn(m, k, generator=g)
    w = torch.randn(n, k, generator=g) * k ** -0.5
    bias = torch.randn(n, generator=g) * 0.1
    got32 = relation_linear(x.to(device), w.to(device), bias.to(device))
    x16, w16 = x.bfloat16(), w.bfloat16()
    got16 = relation_linear(x16.to(device), w16.to(device), bias.to(device),
                            out_dtype=torch.float32)
    gotmix = relation_linear(x.to(device), w16.to(device), None, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert rel_err(host(got32), ored.linear(x.numpy(), w.numpy(), bias.numpy())) <= FP32_REL
    exp16 = ored.linear(x16.float().numpy(), w16.float().numpy(), bias.numpy())
    assert rel_err(host(got16), exp16) <= FP32_REL
    expmix = ored.linear(x16.float().numpy(), w16.float().numpy())
    assert rel_err(host(gotmix), expmix) <= FP32_REL


@pytest.mark.parametrize("bias_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m,n,k", [(4096, 1024, 128), (200, 264, 64), (77, 48, 32), (70, 77, 96)])
def test_linear_small_k_bf16_out(device, m, n, k, bias_dtype):
    """K <= 128 takes the one-round-trip small-K kernel; bf16 output as the expanded cache.
    An odd N ends the 16-bit bias mid-dword and leaves partial edge tiles."""
    g = torch.Generator().manual_seed(m + 3 * n + k)
    x = torch.randn(m, k, generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) * k ** -0.5).bfloat16()
    bias = (torch.randn(n, generator=g) * 0.1).to(bias_dtype)
    got = relation_linear(x.to(device), w.to(device), bias.to(device))
    torch.cuda.synchronize()
    assert got.dtype == torch.bfloat16 and got.shape == (m, n)
    expected = ored.linear(x.float().numpy(), w.float().numpy(), bias.float().numpy())
    assert abs_err(host(got), expected) <= BF16_ABS
    assert abs_err(host(got), ored.round_to(expected, "bfloat16")) <= 2 ** -7 * max(
        1.0, float(np.abs(expected).max()))


def test_graph_replay_matches_eager(device):
    """Decode chain captured in a HIP graph; every replay equals the eager result."""
    cfg = CONFIGS["cfg3"]
    sel_in = selection_inputs(cfg, queries=1, device=device)
    red = reduce_inputs(cfg, device=device)
    from relation_lm.kernels.relation_select import relation_select_packed

    expanded = relation_linear(red["operand_cache"], red["expanded_weight"], red["expanded_bias"])

    def step():
        a, s, p, ps = relation_select_packed(*select_args(sel_in, cfg))
        hidden = relation_hidden_cached(expanded, red["operand_cache"], a, p,
                                        red["product_weight"])
        raw = relation_linear(hidden, red["second_weight"], red["second_bias"],
                              out_dtype=torch.float32)
        return relation_norm_reduce(raw, ps, red["norm_weight"], red["norm_bias"],
                                    sel_in["position"], 1e-5)

    eager = step().clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        other = step()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(other, eager)


@pytest.mark.parametrize("m", [8, 300])
def test_linear_row_strided_input(device, m):
    """A cache column (cache[:, t], row stride T*R) goes in without a copy."""
    g = torch.Generator().manual_seed(4242 + m)
    cache = torch.randn(m, 6, 128, generator=g).bfloat16()
    w = (torch.randn(256, 128, generator=g) * 128 ** -0.5).bfloat16()
    bias = torch.randn(256, generator=g) * 0.1
    column = cache.to(device)[:, 3]
    assert not column.is_contiguous()
    got = relation_linear(column, w.to(device), bias.to(device), out_dtype=torch.float32)
    torch.cuda.synchronize()
    expected = ored.linear(cache[:, 3].float().numpy(), w.float().numpy(), bias.numpy())
    assert rel_err(host(got), expected) <= FP32_REL


def test_linear_second_linear_shape(device):
    """cfg2's second linear: fp32 hidden x bf16 weight -> fp32, checked on a row sample."""
    g = torch.Generator().manual_seed(777)
    hidden = torch.randn(32768, 512, generator=g)
    w = (torch.randn(512, 512, generator=g) * 512 ** -0.5).bfloat16()
    bias = (torch.randn(512, generator=g) * 0.01).bfloat16()
    got = relation_linear(hidden.to(device), w.to(device), bias.to(device),
                          out_dtype=torch.float32)
    torch.cuda.synchronize()
    rows = torch.randperm(32768, generator=g)[:512].sort().values
    x16 = hidden[rows].bfloat16().float().numpy()
    expected = ored.linear(x16, w.float().numpy(), bias.float().numpy())
    assert rel_err(host(got)[rows.numpy()], expected) <= FP32_REL


@pytest.mark.parametrize("dtype,batch", [(torch.bfloat16, 8), (torch.bfloat16, 1), (torch.float32, 3)])
def test_linear_out_into_cache_column(device, dtype, batch):
    """relation_linear_out writes a cache column (rows strided by the cache row
    pitch) in place: the decode step's separate expanded-row update.  Equal to
    relation_linear's result; every other cache row is untouched."""
    g = torch.Generator().manual_seed(41 + batch)
    operand = torch.randn(batch, 64, 128, generator=g).to(device=device, dtype=dtype)
    weight = (torch.randn(2 * 2304, 128, generator=g) * 0.08).to(device=device, dtype=dtype)
    bias = torch.randn(2 * 2304, generator=g).to(device=device, dtype=dtype)
    cache = torch.randn(batch, 64, 2 * 2304, generator=g).to(device=device, dtype=dtype)
    before = cache.clone()
    t = 37
    relation_linear_out(operand[:, t], weight, bias, cache[:, t])
    expected = relation_linear(operand[:, t].contiguous(), weight, bias)
    torch.cuda.synchronize()
    assert torch.equal(cache[:, t], expected)
    keep = torch.ones(64, dtype=torch.bool)
    keep[t] = False
    assert torch.equal(cache[:, keep], before[:, keep])


@pytest.mark.parametrize("hidden_dim,relation_dim", [(3072, 128), (512, 64)])
def test_hidden_seq_out_bf16_feeds_the_linear_unchanged(device, hidden_dim, relation_dim):
    """relation_hidden_cached_seq_out with a bf16 out: every element is the fp32
    hidden rounded to nearest even, so a bf16 second Linear (which rounds its
    fp32 input the same way before the products) gives bit-identical raw rows
    from either hidden -- the multi-anchor relation MLP stores bf16."""
    from relation_lm.kernels.relation_reduce import relation_hidden_cached_seq_out
    g = torch.Generator().manual_seed(hidden_dim)
    b, t, k = 1, 256, 6
    operand = torch.randn(b, t, relation_dim, generator=g).to(device, torch.bfloat16)
    expanded = torch.randn(b, t, 2 * hidden_dim, generator=g).to(device, torch.bfloat16)
    wm = (torch.randn(hidden_dim, relation_dim, generator=g) * relation_dim ** -0.5).to(
        device, torch.bfloat16)
    a = torch.randint(0, t, (b, 4 * t), generator=g).to(device)
    p = torch.randint(0, t, (b, 4 * t, k), generator=g).to(device)
    w2 = (torch.randn(768, hidden_dim, generator=g) * hidden_dim ** -0.5).to(device, torch.bfloat16)
    b2 = torch.randn(768, generator=g).to(device, torch.bfloat16)
    h32 = relation_hidden_cached_seq(expanded, operand, a, p, wm)
    h16 = torch.empty(h32.shape, dtype=torch.bfloat16, device=device)
    relation_hidden_cached_seq_out(expanded, operand, a, p, wm, h16)
    h32b = torch.empty_like(h32)
    relation_hidden_cached_seq_out(expanded, operand, a, p, wm, h32b)
    raw32 = relation_linear(h32, w2, b2, out_dtype=torch.float32)
    raw16 = relation_linear(h16, w2, b2, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(h32b, h32)
    assert torch.equal(h16, h32.to(torch.bfloat16))
    assert torch.equal(raw16, raw32)


@pytest.mark.parametrize("b,t,tq,k,r,h,out_dtype", [
    (2, 256, 256, 8, 128, 768, torch.float32),    # 4096 rows, a partial column tile
    (1, 512, 600, 7, 64, 520, torch.bfloat16),    # 4200 rows (partial row tile), R = 64
    (1, 512, 600, 7, 64, 520, torch.float32),
    (1, 4096, 1024, 6, 128, 3072, torch.bfloat16),  # the multi-anchor block's widths
])
def test_hidden_seq_tile_path(device, b, t, tq, k, r, h, out_dtype):
    """relation_hidden_cached_seq(_out) with many rows (the 128 x 256 tile kernel)
    against the float64 oracle: fp32 within 1e-5 relative, bf16 within that
    plus one rounding of the element.  Some partner indices are out of
    range (the selection's negative sentinel, and past the cache), which read
    as zero rows."""
    from relation_lm.kernels.relation_reduce import relation_hidden_cached_seq_out
    g = torch.Generator().manual_seed(b * 1000 + tq + k + r + h)
    operand = torch.randn(b, t, r, generator=g).to(torch.bfloat16)
    expanded = torch.randn(b, t, 2 * h, generator=g).to(torch.bfloat16)
    wm = (torch.randn(h, r, generator=g) * r ** -0.5).to(torch.bfloat16)
    anchor = torch.randint(0, t, (b, tq), generator=g)
    partner = torch.randint(0, t, (b, tq, k), generator=g)
    partner[:, ::17, 0] = -3          # sentinel of an exhausted partner slot
    partner[:, 5::23, 1] = t + 2      # past the cache
    print(f"hidden tile path B={b} Tq={tq} K={k} R={r} H={h} {out_dtype}", flush=True)
    out = torch.empty(b, tq, k, h, dtype=out_dtype, device=device)
    relation_hidden_cached_seq_out(expanded.to(device), operand.to(device), anchor.to(device),
                                   partner.to(device), wm.to(device), out)
    torch.cuda.synchronize()
    exp = ored.relation_hidden_cached_seq(host(expanded), host(operand), host(anchor),
                                          host(partner), host(wm))
    got = host(out)
    # fp32: the relative bound; bf16: one rounding of the element on top of it
    # (the fp32 floor covers the GELU tail, where outputs of ~1e-7 carry the
    # erf approximation's absolute error).
    bound = FP32_REL * np.abs(exp).max()
    if out_dtype != torch.float32:
        bound = bound + np.exp2(np.floor(np.log2(np.maximum(np.abs(exp), 1e-30))) - 7)
    excess = np.abs(got - exp) - bound
    worst = np.unravel_index(np.argmax(excess), excess.shape)
    assert excess[worst] <= 0, (worst, float(got[worst]), float(exp[worst]),
                                int((excess > 0).sum()))
