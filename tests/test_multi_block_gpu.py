"""GPU parity of the multi-anchor relation block (RelationBlockStack at cfg5).

* relation_lm::multi_relation_reduce_seq / layer_norm / block_statistics against
  oracle/multi_block.py (float64) on random inputs, fp32 and bf16;
* the routed HIP block against the reference block's dense structure
  (oracle/dense_block.py, float64 CPU) where routing keeps every causal position
  (T <= local window): same anchors and partner sets, same output within fp32
  rounding;
* with routing active, the block's selection against the selection oracle
  (bit-exact) and its relation / mixing steps against the factorized path
  oracle (relate_rows) on the block's own caches;
* one layer and the 4-layer stack at the full cfg5 shape (B=4, T=4096, d=768,
  4 slots x K=6, block 64, local 128, top 8, bf16): selection bit-exact and the
  fp32 relation context within 5e-3 of the oracle on 256 sampled queries per
  layer, and on every query of one batch row for one layer.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import multi_block as omb
from oracle import select as osel
from relation_lm.models import MultiRelationBlockConfig, RelationBlockStack
from relation_lm.models.multi_relation_blocks import MultiAnchorRelationBlock
from oracle.dense_block import DenseBlock

pytestmark = pytest.mark.gpu
ops = torch.ops.relation_lm


def host(t):
    return t.detach().float().cpu().numpy() if t.dtype.is_floating_point else t.cpu().numpy()


def bf16_round(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


# ---------------------------------------------------------------------------
# Ops
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape", [(2, 37, 4, 6, 768), (1, 9, 3, 5, 12), (2, 5, 1, 1, 64),
                                   (1, 6, 8, 8, 256)])
@pytest.mark.parametrize("raw_dtype,hid_dtype", [(torch.float32, torch.float32),
                                                 (torch.float32, torch.bfloat16),
                                                 (torch.bfloat16, torch.bfloat16)])
@pytest.mark.parametrize("pos2d", [False, True])
def test_multi_reduce_op(device, shape, raw_dtype, hid_dtype, pos2d):
    b, tq, s, k, d = shape
    g = torch.Generator().manual_seed(b * 1000 + tq * 10 + s + k + d)
    raw = (torch.randn(shape, generator=g) * 2 + 0.5).to(raw_dtype)
    scores = torch.randn(b, tq, s, k, generator=g)
    scores[torch.rand(scores.shape, generator=g) < 0.25] = -torch.inf
    scores[0, min(1, tq - 1), 0] = -torch.inf  # a slot with no active partner
    w = 1 + 0.1 * torch.randn(d, generator=g)
    bias = 0.1 * torch.randn(d, generator=g)
    logits = torch.randn(s, generator=g)
    gate = torch.tensor(0.7)
    hidden = torch.randn(b, tq, d, generator=g).to(hid_dtype)
    if pos2d:
        pos = torch.randint(0, 3 * s, (b, tq), generator=g, dtype=torch.int32)
    else:
        pos = torch.arange(tq)
    dev = lambda t: t.to(device)
    got = ops.multi_relation_reduce_seq(dev(raw), dev(scores), dev(w), dev(bias), dev(logits),
                                        dev(gate), dev(hidden), dev(pos), 1e-5)
    torch.cuda.synchronize()
    expected, _ = omb.multi_relation_reduce_seq(host(raw), host(scores), host(w), host(bias),
                                                host(logits), 0.7, host(hidden), host(pos), 1e-5)
    got = host(got)
    assert got.shape == expected.shape
    if hid_dtype == torch.float32:
        np.testing.assert_allclose(got, expected, rtol=0, atol=3e-5)
    else:  # the output rounds once to bf16: within one bf16 ulp of the exact value
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(expected), 1e-30))) - 7)
        assert (np.abs(got - expected) <= ulp + 1e-5).all()


@pytest.mark.parametrize("bias_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d", [768, 200])
def test_multi_reduce_raw_bias(device, bias_dtype, d):
    # raw_bias is added (fp32) to every raw row as the rows are loaded: the
    # result equals the op on raw + bias bit for bit.  d = 200 leaves lanes of
    # the last column group past the row (they must stay zero).
    g = torch.Generator().manual_seed(77)
    b, tq, s, k = 2, 9, 4, 6
    raw = torch.randn(b, tq, s, k, d, generator=g)
    scores = torch.randn(b, tq, s, k, generator=g)
    rb = (0.5 * torch.randn(d, generator=g)).to(bias_dtype)
    w = 1 + 0.1 * torch.randn(d, generator=g)
    nb = 0.1 * torch.randn(d, generator=g)
    args = [t.to(device) for t in (scores, w, nb, torch.randn(s, generator=g), torch.tensor(0.3),
                                   torch.randn(b, tq, d, generator=g).to(torch.bfloat16),
                                   torch.arange(tq))]
    got = ops.multi_relation_reduce_seq(raw.to(device), *args, 1e-5, rb.to(device))
    ref = ops.multi_relation_reduce_seq((raw + rb.float()).to(device), *args, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("shape,dtype", [((3, 5, 768), torch.float32), ((3, 5, 768), torch.bfloat16),
                                         ((7, 64), torch.float32), ((2, 3, 4, 2048), torch.bfloat16),
                                         ((11, 12), torch.float32)])
def test_layer_norm_op(device, shape, dtype):
    g = torch.Generator().manual_seed(len(shape) * 100 + shape[-1])
    x = (torch.randn(shape, generator=g) * 3 + 1).to(dtype)
    w = 1 + 0.1 * torch.randn(shape[-1], generator=g)
    b = 0.1 * torch.randn(shape[-1], generator=g)
    got = host(ops.layer_norm(x.to(device), w.to(device), b.to(device), 1e-5))
    expected = omb.layer_norm(host(x), host(w), host(b), 1e-5)
    if dtype == torch.float32:
        np.testing.assert_allclose(got, expected, rtol=0, atol=2e-5)
    else:
        np.testing.assert_allclose(got, bf16_round(expected), rtol=0, atol=0.02)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_statistics_op(device, dtype):
    g = torch.Generator().manual_seed(3)
    keys = (torch.randn(2, 256, 64, generator=g) * 2 + 0.3).to(dtype)
    mean, std = ops.block_statistics(keys.to(device), 32)
    em, es = omb.block_statistics(host(keys), 32)
    np.testing.assert_allclose(host(mean), em, rtol=0, atol=1e-5)
    np.testing.assert_allclose(host(std), es, rtol=0, atol=1e-5)


# ---------------------------------------------------------------------------
# Block
# ---------------------------------------------------------------------------

def randomize(module, seed):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in module.named_parameters():
            if "norm" in name or name.startswith("relation_mlp.3"):
                p.copy_((1.0 if name.endswith("weight") else 0.0)
                        + 0.1 * torch.randn(p.shape, generator=g))
            elif p.dim() >= 2:
                p.copy_(torch.randn(p.shape, generator=g) / np.sqrt(p.shape[-1]))
            else:
                p.copy_(0.5 * torch.randn(p.shape, generator=g))


def dense_copy(block: MultiAnchorRelationBlock) -> DenseBlock:
    cfg = block.cfg
    dense = DenseBlock(cfg.d_model, cfg.gate_dim, cfg.relation_dim, cfg.anchors_per_block,
                       cfg.partners_per_anchor, cfg.ff_mult).double()
    own = {k: v.detach().double().cpu() for k, v in block.state_dict().items()}
    missing = [k for k in dense.state_dict() if k not in own]
    assert not missing, missing
    dense.load_state_dict({k: own[k] for k in dense.state_dict()})
    return dense


def small_cfg(**kw):
    base = dict(d_model=64, gate_dim=64, relation_dim=32, ff_mult=2, anchors_per_block=4,
                partners_per_anchor=6, block_size=16, local_window=64, top_blocks=2)
    base.update(kw)
    return MultiRelationBlockConfig(**base)


@pytest.mark.parametrize("seed", [0, 1])
def test_block_equals_dense_reference_without_routing(device, seed):
    """T <= local window: every causal position is a candidate, so the routed
    block computes the reference block's dense function."""
    cfg = small_cfg()
    block = MultiAnchorRelationBlock(cfg)
    randomize(block, 50 + seed)
    dense = dense_copy(block)
    block = block.to(device)
    g = torch.Generator().manual_seed(60 + seed)
    hidden = torch.randn(2, 64, cfg.d_model, generator=g)
    memory = torch.randn(2, 64, cfg.d_model, generator=g)
    with torch.no_grad():
        out, diag = block(hidden.to(device), memory.to(device))
        ref, rdiag = dense(hidden.double(), memory.double())
    active = host(diag["anchor_active"])
    np.testing.assert_array_equal(np.where(active, host(diag["anchor_index"]), 0),
                                  np.where(active, rdiag["anchor_index"].numpy(), 0))
    finite = np.isfinite(rdiag["top"].numpy())
    assert (finite == host(diag["partner_active"])).all()
    got_sets = np.sort(np.where(finite, host(diag["partner_index"]), -1), axis=-1)
    ref_sets = np.sort(np.where(finite, rdiag["partner_index"].numpy(), -1), axis=-1)
    np.testing.assert_array_equal(got_sets, ref_sets)
    np.testing.assert_allclose(host(out), ref.numpy(), rtol=0, atol=2e-4)


def check_layer_on_rows(block, x, memory, sel, y, rows_b, rows_t, hidden_dtype, atol):
    """Selection of the sampled queries bit-exact against the selection oracle fed
    the block's own selection inputs; relation / mixing against relate_rows."""
    args = sel["select_args"]
    take = lambda t: t[rows_b, rows_t]
    query_side = {0, 2, 7}  # anchor_query, anchor_router_query, partner_base
    qargs = []
    for i, a in enumerate(args[:14]):
        if i in query_side:
            v = host(take(a))
            qargs.append(v[:, None] if v.ndim >= 1 else v)
        else:
            qargs.append(host(a))
    # One query per batch row slot: regroup the samples as [B, n] queries.
    batch = x.shape[0]
    n = len(rows_b) // batch
    order = np.argsort(rows_b, kind="stable")
    rb, rt = rows_b[order], rows_t[order]
    qargs = [v[order].reshape((batch, n) + v.shape[2:]) if i in query_side else v
             for i, v in enumerate(qargs)]
    positions = rt.reshape(batch, n)
    cfg = block.cfg
    exp = osel.multi_relation_select_seq(*qargs, positions, cfg.local_window, cfg.top_blocks,
                                         cfg.partners_per_anchor, cfg.strict_valid)
    got = [host(sel[k][rb, rt]).reshape((batch, n) + tuple(sel[k].shape[2:]))
           for k in ("anchor", "anchor_score", "partner", "partner_score")]
    for name, g_, e_ in zip(("anchor", "anchor_score", "partner", "partner_score"), got, exp):
        np.testing.assert_array_equal(g_, e_, err_msg=name)
    mlp = block.relation_mlp
    out, _ = omb.relate_rows(
        host(sel["expanded_cache"]), host(sel["operand_cache"]), host(sel["product_weight"]),
        host(mlp[2].weight), host(mlp[2].bias), host(mlp[3].weight), host(mlp[3].bias),
        host(block.slot_mix_logits), float(block.residual_gate.detach()), host(x[rb, rt]), rb, rt,
        host(sel["anchor"][rb, rt]), host(sel["partner"][rb, rt]),
        host(sel["partner_score"][rb, rt]), mlp[3].eps, hidden_dtype)
    np.testing.assert_allclose(host(y[rb, rt]), out, rtol=0, atol=atol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_routed_block_against_oracles(device, dtype):
    cfg = small_cfg(local_window=32, top_blocks=3, block_size=32, ff_mult=4)
    block = MultiAnchorRelationBlock(cfg)
    randomize(block, 7)
    block = block.to(device=device, dtype=dtype)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(2, 256, cfg.d_model, generator=g).to(device=device, dtype=dtype)
    memory = torch.randn(2, 256, cfg.d_model, generator=g).to(device=device, dtype=dtype)
    with torch.no_grad():
        sel = block.select(x, memory)
        y = block.relate(x, sel)
        full, _ = block(x, memory)
    assert torch.equal(full, y)
    rows_t = np.tile(np.arange(256), 2)
    rows_b = np.repeat(np.arange(2), 256)
    bf = dtype == torch.bfloat16
    check_layer_on_rows(block, x, memory, sel, y, rows_b, rows_t,
                        "bfloat16" if bf else np.float32, 0.02 if bf else 2e-4)


def cfg5_block_config():
    # cfg5: d 768, block 64, local 128, top 8, 4 anchor slots x K=6; exact (gate)
    # and router dims 64 as the selection benchmarks; relation dim 128, MLP 4x.
    return MultiRelationBlockConfig(d_model=768, gate_dim=64, relation_dim=128, ff_mult=4,
                                    anchors_per_block=4, partners_per_anchor=6, block_size=64,
                                    local_window=128, top_blocks=8)


def cfg5_inputs(device, seed=20261205):
    g = torch.Generator().manual_seed(seed)
    hidden = torch.randn(4, 4096, 768, generator=g).to(device=device, dtype=torch.bfloat16)
    memory = torch.randn(4, 4096, 768, generator=g).to(device=device, dtype=torch.bfloat16)
    return hidden, memory


def sample_rows(seed, batch=4, length=4096, per_row=64):
    rng = np.random.default_rng(seed)
    fixed = np.array([0, 1, 2, 3, 127, 128, length - 1])[:per_row]
    t = np.concatenate([fixed, rng.integers(0, length, size=per_row - len(fixed))])
    return np.repeat(np.arange(batch), per_row), np.tile(t, batch)


CONTEXT_ABS = 2e-2     # bf16 bar of the relation state
CONTEXT_TIGHT = 5e-3   # observed margin of the fp32-accumulated path


def check_cfg5_layer(block, x, memory, rows_b, rows_t):
    """One cfg5 layer: the block's fp32 relation context and bf16 output on the
    sampled queries against the oracles (selection bit-exact, context within
    CONTEXT_TIGHT, output within the context bound plus the bf16 rounding of
    the output).  Returns the layer's output."""
    sel = block.select(x, memory)
    context = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    y = block.relate(x, sel, context)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all() and torch.isfinite(context).all()
    check_layer_on_rows(block, x, memory, sel, y, rows_b, rows_t, "bfloat16", 0.03)
    mlp = block.relation_mlp
    _, expected = omb.relate_rows(
        host(sel["expanded_cache"]), host(sel["operand_cache"]), host(sel["product_weight"]),
        host(mlp[2].weight), host(mlp[2].bias), host(mlp[3].weight), host(mlp[3].bias),
        host(block.slot_mix_logits), float(block.residual_gate.detach()),
        host(x[rows_b, rows_t]), rows_b, rows_t, host(sel["anchor"][rows_b, rows_t]),
        host(sel["partner"][rows_b, rows_t]), host(sel["partner_score"][rows_b, rows_t]),
        mlp[3].eps, "bfloat16")
    err = np.abs(host(context[rows_b, rows_t]) - expected)
    assert err.max() <= CONTEXT_ABS, err.max()
    assert err.max() <= CONTEXT_TIGHT, err.max()
    # out = bf16(hidden + sigmoid(gate) * context): the context error plus one
    # bf16 rounding of the output value.
    gate = 1.0 / (1.0 + np.exp(-float(block.residual_gate.detach())))
    exp_out = host(x[rows_b, rows_t]).astype(np.float64) + gate * expected
    half_ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(exp_out), 1e-30))) - 8)
    out_err = np.abs(host(y[rows_b, rows_t]) - exp_out)
    assert (out_err <= half_ulp + gate * CONTEXT_TIGHT + 1e-6).all(), float(out_err.max())
    return y


def test_cfg5_one_layer(device):
    cfg = cfg5_block_config()
    torch.manual_seed(0)
    block = MultiAnchorRelationBlock(cfg)
    randomize(block, 11)
    block = block.to(device=device, dtype=torch.bfloat16)
    x, memory = cfg5_inputs(device)
    rows_b, rows_t = sample_rows(1)
    print("cfg5 one layer: 256 sampled queries", flush=True)
    with torch.no_grad():
        check_cfg5_layer(block, x, memory, rows_b, rows_t)
        # The whole of batch row 0 (4096 queries): context against the oracle.
        sel = block.select(x, memory)
        context = torch.empty(x.shape, dtype=torch.float32, device=device)
        block.relate(x, sel, context)
    torch.cuda.synchronize()
    mlp = block.relation_mlp
    rb, rt = np.zeros(4096, dtype=np.int64), np.arange(4096)
    print("cfg5 one layer: every query of batch row 0", flush=True)
    for lo in range(0, 4096, 1024):
        sl = slice(lo, lo + 1024)
        _, expected = omb.relate_rows(
            host(sel["expanded_cache"]), host(sel["operand_cache"]), host(sel["product_weight"]),
            host(mlp[2].weight), host(mlp[2].bias), host(mlp[3].weight), host(mlp[3].bias),
            host(block.slot_mix_logits), float(block.residual_gate.detach()),
            host(x[rb[sl], rt[sl]]), rb[sl], rt[sl], host(sel["anchor"][0, sl]),
            host(sel["partner"][0, sl]), host(sel["partner_score"][0, sl]), mlp[3].eps,
            "bfloat16")
        err = np.abs(host(context[0, sl]) - expected).max()
        assert err <= CONTEXT_TIGHT, (lo, err)


def test_cfg5_stack(device):
    cfg = cfg5_block_config()
    stack = RelationBlockStack(cfg, 4)
    randomize(stack, 12)
    stack = stack.to(device=device, dtype=torch.bfloat16)
    x, memory = cfg5_inputs(device, seed=20261206)
    rows_b, rows_t = sample_rows(2)
    with torch.no_grad():
        out, diags = stack(x, memory)
        torch.cuda.synchronize()
        assert len(diags) == 4 and torch.isfinite(out.float()).all()
        # Layer by layer, the same kernels as forward, each checked on samples.
        h = x
        for i, block in enumerate(stack.blocks):
            print(f"cfg5 stack: layer {i}", flush=True)
            h = check_cfg5_layer(block, h, memory, rows_b, rows_t)
    final = stack.final_norm
    expected = omb.layer_norm(host(h[rows_b, rows_t]), host(final.weight), host(final.bias),
                              final.eps)
    # The final LayerNorm of the device's own last-layer output: the bf16 result is
    # the oracle's value rounded to bf16, or its neighbour (one step, at most 2^-7
    # of the value) where the fp32 statistics fall near a rounding boundary.
    np.testing.assert_allclose(host(out[rows_b, rows_t]), bf16_round(expected), rtol=2.0**-7,
                               atol=1e-4)
