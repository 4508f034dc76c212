"""GPU parity of relation_hidden_linear_seq_out: the multi-anchor block's relation MLP
(multi_relation_blocks.py:47-52,163 of the reference: Linear -> GELU -> Linear, the first
Linear factorized as relation_hidden_cached, relation_reduce.py:149-183) up to its closing
LayerNorm, bias-free, in one kernel whose bf16 hidden never reaches memory.

Checked
  * bit for bit against the two launches it replaces (relation_hidden_cached_seq_out into
    a bf16 buffer, then relation_linear with an fp32 output and no bias): the kernel runs
    the same MFMA sums, fp32 adds, GELU and bf16 rounding for the hidden and the same
    k-ordered MFMA accumulation for the Linear;
  * against the float64 oracle (relation_hidden_cached_seq, bf16 rounding of the hidden,
    linear) within fp32 accumulation of the exact products: 1e-5 of sum |w2 h| plus one
    bf16 ulp of a hidden value that rounds the other way, times |w2|;
  * on the cfg5 shape (relation dim 128, hidden 3072, d_model 768), the other d_model /
    relation dims it takes, ragged row counts, int32 / int64 indices, indices outside the
    cache (zero rows) and repeated calls.
The weights enter in MFMA fragment order (mfma_fragments, checked against a reshape of
the plain weight).  Shapes outside relation_hidden_linear_seq_fits raise.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reduce as ored
from relation_lm.kernels.relation_reduce import (mfma_fragments,
                                                 relation_hidden_cached_seq_out,
                                                 relation_hidden_linear_seq_fits,
                                                 relation_hidden_linear_seq_out,
                                                 relation_linear)

pytestmark = pytest.mark.gpu


def host(t):
    return t.detach().float().cpu().numpy()


def make_case(b, t, tq, k, r, h, d, seed, device, index_dtype=torch.int64, bad=True):
    g = torch.Generator().manual_seed(seed)
    anchor = torch.randint(0, t, (b, tq), generator=g)
    partner = torch.randint(0, t, (b, tq, k), generator=g)
    if bad:
        anchor[0, 0] = -1                       # outside the cache: zero rows
        partner[-1, -1, 0] = t + 3
        partner[0, tq // 2, k - 1] = -5
    return {
        "expanded": (torch.randn(b, t, 2 * h, generator=g) * 0.5).to(device, torch.bfloat16),
        "operand": torch.randn(b, t, r, generator=g).to(device, torch.bfloat16),
        "anchor": anchor.to(device, index_dtype),
        "partner": partner.to(device, index_dtype),
        "wm": (torch.randn(h, r, generator=g) * r ** -0.5).to(device, torch.bfloat16),
        "w2": (torch.randn(d, h, generator=g) * h ** -0.5).to(device, torch.bfloat16),
    }


def run_fused(c):
    b, tq, k = c["partner"].shape
    out = torch.full((b, tq, k, c["w2"].shape[0]), float("nan"), device=c["w2"].device)
    relation_hidden_linear_seq_out(c["expanded"], c["operand"], c["anchor"], c["partner"],
                                   mfma_fragments(c["wm"]), mfma_fragments(c["w2"]), out)
    return out


def test_mfma_fragments_layout(device):
    # Fragment (nb, g), lane l = weight[32 nb + l % 32, 16 g + 8 (l // 32) : +8].
    g = torch.Generator().manual_seed(1)
    w = torch.randn(96, 48, generator=g).to(device, torch.bfloat16)
    f = mfma_fragments(w).cpu()
    ref = w.cpu().view(3, 32, 3, 2, 8).permute(0, 2, 3, 1, 4).reshape(3, 3, 64, 8)
    assert torch.equal(f, ref)


def run_two_ops(c):
    b, tq, k = c["partner"].shape
    hidden = torch.empty((b, tq, k, c["wm"].shape[0]), dtype=torch.bfloat16,
                         device=c["w2"].device)
    relation_hidden_cached_seq_out(c["expanded"], c["operand"], c["anchor"], c["partner"],
                                   c["wm"], hidden)
    return relation_linear(hidden, c["w2"], None, torch.float32)


# The two-op path runs its tile kernels (the arithmetic the fused kernel repeats) from
# 4096 relation rows on: every bit-identity case has at least that many.
CASES = [
    # b, t, tq, k, r, h, d
    (1, 512, 1024, 6, 128, 3072, 768),    # cfg5: hidden 3072, d_model 768, K = 6
    (2, 300, 700, 3, 64, 256, 256),       # ragged: 4200 rows, not a multiple of 64
    (3, 64, 300, 5, 128, 384, 512),
]
SMALL = [
    (2, 100, 37, 3, 64, 256, 256),        # 222 rows
    (1, 40, 9, 1, 64, 128, 768),          # one partner, one chunk, under one row tile
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("index_dtype", [torch.int64, torch.int32])
def test_bit_identical_to_hidden_then_linear(device, case, index_dtype):
    print("case", case, index_dtype, flush=True)
    c = make_case(*case, seed=sum(case), device=device, index_dtype=index_dtype)
    assert relation_hidden_linear_seq_fits(c["expanded"], c["operand"], mfma_fragments(c["wm"]),
                                           mfma_fragments(c["w2"]))
    got = run_fused(c)
    ref = run_two_ops(c)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    assert torch.equal(got, ref), (got - ref).abs().max().item()


@pytest.mark.parametrize("case", SMALL + [(1, 64, 30, 4, 128, 384, 512)])
def test_against_float64_oracle(device, case):
    c = make_case(*case, seed=7 + sum(case), device=device)
    got = host(run_fused(c))
    hidden = ored.relation_hidden_cached_seq(host(c["expanded"]), host(c["operand"]),
                                             c["anchor"].cpu().numpy(),
                                             c["partner"].cpu().numpy(), host(c["wm"]))
    hb = ored.round_to(hidden, "bf16")
    w2 = host(c["w2"]).astype(np.float64)
    expected = ored.linear(hb, w2)
    # fp32 accumulation of exact bf16 products, plus a hidden value within 2^-8 of a
    # bf16 rounding boundary that the fp32 hidden rounds the other way (one bf16 ulp).
    mag = np.abs(hb) @ np.abs(w2).T
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(hidden), 1e-30))) - 7)
    tol = 1e-5 * mag + 2 * (ulp @ np.abs(w2).T) + 1e-6
    assert (np.abs(got - expected) <= tol).all(), np.abs(got - expected).max()


def test_repeated_calls_and_rows_past_the_end(device):
    # The output rows past the relation rows are never written; repeated calls agree.
    c = make_case(2, 100, 37, 3, 64, 256, 256, seed=11, device=device)
    a = run_fused(c)
    b = run_fused(c)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    big = torch.full((2 * 37 * 3 + 64, 256), 7.0, device=device)
    view = big[: 2 * 37 * 3].view(2, 37, 3, 256)
    relation_hidden_linear_seq_out(c["expanded"], c["operand"], c["anchor"], c["partner"],
                                   mfma_fragments(c["wm"]), mfma_fragments(c["w2"]), view)
    torch.cuda.synchronize()
    assert torch.equal(view, a)
    assert (big[2 * 37 * 3:] == 7.0).all()


def test_unsupported_shapes_raise(device):
    c = make_case(1, 64, 8, 2, 128, 256, 576, seed=3, device=device)   # d_model 576
    wm, w2 = mfma_fragments(c["wm"]), mfma_fragments(c["w2"])
    assert not relation_hidden_linear_seq_fits(c["expanded"], c["operand"], wm, w2)
    out = torch.empty((1, 8, 2, 576), device=device)
    with pytest.raises(RuntimeError, match="d_model 256, 512 or 768"):
        relation_hidden_linear_seq_out(c["expanded"], c["operand"], c["anchor"], c["partner"],
                                       wm, w2, out)
    with pytest.raises(RuntimeError, match="expected a 4-d tensor"):        # plain [D, H] weight
        relation_hidden_linear_seq_out(c["expanded"], c["operand"], c["anchor"], c["partner"],
                                       wm, c["w2"], out)
