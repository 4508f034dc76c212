"""GPU parity of relation_lm::relation_linear on its large-M 16-bit path (the
LDS-DMA tile GEMM: 256x256 tiles when the problem fills the chip, 128x128
otherwise) against a float64 product of the same 16-bit operands.

The relation MLP's second Linear of the multi-anchor block (cfg5:
[98304, 3072] x [3072, 768], bf16) and the reference's second linear G3
(benchmark_relation_reduce.py:63) run here.  Shapes cover both tile sizes,
edges in M and N, a row-strided input, fp16 weights, fp32 and bf16 outputs
and the bias in the epilogue; the small-K kernel (K <= 128, the expanded-cache
projection) on its own shapes.  fp32 outputs: within fp32 accumulation of the
exact products (1e-5 of sum |a w|); 16-bit outputs: that plus half an ulp of
the output type.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from relation_lm import _native  # noqa: F401  (registers torch.ops.relation_lm)

pytestmark = pytest.mark.gpu
ops = torch.ops.relation_lm


def reference(a, w, bias):
    a64, w64 = a.double().cpu(), w.double().cpu()
    out = a64 @ w64.T
    mag = a64.abs() @ w64.abs().T
    if bias is not None:
        out = out + bias.double().cpu()
        mag = mag + bias.double().cpu().abs()
    return out.numpy(), mag.numpy()


def check(got, a, w, bias):
    exp, mag = reference(a, w, bias)
    g = got.double().cpu().numpy()
    tol = 1e-5 * mag + 1e-6
    if got.dtype != torch.float32:
        bits = 8 if got.dtype == torch.bfloat16 else 11
        tol = tol + np.exp2(np.floor(np.log2(np.maximum(np.abs(exp), 1e-30))) - bits)
    bad = np.abs(g - exp) > tol
    assert not bad.any(), (int(bad.sum()), float(np.abs(g - exp).max()))


CASES = [
    # (M, N, K, weight dtype, out dtype, bias, input row padding)
    (32768, 512, 512, torch.bfloat16, torch.float32, True, 0),    # 256x256 tiles (A8 shape)
    (32768, 512, 512, torch.bfloat16, torch.bfloat16, False, 0),
    (16384, 768, 768, torch.bfloat16, torch.bfloat16, True, 0),   # 256x256 tiles, cfg5 projection
    (1000, 300, 192, torch.bfloat16, torch.float32, True, 0),     # 128x128, edges in M and N
    (4100, 264, 320, torch.bfloat16, torch.float32, False, 64),   # edges, row-strided input
    (3000, 512, 256, torch.float16, torch.float32, True, 0),      # fp16 weights
    (2048, 768, 3072, torch.bfloat16, torch.float32, True, 0),    # cfg5 second-Linear widths
]


@pytest.mark.parametrize("m,n,k,wdt,odt,with_bias,pad", CASES)
def test_relation_linear_dma_path(device, m, n, k, wdt, odt, with_bias, pad):
    g = torch.Generator().manual_seed(m + n + k)
    base = torch.randn(m, k + pad, generator=g).to(wdt)
    a = base[:, :k]
    w = (torch.randn(n, k, generator=g) / np.sqrt(k)).to(wdt)
    bias = (0.5 * torch.randn(n, generator=g)).to(wdt) if with_bias else None
    print(f"relation_linear M={m} N={n} K={k} {wdt} -> {odt} bias={with_bias} pad={pad}",
          flush=True)
    a_dev = base.to(device)[:, :k]
    got = ops.relation_linear(a_dev, w.to(device), None if bias is None else bias.to(device), odt)
    torch.cuda.synchronize()
    assert got.shape == (m, n) and got.dtype == odt
    check(got, a, w, bias)


SMALLK_CASES = [
    # (M, N, K, weight dtype, out dtype, bias, input row padding): K <= 128, the
    # expanded-cache projection's kernel (smallk_kernel)
    (4096, 1024, 128, torch.bfloat16, torch.bfloat16, True, 0),   # cfg2 expanded projection
    (4096, 1024, 128, torch.bfloat16, torch.float32, False, 0),
    (1000, 256, 32, torch.bfloat16, torch.bfloat16, True, 0),     # a partial last tile in M
    (777, 384, 96, torch.float16, torch.bfloat16, True, 16),      # fp16, row-strided input
    (300, 128, 64, torch.bfloat16, torch.float32, True, 0),
    (520, 200, 128, torch.bfloat16, torch.bfloat16, True, 0),     # a partial last tile in N
]


@pytest.mark.parametrize("m,n,k,wdt,odt,with_bias,pad", SMALLK_CASES)
def test_relation_linear_small_k(device, m, n, k, wdt, odt, with_bias, pad):
    g = torch.Generator().manual_seed(m + n + k + 7)
    base = torch.randn(m, k + pad, generator=g).to(wdt)
    a = base[:, :k]
    w = (torch.randn(n, k, generator=g) / np.sqrt(k)).to(wdt)
    bias = (0.5 * torch.randn(n, generator=g)).to(wdt) if with_bias else None
    print(f"relation_linear small K: M={m} N={n} K={k} {wdt} -> {odt} bias={with_bias} "
          f"pad={pad}", flush=True)
    got = ops.relation_linear(base.to(device)[:, :k], w.to(device),
                              None if bias is None else bias.to(device), odt)
    torch.cuda.synchronize()
    assert got.shape == (m, n) and got.dtype == odt
    check(got, a, w, bias)


@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float32])
def test_relation_linear_small_k_edge_tiles_equal_full_tiles(device, odt):
    # N = 1024 is whole 128-column tiles (vector stores), N = 1000 ends in an
    # edge tile (element stores); every output takes the same k-steps, so the
    # bits agree.
    g = torch.Generator().manual_seed(31)
    a = torch.randn(4096, 128, generator=g).to(torch.bfloat16).to(device)
    w = (torch.randn(1024, 128, generator=g) / np.sqrt(128)).to(torch.bfloat16).to(device)
    b = (0.5 * torch.randn(1024, generator=g)).to(torch.bfloat16).to(device)
    print(f"relation_linear small K, full vs edge tiles -> {odt}", flush=True)
    full = ops.relation_linear(a, w, b, odt)
    part = ops.relation_linear(a, w[:1000].contiguous(), b[:1000].contiguous(), odt)
    torch.cuda.synchronize()
    assert torch.equal(full[:, :1000], part)


def test_relation_linear_dma_repeat_identical(device):
    # Same inputs, same bits: no atomics or order-dependent accumulation.
    g = torch.Generator().manual_seed(5)
    a = torch.randn(8192, 1024, generator=g).to(torch.bfloat16).to(device)
    w = (torch.randn(768, 1024, generator=g) / 32).to(torch.bfloat16).to(device)
    b = torch.randn(768, generator=g).to(device)
    first = ops.relation_linear(a, w, b, torch.float32)
    second = ops.relation_linear(a, w, b, torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(first, second)


@pytest.mark.parametrize("m,n,k,with_bias", [(1, 512, 576, False), (8, 512, 576, True),
                                             (3, 37, 100, True), (17, 300, 1000, False),
                                             (64, 130, 2308, True)])
def test_relation_linear_fp32_skinny(device, m, n, k, with_bias):
    # fp32 weights, M <= 64: the fp32 FMA skinny kernel (decode shapes, the
    # reference's fp32 packed-projection benchmark at B=1 / B=8).
    g = torch.Generator().manual_seed(m * 7 + n + k)
    a = torch.randn(m, k, generator=g)
    w = torch.randn(n, k, generator=g) * 0.02
    bias = torch.randn(n, generator=g) if with_bias else None
    print(f"relation_linear fp32 M={m} N={n} K={k} bias={with_bias}", flush=True)
    got = ops.relation_linear(a.to(device), w.to(device),
                              None if bias is None else bias.to(device))
    torch.cuda.synchronize()
    assert got.dtype == torch.float32
    check(got, a, w, bias)


@pytest.mark.parametrize("batch", [1, 8])
def test_packed_projection_fp32(device, batch):
    # The reference's packed-cache benchmark inputs: fp32 memory [B, 576] and
    # six fp32 weights (benchmarks/benchmark_packed_cache.py:36-47).
    from relation_lm.inference import pack_sparse_cache_projection_weights

    g = torch.Generator().manual_seed(20260822 + batch)
    memory = torch.randn(batch, 576, generator=g)
    weights = [torch.randn(wd, 576, generator=g) * 0.02 for wd in (64, 64, 128, 128, 64, 64)]
    proj = pack_sparse_cache_projection_weights([x.to(device) for x in weights])
    parts = proj.project(memory.to(device))
    torch.cuda.synchronize()
    for got, wt in zip(parts, weights):
        check(got, memory, wt, None)
