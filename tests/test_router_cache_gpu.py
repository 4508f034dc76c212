"""GPU parity of relation_lm::router_cache_update against the oracle.

Mirrors the reference's tests/test_router_cache_update_gpu.py: the same shapes
(router dim 64 = 4 heads x 16, block 8, cache 512), raw rows taken as strided
views of a packed [B, 512] projection (row stride 512), positions 95/96 (block
boundary) and 447/448, batch 1 and 8, every output and every mutated buffer
within atol = rtol = 1e-6 (the reference's bound).  The inputs come from a
CPU generator, since the reference's device RNG streams cannot be reproduced.
Also: a token-by-token replay from empty caches, bf16 inputs, replays of a
captured HIP graph, positions outside the cache and rejected shapes.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import router
from relation_lm.kernels.router_cache import router_cache_update

pytestmark = pytest.mark.gpu

BUFFERS = ("anchor_raw_cache", "partner_raw_cache", "anchor_conv_cache", "partner_conv_cache",
           "anchor_mean", "anchor_std", "partner_mean", "partner_std")


def make_case(batch, position, device, dtype=torch.float32, seed=0, max_context=512,
              block_size=8):
    g = torch.Generator().manual_seed(20260824 + batch + position + seed)
    dim, heads, head_dim = 64, 4, 16
    packed = torch.randn(batch, 512, generator=g).to(dtype)
    raw_cache = {s: torch.zeros(batch, max_context, dim) for s in ("anchor", "partner")}
    for s in raw_cache:
        raw_cache[s][:, :position] = torch.randn(batch, position, dim, generator=g)
    weight = {s: (torch.randn(dim, 3, generator=g) * 0.1) for s in ("anchor", "partner")}
    conv_cache = {}
    for s in ("anchor", "partner"):
        conv = router.causal_conv(raw_cache[s].numpy(), weight[s][:, None, :].numpy())
        conv[:, position:] = 0.0
        conv_cache[s] = torch.from_numpy(conv).float()
    blocks = max_context // block_size
    case = {
        "packed": packed,
        "anchor_raw_cache": raw_cache["anchor"].to(dtype),
        "partner_raw_cache": raw_cache["partner"].to(dtype),
        "anchor_conv_cache": conv_cache["anchor"].to(dtype),
        "partner_conv_cache": conv_cache["partner"].to(dtype),
        "anchor_mean": torch.zeros(batch, blocks, heads, head_dim, dtype=dtype),
        "anchor_std": torch.zeros(batch, blocks, heads, head_dim, dtype=dtype),
        "partner_mean": torch.zeros(batch, blocks, heads, head_dim, dtype=dtype),
        "partner_std": torch.zeros(batch, blocks, heads, head_dim, dtype=dtype),
        "anchor_weight": weight["anchor"].to(dtype),
        "partner_weight": weight["partner"].to(dtype),
        "position": torch.tensor(position, dtype=torch.long),
        "block_size": block_size,
    }
    host = {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in case.items()}
    dev = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in case.items()}
    return host, dev


def run_gpu(dev):
    packed = dev["packed"]
    return router_cache_update(packed[:, 384:448], packed[:, 448:512], dev["anchor_raw_cache"],
                               dev["partner_raw_cache"], dev["anchor_conv_cache"],
                               dev["partner_conv_cache"], dev["anchor_mean"], dev["anchor_std"],
                               dev["partner_mean"], dev["partner_std"], dev["anchor_weight"],
                               dev["partner_weight"], dev["position"], dev["block_size"])


def run_oracle(host, position=None):
    f = lambda t: t.float().numpy()  # noqa: E731
    packed = f(host["packed"])
    return router.router_cache_update(
        packed[:, 384:448], packed[:, 448:512], *[f(host[k]) for k in BUFFERS],
        f(host["anchor_weight"]), f(host["partner_weight"]),
        int(host["position"]) if position is None else position, host["block_size"])


def assert_close(got, expected, atol, rtol):
    np.testing.assert_allclose(got.float().cpu().numpy(), expected, atol=atol, rtol=rtol)


@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("position", [95, 96, 447, 448])
def test_router_cache_update_state(device, batch, position):
    host, dev = make_case(batch, position, device)
    assert dev["packed"][:, 384:448].stride(0) == 512
    out = run_gpu(dev)
    torch.cuda.synchronize()
    expected_out, expected = run_oracle(host)
    assert out.shape == (batch, 2, 64) and out.dtype == torch.float32
    assert_close(out, expected_out, 1e-6, 1e-6)
    for name in BUFFERS:
        assert_close(dev[name], expected[name], 1e-6, 1e-6)


def test_replay_from_empty_caches(device):
    """Tokens 0..47 one at a time from zeroed caches, oracle replayed alongside."""
    host, dev = make_case(2, 0, device, max_context=48)
    for name in BUFFERS:
        host[name].zero_()
        dev[name].zero_()
    g = torch.Generator().manual_seed(99)
    state = {k: host[k].float().numpy() for k in BUFFERS}
    wa, wp = host["anchor_weight"].float().numpy(), host["partner_weight"].float().numpy()
    for t in range(48):
        packed = torch.randn(2, 512, generator=g)
        dev["packed"] = packed.to(device)
        dev["position"] = torch.tensor(t, device=device, dtype=torch.int32)
        out = run_gpu(dev)
        expected_out, state = router.router_cache_update(
            packed[:, 384:448].numpy(), packed[:, 448:512].numpy(), *[state[k] for k in BUFFERS],
            wa, wp, t, 8)
        torch.cuda.synchronize()
        assert_close(out, expected_out, 1e-6, 1e-6)
    for name in BUFFERS:
        assert_close(dev[name], state[name], 1e-6, 1e-5)


def test_bf16_buffers(device):
    host, dev = make_case(4, 200, device, dtype=torch.bfloat16)
    out = run_gpu(dev)
    torch.cuda.synchronize()
    expected_out, expected = run_oracle(host)
    assert_close(out, expected_out, 1e-5, 1e-5)  # conv is fp32 from bf16 inputs
    for name in BUFFERS:
        # the kernel rounds its fp32 results to bf16 once; the oracle rounds float64
        assert_close(dev[name], expected[name], 2e-2, 1e-2)


def test_graph_replay_matches_eager(device):
    """Captured once, replayed: each replay redoes the same update on fresh buffers."""
    host, eager_dev = make_case(8, 447, device)
    _, dev = make_case(8, 447, device)
    eager_out = run_gpu(eager_dev).clone()
    torch.cuda.synchronize()
    originals = {k: dev[k].clone() for k in BUFFERS}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run_gpu(dev)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run_gpu(dev)
    for _ in range(3):
        for k in BUFFERS:
            dev[k].copy_(originals[k])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager_out)
        for k in BUFFERS:
            assert torch.equal(dev[k], eager_dev[k]), k


@pytest.mark.parametrize("position", [-1, 512])
def test_position_outside_cache(device, position):
    host, dev = make_case(2, 100, device)
    dev["position"] = torch.tensor(position, device=device)
    before = {k: dev[k].clone() for k in BUFFERS}
    out = run_gpu(dev)
    torch.cuda.synchronize()
    assert not out.any()
    for k in BUFFERS:
        assert torch.equal(dev[k], before[k])


def test_rejects_bad_shapes(device):
    host, dev = make_case(2, 10, device)
    dev["anchor_weight"] = dev["anchor_weight"][:, :2].contiguous()
    with pytest.raises(RuntimeError, match="anchor_conv_weight"):
        run_gpu(dev)
    host, dev = make_case(2, 10, device)
    dev["anchor_mean"] = dev["anchor_mean"][:, :, :2].contiguous()
    with pytest.raises(RuntimeError, match="anchor_mean"):
        run_gpu(dev)
