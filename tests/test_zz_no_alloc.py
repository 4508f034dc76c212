"""rlm_relation_linear_norm_reduce_output_noalloc through the C ABI: the
allocation-free form (partials in the library's static per-GPU workspace) must
give the workspace form's exact bits for the same split count, on two calls in
a row (the second smaller, so stale workspace contents from the first must not
leak in), and must reject a size beyond its workspace before launching."""
from __future__ import annotations

import ctypes
import os

import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "relation-lm_amd", "relation_lm", "_lib", "librlm_hip.so")
DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.int32: 3, torch.int64: 4}
HIP_SUCCESS, HIP_ERROR_INVALID_VALUE = 0, 1


class RlmTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("shape", ctypes.c_int64 * 4), ("stride", ctypes.c_int64 * 4)]


def desc(t):
    d = RlmTensor()
    d.data = t.data_ptr()
    d.dtype = DTYPES[t.dtype]
    d.ndim = t.dim()
    for i in range(t.dim()):
        d.shape[i] = t.shape[i]
        d.stride[i] = t.stride(i)
    return d


@pytest.fixture(scope="module")
def lib():
    import relation_lm  # noqa: F401  (loads the library into the process first)
    handle = ctypes.CDLL(LIB)
    handle.rlm_last_error.restype = ctypes.c_char_p
    return handle


def case(batch, k_out, hidden_dim, d, seed, device):
    g = torch.Generator().manual_seed(seed)
    t = {
        "hidden": torch.randn(batch, k_out, hidden_dim, generator=g).to(device),
        "w2": (torch.randn(d, hidden_dim, generator=g) * hidden_dim ** -0.5).to(device,
                                                                             torch.bfloat16),
        "b2": (0.1 * torch.randn(d, generator=g)).to(device),
        "scores": torch.randn(batch, k_out, generator=g).to(device),
        "nw": (1 + 0.1 * torch.randn(d, generator=g)).to(device),
        "nb": (0.1 * torch.randn(d, generator=g)).to(device),
        "pos": torch.tensor(300, device=device),
        "query": torch.randn(batch, d, generator=g).to(device, torch.bfloat16),
        "mix": torch.tensor(-0.5, device=device),
        "ow": (1 + 0.1 * torch.randn(d, generator=g)).to(device, torch.bfloat16),
        "ob": (0.1 * torch.randn(d, generator=g)).to(device),
    }
    return t


def run(lib, t, splits, noalloc):
    batch, k_out, _ = t["hidden"].shape
    d = t["w2"].shape[0]
    ctx = torch.full((batch, d), float("nan"), device=t["hidden"].device)
    final = torch.zeros(batch, d, dtype=torch.bfloat16, device=t["hidden"].device)
    keep = [desc(t[k]) for k in ("hidden", "w2", "b2", "scores", "nw", "nb", "pos")]
    head = [desc(t[k]) for k in ("query", "mix", "ow", "ob")]
    outs = [desc(ctx), desc(final)]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [ctypes.byref(x) for x in keep] + [ctypes.c_double(1e-5)]
    args += [ctypes.byref(x) for x in head] + [ctypes.c_double(1e-5)]
    if noalloc:
        args += [ctypes.c_int32(splits)]
        fn = lib.rlm_relation_linear_norm_reduce_output_noalloc
        parts = None
    else:
        parts = torch.empty(splits, batch * k_out, d, device=t["hidden"].device)
        pd = desc(parts)
        args += [ctypes.byref(pd)]
        fn = lib.rlm_relation_linear_norm_reduce_output
    args += [ctypes.byref(x) for x in outs] + [stream]
    rc = fn(*args)
    assert rc == HIP_SUCCESS, lib.rlm_last_error()
    torch.cuda.synchronize()
    return ctx, final


def test_matches_workspace_form_on_two_calls(device, lib):
    big = case(8, 8, 2304, 576, 1, device)      # 3 x 64 x 576 partials
    small = case(1, 6, 1024, 512, 2, device)    # 4 x 6 x 512 partials, inside the first's
    for t, splits in ((big, 3), (small, 4)):
        ctx_n, fin_n = run(lib, t, splits, True)
        ctx_w, fin_w = run(lib, t, splits, False)
        assert torch.isfinite(ctx_n).all()
        assert torch.equal(ctx_n, ctx_w)
        assert torch.equal(fin_n, fin_w)


def test_rejects_sizes_beyond_the_workspace(device, lib):
    t = case(9, 8, 256, 1024, 3, device)        # 4 x 72 x 1024 > 4 x 64 x 1024
    batch, k_out, _ = t["hidden"].shape
    ctx = torch.zeros(batch, 1024, device=device)
    final = torch.zeros(batch, 1024, dtype=torch.bfloat16, device=device)
    d = [desc(t[k]) for k in ("hidden", "w2", "b2", "scores", "nw", "nb", "pos", "query", "mix",
                              "ow", "ob")] + [desc(ctx), desc(final)]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.rlm_relation_linear_norm_reduce_output_noalloc(
        *[ctypes.byref(x) for x in d[:7]], ctypes.c_double(1e-5),
        *[ctypes.byref(x) for x in d[7:11]], ctypes.c_double(1e-5), ctypes.c_int32(4),
        ctypes.byref(d[11]), ctypes.byref(d[12]), stream)
    assert rc == HIP_ERROR_INVALID_VALUE
    assert b"static workspace" in lib.rlm_last_error()
    rc = lib.rlm_relation_linear_norm_reduce_output_noalloc(
        *[ctypes.byref(x) for x in d[:7]], ctypes.c_double(1e-5),
        *[ctypes.byref(x) for x in d[7:11]], ctypes.c_double(1e-5), ctypes.c_int32(5),
        ctypes.byref(d[11]), ctypes.byref(d[12]), stream)
    assert rc == HIP_ERROR_INVALID_VALUE
    assert b"splits" in lib.rlm_last_error()
