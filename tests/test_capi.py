"""C ABI of librlm_hip.so: exports and host-side argument validation (no GPU needed).

Validation runs on the host before anything is launched, so malformed
descriptors can be exercised on a machine without a GPU; every call here
returns hipErrorInvalidValue with a message and launches nothing.
"""
from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "relation_lm_hip.h")
LIB = os.path.join(ROOT, "relation-lm_amd", "relation_lm", "_lib", "librlm_hip.so")
HIP_ERROR_INVALID_VALUE = 1

RLM_F32, RLM_BF16, RLM_F16, RLM_I32, RLM_I64 = range(5)


class RlmTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("shape", ctypes.c_int64 * 4), ("stride", ctypes.c_int64 * 4)]


def tensor(shape, dtype=RLM_F32, data=0x1000, stride=None):
    t = RlmTensor()
    t.data = data
    t.dtype = dtype
    t.ndim = len(shape)
    if stride is None:
        stride, acc = [], 1
        for s in reversed(shape):
            stride.insert(0, acc)
            acc *= s
    for i, (s, st) in enumerate(zip(shape, stride)):
        t.shape[i] = s
        t.stride[i] = st
    return t


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built; run __graft_entry__.build()")
    handle = ctypes.CDLL(LIB)
    handle.rlm_last_error.restype = ctypes.c_char_p
    handle.rlm_version.restype = ctypes.c_char_p
    return handle


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:hipError_t|const char\*|int)\s+(rlm_\w+)\s*\(", text,
                                 flags=re.M)))


def test_header_declares_the_reference_ops():
    names = declared_functions()
    for op in ("rlm_relation_select_packed", "rlm_anchor_select", "rlm_partner_topk",
               "rlm_relation_hidden_cached", "rlm_relation_hidden_cache_update",
               "rlm_relation_norm_reduce", "rlm_packed_sparse_cache_projection"):
        assert op in names


def test_library_exports_every_declared_symbol(lib):
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing, missing
    assert b"gfx950" in lib.rlm_version()


def test_fused_reduce_fits_predicate(lib):
    """rlm_relation_reduce_fused_seq_fits reads descriptors only: 1 for the shapes
    the fused kernel takes, 0 for those the op runs as the three-op chain."""
    base = {"expanded": tensor([2, 64, 1024], RLM_BF16), "operand": tensor([2, 64, 64], RLM_BF16),
            "partner": tensor([2, 8, 8], RLM_I32), "wm": tensor([512, 64], RLM_BF16),
            "w2": tensor([512, 512], RLM_BF16)}

    def fits(**override):
        d = {**base, **override}
        return lib.rlm_relation_reduce_fused_seq_fits(
            *(ctypes.byref(d[k]) for k in ("expanded", "operand", "partner", "wm", "w2")))

    assert fits() == 1
    assert fits(partner=tensor([2, 8, 5], RLM_I64)) == 1
    assert fits(w2=tensor([576, 512], RLM_BF16)) == 0                    # d_model 576
    assert fits(operand=tensor([2, 64, 64], RLM_F32)) == 0               # fp32 operands
    assert fits(w2=tensor([512, 512], RLM_F32)) == 0
    assert fits(partner=tensor([2, 8, 17], RLM_I32)) == 0                # K > 16
    assert fits(wm=tensor([500, 64], RLM_BF16)) == 0                     # H % 128 != 0
    assert fits(operand=tensor([2, 64, 48], RLM_BF16)) == 0              # R not 32/64/128
    assert fits(w2=tensor([512, 512], RLM_BF16, data=0x1008)) == 0       # misaligned


def test_relation_mlp_fits_and_validation(lib):
    """rlm_relation_hidden_linear_seq_fits reads descriptors only; the entry point rejects
    shapes the kernel does not take before launching anything."""
    base = {"expanded": tensor([2, 64, 6144], RLM_BF16), "operand": tensor([2, 64, 128], RLM_BF16),
            "wm": tensor([96, 8, 64, 8], RLM_BF16), "w2": tensor([24, 192, 64, 8], RLM_BF16)}

    def fits(**override):
        d = {**base, **override}
        return lib.rlm_relation_hidden_linear_seq_fits(
            *(ctypes.byref(d[k]) for k in ("expanded", "operand", "wm", "w2")))

    assert fits() == 1
    assert fits(w2=tensor([16, 192, 64, 8], RLM_BF16)) == 1              # d_model 512
    assert fits(w2=tensor([18, 192, 64, 8], RLM_BF16)) == 0              # d_model 576
    assert fits(w2=tensor([768, 3072], RLM_BF16)) == 0                   # not fragment order
    assert fits(w2=tensor([24, 192, 64, 8], RLM_F32)) == 0               # fp32 weight
    assert fits(operand=tensor([2, 64, 96], RLM_BF16),
                wm=tensor([96, 6, 64, 8], RLM_BF16)) == 0                # R not 64/128
    assert fits(wm=tensor([94, 8, 64, 8], RLM_BF16), w2=tensor([24, 188, 64, 8], RLM_BF16),
                expanded=tensor([2, 64, 6016], RLM_BF16)) == 0           # H % 128 != 0
    assert fits(w2=tensor([24, 192, 64, 8], RLM_BF16, data=0x1008)) == 0  # misaligned

    anchor, partner = tensor([2, 16], RLM_I64), tensor([2, 16, 3], RLM_I64)
    out = tensor([2, 16, 3, 576])
    rc = lib.rlm_relation_hidden_linear_seq(
        ctypes.byref(base["expanded"]), ctypes.byref(base["operand"]), ctypes.byref(anchor),
        ctypes.byref(partner), ctypes.byref(base["wm"]),
        ctypes.byref(tensor([18, 192, 64, 8], RLM_BF16)), ctypes.byref(out), None)
    assert rc == HIP_ERROR_INVALID_VALUE
    assert b"d_model 256, 512 or 768" in lib.rlm_last_error()
    rc = lib.rlm_mfma_fragments(ctypes.byref(tensor([48, 40], RLM_BF16)),
                                ctypes.byref(tensor([1, 2, 64, 8], RLM_BF16)), None)
    assert rc == HIP_ERROR_INVALID_VALUE                                 # 48 rows: not 32k
    assert b"multiple of 32" in lib.rlm_last_error()
    rc = lib.rlm_relation_hidden_linear_seq(
        ctypes.byref(base["expanded"]), ctypes.byref(base["operand"]), ctypes.byref(anchor),
        ctypes.byref(partner), ctypes.byref(base["wm"]), ctypes.byref(base["w2"]),
        ctypes.byref(tensor([2, 16, 3, 768], RLM_BF16)), None)
    assert rc == HIP_ERROR_INVALID_VALUE                                 # bf16 out


def _select_packed_args(b=2, t=64, e=64, nb=8, k=4, **override):
    d = {
        "anchor_query": tensor([b, e]), "anchor_keys": tensor([b, t, e]),
        "anchor_router_query": tensor([b, e]), "anchor_block_mean": tensor([b, nb, 4, e // 4]),
        "anchor_block_std": tensor([b, nb, 4, e // 4]), "anchor_gamma": tensor([4]),
        "anchor_bias": tensor([4, 16]), "partner_base": tensor([b, 2 * e]),
        "partner_anchor_cache": tensor([b, t, 2 * e]), "partner_keys": tensor([b, t, e]),
        "partner_block_mean": tensor([b, nb, 4, e // 4]),
        "partner_block_std": tensor([b, nb, 4, e // 4]), "partner_gamma": tensor([4]),
        "partner_bias": tensor([4, 16]), "position": tensor([], RLM_I64),
        "out_anchor": tensor([b], RLM_I32), "out_anchor_score": tensor([b]),
        "out_partner": tensor([b, k], RLM_I32), "out_partner_score": tensor([b, k]),
    }
    d.update(override)
    return d


def _call_select_packed(lib, d, local=16, top=2, k=4, strict=0):
    names = ["anchor_query", "anchor_keys", "anchor_router_query", "anchor_block_mean",
             "anchor_block_std", "anchor_gamma", "anchor_bias", "partner_base",
             "partner_anchor_cache", "partner_keys", "partner_block_mean", "partner_block_std",
             "partner_gamma", "partner_bias", "position"]
    outs = ["out_anchor", "out_anchor_score", "out_partner", "out_partner_score"]
    args = [ctypes.byref(d[n]) for n in names] + [ctypes.c_int64(local), ctypes.c_int64(top),
                                                    ctypes.c_int64(k), ctypes.c_int32(strict)]
    args += [ctypes.byref(d[n]) for n in outs] + [ctypes.c_void_p(0)]
    return lib.rlm_relation_select_packed(*args), lib.rlm_last_error().decode()


@pytest.mark.parametrize("override,needle", [
    ({"anchor_keys": tensor([2, 64, 32])}, "anchor_keys"),
    ({"anchor_keys": tensor([2, 64, 64], RLM_BF16)}, "anchor_keys"),
    ({"partner_base": tensor([2, 64])}, "partner_base"),
    ({"position": tensor([1], RLM_I64)}, "position"),
    ({"position": tensor([], RLM_F32)}, "position"),
    ({"out_partner": tensor([2, 5], RLM_I32)}, "out_partner"),
    ({"out_anchor": tensor([2], RLM_I64)}, "out_anchor"),
    ({"anchor_keys": tensor([2, 64, 64], stride=[64 * 64, 1, 64])}, "contiguous"),
    ({"anchor_router_query": tensor([2, 32])}, "anchor_router_query"),
])
def test_select_packed_rejects_malformed_arguments(lib, override, needle):
    status, message = _call_select_packed(lib, _select_packed_args(**override))
    assert status == HIP_ERROR_INVALID_VALUE
    assert needle in message


def test_select_packed_rejects_bad_hyperparameters(lib):
    status, message = _call_select_packed(lib, _select_packed_args(), local=0)
    assert status == HIP_ERROR_INVALID_VALUE and "local_window" in message
    status, message = _call_select_packed(lib, _select_packed_args(), top=-1)
    assert status == HIP_ERROR_INVALID_VALUE and "top_blocks" in message


def test_norm_reduce_rejects_bad_shapes(lib):
    raw = tensor([2, 4, 8])
    scores = tensor([2, 5])
    w, bias = tensor([8]), tensor([8])
    pos = tensor([], RLM_I64)
    out = tensor([2, 8])
    status = lib.rlm_relation_norm_reduce(ctypes.byref(raw), ctypes.byref(scores), ctypes.byref(w),
                                          ctypes.byref(bias), ctypes.byref(pos),
                                          ctypes.c_double(1e-5), ctypes.byref(out),
                                          ctypes.c_void_p(0))
    assert status == HIP_ERROR_INVALID_VALUE
    assert "partner_scores" in lib.rlm_last_error().decode()


def test_linear_rejects_mismatched_reduction_dim(lib):
    x, w, out = tensor([4, 16], RLM_BF16), tensor([8, 12], RLM_BF16), tensor([4, 8], RLM_BF16)
    status = lib.rlm_linear(ctypes.byref(x), ctypes.byref(w), None, ctypes.byref(out),
                            ctypes.c_void_p(0))
    assert status == HIP_ERROR_INVALID_VALUE
    assert "weight" in lib.rlm_last_error().decode()


def test_hidden_rejects_index_dtype(lib):
    exp, op = tensor([1, 8, 6]), tensor([1, 8, 4])
    a, p = tensor([1], RLM_F32), tensor([1, 2], RLM_I32)
    wm, out = tensor([3, 4]), tensor([1, 2, 3])
    status = lib.rlm_relation_hidden_cached(ctypes.byref(exp), ctypes.byref(op), ctypes.byref(a),
                                            ctypes.byref(p), ctypes.byref(wm), ctypes.byref(out),
                                            ctypes.c_void_p(0))
    assert status == HIP_ERROR_INVALID_VALUE
    assert "int32 or int64" in lib.rlm_last_error().decode()


def test_torch_ops_registered_with_reference_schemas():
    import torch

    from relation_lm import _native  # noqa: F401

    schema = str(torch.ops.relation_lm.relation_select_packed.default._schema)
    assert schema.endswith("SymInt local_window, SymInt top_blocks, SymInt k_out, "
                           "bool strict_valid) -> (Tensor, Tensor, Tensor, Tensor)")
    assert "Tensor(a!) expanded_cache" in str(
        torch.ops.relation_lm.relation_hidden_cache_update.default._schema)
    assert "SymInt k_out" in str(torch.ops.relationlex.partner_topk.default._schema)
    assert "float norm_eps" in str(torch.ops.relation_lm.relation_norm_reduce.default._schema)
    # triton_op infers SymInt for the reference's `block_size: int` (router_cache.py:188-203).
    for op in (torch.ops.relation_lm.router_cache_update, torch.ops.relation_lm.router_cache_update_ring):
        assert str(op.default._schema).endswith("Tensor position, SymInt block_size) -> Tensor")


def test_cpu_tensors_fail_loudly():
    import torch

    from relation_lm.kernels.relation_reduce import relation_norm_reduce

    with pytest.raises(NotImplementedError):
        relation_norm_reduce(torch.zeros(1, 2, 8), torch.zeros(1, 2), torch.ones(8),
                             torch.zeros(8), torch.tensor(3), 1e-5)


def test_fake_kernels_give_shapes():
    import torch
    from torch._subclasses.fake_tensor import FakeTensorMode

    from relation_lm.kernels.relation_select import relation_select_packed_seq
    from relation_lm.kernels.relation_reduce import relation_hidden_cached_seq

    with FakeTensorMode():
        b, t, e = 2, 64, 64
        args = [torch.empty(b, t, e), torch.empty(b, t, e), torch.empty(b, t, e),
                torch.empty(b, 4, 4, 16), torch.empty(b, 4, 4, 16), torch.empty(4),
                torch.empty(4, 16), torch.empty(b, t, 2 * e), torch.empty(b, t, 2 * e),
                torch.empty(b, t, e), torch.empty(b, 4, 4, 16), torch.empty(b, 4, 4, 16),
                torch.empty(4), torch.empty(4, 16), torch.empty(t, dtype=torch.long)]
        a, s, p, ps = relation_select_packed_seq(*args, 16, 2, 6, False)
        assert a.shape == (b, t) and p.shape == (b, t, 6) and p.dtype == torch.int32
        h = relation_hidden_cached_seq(torch.empty(b, t, 64), torch.empty(b, t, 8),
                                       torch.empty(b, t, dtype=torch.int32),
                                       torch.empty(b, t, 6, dtype=torch.int32),
                                       torch.empty(32, 8))
        assert h.shape == (b, t, 6, 32) and h.dtype == torch.float32


def _multi_args(b=2, t=64, e=64, nb=4, s=3, k=4, tq=8, **override):
    d = {
        "anchor_query": tensor([b, tq, s, e]), "anchor_keys": tensor([b, t, s, e]),
        "anchor_router_query": tensor([b, tq, e]), "anchor_block_mean": tensor([b, nb, 4, e // 4]),
        "anchor_block_std": tensor([b, nb, 4, e // 4]), "anchor_gamma": tensor([4]),
        "anchor_bias": tensor([4, 16]), "partner_base": tensor([b, tq, s, 2 * e]),
        "partner_anchor_cache": tensor([b, t, s, 2 * e]), "partner_keys": tensor([b, t, s, e]),
        "partner_block_mean": tensor([b, nb, 4, e // 4]),
        "partner_block_std": tensor([b, nb, 4, e // 4]), "partner_gamma": tensor([4]),
        "partner_bias": tensor([4, 16]), "positions": tensor([tq], RLM_I64),
        "out_anchor": tensor([b, tq, s], RLM_I32), "out_anchor_score": tensor([b, tq, s]),
        "out_partner": tensor([b, tq, s, k], RLM_I32), "out_partner_score": tensor([b, tq, s, k]),
    }
    d.update(override)
    return d


def _call_multi(lib, d, local=16, top=2, k=4, strict=0):
    names = ["anchor_query", "anchor_keys", "anchor_router_query", "anchor_block_mean",
             "anchor_block_std", "anchor_gamma", "anchor_bias", "partner_base",
             "partner_anchor_cache", "partner_keys", "partner_block_mean", "partner_block_std",
             "partner_gamma", "partner_bias", "positions"]
    outs = ["out_anchor", "out_anchor_score", "out_partner", "out_partner_score"]
    args = [ctypes.byref(d[n]) for n in names] + [ctypes.c_int64(local), ctypes.c_int64(top),
                                                    ctypes.c_int64(k), ctypes.c_int32(strict)]
    args += [ctypes.byref(d[n]) for n in outs] + [ctypes.c_void_p(0)]
    return lib.rlm_multi_relation_select_seq(*args), lib.rlm_last_error().decode()


@pytest.mark.parametrize("override,needle", [
    ({"anchor_keys": tensor([2, 64, 2, 64])}, "anchor_keys"),
    ({"partner_keys": tensor([2, 64, 3, 64], RLM_BF16)}, "partner_keys"),
    ({"partner_base": tensor([2, 8, 3, 64])}, "partner_base"),
    ({"partner_anchor_cache": tensor([2, 64, 3, 64])}, "partner_anchor_cache"),
    ({"anchor_router_query": tensor([2, 8, 32])}, "anchor_router_query"),
    ({"positions": tensor([7], RLM_I64)}, "positions"),
    ({"out_partner": tensor([2, 8, 3, 5], RLM_I32)}, "out_partner"),
    ({"out_anchor": tensor([2, 8, 2], RLM_I32)}, "out_anchor"),
    ({"partner_block_mean": tensor([2, 4, 4, 8])}, "partner_block_mean"),
])
def test_multi_select_rejects_malformed_arguments(lib, override, needle):
    status, message = _call_multi(lib, _multi_args(**override))
    assert status == HIP_ERROR_INVALID_VALUE
    assert needle in message


def test_multi_select_rejects_bad_slot_counts(lib):
    status, message = _call_multi(lib, _multi_args(), local=2)
    assert status == HIP_ERROR_INVALID_VALUE and "local_window" in message
    d = _multi_args(s=9, **{})
    status, message = _call_multi(lib, d)
    assert status == HIP_ERROR_INVALID_VALUE and "slots" in message


def test_multi_select_fake_shapes():
    import torch
    from torch._subclasses.fake_tensor import FakeTensorMode

    from relation_lm.kernels.relation_select import multi_relation_select_seq

    with FakeTensorMode():
        b, t, s, e = 2, 64, 4, 64
        args = [torch.empty(b, t, s, e), torch.empty(b, t, s, e), torch.empty(b, t, e),
                torch.empty(b, 4, 4, 16), torch.empty(b, 4, 4, 16), torch.empty(4),
                torch.empty(4, 16), torch.empty(b, t, s, 2 * e), torch.empty(b, t, s, 2 * e),
                torch.empty(b, t, s, e), torch.empty(b, 4, 4, 16), torch.empty(b, 4, 4, 16),
                torch.empty(4), torch.empty(4, 16), torch.empty(t, dtype=torch.long)]
        a, sc, p, ps = multi_relation_select_seq(*args, 16, 2, 6, False)
        assert a.shape == (b, t, s) and p.shape == (b, t, s, 6) and ps.dtype == torch.float32


def test_fused_reduce_fits_from_python():
    """relation_reduce_fused_seq_fits (Python) asks the C library's predicate about torch
    tensors; CPU tensors serve, since it reads only their descriptors."""
    from relation_lm.kernels.relation_reduce import relation_reduce_fused_seq_fits

    bf = torch.bfloat16
    e, o = torch.empty(2, 64, 1024, dtype=bf), torch.empty(2, 64, 64, dtype=bf)
    pi, wm = torch.empty(2, 8, 8, dtype=torch.int32), torch.empty(512, 64, dtype=bf)
    assert relation_reduce_fused_seq_fits(e, o, pi, wm, torch.empty(512, 512, dtype=bf))
    assert not relation_reduce_fused_seq_fits(e, o, pi, wm, torch.empty(576, 512, dtype=bf))
    assert not relation_reduce_fused_seq_fits(e, o.float(), pi, wm,
                                              torch.empty(512, 512, dtype=bf))
