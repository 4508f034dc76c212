"""Loads the HIP operator library and registers fake (meta) kernels.

Importing this module makes ``torch.ops.relation_lm.*`` and
``torch.ops.relationlex.*`` available.  There is no fallback: when the built
library is missing the import fails with instructions to build it, and calling
an op with CPU tensors raises (only the ROCm-device implementation exists) --
except ``packed_sparse_cache_projection``, whose CPU tensors take ``at::linear``
as the reference's ``F.linear`` does.
"""
from __future__ import annotations

import os

import torch

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib")
TORCH_LIBRARY = os.path.join(LIB_DIR, "_rlm_torch.so")
C_LIBRARY = os.path.join(LIB_DIR, "librlm_hip.so")

_loaded = False
_c_library = None


def load() -> None:
    """Load the operator library once (idempotent)."""
    global _loaded
    if _loaded:
        return
    if not os.path.exists(TORCH_LIBRARY) or not os.path.exists(C_LIBRARY):
        raise ImportError(
            "relation_lm HIP library not built: expected "
            f"{TORCH_LIBRARY} and {C_LIBRARY}. Run `make -C relation-lm_amd/csrc` "
            "(or __graft_entry__.build()) first.")
    torch.ops.load_library(TORCH_LIBRARY)
    _register_fakes()
    _loaded = True


def c_library():
    """The C-ABI library (``ctypes.CDLL``), for the host-only queries it exports."""
    global _c_library
    if _c_library is None:
        load()
        import ctypes

        _c_library = ctypes.CDLL(C_LIBRARY)
        _c_library.rlm_last_error.restype = ctypes.c_char_p
    return _c_library


def _register_fakes() -> None:
    def fake_select(anchor_query, *rest):
        k_out = rest[-2]
        seq = anchor_query.dim() == 3
        qshape = tuple(anchor_query.shape[:2] if seq else anchor_query.shape[:1])
        return (anchor_query.new_empty(qshape, dtype=torch.int32),
                anchor_query.new_empty(qshape, dtype=torch.float32),
                anchor_query.new_empty(qshape + (k_out,), dtype=torch.int32),
                anchor_query.new_empty(qshape + (k_out,), dtype=torch.float32))

    torch.library.register_fake("relation_lm::relation_select_packed")(fake_select)
    torch.library.register_fake("relation_lm::relation_select_packed_seq")(fake_select)
    torch.library.register_fake("relation_lm::relation_select_packed_ring")(fake_select)
    torch.library.register_fake("relation_lm::relation_select_packed_expand_row")(
        lambda anchor_query, *rest: fake_select(anchor_query, *rest[:18]))
    torch.library.register_fake("relation_lm::relation_select_packed_seq_expand")(
        lambda anchor_query, *rest: fake_select(anchor_query, *rest[:18]))

    @torch.library.register_fake("relation_lm::multi_relation_select_seq")
    def _(anchor_query, *rest):
        k_out = rest[-2]
        qshape = tuple(anchor_query.shape[:3])
        return (anchor_query.new_empty(qshape, dtype=torch.int32),
                anchor_query.new_empty(qshape, dtype=torch.float32),
                anchor_query.new_empty(qshape + (k_out,), dtype=torch.int32),
                anchor_query.new_empty(qshape + (k_out,), dtype=torch.float32))

    @torch.library.register_fake("relationlex::anchor_select")
    def _(anchor_query, *rest):
        b = anchor_query.shape[0]
        return (anchor_query.new_empty((b,), dtype=torch.int32),
                anchor_query.new_empty((b,), dtype=torch.float32))

    @torch.library.register_fake("relationlex::partner_topk")
    def _(partner_query, *rest):
        b, k_out = partner_query.shape[0], rest[-2]
        return (partner_query.new_empty((b, k_out), dtype=torch.int32),
                partner_query.new_empty((b, k_out), dtype=torch.float32))

    def fake_hidden(expanded_cache, operand_cache, anchor_index, partner_index, product_weight,
                    *rest):
        return operand_cache.new_empty(tuple(partner_index.shape) + (product_weight.shape[0],),
                                       dtype=torch.float32)

    torch.library.register_fake("relation_lm::relation_hidden_cached")(fake_hidden)
    torch.library.register_fake("relation_lm::relation_hidden_cached_seq")(fake_hidden)
    torch.library.register_fake("relation_lm::relation_hidden_cache_update")(fake_hidden)
    torch.library.register_fake("relation_lm::relation_hidden_cached_ring")(fake_hidden)
    torch.library.register_fake("relation_lm::relation_hidden_cache_update_ring")(fake_hidden)

    def fake_norm(raw, *rest):
        return raw.new_empty(tuple(raw.shape[:-2]) + (raw.shape[-1],), dtype=torch.float32)

    torch.library.register_fake("relation_lm::relation_norm_reduce")(fake_norm)
    torch.library.register_fake("relation_lm::relation_norm_reduce_seq")(fake_norm)

    def fake_router(anchor_raw, *rest):
        return anchor_raw.new_empty((anchor_raw.shape[0], 2, anchor_raw.shape[1]),
                                    dtype=torch.float32)

    torch.library.register_fake("relation_lm::router_cache_update")(fake_router)
    torch.library.register_fake("relation_lm::router_cache_update_ring")(fake_router)

    @torch.library.register_fake("relation_lm::relation_reduce_fused_seq")
    def _(expanded_cache, operand_cache, anchor_index, partner_index, product_weight,
          second_weight, *rest):
        d_model = second_weight.shape[0] * (32 if second_weight.dim() == 4 else 1)
        return operand_cache.new_empty(tuple(partner_index.shape[:2]) + (d_model,),
                                       dtype=torch.float32)

    @torch.library.register_fake("relation_lm::packed_projection_to_caches")
    def _(memory, weight, *rest):
        return memory.new_empty((memory.shape[0], weight.shape[0]))

    @torch.library.register_fake("relation_lm::packed_projection_router_update")
    def _(memory, weight, anchor_keys, partner_keys, operand_cache, partner_anchor_cache,
          position, ring, anchor_raw_cache, *rest):
        return (memory.new_empty((memory.shape[0], weight.shape[0])),
                memory.new_empty((memory.shape[0], 2, anchor_raw_cache.shape[2]),
                                 dtype=torch.float32))

    @torch.library.register_fake("relation_lm::packed_sparse_cache_projection")
    def _(memory, weight):
        return memory.new_empty(tuple(memory.shape[:-1]) + (weight.shape[0],))

    @torch.library.register_fake("relation_lm::relation_linear")
    def _(input, weight, bias=None, out_dtype=None):
        return input.new_empty(tuple(input.shape[:-1]) + (weight.shape[0],),
                               dtype=out_dtype or input.dtype)

    @torch.library.register_fake("relation_lm::relation_linear_out")
    def _(input, weight, bias, out):
        return None

    @torch.library.register_fake("relation_lm::relation_hidden_cached_seq_out")
    def _(expanded_cache, operand_cache, anchor_index, partner_index, product_weight, out):
        return None

    @torch.library.register_fake("relation_lm::mfma_fragments")
    def _(weight):
        return weight.new_empty((weight.shape[0] // 32, weight.shape[1] // 16, 64, 8))

    @torch.library.register_fake("relation_lm::relation_hidden_linear_seq_out")
    def _(expanded_cache, operand_cache, anchor_index, partner_index, product_weight,
          second_weight, out):
        return None

    @torch.library.register_fake("relation_lm::multi_relation_reduce_seq")
    def _(raw, partner_scores, norm_weight, norm_bias, slot_mix_logits, residual_gate, hidden,
          positions, norm_eps, raw_bias=None):
        return torch.empty_like(hidden, memory_format=torch.contiguous_format)

    @torch.library.register_fake("relation_lm::multi_relation_reduce_seq_out")
    def _(raw, partner_scores, norm_weight, norm_bias, slot_mix_logits, residual_gate, hidden,
          positions, norm_eps, raw_bias, out, context=None):
        return None

    def fake_norm_output(raw, partner_scores, norm_weight, norm_bias, position, norm_eps, query,
                         mix_logit, output_weight, output_bias, output_eps):
        shape = tuple(raw.shape[:-2]) + (raw.shape[-1],)
        return (raw.new_empty(shape, dtype=torch.float32),
                query.new_empty(shape))

    torch.library.register_fake("relation_lm::relation_norm_reduce_output")(fake_norm_output)
    torch.library.register_fake("relation_lm::relation_norm_reduce_output_seq")(fake_norm_output)

    @torch.library.register_fake("relation_lm::relation_linear_norm_reduce_output")
    def _(hidden, second_weight, second_bias, partner_scores, norm_weight, norm_bias, position,
          norm_eps, query, mix_logit, output_weight, output_bias, output_eps):
        shape = (hidden.shape[0], second_weight.shape[0])
        return (hidden.new_empty(shape, dtype=torch.float32), query.new_empty(shape))

    @torch.library.register_fake("relation_lm::relation_hidden_linear_norm_reduce_output")
    def _(expanded_cache, operand_cache, anchor_index, partner_index, product_weight,
          second_weight, second_bias, partner_scores, norm_weight, norm_bias, position, norm_eps,
          query, mix_logit, output_weight, output_bias, output_eps, ring=False):
        shape = (operand_cache.shape[0], second_weight.shape[0])
        return (operand_cache.new_empty(shape, dtype=torch.float32), query.new_empty(shape))

    @torch.library.register_fake("relation_lm::layer_norm")
    def _(input, weight, bias, eps):
        return torch.empty_like(input, memory_format=torch.contiguous_format)

    @torch.library.register_fake("relation_lm::block_statistics")
    def _(keys, block_size):
        shape = (keys.shape[0], keys.shape[1] // block_size, keys.shape[2])
        return (keys.new_empty(shape, dtype=torch.float32),
                keys.new_empty(shape, dtype=torch.float32))


load()
