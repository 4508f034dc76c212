"""Factorized relation reduce on gfx950.

Mirrors src/relation_lm/kernels/relation_reduce.py:
  * ``FactorizedRelationWeights`` / ``factor_relation_first_layer`` (:11-57) --
    host-side weight algebra, pure torch, identical contract and errors;
  * ``recommended_relation_cache_mode`` (:60-69);
  * ``relation_hidden_cached`` (:149-183), ``relation_hidden_cache_update``
    (:312-357) and ``relation_norm_reduce`` (:420-450) -- HIP kernels behind the
    same ``torch.ops.relation_lm`` schemas;
plus the sequence forms ``relation_hidden_cached_seq`` /
``relation_norm_reduce_seq`` and ``relation_linear`` (the MFMA GEMM used for the
expanded-cache projection and the relation MLP's second linear).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch
from torch import Tensor

from relation_lm import _native  # noqa: F401  (registers torch.ops.relation_lm)


@dataclass(frozen=True)
class FactorizedRelationWeights:
    """First Relation-MLP layer split into reusable token contributions."""

    anchor_weight: Tensor
    partner_weight: Tensor
    product_weight: Tensor
    first_bias: Tensor
    expanded_weight: Tensor
    expanded_bias: Tensor


def factor_relation_first_layer(
    first_weight: Tensor,
    first_bias: Tensor,
    relation_dim: int,
) -> FactorizedRelationWeights:
    """Factor ``W[a,p,a*p,a-p]+b`` into anchor, partner, and product terms.

    ``(W_a + W_d) a + (W_p - W_d) p + W_m (a * p) + b`` equals the unfactorized
    layer exactly in real arithmetic.  ``expanded_weight`` = ``[W_a+W_d; W_p-W_d]``
    projects a cached operand into ``[anchor_base, partner_base]``;
    ``expanded_bias`` = ``[b; 0]`` applies the bias once.
    """
    if first_weight.ndim != 2 or first_bias.ndim != 1:
        raise ValueError("first_weight must be 2D and first_bias must be 1D")
    relation_dim = int(relation_dim)
    if first_weight.size(1) != 4 * relation_dim:
        raise ValueError("first_weight input dimension must equal 4 * relation_dim")
    blocks = first_weight.split(relation_dim, dim=1)
    anchor_weight = (blocks[0] + blocks[3]).contiguous()
    partner_weight = (blocks[1] - blocks[3]).contiguous()
    product_weight = blocks[2].contiguous()
    return FactorizedRelationWeights(
        anchor_weight=anchor_weight,
        partner_weight=partner_weight,
        product_weight=product_weight,
        first_bias=first_bias.contiguous(),
        expanded_weight=torch.cat((anchor_weight, partner_weight), dim=0).contiguous(),
        expanded_bias=torch.cat((first_bias, torch.zeros_like(first_bias)), dim=0).contiguous(),
    )


def recommended_relation_cache_mode(batch_size: int) -> str:
    """Cache-update policy for decode: fuse the current-row update at batch 1.

    Same contract as the reference (relation_reduce.py:60-69): "fused_update"
    for batch 1, "separate_update" otherwise, ValueError for batch < 1.
    """
    if batch_size < 1:
        raise ValueError("batch_size must be positive")
    return "fused_update" if batch_size == 1 else "separate_update"


def relation_hidden_cached(
    expanded_cache: Tensor,
    operand_cache: Tensor,
    anchor_index: Tensor,
    partner_index: Tensor,
    product_weight: Tensor,
) -> Tensor:
    """GELU(W_m (op[a] * op[p]) + X[a, :H] + X[p, H:]) -> f32 [B, K, H]."""
    return torch.ops.relation_lm.relation_hidden_cached(
        expanded_cache, operand_cache, anchor_index, partner_index, product_weight)


def relation_hidden_cached_seq(
    expanded_cache: Tensor,
    operand_cache: Tensor,
    anchor_index: Tensor,
    partner_index: Tensor,
    product_weight: Tensor,
) -> Tensor:
    """Sequence form: anchor [B,Tq], partner [B,Tq,K] -> f32 [B,Tq,K,H]."""
    return torch.ops.relation_lm.relation_hidden_cached_seq(
        expanded_cache, operand_cache, anchor_index, partner_index, product_weight)


def relation_hidden_cached_seq_out(
    expanded_cache: Tensor,
    operand_cache: Tensor,
    anchor_index: Tensor,
    partner_index: Tensor,
    product_weight: Tensor,
    out: Tensor,
) -> None:
    """relation_hidden_cached_seq into ``out`` [B,Tq,K,H], fp32 or bf16.  A bf16
    ``out`` holds each value rounded to nearest even -- the operand a bf16 Linear
    rounds the fp32 hidden to, so the Linear's result is the same either way."""
    torch.ops.relation_lm.relation_hidden_cached_seq_out(
        expanded_cache, operand_cache, anchor_index, partner_index, product_weight, out)


def mfma_fragments(weight: Tensor) -> Tensor:
    """A [N, K] bf16 / f16 weight in MFMA fragment order, [N/32, K/16, 64, 8]: fragment
    (nb, g) holds, for lane l, ``weight[32 nb + l % 32, 16 g + 8 (l // 32) : +8]`` -- what a
    wave's 32x32x16 matrix instruction reads, contiguous per fragment.  A packing step
    run once per weight (N % 32 == 0, K % 16 == 0)."""
    return torch.ops.relation_lm.mfma_fragments(weight)


def relation_hidden_linear_seq_fits(
    expanded_cache: Tensor,
    operand_cache: Tensor,
    product_weight: Tensor,
    second_weight: Tensor,
) -> bool:
    """True when ``relation_hidden_linear_seq_out`` takes these operands (bf16 caches and
    weights, the weights in fragment order, relation dim 64 or 128, hidden dim a multiple
    of 128, d_model 256, 512 or 768, 16-byte aligned).  Reads only shapes, dtypes and
    pointer alignment."""
    lib = _native.c_library()
    return bool(lib.rlm_relation_hidden_linear_seq_fits(
        *(ctypes.byref(_desc(t)) for t in (expanded_cache, operand_cache, product_weight,
                                           second_weight))))


def relation_hidden_linear_seq_out(
    expanded_cache: Tensor,
    operand_cache: Tensor,
    anchor_index: Tensor,
    partner_index: Tensor,
    product_weight: Tensor,
    second_weight: Tensor,
    out: Tensor,
) -> None:
    """The relation MLP's hidden and bias-free second Linear in one launch, into ``out``
    f32 [B,Tq,K,D]: ``second_weight . bf16(hidden)`` with the hidden of
    ``relation_hidden_cached_seq`` (multi_relation_blocks.py:47-52,163 of the reference:
    Linear -> GELU -> Linear, the first Linear factorized).  ``product_weight`` [H, R] and
    ``second_weight`` [D, H] come in fragment order (``mfma_fragments``).  The hidden never
    reaches memory; the result is bit-identical to ``relation_hidden_cached_seq_out`` into
    a bf16 buffer followed by ``relation_linear(..., None, torch.float32)``.  Shapes outside
    ``relation_hidden_linear_seq_fits`` raise."""
    torch.ops.relation_lm.relation_hidden_linear_seq_out(
        expanded_cache, operand_cache, anchor_index, partner_index, product_weight,
        second_weight, out)


def relation_hidden_cache_update(
    expanded_cache: Tensor,
    operand_cache: Tensor,
    anchor_index: Tensor,
    partner_index: Tensor,
    anchor_weight: Tensor,
    partner_weight: Tensor,
    product_weight: Tensor,
    first_bias: Tensor,
    position: Tensor,
) -> Tensor:
    """Writes ``expanded_cache[:, position]`` and returns the relation hidden f32 [B,K,H]."""
    return torch.ops.relation_lm.relation_hidden_cache_update(
        expanded_cache, operand_cache, anchor_index, partner_index, anchor_weight,
        partner_weight, product_weight, first_bias, position)


def relation_norm_reduce(
    raw: Tensor,
    partner_scores: Tensor,
    norm_weight: Tensor,
    norm_bias: Tensor,
    position: Tensor,
    norm_eps: float,
) -> Tensor:
    """Per-partner LayerNorm, active-K softmax and weighted sum -> f32 [B, D]."""
    return torch.ops.relation_lm.relation_norm_reduce(
        raw, partner_scores, norm_weight, norm_bias, position, float(norm_eps))


def relation_norm_reduce_seq(
    raw: Tensor,
    partner_scores: Tensor,
    norm_weight: Tensor,
    norm_bias: Tensor,
    positions: Tensor,
    norm_eps: float,
) -> Tensor:
    """Sequence form: raw [B,Tq,K,D], scores [B,Tq,K], positions [Tq] or [B,Tq] -> f32 [B,Tq,D]."""
    return torch.ops.relation_lm.relation_norm_reduce_seq(
        raw, partner_scores, norm_weight, norm_bias, positions, float(norm_eps))


def relation_norm_reduce_output(
    raw: Tensor,
    partner_scores: Tensor,
    norm_weight: Tensor,
    norm_bias: Tensor,
    position: Tensor,
    norm_eps: float,
    query: Tensor,
    mix_logit: Tensor,
    output_weight: Tensor,
    output_bias: Tensor,
    output_eps: float,
) -> tuple[Tensor, Tensor]:
    """relation_norm_reduce with the last-token output preparation fused in (the
    reference's roadmap item, README.md:150-151): returns (context f32 [B,D],
    final [B,D]) with final = output_norm(query + sigmoid(mix_logit) * context)
    as RelationLexLM.forward (relation_lm.py:203-206), in query's dtype."""
    return torch.ops.relation_lm.relation_norm_reduce_output(
        raw, partner_scores, norm_weight, norm_bias, position, float(norm_eps), query, mix_logit,
        output_weight, output_bias, float(output_eps))


def relation_norm_reduce_output_seq(
    raw: Tensor,
    partner_scores: Tensor,
    norm_weight: Tensor,
    norm_bias: Tensor,
    positions: Tensor,
    norm_eps: float,
    query: Tensor,
    mix_logit: Tensor,
    output_weight: Tensor,
    output_bias: Tensor,
    output_eps: float,
) -> tuple[Tensor, Tensor]:
    """Sequence form of relation_norm_reduce_output: query [B,Tq,D]."""
    return torch.ops.relation_lm.relation_norm_reduce_output_seq(
        raw, partner_scores, norm_weight, norm_bias, positions, float(norm_eps), query,
        mix_logit, output_weight, output_bias, float(output_eps))


def relation_linear_norm_reduce_output(
    hidden: Tensor,
    second_weight: Tensor,
    second_bias: Tensor,
    partner_scores: Tensor,
    norm_weight: Tensor,
    norm_bias: Tensor,
    position: Tensor,
    norm_eps: float,
    query: Tensor,
    mix_logit: Tensor,
    output_weight: Tensor,
    output_bias: Tensor,
    output_eps: float,
) -> tuple[Tensor, Tensor]:
    """The decode step's second linear folded into relation_norm_reduce_output:
    hidden [B,K,H] -> (context f32 [B,D], final [B,D]), the result of
    ``relation_norm_reduce_output(relation_linear(hidden, second_weight, second_bias,
    torch.float32), ...)`` (benchmarks/benchmark_relation_reduce.py:80-81 then
    relation_lm.py:203-206).

    With bf16/f16 weights and at most 64 hidden rows the linear writes fp32 partial
    products of a few hidden-dim splits into a workspace and the per-query norm kernel
    adds them (and the bias) in split order as it loads them; the summation order is
    then not the one-launch linear's, so the raw rows agree with it to fp32 rounding,
    not bit for bit.  Other shapes run the two ops."""
    return torch.ops.relation_lm.relation_linear_norm_reduce_output(
        hidden, second_weight, second_bias, partner_scores, norm_weight, norm_bias, position,
        float(norm_eps), query, mix_logit, output_weight, output_bias, float(output_eps))


def relation_hidden_linear_norm_reduce_output(
    expanded_cache: Tensor,
    operand_cache: Tensor,
    anchor_index: Tensor,
    partner_index: Tensor,
    product_weight: Tensor,
    second_weight: Tensor,
    second_bias: Tensor,
    partner_scores: Tensor,
    norm_weight: Tensor,
    norm_bias: Tensor,
    position: Tensor,
    norm_eps: float,
    query: Tensor,
    mix_logit: Tensor,
    output_weight: Tensor,
    output_bias: Tensor,
    output_eps: float,
    ring: bool = False,
) -> tuple[Tensor, Tensor]:
    """The decode step's relation tail: relation_hidden_cached (relation_reduce.py:149-183;
    ``ring``: the ring-buffer form) followed by relation_linear_norm_reduce_output -- the
    second linear, relation_norm_reduce (relation_reduce.py:420-450) and the output-head
    preparation (relation_lm.py:203-206) -- returning (context f32 [B,D], final [B,D]).

    With bf16 caches and weights, relation dim 64 or 128, hidden dim a multiple of 64 up
    to 3072, at most 8 partners and d_model up to 768 this is one launch: each workgroup
    forms a 64-column slice of the hidden rows and that slice's partial products of the
    second linear, and the last workgroups to finish sum the partials (in a fixed order)
    and run the norm-reduce.  The hidden is rounded to bf16 for the linear, as the
    two-op form's 16-bit linear does, and the partial sums are added in another order, so
    the raw rows agree with the two-op form to fp32 rounding.  Other shapes run the two
    ops (relation_hidden_linear_norm_reduce_output_fits in the C library tells which)."""
    return torch.ops.relation_lm.relation_hidden_linear_norm_reduce_output(
        expanded_cache, operand_cache, anchor_index, partner_index, product_weight,
        second_weight, second_bias, partner_scores, norm_weight, norm_bias, position,
        float(norm_eps), query, mix_logit, output_weight, output_bias, float(output_eps),
        bool(ring))


_DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.int32: 3,
               torch.int64: 4}


class _TensorDesc(ctypes.Structure):
    """The C library's ``rlm_tensor`` descriptor (include/relation_lm_hip.h)."""

    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("shape", ctypes.c_int64 * 4), ("stride", ctypes.c_int64 * 4)]


def _desc(t: Tensor) -> _TensorDesc:
    if t.dim() > 4 or t.dtype not in _DTYPE_CODE:
        raise ValueError(f"unsupported tensor for the C library: {t.dtype}, {t.dim()}-d")
    d = _TensorDesc(t.data_ptr(), _DTYPE_CODE[t.dtype], t.dim())
    for i, (n, st) in enumerate(zip(t.shape, t.stride())):
        d.shape[i], d.stride[i] = n, st
    return d


def relation_reduce_fused_seq_fits(
    expanded_cache: Tensor,
    operand_cache: Tensor,
    partner_index: Tensor,
    product_weight: Tensor,
    second_weight: Tensor,
) -> bool:
    """True when ``relation_reduce_fused_seq`` runs these operands as one fused kernel, False
    when it runs the three-launch chain instead (fp32, d_model 576, K > 16, ...).  Reads only
    shapes, dtypes and pointer alignment; launches nothing."""
    lib = _native.c_library()
    return bool(lib.rlm_relation_reduce_fused_seq_fits(
        *(ctypes.byref(_desc(t)) for t in (expanded_cache, operand_cache, partner_index,
                                           product_weight, second_weight))))


def relation_reduce_fused_seq(
    expanded_cache: Tensor,
    operand_cache: Tensor,
    anchor_index: Tensor,
    partner_index: Tensor,
    product_weight: Tensor,
    second_weight: Tensor,
    second_bias: Tensor,
    partner_scores: Tensor,
    norm_weight: Tensor,
    norm_bias: Tensor,
    positions: Tensor,
    norm_eps: float,
) -> Tensor:
    """Relation hidden -> second linear -> norm-reduce in one kernel -> f32 [B, Tq, D].

    Same result as ``relation_norm_reduce_seq(relation_linear(relation_hidden_cached_seq(...),
    second_weight, second_bias), ...)`` (the reference's three-call sequence,
    benchmarks/benchmark_relation_reduce.py:55-64) with bf16 caches and weights: the
    hidden is rounded to bf16 before the second linear, as the unfused bf16 linear does.
    Operands the fused kernel does not take (fp32, d_model outside {128, 256, 384,
    512}, K > 16, ...) run that three-op chain on HIP instead, so every shape the
    reference's ops accept goes through this op.
    """
    return torch.ops.relation_lm.relation_reduce_fused_seq(
        expanded_cache, operand_cache, anchor_index, partner_index, product_weight,
        second_weight, second_bias, partner_scores, norm_weight, norm_bias, positions,
        float(norm_eps))


def relation_linear(input: Tensor, weight: Tensor, bias: Tensor | None = None,
                    out_dtype: torch.dtype | None = None) -> Tensor:
    """``input @ weight.T + bias`` on MFMA (bf16/f16 weights) or fp32 FMA (fp32 weights)."""
    return torch.ops.relation_lm.relation_linear(input, weight, bias, out_dtype)


def relation_linear_out(input: Tensor, weight: Tensor, bias: Tensor | None, out: Tensor) -> None:
    """``out[:] = input @ weight.T + bias`` into a 2-d view whose rows may be strided
    (e.g. ``expanded_cache[:, t]``: the decode step's separate cache-row update
    written in place, relation_reduce.py:60-69's "separate_update" mode)."""
    torch.ops.relation_lm.relation_linear_out(input, weight, bias, out)
