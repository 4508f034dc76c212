"""Multi-anchor relation block and block stack on the routed HIP path.

Mirrors ``relation_lm.models.multi_relation_blocks`` of the reference
(src/relation_lm/models/multi_relation_blocks.py:10-207): the same config
fields, parameter names and forward contract ``(hidden, memory) -> (output,
diagnostics)``, with the dense O(T^2) selection replaced by the routed
multi-anchor selection (local window plus the top blocks of a block router,
``multi_relation_select_seq``) and every step run by the HIP library:

  input_norm                      relation_lm::layer_norm
  projections of hidden / memory  relation_lm::relation_linear (MFMA)
  router block statistics         relation_lm::block_statistics
  distinct anchors, partners      relation_lm::multi_relation_select_seq
  relation MLP Linear -> GELU     relation_lm::relation_hidden_linear_seq_out: one
    -> Linear (bias-free)           kernel (factorized first Linear: operand cache,
                                    expanded cache = [W_a+W_d; W_p-W_d] op + [b; 0];
                                    the bf16 hidden stays on chip; fp32 output)
    other shapes                    relation_lm::relation_hidden_cached_seq_out, then
                                    relation_lm::relation_linear (MFMA DMA-tile GEMM)
  second Linear's bias, LayerNorm, relation_lm::multi_relation_reduce_seq
    partner softmax, slot mix,
    residual gate
  final_norm (stack)              relation_lm::layer_norm

When the sequence is no longer than the local window every causal position is
a candidate and the routed selection equals the reference's dense one, so the
block then computes the reference block's function (tests/test_multi_block_gpu.py).

Routing parameters beyond the reference's: per-side router projections of the
query (``anchor_router_query``, and per slot ``partner_router_query`` over
cat(query, anchor) like ``partner_query``) and of the memory
(``anchor_router_key`` / ``partner_router_key``, whose block mean and std feed
the block scores), plus the per-head ``*_router_gamma`` and distance-bucket
``*_router_bias`` of DistilledBlockRouter (routing/block_router.py).

Inference only: dropout is not applied (the reference's ``nn.Dropout`` in eval
mode), and parameters are packed for the kernels on first use and re-packed
whenever one of them changes.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor, nn

from relation_lm import _native  # noqa: F401  (registers torch.ops.relation_lm)
from relation_lm.kernels.relation_reduce import (factor_relation_first_layer, mfma_fragments,
                                                 relation_hidden_linear_seq_fits)

ops = torch.ops.relation_lm


@dataclass
class MultiRelationBlockConfig:
    d_model: int
    gate_dim: int
    relation_dim: int
    ff_mult: int = 4
    anchors_per_block: int = 2
    partners_per_anchor: int = 4
    dropout: float = 0.0
    # Routing (no counterpart in the reference's dense block).
    block_size: int = 64
    local_window: int = 128
    top_blocks: int = 8
    router_heads: int = 4
    router_head_dim: int = 16
    rel_buckets: int = 16
    strict_valid: bool = False
    norm_eps: float = 1e-5


class MultiAnchorRelationBlock(nn.Module):
    """A causal relation layer with several anchor slots per query (routed).

    As the reference: active anchor slots are distinct, partner selection
    excludes every active anchor of the query, and only min(H, t + 1) slots are
    active at position t.
    """

    def __init__(self, cfg: MultiRelationBlockConfig) -> None:
        super().__init__()
        self.cfg = cfg
        h, d, g, r = cfg.anchors_per_block, cfg.d_model, cfg.gate_dim, cfg.relation_dim
        rd = cfg.router_heads * cfg.router_head_dim
        hidden = cfg.ff_mult * d
        self.input_norm = nn.LayerNorm(d)
        self.anchor_query = nn.Linear(d, h * g, bias=False)
        self.anchor_key = nn.Linear(d, h * g, bias=False)
        self.partner_query = nn.ModuleList(nn.Linear(2 * d, g, bias=False) for _ in range(h))
        self.partner_key = nn.Linear(d, h * g, bias=False)
        self.operand = nn.Linear(d, r, bias=False)
        self.relation_mlp = nn.Sequential(
            nn.Linear(4 * r, hidden),
            nn.GELU(),
            nn.Linear(hidden, d),
            nn.LayerNorm(d),
        )
        self.slot_mix_logits = nn.Parameter(torch.zeros(h))
        self.residual_gate = nn.Parameter(torch.tensor(-1.5))
        self.dropout = nn.Dropout(cfg.dropout)
        self.anchor_router_query = nn.Linear(d, rd, bias=False)
        self.anchor_router_key = nn.Linear(d, rd, bias=False)
        self.partner_router_query = nn.ModuleList(nn.Linear(2 * d, rd, bias=False)
                                                  for _ in range(h))
        self.partner_router_key = nn.Linear(d, rd, bias=False)
        self.anchor_router_gamma = nn.Parameter(torch.zeros(cfg.router_heads))
        self.anchor_router_bias = nn.Parameter(torch.zeros(cfg.router_heads, cfg.rel_buckets))
        self.partner_router_gamma = nn.Parameter(torch.zeros(cfg.router_heads))
        self.partner_router_bias = nn.Parameter(torch.zeros(cfg.router_heads, cfg.rel_buckets))
        self._packed = None
        self._packed_key = None

    # -- kernel-side parameter layout ---------------------------------------
    def _pack(self) -> dict:
        key = tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in self.parameters())
        if self._packed is not None and self._packed_key == key:
            return self._packed
        d = self.cfg.d_model
        with torch.no_grad():
            query_side = [torch.cat((q.weight[:, :d], rq.weight[:, :d]), dim=0)
                          for q, rq in zip(self.partner_query, self.partner_router_query)]
            memory_side = [torch.cat((q.weight[:, d:], rq.weight[:, d:]), dim=0)
                           for q, rq in zip(self.partner_query, self.partner_router_query)]
            mlp = self.relation_mlp
            factors = factor_relation_first_layer(mlp[0].weight, mlp[0].bias, self.cfg.relation_dim)
            self._packed = {
                "partner_base_weight": torch.cat(query_side, dim=0).contiguous(),
                "partner_cache_weight": torch.cat(memory_side, dim=0).contiguous(),
                "expanded_weight": factors.expanded_weight,
                "expanded_bias": factors.expanded_bias,
                "product_weight": factors.product_weight,
            }
            # The relation MLP's product and second-Linear weights in MFMA fragment
            # order, for the one-launch relation MLP (bf16 on the GPU only).
            wm, w2 = factors.product_weight, mlp[2].weight
            if (wm.is_cuda and wm.dtype == torch.bfloat16 and w2.dtype == torch.bfloat16
                    and wm.shape[0] % 32 == 0 and wm.shape[1] % 16 == 0
                    and w2.shape[0] % 32 == 0 and w2.shape[1] % 16 == 0):
                self._packed["product_weight_frags"] = mfma_fragments(wm.contiguous())
                self._packed["second_weight_frags"] = mfma_fragments(w2.contiguous())
        self._packed_key = key
        return self._packed

    def _memory_side(self, memory: Tensor, packed: dict) -> dict:
        """Everything the layer derives from the memory alone (keys, caches, block
        statistics): the routed form of anchor_key / partner_key / operand applied
        to every memory row once."""
        cfg = self.cfg
        b, t, _ = memory.shape
        h, g, r = cfg.anchors_per_block, cfg.gate_dim, cfg.relation_dim
        nh, hd = cfg.router_heads, cfg.router_head_dim
        out = {
            "anchor_keys": ops.relation_linear(memory, self.anchor_key.weight).view(b, t, h, g),
            "partner_keys": ops.relation_linear(memory, self.partner_key.weight).view(b, t, h, g),
            "partner_anchor_cache": ops.relation_linear(memory, packed["partner_cache_weight"]
                                                        ).view(b, t, h, g + nh * hd),
        }
        for side, layer in (("anchor", self.anchor_router_key), ("partner", self.partner_router_key)):
            mean, std = ops.block_statistics(ops.relation_linear(memory, layer.weight),
                                             cfg.block_size)
            out[f"{side}_block_mean"] = mean.view(b, t // cfg.block_size, nh, hd)
            out[f"{side}_block_std"] = std.view(b, t // cfg.block_size, nh, hd)
        operand = ops.relation_linear(memory, self.operand.weight)
        out["operand_cache"] = operand
        out["expanded_cache"] = ops.relation_linear(operand, packed["expanded_weight"],
                                                    packed["expanded_bias"])
        assert operand.shape[-1] == r
        return out

    def select(self, hidden: Tensor, memory: Tensor) -> dict:
        """input_norm, the projections, router statistics and the routed selection.
        Returns the selection op's arguments ("select_args") and outputs, and the
        memory-side caches the relation MLP reads."""
        cfg = self.cfg
        batch, length, _ = hidden.shape
        h, k_count, g = cfg.anchors_per_block, cfg.partners_per_anchor, cfg.gate_dim
        if length < k_count:
            raise ValueError("sequence length must be >= partners_per_anchor")
        if length % cfg.block_size != 0:
            raise ValueError("sequence length must be a multiple of block_size")
        packed = self._pack()
        positions = torch.arange(length, device=hidden.device)
        normalized = ops.layer_norm(hidden, self.input_norm.weight, self.input_norm.bias,
                                    self.input_norm.eps)
        mem = self._memory_side(memory, packed)
        rd = cfg.router_heads * cfg.router_head_dim
        args = (
            ops.relation_linear(normalized, self.anchor_query.weight).view(batch, length, h, g),
            mem["anchor_keys"],
            ops.relation_linear(normalized, self.anchor_router_query.weight),
            mem["anchor_block_mean"], mem["anchor_block_std"], self.anchor_router_gamma,
            self.anchor_router_bias,
            ops.relation_linear(normalized, packed["partner_base_weight"]
                                ).view(batch, length, h, g + rd),
            mem["partner_anchor_cache"], mem["partner_keys"], mem["partner_block_mean"],
            mem["partner_block_std"], self.partner_router_gamma, self.partner_router_bias,
            positions, cfg.local_window, cfg.top_blocks, k_count, cfg.strict_valid)
        anchor, anchor_score, partner, partner_score = ops.multi_relation_select_seq(*args)
        return {"select_args": args, "positions": positions, "normalized": normalized,
                "anchor": anchor, "anchor_score": anchor_score, "partner": partner,
                "partner_score": partner_score, "operand_cache": mem["operand_cache"],
                "expanded_cache": mem["expanded_cache"], "product_weight": packed["product_weight"],
                "product_weight_frags": packed.get("product_weight_frags"),
                "second_weight_frags": packed.get("second_weight_frags")}

    def relate(self, hidden: Tensor, sel: dict, context: Tensor | None = None) -> Tensor:
        """The relation MLP over every (query, slot, partner) row of the selection,
        the partner and slot mixing, and the residual gate.  ``context`` (fp32,
        hidden's shape), when given, receives the block's relation context."""
        cfg = self.cfg
        batch, length, d = hidden.shape
        h, k_count = cfg.anchors_per_block, cfg.partners_per_anchor
        mlp = self.relation_mlp
        output = torch.empty_like(hidden, memory_format=torch.contiguous_format)
        wm_frags, w2_frags = sel.get("product_weight_frags"), sel.get("second_weight_frags")
        if wm_frags is not None and relation_hidden_linear_seq_fits(
                sel["expanded_cache"], sel["operand_cache"], wm_frags, w2_frags):
            # The hidden and the bias-free second Linear in one launch (the
            # hidden never reaches memory); the second Linear's bias joins the
            # rows as the slot reduce loads them.  Equal groups of batch rows,
            # each group's fp32 rows below the 2 GiB a kernel addresses.
            raw_bytes = length * h * k_count * d * 4
            most = max(1, min(batch, (2**31 - 1) // raw_bytes))
            group = -(-batch // -(-batch // most))
            raw = torch.empty((group, length * h, k_count, d), dtype=torch.float32,
                              device=hidden.device)
            for b0 in range(0, batch, group):
                b1 = min(batch, b0 + group)
                n = b1 - b0
                part = raw[:n]
                ops.relation_hidden_linear_seq_out(
                    sel["expanded_cache"][b0:b1], sel["operand_cache"][b0:b1],
                    sel["anchor"][b0:b1].reshape(n, length * h),
                    sel["partner"][b0:b1].reshape(n, length * h, k_count), wm_frags, w2_frags,
                    part)
                ops.multi_relation_reduce_seq_out(
                    part.view(n, length, h, k_count, d), sel["partner_score"][b0:b1],
                    mlp[3].weight, mlp[3].bias, self.slot_mix_logits, self.residual_gate,
                    hidden[b0:b1], sel["positions"], mlp[3].eps, mlp[2].bias, output[b0:b1],
                    None if context is None else context[b0:b1])
            return output
        # Other shapes: the hidden, then the second Linear.
        # The MLP hidden in the second Linear's operand dtype: a bf16 Linear
        # rounds an fp32 hidden to bf16 before its products, so storing bf16
        # gives the same result at half the bytes.  A few batch rows at a time:
        # the [rows, T*S, K, hidden] hidden of a group stays below the 2 GiB a
        # kernel addresses, and the groups are of equal size so that each
        # second Linear fills the chip alike.
        hid_dtype = torch.bfloat16 if mlp[2].weight.dtype == torch.bfloat16 else torch.float32
        width = mlp[2].weight.shape[1]
        row_bytes = length * h * k_count * width * torch.empty((), dtype=hid_dtype).element_size()
        most = max(1, min(batch, (2**31 - 1) // row_bytes))
        group = -(-batch // -(-batch // most))
        rows = torch.empty((group, length * h, k_count, width), dtype=hid_dtype,
                           device=hidden.device)
        for b0 in range(0, batch, group):
            b1 = min(batch, b0 + group)
            n = b1 - b0
            part = rows[:n]
            ops.relation_hidden_cached_seq_out(
                sel["expanded_cache"][b0:b1], sel["operand_cache"][b0:b1],
                sel["anchor"][b0:b1].reshape(n, length * h),
                sel["partner"][b0:b1].reshape(n, length * h, k_count), sel["product_weight"],
                part)
            # The second Linear with its bias, fp32 output (the LayerNorm that
            # follows reads the rows unrounded).
            raw = ops.relation_linear(part, mlp[2].weight, mlp[2].bias, torch.float32)
            ops.multi_relation_reduce_seq_out(
                raw.view(n, length, h, k_count, d), sel["partner_score"][b0:b1], mlp[3].weight,
                mlp[3].bias, self.slot_mix_logits, self.residual_gate, hidden[b0:b1],
                sel["positions"], mlp[3].eps, None, output[b0:b1],
                None if context is None else context[b0:b1])
        return output

    def forward(self, hidden: Tensor, memory: Tensor) -> tuple[Tensor, dict[str, Tensor]]:
        sel = self.select(hidden, memory)
        output = self.relate(hidden, sel)
        h = self.cfg.anchors_per_block
        positions = sel["positions"]
        anchor_active = torch.arange(h, device=hidden.device)[None, :] <= positions[:, None]
        return output, {
            "anchor_index": sel["anchor"],
            "anchor_active": anchor_active[None].expand(hidden.shape[0], -1, -1),
            "partner_index": sel["partner"],
            "partner_active": torch.isfinite(sel["partner_score"]),
            "partner_score": sel["partner_score"],
        }


class RelationBlockStack(nn.Module):
    """Sequential relation depth (reference: multi_relation_blocks.py:190-207)."""

    def __init__(self, cfg: MultiRelationBlockConfig, num_blocks: int) -> None:
        super().__init__()
        self.blocks = nn.ModuleList(MultiAnchorRelationBlock(cfg) for _ in range(int(num_blocks)))
        self.final_norm = nn.LayerNorm(cfg.d_model)

    def forward(self, hidden: Tensor, memory: Tensor) -> tuple[Tensor, list[dict[str, Tensor]]]:
        diagnostics = []
        for block in self.blocks:
            hidden, block_diagnostics = block(hidden, memory)
            diagnostics.append(block_diagnostics)
        return (ops.layer_norm(hidden, self.final_norm.weight, self.final_norm.bias,
                               self.final_norm.eps), diagnostics)
