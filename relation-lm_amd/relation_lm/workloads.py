"""Seeded synthetic workloads of the routed relation path.

Shapes follow the benchmark configurations of the routed relation path:

  cfg1  B=1  T=128  d=256, block 16 (8 blocks), local 32, top 2, K=8, fp32
  cfg2  B=8  T=512  d=512, block 32 (16 blocks), local 64, top 4, K=8, bf16
        activations / fp32 scores, relation hidden 512 (full sequence)
  cfg3  decode at t=511 against a 512-row cache, block 32, local 64, top 4,
        K=8, packed 576->512 bf16 projection, R=128 H=2304 D=576, B in {1, 8}
  cfg4  B=8  T=2048 d=512, K=8, hidden 1024 (reduce in isolation)
  cfg5  B=4  T=4096 d=768, block 64 (64 blocks), local 128, top 8, 4 anchor
        slots x K=6 partners, bf16 (routed multi-anchor selection, one layer
        of the 4-layer stack)

Every tensor is drawn on the CPU from one ``torch.Generator`` in a fixed order
and then copied to the device, so a CPU checker sees the same bits as the GPU.
Activations and caches ~ N(0,1); weights ~ N(0, 1/fan_in); gamma and bias ~
N(0,1); block statistics are the mean and biased std of seeded router keys
(the DistilledBlockRouter.block_statistics definition).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from relation_lm.kernels.relation_reduce import factor_relation_first_layer


@dataclass(frozen=True)
class RelationConfig:
    name: str
    batch: int
    context: int
    d_model: int
    block_size: int
    local_window: int
    top_blocks: int
    k_out: int
    dtype: torch.dtype
    relation_dim: int = 128
    hidden_dim: int = 1024
    exact_dim: int = 64
    heads: int = 4
    head_dim: int = 16
    rel_buckets: int = 16
    strict_valid: bool = False
    seed: int = 20261201

    @property
    def blocks(self) -> int:
        return self.context // self.block_size

    @property
    def queries(self) -> int:
        return self.batch * self.context


CONFIGS = {
    "cfg1": RelationConfig("cfg1", 1, 128, 256, 16, 32, 2, 8, torch.float32, hidden_dim=1024,
                           seed=20261201),
    "cfg2": RelationConfig("cfg2", 8, 512, 512, 32, 64, 4, 8, torch.bfloat16, hidden_dim=512,
                           seed=20261202),
    "cfg3": RelationConfig("cfg3", 8, 512, 576, 32, 64, 4, 8, torch.bfloat16, hidden_dim=2304,
                           seed=20261203),
    "cfg4": RelationConfig("cfg4", 8, 2048, 512, 64, 128, 4, 8, torch.bfloat16, hidden_dim=1024,
                           seed=20261204),
}


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _randn(g, *shape, scale: float = 1.0, dtype=torch.float32) -> torch.Tensor:
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def block_statistics(keys: torch.Tensor, block_size: int, heads: int, head_dim: int):
    """Per-block mean and biased std, [B, NB, heads, head_dim] (block_router.py:54-68)."""
    batch, length, _ = keys.shape
    grouped = keys.float().view(batch, length // block_size, block_size, heads, head_dim)
    return grouped.mean(2).contiguous(), grouped.std(2, unbiased=False).contiguous()


def selection_inputs(cfg: RelationConfig, *, queries: int | None = None,
                     device: torch.device | str = "cpu", seed: int | None = None) -> dict:
    """Inputs of relation_select_packed(_seq).

    ``queries=None`` gives the sequence form (one query per cache position, query
    tensors [B,T,*]); ``queries=1`` gives the decode form (query tensors [B,*]).
    """
    g = _gen(cfg.seed if seed is None else seed)
    b, t, e = cfg.batch, cfg.context, cfg.exact_dim
    rd = cfg.heads * cfg.head_dim
    q = t if queries is None else queries
    qshape = (b, q) if queries is None else (b,)
    act = cfg.dtype
    out = {
        "anchor_query": _randn(g, *qshape, e, dtype=act),
        "anchor_keys": _randn(g, b, t, e, dtype=act),
        "anchor_router_query": _randn(g, *qshape, rd, dtype=act),
        "partner_base": _randn(g, *qshape, 2 * e, dtype=act),
        "partner_anchor_cache": _randn(g, b, t, 2 * e, dtype=act),
        "partner_keys": _randn(g, b, t, e, dtype=act),
    }
    for side in ("anchor", "partner"):
        router_keys = _randn(g, b, t, rd, dtype=act)
        mean, std = block_statistics(router_keys, cfg.block_size, cfg.heads, cfg.head_dim)
        out[f"{side}_block_mean"] = mean
        out[f"{side}_block_std"] = std
        out[f"{side}_gamma"] = _randn(g, cfg.heads)
        out[f"{side}_bias"] = _randn(g, cfg.heads, cfg.rel_buckets)
    if queries is None:
        out["positions"] = torch.arange(t, dtype=torch.int64)
    else:
        out["position"] = torch.tensor(t - 1, dtype=torch.int64)
    return {k: v.to(device) for k, v in out.items()}


@dataclass(frozen=True)
class MultiAnchorConfig:
    name: str
    batch: int
    context: int
    d_model: int
    block_size: int
    local_window: int
    top_blocks: int
    slots: int
    k_out: int
    dtype: torch.dtype
    layers: int = 1
    exact_dim: int = 64
    heads: int = 4
    head_dim: int = 16
    rel_buckets: int = 16
    strict_valid: bool = False
    seed: int = 20261205

    @property
    def blocks(self) -> int:
        return self.context // self.block_size

    @property
    def queries(self) -> int:
        return self.batch * self.context


MULTI_CONFIGS = {
    "cfg5": MultiAnchorConfig("cfg5", 4, 4096, 768, 64, 128, 8, 4, 6, torch.bfloat16, layers=4),
}


def multi_selection_inputs(cfg: MultiAnchorConfig, *, positions=None,
                           device: torch.device | str = "cpu", seed: int | None = None) -> dict:
    """Inputs of multi_relation_select_seq: per-slot exact queries/keys
    [B,*,S,E], per-slot partner rows [B,*,S,E+RD], one anchor router query per
    query and block statistics of seeded router keys.  ``positions`` (default:
    every cache position) sets the queries."""
    g = _gen(cfg.seed if seed is None else seed)
    b, t, e, s = cfg.batch, cfg.context, cfg.exact_dim, cfg.slots
    rd = cfg.heads * cfg.head_dim
    pos = torch.arange(t, dtype=torch.int64) if positions is None else torch.as_tensor(
        positions, dtype=torch.int64)
    q = pos.shape[-1]
    act = cfg.dtype
    out = {
        "anchor_query": _randn(g, b, q, s, e, dtype=act),
        "anchor_keys": _randn(g, b, t, s, e, dtype=act),
        "anchor_router_query": _randn(g, b, q, rd, dtype=act),
        "partner_base": _randn(g, b, q, s, e + rd, dtype=act),
        "partner_anchor_cache": _randn(g, b, t, s, e + rd, dtype=act),
        "partner_keys": _randn(g, b, t, s, e, dtype=act),
    }
    for side in ("anchor", "partner"):
        router_keys = _randn(g, b, t, rd, dtype=act)
        mean, std = block_statistics(router_keys, cfg.block_size, cfg.heads, cfg.head_dim)
        out[f"{side}_block_mean"] = mean
        out[f"{side}_block_std"] = std
        out[f"{side}_gamma"] = _randn(g, cfg.heads)
        out[f"{side}_bias"] = _randn(g, cfg.heads, cfg.rel_buckets)
    out["positions"] = pos
    return {k: v.to(device) for k, v in out.items()}


def multi_select_args(inputs: dict, cfg: MultiAnchorConfig) -> tuple:
    """Positional arguments of multi_relation_select_seq."""
    return tuple(inputs[k] for k in SELECT_ORDER) + (
        inputs["positions"], cfg.local_window, cfg.top_blocks, cfg.k_out, cfg.strict_valid)


def router_cache_inputs(cfg: RelationConfig, *, device: torch.device | str = "cpu",
                        seed: int | None = None) -> dict:
    """Decode-time router state of both streams for router_cache_update: raw and
    conv caches [B,T,RD] (fp32, N(0,1)) and depthwise conv weights [RD,3]
    (N(0,1) * 0.1, the scale of the reference's test)."""
    g = _gen((cfg.seed if seed is None else seed) + 7919)
    b, t, rd = cfg.batch, cfg.context, cfg.heads * cfg.head_dim
    out = {}
    for side in ("anchor", "partner"):
        out[f"{side}_raw_cache"] = _randn(g, b, t, rd)
        out[f"{side}_conv_cache"] = _randn(g, b, t, rd)
        out[f"{side}_conv_weight"] = _randn(g, rd, 3, scale=0.1)
    return {k: v.to(device) for k, v in out.items()}


SELECT_ORDER = ("anchor_query", "anchor_keys", "anchor_router_query", "anchor_block_mean",
                "anchor_block_std", "anchor_gamma", "anchor_bias", "partner_base",
                "partner_anchor_cache", "partner_keys", "partner_block_mean",
                "partner_block_std", "partner_gamma", "partner_bias")


def select_args(inputs: dict, cfg: RelationConfig) -> tuple:
    """Positional arguments of relation_select_packed(_seq) in reference order."""
    position = inputs["positions"] if "positions" in inputs else inputs["position"]
    return tuple(inputs[k] for k in SELECT_ORDER) + (
        position, cfg.local_window, cfg.top_blocks, cfg.k_out, cfg.strict_valid)


def reduce_inputs(cfg: RelationConfig, *, device: torch.device | str = "cpu",
                  seed: int | None = None) -> dict:
    """Operand cache, factorized first layer, second linear and LayerNorm parameters."""
    g = _gen((cfg.seed if seed is None else seed) + 7919)
    b, t, r, h, d = cfg.batch, cfg.context, cfg.relation_dim, cfg.hidden_dim, cfg.d_model
    act = cfg.dtype
    operand = _randn(g, b, t, r, dtype=act)
    first_weight = _randn(g, h, 4 * r, scale=(4 * r) ** -0.5)
    first_bias = _randn(g, h, scale=0.01)
    factors = factor_relation_first_layer(first_weight, first_bias, r)
    out = {
        "operand_cache": operand,
        "first_weight": first_weight.to(act),
        "first_bias": first_bias.to(act),
        "anchor_weight": factors.anchor_weight.to(act),
        "partner_weight": factors.partner_weight.to(act),
        "product_weight": factors.product_weight.to(act),
        "expanded_weight": factors.expanded_weight.to(act),
        "expanded_bias": factors.expanded_bias.to(act),
        "second_weight": _randn(g, d, h, scale=h ** -0.5, dtype=act),
        "second_bias": _randn(g, d, scale=0.01, dtype=act),
        "norm_weight": (1.0 + _randn(g, d, scale=0.05)).to(act),
        "norm_bias": _randn(g, d, scale=0.01, dtype=act),
    }
    return {k: v.to(device) for k, v in out.items()}


def packed_projection_inputs(cfg: RelationConfig, *, device="cpu", seed: int | None = None):
    """Memory rows [B, 576] and the six packed weights (widths 64,64,128,128,64,64)."""
    g = _gen((cfg.seed if seed is None else seed) + 104729)
    widths = (64, 64, 128, 128, 64, 64)
    memory = _randn(g, cfg.batch, cfg.d_model, dtype=cfg.dtype)
    weights = tuple(_randn(g, w, cfg.d_model, scale=cfg.d_model ** -0.5, dtype=cfg.dtype)
                    for w in widths)
    return memory.to(device), tuple(w.to(device) for w in weights)


def causal_partner_indices(cfg: RelationConfig, seed: int):
    """Config-4 style reduce inputs: per query one anchor and K partners drawn
    uniformly over the causal history [0, t], partners distinct from the anchor,
    and N(0,1) partner scores.  Query 0 has no position besides its anchor, so
    its partner slots carry the select op's sentinel (t - local_window + 1, -inf).
    Returns (anchor [B,T] int32, partner [B,T,K] int32, scores [B,T,K], positions [T])
    on the CPU."""
    g = _gen(seed)
    B, T, K = cfg.batch, cfg.context, cfg.k_out
    pos = torch.arange(T)
    anchor = (torch.rand(B, T, generator=g) * (pos + 1)).long()
    draw = (torch.rand(B, T, K, generator=g) * pos[None, :, None].clamp(min=1)).long()
    partner = draw + (draw >= anchor[:, :, None]).long()  # uniform over [0, t] without the anchor
    scores = torch.randn(B, T, K, generator=g)
    partner[:, 0, :] = 0 - cfg.local_window + 1
    scores[:, 0, :] = -torch.inf
    return anchor.int(), partner.int(), scores, pos


def decode_state(cfg: RelationConfig, *, device: torch.device | str, position: int | None = None,
                 seed: int | None = None) -> dict:
    """State of the cfg3 decode step: selection inputs (query side for one token,
    caches and block statistics), reduce inputs with the expanded cache, the
    packed 576->512 projection and a memory row, the router state of both
    streams and the output-head preparation inputs (the token's query stream,
    the relation mix logit, output_norm; relation_lm.py:203-206).

    ``position`` (default: the last cache row) is the token's absolute
    position; past the cache length the step runs on ring-buffer caches."""
    from relation_lm.inference import pack_sparse_cache_projection_weights
    from relation_lm.kernels.relation_reduce import relation_linear

    st = {"sel": selection_inputs(cfg, queries=1, device=device, seed=seed),
          "red": reduce_inputs(cfg, device=device, seed=seed),
          "router": router_cache_inputs(cfg, device=device, seed=seed)}
    st["expanded_cache"] = relation_linear(st["red"]["operand_cache"],
                                           st["red"]["expanded_weight"],
                                           st["red"]["expanded_bias"])
    memory, weights = packed_projection_inputs(cfg, device=device, seed=seed)
    st["memory"] = memory
    st["projection"] = pack_sparse_cache_projection_weights(weights)
    t = cfg.context - 1 if position is None else int(position)
    st["sel"]["position"] = torch.tensor(t, dtype=torch.int64, device=device)
    st["ring"] = t >= cfg.context
    g = _gen((cfg.seed if seed is None else seed) + 3)
    st["head"] = {"query": _randn(g, cfg.batch, cfg.d_model, dtype=cfg.dtype).to(device),
                  "mix": torch.tensor(-1.0, device=device),
                  "weight": (1 + _randn(g, cfg.d_model, scale=0.1)).to(device, cfg.dtype),
                  "bias": _randn(g, cfg.d_model, scale=0.1, dtype=cfg.dtype).to(device)}
    return st


# Grid size up to which the one-launch decode tail is the faster form on MI355X.  Two
# of its workgroups fit a CU (122 VGPRs a lane, 55.6 KB of LDS), so cfg3 at B=8 (288
# workgroups) is resident at once, yet its tail takes 24.6 us there against 18.9 us
# for the three launches of the split form; at B=1 (36 workgroups) it takes 14.8 us.
ONE_ROUND_WORKGROUPS = 256


def decode_step(st: dict, cfg: RelationConfig) -> tuple:
    """One decode step on ``decode_state`` tensors, the launch sequence the
    benchmark times:
      1. packed projection of the memory row, writing the token's rows of the
         anchor / partner key, operand and partner-anchor caches, with the
         router cache update of both streams folded in (one launch);
      2. relation_select_packed with the token's expanded-cache row projected by
         extra workgroups of the same launch;
      3. the relation tail: while its grid (one workgroup per query and 64 hidden
         columns; 36 per query at cfg3) stays within ONE_ROUND_WORKGROUPS, one
         launch -- the cached relation hidden, the second linear over slices of the
         hidden dim and the norm-reduce with the output-head preparation
         (relation_hidden_linear_norm_reduce_output); beyond that (cfg3 at B=8)
         the two-launch form is faster on MI355X: relation_hidden_cached(_ring),
         then relation_linear_norm_reduce_output (the split-K linear and the
         norm-reduce).
    The caches are updated in place at the state's position (ring: mod T).
    Returns (anchor, anchor_score, partner, partner_score, context, final)."""
    from relation_lm.kernels.relation_reduce import (
        relation_hidden_cached,
        relation_hidden_linear_norm_reduce_output,
        relation_linear_norm_reduce_output,
    )
    from relation_lm.kernels.relation_select import relation_select_packed_expand_row
    from relation_lm.kernels.ring import relation_hidden_cached_ring

    sel, red, rc, head = st["sel"], st["red"], st["router"], st["head"]
    ring, position, expanded = st["ring"], sel["position"], st["expanded_cache"]
    st["projection"].project_into_routed(
        st["memory"], sel["anchor_keys"], sel["partner_keys"], red["operand_cache"],
        sel["partner_anchor_cache"], position, rc["anchor_raw_cache"], rc["partner_raw_cache"],
        rc["anchor_conv_cache"], rc["partner_conv_cache"], sel["anchor_block_mean"],
        sel["anchor_block_std"], sel["partner_block_mean"], sel["partner_block_std"],
        rc["anchor_conv_weight"], rc["partner_conv_weight"], cfg.block_size, ring=ring)
    a, s, p, ps = relation_select_packed_expand_row(
        *select_args(sel, cfg), red["operand_cache"], red["expanded_weight"],
        red["expanded_bias"], expanded, ring)
    tail = (red["second_weight"], red["second_bias"], ps, red["norm_weight"], red["norm_bias"],
            position, 1e-5, head["query"], head["mix"], head["weight"], head["bias"], 1e-5)
    if a.shape[0] * (red["product_weight"].shape[0] // 64) <= ONE_ROUND_WORKGROUPS:
        context, final = relation_hidden_linear_norm_reduce_output(
            expanded, red["operand_cache"], a, p, red["product_weight"], *tail, ring=ring)
    else:
        cached = relation_hidden_cached_ring if ring else relation_hidden_cached
        hidden = cached(expanded, red["operand_cache"], a, p, red["product_weight"])
        context, final = relation_linear_norm_reduce_output(hidden, *tail)
    return a, s, p, ps, context, final
