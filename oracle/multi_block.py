"""Multi-anchor relation block after selection -- TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py).

Restates in numpy float64, from src/relation_lm/models/multi_relation_blocks.py:
  * the relation features and MLP of every (query, slot, partner) row,
    Linear -> GELU -> Linear -> LayerNorm on [a, p, a*p, a-p] of the operand
    projections of the gathered anchor and partner rows (:47-52, :148-163);
  * the per-slot partner weights: softmax over the K partners with inactive ones
    (non-finite score) at -1e4, times the active mask, renormalised by
    max(sum, 1e-9) -- no k_limit (:164-168);
  * the slot context, masked by slot activity (:169-170);
  * the slot mix: softmax(slot_mix_logits) times activity, renormalised by
    max(sum, 1e-9) (:172-176), and the context (:177);
  * output = hidden + sigmoid(residual_gate) * context (:178);
  * RelationBlockStack: the blocks in order, then final_norm (:190-207);
  * block statistics of router keys (routing/block_router.py:54-68).
Slot s of the query at position t is active iff s <= t (:82-84).

``block_post_selection`` takes the selection (anchor / partner indices and the
partner scores) as given, so it applies to the dense selection of the reference
and to the routed one of this library alike.  ``multi_relation_reduce_seq`` is
the contract of the library op of the same name: the block's steps after the
relation MLP's second Linear.

Parity pins (tests/test_oracle_multi_block.py):
  * against a dense torch forward of the reference's module structure
    (nn.Linear / nn.LayerNorm / nn.GELU modules, F.one_hot masks, torch.topk)
    in float64 on tiny shapes, through the dense selection's outputs;
  * invariants: a residual gate of -inf returns the input; the output does not
    depend on the order of a slot's partners; the slot weights of a query sum
    to 1 over its active slots; a slot whose partners are all inactive adds 0.
"""
from __future__ import annotations

import numpy as np
from scipy.special import erf


def _f64(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float64)


def layer_norm(x, weight, bias, eps: float) -> np.ndarray:
    """Biased-variance LayerNorm over the last axis (nn.LayerNorm)."""
    x = _f64(x)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + float(eps)) * _f64(weight) + _f64(bias)


def gelu(x) -> np.ndarray:
    """Exact-erf GELU (nn.GELU())."""
    x = _f64(x)
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


def slot_activity(positions, slots: int) -> np.ndarray:
    """[..., S] bool: slot s active iff s <= t."""
    t = np.asarray(positions, dtype=np.int64)
    return np.arange(slots)[None, :] <= t.reshape(-1)[:, None]


def partner_weights(scores) -> np.ndarray:
    """Per-slot partner weights from top scores [..., K] (:164-168)."""
    s = _f64(scores)
    active = np.isfinite(s)
    safe = np.where(active, s, -1.0e4)
    e = np.exp(safe - safe.max(axis=-1, keepdims=True))
    prob = e / e.sum(axis=-1, keepdims=True) * active
    return prob / np.maximum(prob.sum(axis=-1, keepdims=True), 1.0e-9)


def slot_weights(slot_mix_logits, active) -> np.ndarray:
    """softmax(logits) * active, renormalised (:172-176); active [Q,S]."""
    z = _f64(slot_mix_logits)
    w = np.exp(z - z.max())
    w = w / w.sum()
    a = w[None, :] * active
    return a / np.maximum(a.sum(axis=-1, keepdims=True), 1.0e-9)


def mix(relation, scores, active, slot_mix_logits, hidden, residual_gate):
    """Partner weights, slot context, slot mix and residual gate (:164-178).

    relation [Q,S,K,D] (the LayerNorm'd MLP output), scores [Q,S,K], active
    [Q,S] bool, hidden [Q,D].  Returns (output [Q,D], context [Q,D])."""
    pw = partner_weights(scores)
    slot_context = np.einsum("qsk,qskd->qsd", pw, _f64(relation)) * active[..., None]
    sw = slot_weights(slot_mix_logits, active)
    context = np.einsum("qs,qsd->qd", sw, slot_context)
    gate = 1.0 / (1.0 + np.exp(-float(residual_gate)))
    return _f64(hidden) + gate * context, context


def block_post_selection(hidden, memory, anchor_index, partner_index, partner_score, params,
                         eps: float = 1e-5):
    """One block after selection for full sequences (queries at positions 0..T-1).

    hidden, memory [B,T,D]; anchor_index [B,T,S]; partner_index [B,T,S,K];
    partner_score [B,T,S,K] (non-finite = inactive partner).  params: operand
    [R,D]; mlp_w1 [Hd,4R], mlp_b1 [Hd]; mlp_w2 [D,Hd], mlp_b2 [D]; mlp_ln_w /
    mlp_ln_b [D]; slot_mix_logits [S]; residual_gate (scalar).
    Returns (output [B,T,D], context [B,T,D])."""
    hidden, memory = _f64(hidden), _f64(memory)
    batch, length, d = hidden.shape
    slots = np.asarray(anchor_index).shape[2]
    active = slot_activity(np.tile(np.arange(length), batch), slots)     # [B*T,S]
    b = np.arange(batch)[:, None, None]
    anchor = memory[b, np.asarray(anchor_index)] * active.reshape(batch, length, slots)[..., None]
    partner = memory[b[..., None], np.asarray(partner_index)]            # [B,T,S,K,D]
    w_op = _f64(params["operand"])
    a_op = anchor @ w_op.T                                               # [B,T,S,R]
    p_op = partner @ w_op.T                                              # [B,T,S,K,R]
    a_op = np.broadcast_to(a_op[:, :, :, None, :], p_op.shape)
    feature = np.concatenate([a_op, p_op, a_op * p_op, a_op - p_op], axis=-1)
    h = gelu(feature @ _f64(params["mlp_w1"]).T + _f64(params["mlp_b1"]))
    r = h @ _f64(params["mlp_w2"]).T + _f64(params["mlp_b2"])
    relation = layer_norm(r, params["mlp_ln_w"], params["mlp_ln_b"], eps)
    out, context = mix(relation.reshape(batch * length, slots, -1, d),
                       _f64(partner_score).reshape(batch * length, slots, -1), active,
                       params["slot_mix_logits"], hidden.reshape(batch * length, d),
                       params["residual_gate"])
    return out.reshape(batch, length, d), context.reshape(batch, length, d)


def relate_rows(expanded, operand, product_weight, second_weight, second_bias, norm_weight,
                norm_bias, slot_mix_logits, residual_gate, hidden_rows, batch_of, t, anchor,
                partner, partner_score, eps: float = 1e-5, hidden_dtype=np.float32):
    """The factorized path of a list of queries (the library's form of :148-178):
    MLP hidden from the expanded / operand caches (oracle/reduce.py, float64,
    rounded to fp32 as the hidden op returns it, then to `hidden_dtype` --
    "bfloat16" when the second Linear takes bf16 operands), second Linear in
    float64, then multi_relation_reduce_seq's steps.
    hidden_rows [Q,D]; batch_of, t [Q]; anchor [Q,S]; partner, partner_score [Q,S,K].
    Returns (output [Q,D], context [Q,D])."""
    from oracle import reduce as ored

    anchor = np.asarray(anchor, dtype=np.int64)
    partner = np.asarray(partner, dtype=np.int64)
    q, slots = anchor.shape
    k = partner.shape[2]
    rows = ored._hidden_flat(expanded, operand, np.repeat(np.asarray(batch_of), slots),
                             anchor.reshape(-1), partner.reshape(-1, k), product_weight)
    rows = ored.round_to(rows, hidden_dtype)
    raw = rows @ _f64(second_weight).T + _f64(second_bias)
    d = raw.shape[-1]
    relation = layer_norm(raw, norm_weight, norm_bias, eps).reshape(q, slots, k, d)
    return mix(relation, _f64(partner_score), slot_activity(t, slots), slot_mix_logits,
               hidden_rows, residual_gate)


def multi_relation_reduce_seq(raw, partner_scores, norm_weight, norm_bias, slot_mix_logits,
                              residual_gate, hidden, positions, norm_eps):
    """Contract of relation_lm::multi_relation_reduce_seq: LayerNorm of every raw row
    [B,Tq,S,K,D] (the relation MLP's second Linear output, bias included), then
    :164-178.  positions [Tq] or [B,Tq].  Returns (output [B,Tq,D], context)."""
    raw = _f64(raw)
    batch, queries, slots, k, d = raw.shape
    pos = np.asarray(positions, dtype=np.int64)
    if pos.ndim == 1:
        pos = np.broadcast_to(pos[None, :], (batch, queries))
    relation = layer_norm(raw, norm_weight, norm_bias, norm_eps).reshape(-1, slots, k, d)
    active = slot_activity(pos.reshape(-1), slots)
    out, context = mix(relation, _f64(partner_scores).reshape(-1, slots, k), active,
                       slot_mix_logits, _f64(hidden).reshape(-1, d), residual_gate)
    return out.reshape(batch, queries, d), context.reshape(batch, queries, d)


def block_statistics(keys, block_size: int):
    """Mean and biased std of keys [B,T,C] over each block of block_size rows
    (block_router.py:54-68).  Returns float64 [B,NB,C] each."""
    k = _f64(keys)
    batch, length, c = k.shape
    grouped = k.reshape(batch, length // block_size, block_size, c)
    return grouped.mean(axis=2), grouped.std(axis=2)
