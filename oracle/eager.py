"""Eager fp32 PyTorch restatement of the routed path -- TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py); used as the CPU baseline that bench.py times.

The reference ships no CPU implementation of its routed selection or reduce
(every op is a Triton kernel), so the CPU baseline is this restatement in
plain torch fp32 eager ops, vectorised over all queries:
  * ``_relation_select_packed_kernel``  src/relation_lm/kernels/relation_select.py:9-308
    (block scores :53-106, sequential block picks :229-242, local window plus
    picked blocks :244-284, exact top-1 / top-k with ties to the lower lane
    :114-163 / :286-308);
  * ``_relation_hidden_cached_kernel``  src/relation_lm/kernels/relation_reduce.py:72-146;
  * the caller's second linear          benchmarks/benchmark_relation_reduce.py:63;
  * ``_relation_norm_reduce_kernel``    src/relation_lm/kernels/relation_reduce.py:360-417;
  * ``PackedSparseCacheProjection.project``  src/relation_lm/inference/packed_cache.py:52-57.

Numerics: fp32 throughout, as the reference's kernels compute (its dots
accumulate in fp32), not the float64-accumulate contract of oracle/select.py.
Ties are broken toward the lower lane with a stable descending sort.  The
indices therefore equal the float64 oracle's except where two candidates'
fp32 scores differ from their float64-rounded values in opposite directions
(near-ties within an fp32 ulp); tests/test_oracle_eager.py measures that
agreement and the reduced states' error on seeded inputs.
"""
from __future__ import annotations

import math

import torch

NEG_INF = float("-inf")


def _block_geometry(t, blocks, block_size, local_window, strict_valid, rel_buckets):
    """Eligibility [Q,NB], distance bucket [Q,NB] and local start [Q] (relation_select.py:50-65)."""
    end = (torch.arange(blocks) + 1) * block_size - 1
    complete = end[None, :] <= t[:, None]
    local_start = torch.clamp(t - local_window + 1, min=0)
    eligible = complete & (end[None, :] < local_start[:, None]) if strict_valid else complete
    distance = torch.clamp(t[:, None] - end[None, :], min=0)
    bucket = torch.clamp(torch.floor(torch.log2((distance + 1).float())).long(), max=rel_buckets - 1)
    return eligible, bucket, local_start


def _block_scores(router_query, block_mean, block_std, gamma, bias, batch_of, t, block_size,
                  local_window, strict_valid):
    """Per-head content + softplus(gamma) * uncertainty, bucket bias, log-sum-exp over heads,
    -inf where not eligible (relation_select.py:68-106)."""
    blocks, heads, head_dim = block_mean.shape[1], block_mean.shape[2], block_mean.shape[3]
    q = router_query.reshape(-1, heads, head_dim)
    eligible, bucket, _ = _block_geometry(t, blocks, block_size, local_window, strict_valid,
                                          bias.shape[1])
    mean = block_mean[batch_of]
    std = block_std[batch_of]
    content = torch.einsum("qjhd,qhd->qjh", mean, q)
    uncertainty = torch.einsum("qjhd,qhd->qjh", std, q.abs())
    per_head = (content + torch.log1p(torch.exp(gamma))[None, None, :] * uncertainty)
    per_head = per_head * (1.0 / math.sqrt(head_dim)) + bias[:, bucket].permute(1, 2, 0)
    score = torch.logsumexp(per_head, dim=-1)
    return score.masked_fill(~eligible, NEG_INF)


def _candidates(scores, t, local_window, top_blocks, block_size, max_t, local_start):
    """Lane positions and validity: local window, then the picked blocks in pick order."""
    order = torch.sort(scores, dim=1, descending=True, stable=True)
    picked = order.indices[:, :top_blocks]
    picked_ok = order.values[:, :top_blocks] > -1.0e30
    lpos = t[:, None] - local_window + 1 + torch.arange(local_window)[None, :]
    lvalid = (lpos >= 0) & (lpos <= t[:, None]) & (lpos < max_t)
    rpos = (picked[:, :, None] * block_size + torch.arange(block_size)).reshape(len(t), -1)
    rvalid = (picked_ok.repeat_interleave(block_size, dim=1) & (rpos <= t[:, None])
              & (rpos < local_start[:, None]) & (rpos < max_t))
    return torch.cat([lpos, rpos], dim=1), torch.cat([lvalid, rvalid], dim=1)


def _lane_scores(keys, batch_of, pos, valid, query):
    safe = torch.where(valid, pos, torch.zeros_like(pos))
    k = keys[batch_of[:, None], safe]
    score = torch.einsum("qce,qe->qc", k, query) * (1.0 / math.sqrt(keys.shape[2]))
    return score.masked_fill(~valid, NEG_INF)


def relation_select_packed_flat(aq, ak, arq, amean, astd, agamma, abias, pbase, pcache, pk,
                                pmean, pstd, pgamma, pbias, batch_of, t, local_window,
                                top_blocks, k_out, strict_valid):
    """Anchor and partners of the flat query list (batch row batch_of[i], position t[i])."""
    max_t, exact_dim = ak.shape[1], ak.shape[2]
    block_size = max_t // amean.shape[1]
    _, _, local_start = _block_geometry(t, amean.shape[1], block_size, local_window,
                                        strict_valid, abias.shape[1])
    # Anchor: top-1, ties to the lowest position.
    scores = _block_scores(arq, amean, astd, agamma, abias, batch_of, t, block_size,
                           local_window, strict_valid)
    pos, valid = _candidates(scores, t, local_window, top_blocks, block_size, max_t, local_start)
    s = _lane_scores(ak, batch_of, pos, valid, aq)
    best = s.max(dim=1).values
    big = torch.iinfo(torch.int64).max
    anchor = torch.where(s == best[:, None], pos, torch.full_like(pos, big)).min(dim=1).values
    # Factorized partner query (relation_select.py:165-193).
    contribution = pcache[batch_of, anchor]
    pq = pbase[:, :exact_dim] + contribution[:, :exact_dim]
    prq = pbase[:, exact_dim:] + contribution[:, exact_dim:]
    scores = _block_scores(prq, pmean, pstd, pgamma, pbias, batch_of, t, block_size,
                           local_window, strict_valid)
    pos, valid = _candidates(scores, t, local_window, top_blocks, block_size, max_t, local_start)
    valid = valid & (pos != anchor[:, None])
    s = _lane_scores(pk, batch_of, pos, valid, pq)
    order = torch.sort(s, dim=1, descending=True, stable=True)
    lanes = order.indices[:, :k_out]
    top = order.values[:, :k_out]
    have = top > NEG_INF
    lanes = torch.where(have, lanes, torch.zeros_like(lanes))  # exhausted slots repeat lane 0
    partner = torch.gather(pos, 1, lanes)
    return (anchor.int(), best, partner.int(), torch.where(have, top, torch.full_like(top, NEG_INF)))


def relation_select_packed_seq(anchor_query, anchor_keys, anchor_router_query, anchor_block_mean,
                               anchor_block_std, anchor_gamma, anchor_bias, partner_base,
                               partner_anchor_cache, partner_keys, partner_block_mean,
                               partner_block_std, partner_gamma, partner_bias, positions,
                               local_window, top_blocks, k_out, strict_valid):
    """Sequence form: query tensors [B,Tq,*], positions [Tq] or [B,Tq]."""
    batch, queries = anchor_query.shape[0], anchor_query.shape[1]
    pos = torch.as_tensor(positions).long()
    if pos.dim() == 1:
        pos = pos[None, :].expand(batch, queries)
    batch_of = torch.arange(batch).repeat_interleave(queries)
    flat = [x.reshape(batch * queries, -1) for x in (anchor_query, anchor_router_query,
                                                     partner_base)]
    a, s, p, ps = relation_select_packed_flat(
        flat[0], anchor_keys, flat[1], anchor_block_mean, anchor_block_std, anchor_gamma,
        anchor_bias, flat[2], partner_anchor_cache, partner_keys, partner_block_mean,
        partner_block_std, partner_gamma, partner_bias, batch_of, pos.reshape(-1),
        int(local_window), int(top_blocks), int(k_out), bool(strict_valid))
    return (a.reshape(batch, queries), s.reshape(batch, queries),
            p.reshape(batch, queries, -1), ps.reshape(batch, queries, -1))


def relation_hidden_cached_seq(expanded, operand, anchor, partner, product_weight):
    """GELU(W_m (op[a] * op[p]) + X[a, :H] + X[p, H:]) -> [B,Tq,K,H] (relation_reduce.py:87-146)."""
    hidden_dim = product_weight.shape[0]
    batch = operand.shape[0]
    b = torch.arange(batch)[:, None]
    a = anchor.long()
    p = partner.long()
    op_a = operand[b, a]                          # [B,Tq,R]
    op_p = operand[b[:, :, None], p]              # [B,Tq,K,R]
    pre = torch.matmul(op_p * op_a[:, :, None, :], product_weight.t())
    pre = pre + expanded[b, a][..., None, :hidden_dim] + expanded[b[:, :, None], p][..., hidden_dim:]
    return torch.nn.functional.gelu(pre)


def relation_norm_reduce_seq(raw, scores, norm_weight, norm_bias, positions, eps):
    """LayerNorm per partner, softmax over the active partners (rank < k_limit and
    score > -1e30), weighted sum (relation_reduce.py:360-417)."""
    batch, queries, k, d = raw.shape
    pos = torch.as_tensor(positions).long()
    if pos.dim() == 1:
        pos = pos[None, :].expand(batch, queries)
    normalized = torch.nn.functional.layer_norm(raw, (d,), norm_weight, norm_bias, eps)
    limit = torch.clamp(torch.ceil(torch.log2((pos + 2).double())).long(), 1, k)
    active = (torch.arange(k)[None, None, :] < limit[..., None]) & (scores > -1.0e30)
    safe = torch.where(active, scores, torch.full_like(scores, -1.0e4))
    prob = torch.exp(safe - safe.max(dim=-1, keepdim=True).values) * active
    prob = prob / torch.clamp(prob.sum(dim=-1, keepdim=True), min=1.0e-9)
    return torch.einsum("bqk,bqkd->bqd", prob, normalized)


def relation_chain_seq(sel, red, cfg):
    """Expanded projection, select, hidden, second linear, norm-reduce of the sequence
    form; `sel` / `red` hold fp32 CPU tensors (workloads.selection_inputs / reduce_inputs)."""
    operand = red["operand_cache"]
    expanded = torch.nn.functional.linear(operand, red["expanded_weight"], red["expanded_bias"])
    a, _, p, ps = relation_select_packed_seq(
        sel["anchor_query"], sel["anchor_keys"], sel["anchor_router_query"],
        sel["anchor_block_mean"], sel["anchor_block_std"], sel["anchor_gamma"],
        sel["anchor_bias"], sel["partner_base"], sel["partner_anchor_cache"],
        sel["partner_keys"], sel["partner_block_mean"], sel["partner_block_std"],
        sel["partner_gamma"], sel["partner_bias"], sel["positions"], cfg.local_window,
        cfg.top_blocks, cfg.k_out, cfg.strict_valid)
    hidden = relation_hidden_cached_seq(expanded, operand, a, p, red["product_weight"])
    raw = torch.nn.functional.linear(hidden, red["second_weight"], red["second_bias"])
    ctx = relation_norm_reduce_seq(raw, ps, red["norm_weight"], red["norm_bias"],
                                   sel["positions"], 1e-5)
    return a, p, ctx


def expanded_cache(red):
    """The expanded cache [B,T,2H] = [W_a op + b1, W_p op] of every operand row: decode
    state, kept across steps (relation_reduce.py:23-57 factorization)."""
    return torch.nn.functional.linear(red["operand_cache"], red["expanded_weight"],
                                      red["expanded_bias"])


def relation_decode_step(sel, red, expanded, memory, packed_weight, cfg):
    """One decode step of the routed path for every batch row at the shared position:
    the packed 576->512 projection of the memory rows (packed_cache.py:52-57), the
    packed selection (decode form, relation_select.py:311-382), hidden from the
    expanded cache state (relation_reduce.py:87-146), second linear and norm-reduce.
    `sel` is workloads.selection_inputs(cfg, queries=1) in fp32."""
    projected = torch.nn.functional.linear(memory, packed_weight)
    batch = sel["anchor_query"].shape[0]
    t = torch.full((batch,), int(sel["position"]), dtype=torch.long)
    a, _, p, ps = relation_select_packed_flat(
        sel["anchor_query"], sel["anchor_keys"], sel["anchor_router_query"],
        sel["anchor_block_mean"], sel["anchor_block_std"], sel["anchor_gamma"],
        sel["anchor_bias"], sel["partner_base"], sel["partner_anchor_cache"],
        sel["partner_keys"], sel["partner_block_mean"], sel["partner_block_std"],
        sel["partner_gamma"], sel["partner_bias"], torch.arange(batch), t, cfg.local_window,
        cfg.top_blocks, cfg.k_out, cfg.strict_valid)
    hidden = relation_hidden_cached_seq(expanded, red["operand_cache"], a[:, None], p[:, None],
                                        red["product_weight"])
    raw = torch.nn.functional.linear(hidden, red["second_weight"], red["second_bias"])
    ctx = relation_norm_reduce_seq(raw, ps[:, None], red["norm_weight"], red["norm_bias"],
                                   t[:, None], 1e-5)
    return projected, a, p, ctx[:, 0]
