"""Routed selection oracle -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates, in numpy, the selection kernels of the reference:
  * ``_relation_select_packed_kernel``  src/relation_lm/kernels/relation_select.py:9-308
  * ``_anchor_select_kernel``           src/relation_lm/kernels/triton_select.py:9-120
  * ``_partner_topk_kernel``            src/relation_lm/kernels/triton_select.py:123-252
in a form vectorised over an arbitrary list of queries (batch row ``b``,
position ``t``), so the same code is the decode oracle (one query per row at
the shared position) and the sequence/prefill oracle (one query per position).

Parity pins (tests/test_oracle_select.py):
  * block scores  == DistilledBlockRouter._scores restated (logsumexp over heads
    minus log H; block_router.py:70-101) -- independent formulation;
  * T <= LOCAL, or compat mode with every complete block selected: selection
    equals the dense causal argmax / top-k of RelationLexLM.relation_context
    (relation_lm.py:158-167) computed with torch on the full score matrix;
  * strict mode: brute-force set construction from the block ranking;
  * hand-built exact ties (duplicate keys) and the invalid-slot sentinel;
  * packed == two-op composition (tests/test_relation_select_gpu.py:33-87).
"""
from __future__ import annotations

import math

import numpy as np

NEG_INF32 = np.float32(-np.inf)
_CHUNK = 256


def _f64(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float64)


def _f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32)


def floor_log2(n: np.ndarray) -> np.ndarray:
    """floor(log2(n)) for integers n >= 1.

    The reference evaluates ``floor(log2(float(n)))`` in fp32
    (relation_select.py:61-65); both agree for n < 2**21 and buckets are
    clamped to REL_BUCKETS-1 long before that.
    """
    n = np.asarray(n, dtype=np.int64)
    out = np.zeros(n.shape, dtype=np.int64)
    m = n.copy()
    for shift in (32, 16, 8, 4, 2, 1):
        big = m >= (1 << shift)
        out = np.where(big, out + shift, out)
        m = np.where(big, m >> shift, m)
    return out


def block_geometry(t: np.ndarray, blocks: int, block_size: int, local_window: int,
                   strict_valid: bool, rel_buckets: int):
    """Eligibility, distance bucket and local_start per (query, block).

    relation_select.py:50-65 / triton_select.py:23-38.
    Returns (eligible [Q,NB] bool, bucket [Q,NB] int, local_start [Q] int).
    """
    t = np.asarray(t, dtype=np.int64)
    end = (np.arange(blocks, dtype=np.int64) + 1) * block_size - 1
    complete = end[None, :] <= t[:, None]
    local_start = np.maximum(t - local_window + 1, 0)
    if strict_valid:
        eligible = complete & (end[None, :] < local_start[:, None])
    else:
        eligible = complete
    distance = np.maximum(t[:, None] - end[None, :], 0)
    bucket = np.minimum(floor_log2(distance + 1), rel_buckets - 1)
    return eligible, bucket, local_start


def softplus_kernel_form(gamma) -> np.ndarray:
    """log(1 + exp(gamma)) without threshold, as relation_select.py:87."""
    g = _f64(gamma)
    return np.log(1.0 + np.exp(g))


def block_scores(router_query, block_mean, block_std, gamma, bias, batch_of, t, *,
                 block_size: int, local_window: int, strict_valid: bool) -> np.ndarray:
    """Router block scores, float32 [Q, NB] with -inf where not eligible.

    Per head h (relation_select.py:70-96):
        s_h = (sum_d mean*q_h + softplus(gamma_h) * sum_d std*|q_h|) * HD^-0.5
              + bias[h, bucket]
    combined by log-sum-exp over heads (:97-103, see logsumexp_heads), masked
    (:104-106).
    """
    blocks, heads, head_dim = block_mean.shape[1], block_mean.shape[2], block_mean.shape[3]
    rel_buckets = bias.shape[1]
    q = _f64(router_query).reshape(-1, heads, head_dim)
    eligible, bucket, _ = block_geometry(t, blocks, block_size, local_window, strict_valid,
                                         rel_buckets)
    mean = _f64(block_mean)[batch_of]
    std = _f64(block_std)[batch_of]
    content = np.einsum("qjhd,qhd->qjh", mean, q)
    uncertainty = np.einsum("qjhd,qhd->qjh", std, np.abs(q))
    sp = softplus_kernel_form(gamma)
    head_scale = 1.0 / math.sqrt(head_dim)
    bias64 = _f64(bias)
    per_head = (content + sp[None, None, :] * uncertainty) * head_scale
    per_head = per_head + np.transpose(bias64[:, bucket], (1, 2, 0))
    acc = logsumexp_heads(per_head)
    out = acc.astype(np.float32)
    out[~eligible] = NEG_INF32
    return out


def logsumexp_heads(per_head: np.ndarray) -> np.ndarray:
    """log(sum_h exp(s_h)) over the last axis in float64, as m + log(sum_h exp(s_h - m)).

    The reference kernel folds the heads pairwise in head order
    (relation_select.py:97-103: acc = m + log(exp(acc - m) + exp(s_h - m))); its
    block router writes the same quantity as one logsumexp (block_router.py:99).
    Both are the same real number; evaluated in float64 they agree to a few
    float64 ulps (tests/test_oracle_select.py pins this), far below the one
    rounding to float32 that every comparison sees.
    """
    mx = per_head.max(axis=-1, keepdims=True)
    return mx[..., 0] + np.log(np.exp(per_head - mx).sum(axis=-1))


def logsumexp_heads_pairwise(per_head: np.ndarray) -> np.ndarray:
    """The reference kernel's pairwise fold in head order (relation_select.py:97-103)."""
    acc = per_head[..., 0]
    for h in range(1, per_head.shape[-1]):
        s = per_head[..., h]
        mx = np.maximum(acc, s)
        acc = mx + np.log(np.exp(acc - mx) + np.exp(s - mx))
    return acc


def pick_blocks(scores: np.ndarray, top_blocks: int):
    """TOP sequential argmax picks, ties to the lowest block (relation_select.py:229-242).

    Returns (selected [Q,TOP] int64, valid [Q,TOP] bool); a pick is valid iff
    its value is > -1e30 (:237).  Picks after the eligible blocks run out land
    on -inf entries and are invalid.
    """
    work = scores.copy()
    rows = np.arange(work.shape[0])
    selected = np.zeros((work.shape[0], top_blocks), dtype=np.int64)
    valid = np.zeros((work.shape[0], top_blocks), dtype=bool)
    for rank in range(top_blocks):
        index = np.argmax(work, axis=1)
        value = work[rows, index]
        selected[:, rank] = index
        valid[:, rank] = value > -1.0e30
        work[rows, index] = NEG_INF32
    return selected, valid


def exact_scores(keys, batch_of, pos, valid, query, scale: float) -> np.ndarray:
    """fp32(sum_d key[b,pos,d] * query[d] * scale) for valid lanes, -inf otherwise.

    relation_select.py:114-122 / :286-296 under the float64-accumulation contract.
    """
    safe = np.where(valid, pos, 0)
    k = _f64(keys)[batch_of[:, None], safe]
    dot = np.einsum("qce,qe->qc", k, _f64(query))
    out = (dot * scale).astype(np.float32)
    out[~valid] = NEG_INF32
    return out


def _remote_lanes(selected, sel_valid, t, local_start, block_size, max_t):
    """Positions/validity of the TOP*BS remote lanes in pick order (:244-283)."""
    offsets = np.arange(block_size, dtype=np.int64)
    pos = (selected[:, :, None] * block_size + offsets[None, None, :]).reshape(len(t), -1)
    ok = np.repeat(sel_valid, block_size, axis=1)
    valid = (ok & (pos >= 0) & (pos <= t[:, None]) & (pos < local_start[:, None])
             & (pos < max_t))
    return pos, valid


def _local_lanes(t, local_window, max_t):
    pos = t[:, None] - local_window + 1 + np.arange(local_window, dtype=np.int64)[None, :]
    valid = (pos >= 0) & (pos <= t[:, None]) & (pos < max_t)
    return pos, valid


def _anchor_core(aq, ak, arq, amean, astd, agamma, abias, batch_of, t, local_window,
                 top_blocks, strict_valid):
    """Exact top-1 anchor; ties to the lowest position (relation_select.py:68-163)."""
    max_t, exact_dim = ak.shape[1], ak.shape[2]
    blocks = amean.shape[1]
    block_size = max_t // blocks
    scores = block_scores(arq, amean, astd, agamma, abias, batch_of, t,
                          block_size=block_size, local_window=local_window,
                          strict_valid=strict_valid)
    selected, sel_valid = pick_blocks(scores, top_blocks)
    _, _, local_start = block_geometry(t, blocks, block_size, local_window, strict_valid,
                                       abias.shape[1])
    lpos, lvalid = _local_lanes(t, local_window, max_t)
    rpos, rvalid = _remote_lanes(selected, sel_valid, t, local_start, block_size, max_t)
    pos = np.concatenate([lpos, rpos], axis=1)
    valid = np.concatenate([lvalid, rvalid], axis=1)
    score = exact_scores(ak, batch_of, pos, valid, aq, 1.0 / math.sqrt(exact_dim))
    best = score.max(axis=1)
    tie = score == best[:, None]
    big = np.iinfo(np.int64).max
    anchor = np.where(tie, pos, big).min(axis=1)
    return anchor.astype(np.int32), best.astype(np.float32)


def _partner_core(pq, pk, prq, pmean, pstd, pgamma, pbias, batch_of, t, anchor,
                  local_window, top_blocks, k_out, strict_valid):
    """Exact top-k partners with anchor exclusion; ties to the lowest lane.

    relation_select.py:177-308 / triton_select.py:157-252.  Lanes are the local
    window followed by the picked remote blocks in pick order; the k sequential
    argmaxes equal a stable descending sort over lanes.  Once the finite lanes
    are exhausted every slot repeats lane 0: position t-LOCAL+1, score -inf.
    """
    max_t, exact_dim = pk.shape[1], pk.shape[2]
    blocks = pmean.shape[1]
    block_size = max_t // blocks
    scores = block_scores(prq, pmean, pstd, pgamma, pbias, batch_of, t,
                          block_size=block_size, local_window=local_window,
                          strict_valid=strict_valid)
    selected, sel_valid = pick_blocks(scores, top_blocks)
    _, _, local_start = block_geometry(t, blocks, block_size, local_window, strict_valid,
                                       pbias.shape[1])
    lpos, lvalid = _local_lanes(t, local_window, max_t)
    rpos, rvalid = _remote_lanes(selected, sel_valid, t, local_start, block_size, max_t)
    pos = np.concatenate([lpos, rpos], axis=1)
    valid = np.concatenate([lvalid, rvalid], axis=1)
    valid &= pos != np.asarray(anchor, dtype=np.int64)[:, None]
    score = exact_scores(pk, batch_of, pos, valid, pq, 1.0 / math.sqrt(exact_dim))
    order = np.argsort(-score, axis=1, kind="stable")
    available = (score > NEG_INF32).sum(axis=1)
    rows = np.arange(score.shape[0])[:, None]
    slot = np.arange(k_out)[None, :]
    lanes = np.zeros((score.shape[0], k_out), dtype=np.int64)
    take = min(k_out, order.shape[1])
    lanes[:, :take] = order[:, :take]
    lanes = np.where(slot < available[:, None], lanes, 0)
    out_pos = pos[rows, lanes]
    out_score = np.where(slot < available[:, None], score[rows, lanes], NEG_INF32)
    return out_pos.astype(np.int32), out_score.astype(np.float32)


def _flatten_queries(batch: int, queries: int, positions) -> tuple[np.ndarray, np.ndarray]:
    pos = np.asarray(positions, dtype=np.int64)
    if pos.ndim == 0:
        pos = np.full((batch, queries), int(pos), dtype=np.int64)
    elif pos.ndim == 1:
        pos = np.broadcast_to(pos[None, :], (batch, queries))
    batch_of = np.repeat(np.arange(batch, dtype=np.int64), queries)
    return batch_of, np.ascontiguousarray(pos).reshape(-1)


def _packed_flat(aq, ak, arq, amean, astd, agamma, abias, pbase, pcache, pk, pmean, pstd,
                 pgamma, pbias, batch_of, t, local_window, top_blocks, k_out, strict_valid):
    exact_dim = ak.shape[2]
    n = len(t)
    anchor = np.zeros(n, np.int32)
    anchor_score = np.zeros(n, np.float32)
    partner = np.zeros((n, k_out), np.int32)
    partner_score = np.zeros((n, k_out), np.float32)
    for lo in range(0, n, _CHUNK):
        sl = slice(lo, min(n, lo + _CHUNK))
        b, tt = batch_of[sl], t[sl]
        a, s = _anchor_core(aq[sl], ak, arq[sl], amean, astd, agamma, abias, b, tt,
                            local_window, top_blocks, strict_valid)
        # Factorized partner query, fp32 adds (relation_select.py:165-193).
        contribution = _f32(pcache)[b, a.astype(np.int64)]
        base = _f32(pbase[sl])
        pq = base[:, :exact_dim] + contribution[:, :exact_dim]
        prq = base[:, exact_dim:] + contribution[:, exact_dim:]
        p, ps = _partner_core(pq, pk, prq, pmean, pstd, pgamma, pbias, b, tt, a,
                              local_window, top_blocks, k_out, strict_valid)
        anchor[sl], anchor_score[sl], partner[sl], partner_score[sl] = a, s, p, ps
    return anchor, anchor_score, partner, partner_score


def relation_select_packed(anchor_query, anchor_keys, anchor_router_query, anchor_block_mean,
                           anchor_block_std, anchor_gamma, anchor_bias, partner_base,
                           partner_anchor_cache, partner_keys, partner_block_mean,
                           partner_block_std, partner_gamma, partner_bias, position,
                           local_window, top_blocks, k_out, strict_valid):
    """Decode form: one query per row at the shared position (relation_select.py:311-382)."""
    batch = anchor_query.shape[0]
    batch_of, t = _flatten_queries(batch, 1, position)
    return _packed_flat(anchor_query, anchor_keys, anchor_router_query, anchor_block_mean,
                        anchor_block_std, anchor_gamma, anchor_bias, partner_base,
                        partner_anchor_cache, partner_keys, partner_block_mean,
                        partner_block_std, partner_gamma, partner_bias, batch_of, t,
                        int(local_window), int(top_blocks), int(k_out), bool(strict_valid))


def relation_select_packed_seq(anchor_query, anchor_keys, anchor_router_query,
                               anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias,
                               partner_base, partner_anchor_cache, partner_keys,
                               partner_block_mean, partner_block_std, partner_gamma,
                               partner_bias, positions, local_window, top_blocks, k_out,
                               strict_valid):
    """Sequence form: query tensors [B,Tq,*], positions [Tq] or [B,Tq]."""
    batch, queries = anchor_query.shape[0], anchor_query.shape[1]
    batch_of, t = _flatten_queries(batch, queries, positions)

    def flat(x):
        return np.asarray(x).reshape(batch * queries, -1)

    a, s, p, ps = _packed_flat(flat(anchor_query), anchor_keys, flat(anchor_router_query),
                               anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias,
                               flat(partner_base), partner_anchor_cache, partner_keys,
                               partner_block_mean, partner_block_std, partner_gamma,
                               partner_bias, batch_of, t, int(local_window), int(top_blocks),
                               int(k_out), bool(strict_valid))
    k = int(k_out)
    return (a.reshape(batch, queries), s.reshape(batch, queries),
            p.reshape(batch, queries, k), ps.reshape(batch, queries, k))


def anchor_select(anchor_query, anchor_keys, router_query, block_mean, block_std, gamma, bias,
                  position, local_window, top_blocks, strict_valid):
    """triton_select.py:255-295."""
    batch = anchor_query.shape[0]
    batch_of, t = _flatten_queries(batch, 1, position)
    return _anchor_core(anchor_query, anchor_keys, router_query, block_mean, block_std, gamma,
                        bias, batch_of, t, int(local_window), int(top_blocks),
                        bool(strict_valid))


def partner_topk(partner_query, partner_keys, router_query, block_mean, block_std, gamma, bias,
                 position, anchor_index, local_window, top_blocks, k_out, strict_valid):
    """triton_select.py:298-346 (partner and router queries precomputed by the caller)."""
    batch = partner_query.shape[0]
    batch_of, t = _flatten_queries(batch, 1, position)
    return _partner_core(_f32(partner_query), partner_keys, _f32(router_query), block_mean,
                         block_std, gamma, bias, batch_of, t,
                         np.asarray(anchor_index, dtype=np.int64), int(local_window),
                         int(top_blocks), int(k_out), bool(strict_valid))


# ---------------------------------------------------------------------------
# Routed multi-anchor selection (no reference kernel; dense semantics at
# src/relation_lm/models/multi_relation_blocks.py:69-147)
# ---------------------------------------------------------------------------

def _topk_lanes(score: np.ndarray, pos: np.ndarray, k_out: int):
    """Stable descending top-k over candidate lanes; exhausted slots repeat
    lane 0 with score -inf (the convention of _partner_core)."""
    order = np.argsort(-score, axis=1, kind="stable")
    available = (score > NEG_INF32).sum(axis=1)
    rows = np.arange(score.shape[0])[:, None]
    slot = np.arange(k_out)[None, :]
    lanes = np.zeros((score.shape[0], k_out), dtype=np.int64)
    take = min(k_out, order.shape[1])
    lanes[:, :take] = order[:, :take]
    lanes = np.where(slot < available[:, None], lanes, 0)
    out_pos = pos[rows, lanes]
    out_score = np.where(slot < available[:, None], score[rows, lanes], NEG_INF32)
    return out_pos, out_score


def _routed_lanes(router_query, mean, std, gamma, bias, batch_of, t, local_window,
                  top_blocks, strict_valid, max_t):
    """Candidate lanes [local | picked blocks in pick order] and their validity."""
    blocks = mean.shape[1]
    block_size = max_t // blocks
    scores = block_scores(router_query, mean, std, gamma, bias, batch_of, t,
                          block_size=block_size, local_window=local_window,
                          strict_valid=strict_valid)
    selected, sel_valid = pick_blocks(scores, top_blocks)
    _, _, local_start = block_geometry(t, blocks, block_size, local_window, strict_valid,
                                       bias.shape[1])
    lpos, lvalid = _local_lanes(t, local_window, max_t)
    rpos, rvalid = _remote_lanes(selected, sel_valid, t, local_start, block_size, max_t)
    return np.concatenate([lpos, rpos], axis=1), np.concatenate([lvalid, rvalid], axis=1)


def _multi_flat(aq, ak, arq, amean, astd, agamma, abias, pbase, pcache, pk, pmean, pstd,
                pgamma, pbias, batch_of, t, local_window, top_blocks, k_out, strict_valid):
    """S anchor slots per query over one routed anchor candidate set, then per
    slot a routed partner set that excludes every active anchor.

    Follows MultiAnchorRelationBlock (multi_relation_blocks.py):
      * slot s is active iff s <= t (:84); inactive slots report anchor 0 (:94)
        and no partners (:140-142);
      * slot s takes the argmax of its own anchor score over the candidates not
        already taken by slots < s (:86-95), ties to the lowest position;
      * slot s's partner query is the split form of partner_query[s](cat(query,
        anchor)) (:116-124): partner_base[s] + partner_anchor_cache[anchor, s]
        in float32, exact half and router half;
      * every active anchor of the query is excluded from every slot's
        partners (:133-139); top-k as the single-anchor partner pass.
    Routing replaces the dense causal candidate set by [local window | TOP
    picked blocks]: the anchor picks come from the anchor router, shared by all
    slots; each slot's partner picks come from its own router query against the
    shared partner block statistics.
    """
    n = len(t)
    slots = ak.shape[2]
    max_t, exact_dim = ak.shape[1], ak.shape[3]
    scale = 1.0 / math.sqrt(exact_dim)
    anchor = np.zeros((n, slots), np.int32)
    anchor_score = np.full((n, slots), NEG_INF32, np.float32)
    partner = np.zeros((n, slots, k_out), np.int32)
    partner_score = np.full((n, slots, k_out), NEG_INF32, np.float32)
    for lo in range(0, n, _CHUNK):
        sl = slice(lo, min(n, lo + _CHUNK))
        b, tt = batch_of[sl], t[sl]
        m = len(tt)
        active = np.arange(slots)[None, :] <= tt[:, None]  # [m, S]
        pos, valid = _routed_lanes(arq[sl], amean, astd, agamma, abias, b, tt, local_window,
                                   top_blocks, strict_valid, max_t)
        taken = np.zeros((m, 0), np.int64)
        chosen = np.zeros((m, slots), np.int64)
        for s in range(slots):
            v = valid & ~(pos[:, :, None] == taken[:, None, :]).any(axis=2)
            sc = exact_scores(ak[:, :, s], b, pos, v, aq[sl, s], scale)
            best = sc.max(axis=1)
            tie = (sc == best[:, None]) & (sc > NEG_INF32)
            big = np.iinfo(np.int64).max
            a = np.where(tie, pos, big).min(axis=1)
            ok = active[:, s] & (best > NEG_INF32)
            chosen[:, s] = np.where(ok, a, 0)
            anchor_score[sl, s] = np.where(ok, best, NEG_INF32)
            taken = np.concatenate([taken, np.where(ok, a, -1)[:, None]], axis=1)
        anchor[sl] = chosen.astype(np.int32)
        lane0 = tt - local_window + 1
        for s in range(slots):
            have = active[:, s]
            contribution = _f32(pcache)[b, chosen[:, s], s]
            contribution = np.where(have[:, None], contribution, np.float32(0))
            base = _f32(pbase[sl, s])
            pq = base[:, :exact_dim] + contribution[:, :exact_dim]
            prq = base[:, exact_dim:] + contribution[:, exact_dim:]
            ppos, pvalid = _routed_lanes(prq, pmean, pstd, pgamma, pbias, b, tt, local_window,
                                         top_blocks, strict_valid, max_t)
            pvalid &= ~(ppos[:, :, None] == taken[:, None, :]).any(axis=2)
            pvalid &= have[:, None]
            sc = exact_scores(pk[:, :, s], b, ppos, pvalid, pq, scale)
            out_pos, out_score = _topk_lanes(sc, ppos, k_out)
            out_pos = np.where(have[:, None], out_pos, lane0[:, None])
            partner[sl, s] = out_pos.astype(np.int32)
            partner_score[sl, s] = out_score
    return anchor, anchor_score, partner, partner_score


def multi_relation_select_seq(anchor_query, anchor_keys, anchor_router_query, anchor_block_mean,
                              anchor_block_std, anchor_gamma, anchor_bias, partner_base,
                              partner_anchor_cache, partner_keys, partner_block_mean,
                              partner_block_std, partner_gamma, partner_bias, positions,
                              local_window, top_blocks, k_out, strict_valid):
    """Sequence form of the routed multi-anchor selection.

    anchor_query [B,Tq,S,E], anchor_keys [B,T,S,E], anchor_router_query [B,Tq,RD],
    partner_base [B,Tq,S,E+RD], partner_anchor_cache [B,T,S,E+RD],
    partner_keys [B,T,S,E]; statistics, gamma and bias as the single-anchor op;
    positions [Tq] or [B,Tq].  Returns anchor int32 [B,Tq,S], anchor_score f32
    [B,Tq,S], partner int32 [B,Tq,S,K], partner_score f32 [B,Tq,S,K].
    """
    batch, queries, slots = anchor_query.shape[0], anchor_query.shape[1], anchor_query.shape[2]
    batch_of, t = _flatten_queries(batch, queries, positions)

    def flat(x):
        x = np.asarray(x)
        return x.reshape((batch * queries,) + x.shape[2:])

    a, s, p, ps = _multi_flat(flat(anchor_query), np.asarray(anchor_keys),
                              flat(anchor_router_query), anchor_block_mean, anchor_block_std,
                              anchor_gamma, anchor_bias, flat(partner_base),
                              np.asarray(partner_anchor_cache), np.asarray(partner_keys),
                              partner_block_mean, partner_block_std, partner_gamma, partner_bias,
                              batch_of, t, int(local_window), int(top_blocks), int(k_out),
                              bool(strict_valid))
    k = int(k_out)
    return (a.reshape(batch, queries, slots), s.reshape(batch, queries, slots),
            p.reshape(batch, queries, slots, k), ps.reshape(batch, queries, slots, k))


# ---------------------------------------------------------------------------
# Ring-buffer caches (no reference kernel; the reference's roadmap item
# "persistent ring-buffer state and contexts beyond 512", README.md:150)
# ---------------------------------------------------------------------------
#
# A cache of C rows (C = cache length, a power of two) holds the last C
# positions: position p lives in row p mod C, and block-statistics slot j holds
# the newest absolute block jb <= t // BS with jb = j (mod NB), NB = C / BS.
# Positions stay absolute in every input and output.  At position t the
# resident positions are [t-C+1, t]; every block jb in [t//BS - NB + 1, t//BS]
# lies inside that range, so a block is eligible exactly when the linear rule
# holds for its absolute index jb (complete, strict-mode local rule) and
# jb >= 0.  Picks rank by score, ties to the lowest absolute block.

def ring_blocks(t: np.ndarray, blocks: int, block_size: int) -> np.ndarray:
    """Absolute block index held by each statistics slot, [Q, NB] (negative: never written)."""
    cur = np.asarray(t, dtype=np.int64) // block_size
    slot = np.arange(blocks, dtype=np.int64)
    return cur[:, None] - np.mod(cur[:, None] - slot[None, :], blocks)


def ring_block_scores(router_query, block_mean, block_std, gamma, bias, batch_of, t, *,
                      block_size: int, local_window: int, strict_valid: bool):
    """Block scores per statistics slot (formula of block_scores) with the
    eligibility and distance bucket of the slot's absolute block.
    Returns (scores float32 [Q, NB], absolute block [Q, NB])."""
    blocks, heads, head_dim = block_mean.shape[1], block_mean.shape[2], block_mean.shape[3]
    rel_buckets = bias.shape[1]
    t = np.asarray(t, dtype=np.int64)
    jb = ring_blocks(t, blocks, block_size)
    end = (jb + 1) * block_size - 1
    local_start = np.maximum(t - local_window + 1, 0)
    eligible = (jb >= 0) & (end <= t[:, None])
    if strict_valid:
        eligible &= end < local_start[:, None]
    distance = np.maximum(t[:, None] - end, 0)
    bucket = np.minimum(floor_log2(distance + 1), rel_buckets - 1)
    q = _f64(router_query).reshape(-1, heads, head_dim)
    mean = _f64(block_mean)[batch_of]
    std = _f64(block_std)[batch_of]
    content = np.einsum("qjhd,qhd->qjh", mean, q)
    uncertainty = np.einsum("qjhd,qhd->qjh", std, np.abs(q))
    sp = softplus_kernel_form(gamma)
    bias64 = _f64(bias)
    per_head = (content + sp[None, None, :] * uncertainty) * (1.0 / math.sqrt(head_dim))
    per_head = per_head + np.transpose(bias64[:, bucket], (1, 2, 0))
    out = logsumexp_heads(per_head).astype(np.float32)
    out[~eligible] = NEG_INF32
    return out, jb


def ring_pick_blocks(scores: np.ndarray, jb: np.ndarray, top_blocks: int):
    """TOP picks by descending score, ties to the lowest absolute block; returns
    absolute blocks (selected [Q,TOP]) and validity (value > -1e30)."""
    n, blocks = scores.shape
    # stable sort on (-score, absolute block): argsort by block first, then a
    # stable sort by score keeps the lower block first among equal scores
    by_block = np.argsort(jb, axis=1, kind="stable")
    s_sorted = np.take_along_axis(scores, by_block, axis=1)
    order = np.take_along_axis(by_block, np.argsort(-s_sorted, axis=1, kind="stable"), axis=1)
    take = order[:, :top_blocks]
    selected = np.take_along_axis(jb, take, axis=1)
    valid = np.take_along_axis(scores, take, axis=1) > -1.0e30
    if top_blocks > blocks:
        pad = top_blocks - blocks
        selected = np.concatenate([selected, np.zeros((n, pad), np.int64)], axis=1)
        valid = np.concatenate([valid, np.zeros((n, pad), bool)], axis=1)
    return selected, valid


def ring_exact_scores(keys, batch_of, pos, valid, query, scale: float) -> np.ndarray:
    """exact_scores with position p read from cache row p mod C."""
    rows = np.mod(np.where(valid, pos, 0), keys.shape[1])
    return exact_scores(keys, batch_of, rows, valid, query, scale)


def _ring_lanes(router_query, mean, std, gamma, bias, batch_of, t, local_window, top_blocks,
                strict_valid, capacity):
    blocks = mean.shape[1]
    block_size = capacity // blocks
    scores, jb = ring_block_scores(router_query, mean, std, gamma, bias, batch_of, t,
                                   block_size=block_size, local_window=local_window,
                                   strict_valid=strict_valid)
    selected, sel_valid = ring_pick_blocks(scores, jb, top_blocks)
    local_start = np.maximum(t - local_window + 1, 0)
    lpos = t[:, None] - local_window + 1 + np.arange(local_window, dtype=np.int64)[None, :]
    lvalid = (lpos >= 0) & (lpos <= t[:, None])
    offsets = np.arange(block_size, dtype=np.int64)
    rpos = (selected[:, :, None] * block_size + offsets[None, None, :]).reshape(len(t), -1)
    rvalid = (np.repeat(sel_valid, block_size, axis=1) & (rpos >= 0) & (rpos <= t[:, None])
              & (rpos < local_start[:, None]))
    return np.concatenate([lpos, rpos], axis=1), np.concatenate([lvalid, rvalid], axis=1)


def relation_select_packed_ring(anchor_query, anchor_keys, anchor_router_query,
                                anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias,
                                partner_base, partner_anchor_cache, partner_keys,
                                partner_block_mean, partner_block_std, partner_gamma,
                                partner_bias, position, local_window, top_blocks, k_out,
                                strict_valid):
    """Decode-form packed selection over ring-buffer caches of C rows (any t >= 0).

    The chain of relation_select_packed (anchor top-1 ties to the lowest
    position, factorized partner query from the anchor's cache row, partner
    top-k with the anchor excluded, exhausted slots at lane 0 with -inf) with
    rows addressed mod C and slots mapped to absolute blocks as above.
    """
    batch = anchor_query.shape[0]
    batch_of, t = _flatten_queries(batch, 1, position)
    capacity, exact_dim = anchor_keys.shape[1], anchor_keys.shape[2]
    scale = 1.0 / math.sqrt(exact_dim)
    local_window, top_blocks, k_out = int(local_window), int(top_blocks), int(k_out)
    strict_valid = bool(strict_valid)
    pos, valid = _ring_lanes(anchor_router_query, anchor_block_mean, anchor_block_std,
                             anchor_gamma, anchor_bias, batch_of, t, local_window, top_blocks,
                             strict_valid, capacity)
    score = ring_exact_scores(anchor_keys, batch_of, pos, valid, anchor_query, scale)
    best = score.max(axis=1)
    tie = score == best[:, None]
    found = valid.any(axis=1)
    anchor = np.where(tie & valid, pos, np.iinfo(np.int64).max).min(axis=1)
    anchor = np.where(found, anchor, t - local_window + 1)
    anchor_score = np.where(found, best, NEG_INF32).astype(np.float32)
    have = found & (anchor >= 0)
    contribution = _f32(partner_anchor_cache)[batch_of, np.mod(np.where(have, anchor, 0),
                                                                 capacity)]
    contribution = np.where(have[:, None], contribution, np.float32(0))
    base = _f32(partner_base)
    pq = base[:, :exact_dim] + contribution[:, :exact_dim]
    prq = base[:, exact_dim:] + contribution[:, exact_dim:]
    ppos, pvalid = _ring_lanes(prq, partner_block_mean, partner_block_std, partner_gamma,
                               partner_bias, batch_of, t, local_window, top_blocks, strict_valid,
                               capacity)
    pvalid &= ppos != anchor[:, None]
    pscore = ring_exact_scores(partner_keys, batch_of, ppos, pvalid, pq, scale)
    out_pos, out_score = _topk_lanes(pscore, ppos, k_out)
    return (anchor.astype(np.int32), anchor_score, out_pos.astype(np.int32),
            out_score.astype(np.float32))
