"""Relation reduce / projection oracle -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates in numpy:
  * ``factor_relation_first_layer``            relation_reduce.py:23-57
  * expanded-cache projection                  tests/test_relation_reduce_gpu.py:64-68
  * ``_relation_hidden_cached_kernel``         relation_reduce.py:72-146
  * ``_relation_hidden_cache_update_kernel``   relation_reduce.py:186-309
  * ``_relation_norm_reduce_kernel``           relation_reduce.py:360-417
  * ``PackedSparseCacheProjection.project``    inference/packed_cache.py:52-57
  * the last-token output preparation          models/relation_lm.py:203-206
  * the caller's second linear                 benchmarks/benchmark_relation_reduce.py:63

Everything is evaluated in float64 and rounded once to float32 (or to the
cache dtype for stored rows), except the elementwise product a*p which the
reference rounds to fp32 before the dot (relation_reduce.py:129) -- kept.

Parity pins (tests/test_oracle_reduce.py):
  * hidden == GELU(W1 [a, p, a*p, a-p] + b1) through torch.nn.functional on the
    unfactorized features (the reference's own closed form,
    tests/test_relation_reduce_gpu.py:80-101);
  * norm-reduce == torch F.layer_norm + masked softmax + sum (the reference's
    ``_reference_context``, tests/test_relation_reduce_gpu.py:21-43) and the
    dense weights of relation_lm.py:171-177;
  * packed projection == six separate torch linears
    (tests/test_packed_cache_projection.py:17-23);
  * k_limit == ceil(log2(t + 2)) evaluated in float for every t < 2**20;
  * output_prep == torch F.layer_norm(query + sigmoid(mix) * context), and with
    the mix logit at -inf equals the LayerNorm of the query alone.
"""
from __future__ import annotations

import math

import numpy as np
from scipy.special import erf

_CHUNK = 512


def _f64(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float64)


def gelu_erf(x: np.ndarray) -> np.ndarray:
    """Exact-erf GELU (relation_reduce.py:139; nn.GELU() at relation_lm.py:114)."""
    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))


def factor_relation_first_layer(first_weight, first_bias, relation_dim: int):
    """Split W1 [H, 4R] into (W_a+W_d, W_p-W_d, W_m) and the expanded weight/bias.

    relation_reduce.py:42-56.  Returns a dict of float64 arrays.
    """
    w = _f64(first_weight)
    r = int(relation_dim)
    wa, wp, wm, wd = w[:, :r], w[:, r:2 * r], w[:, 2 * r:3 * r], w[:, 3 * r:]
    anchor_weight = wa + wd
    partner_weight = wp - wd
    b = _f64(first_bias)
    return {
        "anchor_weight": anchor_weight,
        "partner_weight": partner_weight,
        "product_weight": wm,
        "first_bias": b,
        "expanded_weight": np.concatenate([anchor_weight, partner_weight], axis=0),
        "expanded_bias": np.concatenate([b, np.zeros_like(b)], axis=0),
    }


def linear(x, weight, bias=None) -> np.ndarray:
    """x @ weight^T (+ bias) in float64 (F.linear)."""
    out = _f64(x) @ _f64(weight).T
    if bias is not None:
        out = out + _f64(bias)
    return out


def _gather_rows(cache, batch_of, index):
    """cache[b, index] with out-of-range indices reading zeros (guarded gather)."""
    index = np.asarray(index, dtype=np.int64)
    ok = (index >= 0) & (index < cache.shape[1])
    safe = np.where(ok, index, 0)
    b = batch_of.reshape(batch_of.shape + (1,) * (index.ndim - 1))
    rows = _f64(cache)[b, safe]
    return np.where(ok[..., None], rows, 0.0)


def _hidden_flat(expanded, operand, batch_of, anchor, partner, product_weight,
                 anchor_current=None, partner_current=None, current_t=None):
    hidden_dim = product_weight.shape[0]
    n, k = partner.shape
    out = np.zeros((n, k, hidden_dim), dtype=np.float32)
    wm = _f64(product_weight)
    for lo in range(0, n, _CHUNK):
        sl = slice(lo, min(n, lo + _CHUNK))
        b, a, p = batch_of[sl], anchor[sl], partner[sl]
        op_a = _gather_rows(operand, b, a).astype(np.float32)          # [q,R]
        op_p = _gather_rows(operand, b, p).astype(np.float32)          # [q,K,R]
        product = (op_p * op_a[:, None, :]).astype(np.float32)          # fp32 product (:129)
        pre = (_f64(product).reshape(-1, wm.shape[1]) @ wm.T).reshape(len(a), k, hidden_dim)
        base_a = _gather_rows(expanded, b, a)[:, :hidden_dim]            # [q,H]
        base_p = _gather_rows(expanded, b, p)[..., hidden_dim:]          # [q,K,H]
        if anchor_current is not None:
            use_a = (np.asarray(a) == current_t)[:, None]
            base_a = np.where(use_a, anchor_current[b], base_a)
            use_p = (np.asarray(p) == current_t)[..., None]
            base_p = np.where(use_p, partner_current[b][:, None, :], base_p)
        out[sl] = gelu_erf(pre + base_a[:, None, :] + base_p).astype(np.float32)
    return out


def relation_hidden_cached(expanded_cache, operand_cache, anchor_index, partner_index,
                           product_weight) -> np.ndarray:
    """hidden f32 [B,K,H] (relation_reduce.py:87-146).  Out-of-range indices read zeros."""
    batch = operand_cache.shape[0]
    return _hidden_flat(expanded_cache, operand_cache, np.arange(batch),
                        np.asarray(anchor_index, np.int64),
                        np.asarray(partner_index, np.int64), product_weight)


def relation_hidden_cached_seq(expanded_cache, operand_cache, anchor_index, partner_index,
                               product_weight) -> np.ndarray:
    """Sequence form: anchor [B,Tq], partner [B,Tq,K] -> hidden f32 [B,Tq,K,H]."""
    batch, queries, k = np.asarray(partner_index).shape
    batch_of = np.repeat(np.arange(batch), queries)
    out = _hidden_flat(expanded_cache, operand_cache, batch_of,
                       np.asarray(anchor_index, np.int64).reshape(-1),
                       np.asarray(partner_index, np.int64).reshape(-1, k), product_weight)
    return out.reshape(batch, queries, k, -1)


def current_expanded_row(operand_cache, anchor_weight, partner_weight, first_bias, position):
    """[W_a op[t] + b1, W_p op[t]] per row in float64 (relation_reduce.py:215-236)."""
    t = int(position)
    current = _f64(operand_cache)[:, t].astype(np.float32)
    anchor_part = linear(current, anchor_weight, first_bias)
    partner_part = linear(current, partner_weight)
    return anchor_part, partner_part


def relation_hidden_cache_update(expanded_cache, operand_cache, anchor_index, partner_index,
                                 anchor_weight, partner_weight, product_weight, first_bias,
                                 position, cache_dtype=np.float32):
    """Returns (hidden f32 [B,K,H], updated expanded cache as float64).

    relation_reduce.py:205-309: row `position` of the cache is rewritten (rounded
    to the cache dtype) while the hidden uses the unrounded fp32 row wherever an
    index equals `position`.  `cache_dtype` names the rounding of the stored row
    (np.float32, or "bfloat16").
    """
    t = int(position)
    hidden_dim = product_weight.shape[0]
    anchor_part, partner_part = current_expanded_row(operand_cache, anchor_weight,
                                                     partner_weight, first_bias, t)
    anchor32 = anchor_part.astype(np.float32).astype(np.float64)
    partner32 = partner_part.astype(np.float32).astype(np.float64)
    updated = _f64(expanded_cache).copy()
    updated[:, t, :hidden_dim] = round_to(anchor32, cache_dtype)
    updated[:, t, hidden_dim:] = round_to(partner32, cache_dtype)
    batch = operand_cache.shape[0]
    hidden = _hidden_flat(expanded_cache, operand_cache, np.arange(batch),
                          np.asarray(anchor_index, np.int64),
                          np.asarray(partner_index, np.int64), product_weight,
                          anchor_current=anchor32, partner_current=partner32, current_t=t)
    return hidden, updated


def round_to(x: np.ndarray, dtype) -> np.ndarray:
    """Round float64/float32 values to float32 or bfloat16 (round-to-nearest-even)."""
    x32 = np.asarray(x, dtype=np.float32)
    if dtype in ("bfloat16", "bf16"):
        bits = x32.view(np.uint32).astype(np.uint64)
        rounding = ((bits >> 16) & 1) + 0x7FFF
        out = ((bits + rounding) >> 16 << 16).astype(np.uint32)
        nan = np.isnan(x32)
        out = np.where(nan, np.uint32(0x7FC00000), out)
        return out.view(np.float32).astype(np.float64)
    return x32.astype(np.float64)


def k_limit(position, k_out: int) -> np.ndarray:
    """clamp(ceil(log2(t + 2)), 1, K) == clamp(bit_length(t + 1), 1, K) (relation_reduce.py:399-401)."""
    t = np.asarray(position, dtype=np.int64)
    bits = np.zeros(t.shape, dtype=np.int64)
    m = t + 1
    while np.any(m > 0):
        bits = np.where(m > 0, bits + 1, bits)
        m = m >> 1
    return np.clip(bits, 1, k_out)


def _norm_reduce_flat(raw, scores, norm_weight, norm_bias, t, eps):
    x = _f64(raw)
    d = x.shape[-1]
    mean = x.sum(-1, keepdims=True) / d
    centered = x - mean
    var = (centered * centered).sum(-1, keepdims=True) / d
    normalized = centered / np.sqrt(var + float(eps)) * _f64(norm_weight) + _f64(norm_bias)
    k = x.shape[1]
    limit = k_limit(t, k)
    s = _f64(scores)
    active = (np.arange(k)[None, :] < limit[:, None]) & (s > -1.0e30)
    safe = np.where(active, s, -1.0e4)
    prob = np.exp(safe - safe.max(axis=1, keepdims=True)) * active
    prob = prob / np.maximum(prob.sum(axis=1, keepdims=True), 1.0e-9)
    return np.einsum("qk,qkd->qd", prob, normalized).astype(np.float32)


def relation_norm_reduce(raw, partner_scores, norm_weight, norm_bias, position,
                         norm_eps) -> np.ndarray:
    """ctx f32 [B,D] (relation_reduce.py:374-417)."""
    batch = raw.shape[0]
    t = np.full(batch, int(position), dtype=np.int64)
    return _norm_reduce_flat(raw, partner_scores, norm_weight, norm_bias, t, norm_eps)


def relation_norm_reduce_seq(raw, partner_scores, norm_weight, norm_bias, positions,
                             norm_eps) -> np.ndarray:
    """Sequence form: raw [B,Tq,K,D], scores [B,Tq,K], positions [Tq] or [B,Tq]."""
    batch, queries, k, d = raw.shape
    pos = np.asarray(positions, dtype=np.int64)
    if pos.ndim == 1:
        pos = np.broadcast_to(pos[None, :], (batch, queries))
    out = _norm_reduce_flat(np.asarray(raw).reshape(-1, k, d),
                            np.asarray(partner_scores).reshape(-1, k), norm_weight, norm_bias,
                            np.ascontiguousarray(pos).reshape(-1), norm_eps)
    return out.reshape(batch, queries, d)


def output_prep(query, context, mix_logit, output_weight, output_bias, eps) -> np.ndarray:
    """output_norm(query + sigmoid(mix_logit) * context) in float64
    (RelationLexLM.forward, relation_lm.py:203-206)."""
    gate = 1.0 / (1.0 + np.exp(-float(mix_logit)))
    y = _f64(query) + gate * _f64(context)
    mean = y.mean(axis=-1, keepdims=True)
    var = ((y - mean) ** 2).mean(axis=-1, keepdims=True)
    return (y - mean) / np.sqrt(var + float(eps)) * _f64(output_weight) + _f64(output_bias)


def packed_sparse_cache_projection(memory, weight) -> np.ndarray:
    """memory @ W^T in float64 (inference/packed_cache.py:56)."""
    return linear(memory, weight)


def relation_hidden_cached_ring(expanded_cache, operand_cache, anchor_index, partner_index,
                                product_weight) -> np.ndarray:
    """relation_hidden_cached with absolute indices over ring caches of C rows
    (no reference op): index p reads row p mod C."""
    cap = np.shape(expanded_cache)[1]
    return relation_hidden_cached(expanded_cache, operand_cache, np.mod(anchor_index, cap),
                                  np.mod(partner_index, cap), product_weight)


def relation_hidden_cache_update_ring(expanded_cache, operand_cache, anchor_index,
                                      partner_index, anchor_weight, partner_weight,
                                      product_weight, first_bias, position,
                                      cache_dtype=np.float32):
    """relation_hidden_cache_update over ring caches of C rows (no reference op).

    Position t's expanded row is computed from operand row t mod C, stored to
    row t mod C (rounded to the cache dtype) and used unrounded wherever an
    index equals t; an index p in the resident range [t-C+1, t] reads row
    p mod C; any other index reads zeros (an older one would alias the row
    being rewritten).  Returns (hidden f32 [B,K,H], updated cache float64).
    """
    cap = np.shape(expanded_cache)[1]
    t = int(position)

    def resident_row(index):
        index = np.asarray(index, dtype=np.int64)
        ok = (index >= 0) & (index <= t) & (index > t - cap)
        return np.where(ok, np.mod(index, cap), -1)

    a, p = resident_row(anchor_index), resident_row(partner_index)
    if t < 0:
        return (relation_hidden_cached(expanded_cache, operand_cache, a, p, product_weight),
                _f64(expanded_cache).copy())
    return relation_hidden_cache_update(expanded_cache, operand_cache, a, p, anchor_weight,
                                        partner_weight, product_weight, first_bias, t % cap,
                                        cache_dtype)
