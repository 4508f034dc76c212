/*
 * relation_lm_hip.h -- C ABI of the MI355X (gfx950) routed relation path.
 *
 * Every entry point mirrors one operator of the reference package
 * (Ahmet2001/relation-lm, src/relation_lm/...) argument for argument: the
 * tensors arrive as plain descriptors (pointer, dtype, shape, strides), the
 * scalar arguments keep their reference names and meaning, outputs are
 * caller-allocated descriptors, and the call is enqueued on `stream`.
 *
 * Conventions shared by every entry point
 *  - Return value: hipSuccess (0) or a hipError_t.  Argument errors return
 *    hipErrorInvalidValue and leave a message for rlm_last_error(); nothing
 *    is launched in that case.
 *  - No entry point allocates device memory, synchronises the stream or
 *    reads device memory on the host: `position` stays on the device, so
 *    every call can be captured into a HIP graph.
 *  - Positions and indices that fall outside [0, max_t) are never
 *    dereferenced: the kernels treat such rows as invalid / all-zero.
 *  - Inputs are borrowed.  Only the tensors documented as mutated are
 *    written besides the outputs.
 */
#ifndef RELATION_LM_HIP_H
#define RELATION_LM_HIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types understood by the library. */
enum rlm_dtype {
  RLM_F32 = 0,
  RLM_BF16 = 1,
  RLM_F16 = 2,
  RLM_I32 = 3,
  RLM_I64 = 4,
};

#define RLM_MAX_DIMS 4

/* A strided view of device memory.  Strides are in elements. */
typedef struct rlm_tensor {
  void* data;
  int32_t dtype;                 /* enum rlm_dtype */
  int32_t ndim;                  /* 0..RLM_MAX_DIMS */
  int64_t shape[RLM_MAX_DIMS];
  int64_t stride[RLM_MAX_DIMS];
} rlm_tensor;

/* Message describing the last failed call on this host thread ("" if none). */
const char* rlm_last_error(void);

/* Library version string. */
const char* rlm_version(void);

/* ------------------------------------------------------------------------
 * Routed selection
 * ---------------------------------------------------------------------- */

/*
 * Replaces relation_lm::relation_select_packed
 *   (src/relation_lm/kernels/relation_select.py:311-382).
 * Anchor block scoring, exact top-1 anchor, factorized partner query,
 * partner block routing and exact top-k partners for one query per batch
 * row at the shared 0-d device `position`.
 *   anchor_query [B,E], anchor_keys [B,T,E], anchor_router_query [B,RD],
 *   anchor_block_mean/std [B,NB,H,HD], anchor_gamma [H], anchor_bias [H,RB],
 *   partner_base [B,2E], partner_anchor_cache [B,T,2E], partner_keys [B,T,E],
 *   partner_block_mean/std [B,NB,H,HD], partner_gamma [H], partner_bias [H,RB],
 *   position: 0-d int64/int32.  RD = H*HD must equal E.
 * Outputs: out_anchor int32 [B], out_anchor_score f32 [B],
 *          out_partner int32 [B,K], out_partner_score f32 [B,K].
 */
hipError_t rlm_relation_select_packed(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias,
    const rlm_tensor* position, int64_t local_window, int64_t top_blocks,
    int64_t k_out, int32_t strict_valid, const rlm_tensor* out_anchor,
    const rlm_tensor* out_anchor_score, const rlm_tensor* out_partner,
    const rlm_tensor* out_partner_score, hipStream_t stream);

/*
 * Sequence (prefill) form of rlm_relation_select_packed: no reference
 * counterpart; the reference op is its Tq=1 case.  Query-side tensors gain a
 * query axis ([B,Tq,E], [B,Tq,RD], [B,Tq,2E]) and `position` holds one
 * position per query, shaped [Tq] (shared by all rows) or [B,Tq].
 * Outputs: int32 [B,Tq], f32 [B,Tq], int32 [B,Tq,K], f32 [B,Tq,K].
 */
hipError_t rlm_relation_select_packed_seq(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias,
    const rlm_tensor* positions, int64_t local_window, int64_t top_blocks,
    int64_t k_out, int32_t strict_valid, const rlm_tensor* out_anchor,
    const rlm_tensor* out_anchor_score, const rlm_tensor* out_partner,
    const rlm_tensor* out_partner_score, hipStream_t stream);

/*
 * rlm_relation_select_packed_seq plus the whole expanded cache: no reference op.
 * Replaces, in one launch where the shapes allow, the sequence selection and
 * the expanded-cache projection the reference runs as its own linear call
 * (tests/test_relation_reduce_gpu.py:64-68: expanded = F.linear(operand_cache,
 * W_e, b_e)): for every cache row r of every batch row b,
 *   expanded_cache[b, r] = expanded_weight . operand_cache[b, r] + expanded_bias,
 * in bf16 with fp32 sums, the same bits as rlm_linear on [B*T, R].  The
 * selection is the same as rlm_relation_select_packed_seq.  operand_cache
 * [B,T,R] bf16 (R in {32,64,96,128}), expanded_weight [N,R] bf16 (N % 16 == 0),
 * expanded_bias [N] or NULL, expanded_cache [B,T,N] bf16.  Where the sequence
 * selection's matrix-core kernel applies, N % 128 == 0 and T >= max(4 R, 272),
 * its workgroups project 128 x 128 cache tiles while their own loads are in
 * flight; otherwise the projection is a launch of its own after the selection.
 */
hipError_t rlm_relation_select_packed_seq_expand(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias,
    const rlm_tensor* positions, int64_t local_window, int64_t top_blocks,
    int64_t k_out, int32_t strict_valid, const rlm_tensor* operand_cache,
    const rlm_tensor* expanded_weight, const rlm_tensor* expanded_bias,
    const rlm_tensor* expanded_cache, const rlm_tensor* out_anchor,
    const rlm_tensor* out_anchor_score, const rlm_tensor* out_partner,
    const rlm_tensor* out_partner_score, hipStream_t stream);

/*
 * rlm_relation_select_packed (decode form) plus the token's expanded-cache row:
 * no reference op.  Replaces, in one launch, relation_select_packed
 * (relation_select.py:311-382) and the reference decode's row projection
 * (docs/benchmarks.md:80-81: "separate cuBLAS cache projection" for B > 1; the
 * fresh row relation_hidden_cache_update writes, relation_reduce.py:215-251,
 * for B == 1): for every batch row b,
 *   expanded_cache[b, r] = expanded_weight . operand_cache[b, r] + expanded_bias,
 * r = position (ring != 0: position mod T), in bf16 with fp32 sums; nothing is
 * written when the position is outside a linear cache.  The selection is the
 * same as rlm_relation_select_packed(_ring).  operand_cache [B,T,R] bf16
 * (R in {32,64,96,128}), expanded_weight [N,R] bf16 (N % 16 == 0),
 * expanded_bias [N] or NULL, expanded_cache [B,T,N] bf16.  Where the decode
 * selection kernel applies, the row is projected by extra workgroups of its
 * launch, beside the B selection workgroups; otherwise by a launch of its own.
 */
hipError_t rlm_relation_select_packed_expand_row(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias,
    const rlm_tensor* position, int64_t local_window, int64_t top_blocks,
    int64_t k_out, int32_t strict_valid, const rlm_tensor* operand_cache,
    const rlm_tensor* expanded_weight, const rlm_tensor* expanded_bias,
    const rlm_tensor* expanded_cache, int32_t ring, const rlm_tensor* out_anchor,
    const rlm_tensor* out_anchor_score, const rlm_tensor* out_partner,
    const rlm_tensor* out_partner_score, hipStream_t stream);

/*
 * Routed multi-anchor selection: no reference kernel.  The reference has only
 * the dense form, MultiAnchorRelationBlock._select_distinct_anchors and
 * forward's partner selection (src/relation_lm/models/multi_relation_blocks.py:69-147);
 * this op restricts its candidates to the routed set of the packed selection.
 *   anchor_query [B,Tq,S,E], anchor_keys [B,T,S,E], anchor_router_query [B,Tq,RD],
 *   anchor_block_mean/std [B,NB,H,HD], anchor_gamma [H], anchor_bias [H,RB],
 *   partner_base [B,Tq,S,E+RD], partner_anchor_cache [B,T,S,E+RD],
 *   partner_keys [B,T,S,E], partner_block_mean/std [B,NB,H,HD] (shared by the
 *   slots), partner_gamma [H], partner_bias [H,RB], positions [Tq] or [B,Tq].
 *   1 <= S <= 8, local_window >= S.
 * Slot s is active iff s <= t; active slots take distinct anchors (argmax over
 * the untaken candidates, slot order), inactive slots report anchor 0 and
 * score -inf.  Each active slot's partners exclude every active anchor of the
 * query; entries past the available candidates (and every entry of an
 * inactive slot) hold position t-local_window+1 and score -inf.
 * Outputs: out_anchor int32 [B,Tq,S], out_anchor_score f32 [B,Tq,S],
 *          out_partner int32 [B,Tq,S,K], out_partner_score f32 [B,Tq,S,K].
 */
hipError_t rlm_multi_relation_select_seq(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias,
    const rlm_tensor* positions, int64_t local_window, int64_t top_blocks,
    int64_t k_out, int32_t strict_valid, const rlm_tensor* out_anchor,
    const rlm_tensor* out_anchor_score, const rlm_tensor* out_partner,
    const rlm_tensor* out_partner_score, hipStream_t stream);

/*
 * Replaces relationlex::anchor_select
 *   (src/relation_lm/kernels/triton_select.py:255-295).
 *   anchor_query [B,E], anchor_keys [B,T,E], router_query [B,RD],
 *   block_mean/std [B,NB,H,HD], gamma [H], bias [H,RB], position 0-d.
 * Outputs: out_index int32 [B], out_score f32 [B].
 */
hipError_t rlm_anchor_select(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* router_query, const rlm_tensor* block_mean,
    const rlm_tensor* block_std, const rlm_tensor* gamma,
    const rlm_tensor* bias, const rlm_tensor* position, int64_t local_window,
    int64_t top_blocks, int32_t strict_valid, const rlm_tensor* out_index,
    const rlm_tensor* out_score, hipStream_t stream);

/*
 * Replaces relationlex::partner_topk
 *   (src/relation_lm/kernels/triton_select.py:298-346).
 *   partner_query [B,E], partner_keys [B,T,E], router_query [B,RD],
 *   block_mean/std [B,NB,H,HD], gamma [H], bias [H,RB], position 0-d,
 *   anchor_index int32/int64 [B].
 * Outputs: out_index int32 [B,K], out_score f32 [B,K].
 */
hipError_t rlm_partner_topk(
    const rlm_tensor* partner_query, const rlm_tensor* partner_keys,
    const rlm_tensor* router_query, const rlm_tensor* block_mean,
    const rlm_tensor* block_std, const rlm_tensor* gamma,
    const rlm_tensor* bias, const rlm_tensor* position,
    const rlm_tensor* anchor_index, int64_t local_window, int64_t top_blocks,
    int64_t k_out, int32_t strict_valid, const rlm_tensor* out_index,
    const rlm_tensor* out_score, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Relation reduce
 * ---------------------------------------------------------------------- */

/*
 * Replaces relation_lm::relation_hidden_cached
 *   (src/relation_lm/kernels/relation_reduce.py:149-183).
 *   hidden[b,k,:] = GELU(W_m (op[a_b] * op[p_bk]) + X[a_b,0:H] + X[p_bk,H:2H])
 *   expanded_cache X [B,T,2H], operand_cache op [B,T,R],
 *   anchor_index [B], partner_index [B,K] (int32/int64), product_weight W_m [H,R].
 * Output: out f32 [B,K,H].
 */
hipError_t rlm_relation_hidden_cached(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* product_weight, const rlm_tensor* out,
    hipStream_t stream);

/*
 * Sequence form of rlm_relation_hidden_cached (no reference counterpart):
 * anchor_index [B,Tq], partner_index [B,Tq,K]; output f32 [B,Tq,K,H].
 */
hipError_t rlm_relation_hidden_cached_seq(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* product_weight, const rlm_tensor* out,
    hipStream_t stream);

/*
 * The relation MLP of MultiAnchorRelationBlock up to its closing LayerNorm
 *   (src/relation_lm/models/multi_relation_blocks.py:47-52,163: Linear -> GELU ->
 * Linear, the first Linear factorized as relation_hidden_cached,
 * src/relation_lm/kernels/relation_reduce.py:149-183), bias-free, in one
 * launch:
 *   out[b,q,k,:] = second_weight . bf16(hidden[b,q,k,:])
 * with hidden as rlm_relation_hidden_cached_seq; the hidden never reaches
 * memory.  Bit-identical to rlm_relation_hidden_cached_seq with a bf16 output
 * followed by rlm_linear with an fp32 output and no bias.
 *   expanded_cache [B,T,2H], operand_cache [B,T,R] (bf16, 16-byte aligned),
 *   anchor_index [B,Tq], partner_index [B,Tq,K] (int32/int64);
 *   product_weight [H/32, R/16, 64, 8] and second_weight [D/32, H/16, 64, 8]:
 *   the [H,R] and [D,H] bf16 weights in MFMA fragment order
 *   (rlm_mfma_fragments, done once per weight).
 * Output: out f32 [B,Tq,K,D].  Shapes: R in {64, 128}, H a multiple of 128,
 * D in {256, 512, 768} (rlm_relation_hidden_linear_seq_fits says whether given
 * tensors qualify; other shapes fail with hipErrorInvalidValue).
 */
hipError_t rlm_relation_hidden_linear_seq(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* product_weight, const rlm_tensor* second_weight,
    const rlm_tensor* out, hipStream_t stream);

/* 1 if rlm_relation_hidden_linear_seq takes these tensors (dtypes, shapes,
 * alignment; the weights in fragment order), else 0. */
int rlm_relation_hidden_linear_seq_fits(const rlm_tensor* expanded_cache,
                                        const rlm_tensor* operand_cache,
                                        const rlm_tensor* product_weight,
                                        const rlm_tensor* second_weight);

/*
 * MFMA fragment order of a [N,K] bf16/f16 weight (no reference counterpart: a
 * weight packing step, like the reference's pack_sparse_cache_projection_weights):
 * out [N/32, K/16, 64, 8], fragment (nb, g) lane l = weight[32 nb + l % 32,
 * 16 g + 8 (l / 32) .. +7] -- the operand a wave's v_mfma_f32_32x32x16 reads,
 * contiguous per fragment.  N % 32 == 0, K % 16 == 0, 16-byte aligned.
 */
hipError_t rlm_mfma_fragments(const rlm_tensor* weight, const rlm_tensor* out,
                              hipStream_t stream);

/*
 * Replaces relation_lm::relation_hidden_cache_update
 *   (src/relation_lm/kernels/relation_reduce.py:312-357).
 * Writes expanded_cache[b, position] = [W_a op[t] + b1, W_p op[t]] (the only
 * mutated input) and returns the hidden of rlm_relation_hidden_cached, using
 * the fresh row wherever an index equals `position`.
 *   anchor_weight, partner_weight, product_weight [H,R], first_bias [H].
 */
hipError_t rlm_relation_hidden_cache_update(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* anchor_weight, const rlm_tensor* partner_weight,
    const rlm_tensor* product_weight, const rlm_tensor* first_bias,
    const rlm_tensor* position, const rlm_tensor* out, hipStream_t stream);

/*
 * Replaces relation_lm::relation_norm_reduce
 *   (src/relation_lm/kernels/relation_reduce.py:420-450).
 *   ctx[b] = sum_k p_k * LayerNorm(raw[b,k]),  p = active-K masked softmax.
 *   raw [B,K,D], partner_scores f32 [B,K], norm_weight/bias [D], position 0-d.
 * Output: out f32 [B,D].
 */
hipError_t rlm_relation_norm_reduce(
    const rlm_tensor* raw, const rlm_tensor* partner_scores,
    const rlm_tensor* norm_weight, const rlm_tensor* norm_bias,
    const rlm_tensor* position, double norm_eps, const rlm_tensor* out,
    hipStream_t stream);

/*
 * Sequence form of rlm_relation_norm_reduce (no reference counterpart):
 * raw [B,Tq,K,D], partner_scores [B,Tq,K], positions [Tq] or [B,Tq];
 * output f32 [B,Tq,D].
 */
hipError_t rlm_relation_norm_reduce_seq(
    const rlm_tensor* raw, const rlm_tensor* partner_scores,
    const rlm_tensor* norm_weight, const rlm_tensor* norm_bias,
    const rlm_tensor* positions, double norm_eps, const rlm_tensor* out,
    hipStream_t stream);

/*
 * rlm_relation_norm_reduce with the last-token output preparation fused as
 * its epilogue (the reference's roadmap item "fuse last-token output
 * preparation", README.md:150-151; the computation is RelationLexLM.forward's
 * output_norm(query + sigmoid(relation_mix_logit) * context),
 * src/relation_lm/models/relation_lm.py:203-206):
 *   query [B,D] (f32/bf16/f16), mix_logit 0-d, output_weight/output_bias [D]
 *   (output_norm), output_eps.
 * Outputs: out_context f32 [B,D] (bit-identical to rlm_relation_norm_reduce),
 *          out_final [B,D] in query's dtype = LayerNorm_out(query + sigmoid(mix) ctx).
 */
hipError_t rlm_relation_norm_reduce_output(
    const rlm_tensor* raw, const rlm_tensor* partner_scores, const rlm_tensor* norm_weight,
    const rlm_tensor* norm_bias, const rlm_tensor* position, double norm_eps,
    const rlm_tensor* query, const rlm_tensor* mix_logit, const rlm_tensor* output_weight,
    const rlm_tensor* output_bias, double output_eps, const rlm_tensor* out_context,
    const rlm_tensor* out_final, hipStream_t stream);

/*
 * The decode step's second linear and norm-reduce with the output-head
 * preparation (no reference op: the reference calls F.linear then
 * relation_norm_reduce, benchmarks/benchmark_relation_reduce.py:80-81; the
 * output-head preparation is its roadmap item 3, README.md:151): the same result as
 *   raw = hidden @ second_weight^T + second_bias   (rlm_linear)
 *   rlm_relation_norm_reduce_output(raw, ...)
 * within fp32 rounding (the reduction is summed in a different order).  The
 * linear runs split-K over `partials` [S, B*K, D] fp32 (a caller-owned
 * workspace; S splits of the hidden dim, each written whole) and the per-query
 * norm-reduce kernel adds the S partial products in order plus the bias as it
 * loads the rows -- deterministic, no atomics.
 *   hidden [B,K,H] f32/bf16/f16, second_weight [D,H] bf16/f16, second_bias [D].
 *   query NULL: context only (out_final unused).  Decode shapes only: B <= 256
 *   queries, B*K <= 64 rows, D % 4 == 0, D <= 1024, K <= 16.
 */
hipError_t rlm_relation_linear_norm_reduce_output(
    const rlm_tensor* hidden, const rlm_tensor* second_weight, const rlm_tensor* second_bias,
    const rlm_tensor* partner_scores, const rlm_tensor* norm_weight,
    const rlm_tensor* norm_bias, const rlm_tensor* position, double norm_eps,
    const rlm_tensor* query, const rlm_tensor* mix_logit, const rlm_tensor* output_weight,
    const rlm_tensor* output_bias, double output_eps, const rlm_tensor* partials,
    const rlm_tensor* out_context, const rlm_tensor* out_final, hipStream_t stream);

/*
 * rlm_relation_linear_norm_reduce_output without the `partials` workspace,
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc); no counterpart in
 * the reference.  The partials live in a static per-GPU device array of
 * 4 x 64 x 1024 fp32 (1 MiB): splits * B*K * D must not exceed that, or the
 * call fails with hipErrorInvalidValue.  `splits` (1..4) is the S of the
 * workspace form; the result equals that form's with the same S.  Allocates
 * nothing; call with the stream's device current.  Calls that overlap on one
 * GPU share the array and race.
 */
hipError_t rlm_relation_linear_norm_reduce_output_noalloc(
    const rlm_tensor* hidden, const rlm_tensor* second_weight, const rlm_tensor* second_bias,
    const rlm_tensor* partner_scores, const rlm_tensor* norm_weight,
    const rlm_tensor* norm_bias, const rlm_tensor* position, double norm_eps,
    const rlm_tensor* query, const rlm_tensor* mix_logit, const rlm_tensor* output_weight,
    const rlm_tensor* output_bias, double output_eps, int32_t splits,
    const rlm_tensor* out_context, const rlm_tensor* out_final, hipStream_t stream);

/*
 * The decode step's relation tail in one launch (no single reference op: the
 * reference calls relation_hidden_cached, src/relation_lm/kernels/
 * relation_reduce.py:149-183, then F.linear and relation_norm_reduce,
 * relation_reduce.py:420-450, benchmarks/benchmark_relation_reduce.py:55-64,
 * and prepares the output head, models/relation_lm.py:203-206): the result of
 *   hidden = rlm_relation_hidden_cached(_ring)(...)       (fp32, [B,K,H])
 *   rlm_relation_linear_norm_reduce_output(hidden, ...)
 * with the hidden rounded to bf16 for the second linear (as that op's 16-bit
 * path does) and the linear's fp32 sums in another order: equal to fp32
 * rounding of the raw rows, not bit for bit.
 *   expanded_cache [B,T,2H], operand_cache [B,T,R], product_weight [H,R],
 *   second_weight [D,H] (all bf16), anchor_index [B], partner_index [B,K]
 *   (int32/int64), second_bias/norm_weight/norm_bias/output_weight/
 *   output_bias [D], partner_scores f32 [B,K], position 0-d, query [B,D],
 *   mix_logit 0-d; ring != 0: ring-buffer caches (T a power of two, index i
 *   in row i mod T), as rlm_relation_hidden_cached_ring.
 *   workspace: fp32 [n] and counters: int32 [m] with n, m from
 *   rlm_relation_hidden_linear_norm_reduce_output_workspace.  The counters
 *   must be zero before the first call and are zero again when each call
 *   ends; calls that overlap on one device must use different counters.
 *   out_context f32 [B,D], out_final [B,D] in the query's dtype.
 * Shapes: R in {64, 128}, H a multiple of 64 up to 3072, 1 <= K <= 8,
 * D a multiple of 4 up to 768 (rlm_relation_hidden_linear_norm_reduce_output_fits
 * says whether given tensors qualify; other shapes fail with
 * hipErrorInvalidValue and run the two ops above).
 */
hipError_t rlm_relation_hidden_linear_norm_reduce_output(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* product_weight, const rlm_tensor* second_weight,
    const rlm_tensor* second_bias, const rlm_tensor* partner_scores,
    const rlm_tensor* norm_weight, const rlm_tensor* norm_bias, const rlm_tensor* position,
    double norm_eps, const rlm_tensor* query, const rlm_tensor* mix_logit,
    const rlm_tensor* output_weight, const rlm_tensor* output_bias, double output_eps,
    int32_t ring, const rlm_tensor* workspace, const rlm_tensor* counters,
    const rlm_tensor* out_context, const rlm_tensor* out_final, hipStream_t stream);

/* Workspace sizes of rlm_relation_hidden_linear_norm_reduce_output for B
 * queries of K partners, hidden dim H (a multiple of 64) and d_model D:
 * *workspace_floats fp32 elements and *counters int32 elements. */
hipError_t rlm_relation_hidden_linear_norm_reduce_output_workspace(
    int64_t batch, int64_t partners, int64_t hidden_dim, int64_t d_model,
    int64_t* workspace_floats, int64_t* counters);

/* 1 if rlm_relation_hidden_linear_norm_reduce_output takes these tensors
 * (dtypes, shapes, alignment), else 0. */
int rlm_relation_hidden_linear_norm_reduce_output_fits(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* partner_index, const rlm_tensor* product_weight,
    const rlm_tensor* second_weight);

/*
 * Sequence form of rlm_relation_norm_reduce_output: raw [B,Tq,K,D],
 * partner_scores [B,Tq,K], positions [Tq] or [B,Tq], query [B,Tq,D];
 * out_context f32 [B,Tq,D], out_final [B,Tq,D].
 */
hipError_t rlm_relation_norm_reduce_output_seq(
    const rlm_tensor* raw, const rlm_tensor* partner_scores, const rlm_tensor* norm_weight,
    const rlm_tensor* norm_bias, const rlm_tensor* positions, double norm_eps,
    const rlm_tensor* query, const rlm_tensor* mix_logit, const rlm_tensor* output_weight,
    const rlm_tensor* output_bias, double output_eps, const rlm_tensor* out_context,
    const rlm_tensor* out_final, hipStream_t stream);

/*
 * Fused relation reduce, sequence form (no reference counterpart: the
 * reference runs relation_hidden_cached -> F.linear -> relation_norm_reduce,
 * src/relation_lm/kernels/relation_reduce.py:149,420 and the call sequence of
 * benchmarks/benchmark_relation_reduce.py:55-64, with fp32 intermediates).
 *   ctx[b,q] = sum_k p_k LayerNorm(W2 h_k + b2),
 *   h_k = GELU(W_m (op[a]*op[p_k]) + X[a,0:H] + X[p_k,H:2H]) rounded to bf16,
 *   p = the active-K softmax of relation_norm_reduce.
 *   expanded_cache [B,T,2H], operand_cache [B,T,R], product_weight [H,R],
 *   second_weight [D,H] or the same weight in MFMA fragment order
 *   [D/32,H/16,64,8] (rlm_mfma_fragments, done once: each fragment load is then
 *   one contiguous 1 KiB; same result bit for bit) (all bf16), second_bias [D],
 *   partner_scores f32 [B,Tq,K], norm_weight/norm_bias [D], anchor_index
 *   [B,Tq], partner_index [B,Tq,K], positions [Tq] or [B,Tq].  1 <= K <= 16,
 *   R in {32,64,128}, H a multiple of 128, D in {128, 256, 384, 512}.
 * Output: out f32 [B,Tq,D].
 */
hipError_t rlm_relation_reduce_fused_seq(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* product_weight, const rlm_tensor* second_weight,
    const rlm_tensor* second_bias, const rlm_tensor* partner_scores,
    const rlm_tensor* norm_weight, const rlm_tensor* norm_bias, const rlm_tensor* positions,
    double norm_eps, const rlm_tensor* out, hipStream_t stream);

/*
 * Whether rlm_relation_reduce_fused_seq takes these operands (no reference
 * counterpart: the capability query behind relation_lm::relation_reduce_fused_seq,
 * which runs the unfused relation_hidden_cached_seq -> relation_linear ->
 * relation_norm_reduce_seq chain for every other shape, e.g. the reference's
 * fp32 D = 576 cases of tests/test_relation_reduce_gpu.py:163-200).  Returns 1
 * for bf16 caches and weights, 1 <= K <= 16, R in {32,64,128}, H a multiple of
 * 128, D in {128, 256, 384, 512} and 16-byte aligned operand_cache,
 * product_weight and second_weight; 0 otherwise.  Reads descriptors only.
 */
int rlm_relation_reduce_fused_seq_fits(const rlm_tensor* expanded_cache,
                                       const rlm_tensor* operand_cache,
                                       const rlm_tensor* partner_index,
                                       const rlm_tensor* product_weight,
                                       const rlm_tensor* second_weight);

/* ------------------------------------------------------------------------
 * Router cache (decode producer of the selection's block statistics)
 * ---------------------------------------------------------------------- */

/*
 * Replaces relation_lm::router_cache_update
 *   (src/relation_lm/kernels/router_cache.py:181-241; kernel :9-178).
 *   anchor_raw / partner_raw [B,D] rows (any row stride, unit column stride),
 *   raw and conv caches [B,T,D], anchor/partner mean and std [B,NB,...] with D
 *   values per block, conv weights [D,3], position 0-d int32/int64 (device).
 *   Writes raw/conv cache row `position`, the statistics of block
 *   position / block_size and out f32 [B,2,D] (the two streams' conv rows).
 *   A position outside [0,T) writes zeros to out and leaves the caches alone.
 */
hipError_t rlm_router_cache_update(
    const rlm_tensor* anchor_raw, const rlm_tensor* partner_raw,
    const rlm_tensor* anchor_raw_cache, const rlm_tensor* partner_raw_cache,
    const rlm_tensor* anchor_conv_cache, const rlm_tensor* partner_conv_cache,
    const rlm_tensor* anchor_mean, const rlm_tensor* anchor_std,
    const rlm_tensor* partner_mean, const rlm_tensor* partner_std,
    const rlm_tensor* anchor_conv_weight, const rlm_tensor* partner_conv_weight,
    const rlm_tensor* position, int64_t block_size, const rlm_tensor* out,
    hipStream_t stream);

/* ------------------------------------------------------------------------
 * Ring-buffer caches: contexts beyond the cache length
 *
 * No reference counterpart: the reference's roadmap item "persistent
 * ring-buffer state and contexts beyond 512" (README.md:150,
 * docs/roadmap.md:8).  Each entry point takes exactly the arguments of its
 * linear form above; positions stay absolute (inputs and outputs) and may
 * exceed the cache length T, a power of two.  Position p lives in cache row
 * p mod T; block statistics slot j holds the newest absolute block
 * jb <= t / BS with jb = j mod NB (NB * BS == T).  The resident positions at
 * t are [t-T+1, t]; only whole resident blocks are eligible for routing, and
 * block picks tie to the lowest absolute block.  For t < T each entry point
 * equals its linear form.
 * ---------------------------------------------------------------------- */

/* Ring form of rlm_relation_select_packed (decode form). */
hipError_t rlm_relation_select_packed_ring(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias,
    const rlm_tensor* position, int64_t local_window, int64_t top_blocks,
    int64_t k_out, int32_t strict_valid, const rlm_tensor* out_anchor,
    const rlm_tensor* out_anchor_score, const rlm_tensor* out_partner,
    const rlm_tensor* out_partner_score, hipStream_t stream);

/* Ring form of rlm_relation_hidden_cached: indices are absolute positions
 * (any value >= 0 reads row index mod T). */
hipError_t rlm_relation_hidden_cached_ring(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* product_weight, const rlm_tensor* out, hipStream_t stream);

/* Ring form of rlm_relation_hidden_cache_update: the fresh row of position t
 * is written to row t mod T and substituted wherever an index equals t. */
hipError_t rlm_relation_hidden_cache_update_ring(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* anchor_weight, const rlm_tensor* partner_weight,
    const rlm_tensor* product_weight, const rlm_tensor* first_bias,
    const rlm_tensor* position, const rlm_tensor* out, hipStream_t stream);

/* Ring form of rlm_router_cache_update: raw/conv rows at t mod T (the conv
 * reads rows t-1, t-2 mod T), statistics of block t/BS in slot (t/BS) mod NB;
 * rows of that block past t count as zero (they still hold positions from T
 * earlier). */
hipError_t rlm_router_cache_update_ring(
    const rlm_tensor* anchor_raw, const rlm_tensor* partner_raw,
    const rlm_tensor* anchor_raw_cache, const rlm_tensor* partner_raw_cache,
    const rlm_tensor* anchor_conv_cache, const rlm_tensor* partner_conv_cache,
    const rlm_tensor* anchor_mean, const rlm_tensor* anchor_std,
    const rlm_tensor* partner_mean, const rlm_tensor* partner_std,
    const rlm_tensor* anchor_conv_weight, const rlm_tensor* partner_conv_weight,
    const rlm_tensor* position, int64_t block_size, const rlm_tensor* out,
    hipStream_t stream);

/* ------------------------------------------------------------------------
 * Dense projections (MFMA)
 * ---------------------------------------------------------------------- */

/*
 * Replaces the F.linear inside PackedSparseCacheProjection.project
 *   (src/relation_lm/inference/packed_cache.py:52-57).
 *   memory [M,Din] (any leading shape flattened by the caller), weight [Dout,Din].
 * Output: out [M,Dout], same dtype as memory.
 */
hipError_t rlm_packed_sparse_cache_projection(
    const rlm_tensor* memory, const rlm_tensor* weight, const rlm_tensor* out,
    hipStream_t stream);

/*
 * rlm_packed_sparse_cache_projection plus the decode-time cache writes, in one
 * kernel: no reference counterpart (the reference projects with F.linear and
 * leaves the cache writes to the caller, packed_cache.py:52-57).  Output
 * columns of the first four segments (anchor_key, partner_key, operand,
 * partner_anchor: SPARSE_CACHE_NAMES order, widths taken from the caches) are
 * also written to row `position` of anchor_keys [B,T,E], partner_keys [B,T,E],
 * operand_cache [B,T,R] and partner_anchor_cache [B,T,2E] (row position mod T
 * when `ring` is set; T a power of two).  B <= 64, 16-bit weights; caches in
 * the output dtype.  `out` [B,Dout] receives every column (the router segments
 * feed rlm_router_cache_update).
 */
hipError_t rlm_packed_projection_to_caches(
    const rlm_tensor* memory, const rlm_tensor* weight, const rlm_tensor* out,
    const rlm_tensor* anchor_keys, const rlm_tensor* partner_keys,
    const rlm_tensor* operand_cache, const rlm_tensor* partner_anchor_cache,
    const rlm_tensor* position, int32_t ring, hipStream_t stream);

/*
 * rlm_packed_projection_to_caches and rlm_router_cache_update(_ring) on its
 * router segments in one launch: the reference's roadmap item "fold the
 * router cache update into the packed projection" (README.md:148-149); no
 * reference op.  The router segments are the last two of the packed output
 * (widths D each, the router caches' last dim); the router tensors are those of
 * rlm_router_cache_update with the raw rows taken from `out`.  Results are
 * bit-identical to the two calls.  16-bit memory/weight/out, B <= 16, Din <= 768,
 * D <= 64, block_size 8/16/32/64 and one fp32 or bf16 dtype for the router
 * state take the single launch; other shapes run the two calls in turn.
 * router_out [B,2,D] fp32 receives the conv rows.
 */
hipError_t rlm_packed_projection_router_update(
    const rlm_tensor* memory, const rlm_tensor* weight, const rlm_tensor* out,
    const rlm_tensor* anchor_keys, const rlm_tensor* partner_keys,
    const rlm_tensor* operand_cache, const rlm_tensor* partner_anchor_cache,
    const rlm_tensor* position, int32_t ring, const rlm_tensor* anchor_raw_cache,
    const rlm_tensor* partner_raw_cache, const rlm_tensor* anchor_conv_cache,
    const rlm_tensor* partner_conv_cache, const rlm_tensor* anchor_mean,
    const rlm_tensor* anchor_std, const rlm_tensor* partner_mean, const rlm_tensor* partner_std,
    const rlm_tensor* anchor_conv_weight, const rlm_tensor* partner_conv_weight,
    int64_t block_size, const rlm_tensor* router_out, hipStream_t stream);

/*
 * out = input @ weight^T (+ bias), the library GEMM behind the expanded-cache
 * projection (tests/test_relation_reduce_gpu.py:64-68 in the reference) and
 * the relation MLP's second linear (benchmarks/benchmark_relation_reduce.py:63).
 *   input [M,Kd] (f32/bf16/f16; rows may be strided), weight [N,Kd] (16-bit
 *   weights take a 16-bit input of their dtype or f32, rounded on load; f32
 *   weights take f32), bias [N] or NULL.
 * Output: out [M,N] (f32/bf16/f16; unit column stride, rows may be strided,
 * e.g. a cache column cache[:, t]).  16-bit weights use MFMA with fp32
 * accumulation; f32 weights use fp32 arithmetic throughout.
 */
hipError_t rlm_linear(const rlm_tensor* input, const rlm_tensor* weight,
                      const rlm_tensor* bias, const rlm_tensor* out,
                      hipStream_t stream);

/* ------------------------------------------------------------------------
 * Multi-anchor relation block (the cfg5 RelationBlockStack)
 * ---------------------------------------------------------------------- */

/*
 * Replaces the post-selection half of MultiAnchorRelationBlock.forward
 *   (src/relation_lm/models/multi_relation_blocks.py:163-178): the relation
 * MLP's closing LayerNorm per (query, slot, partner) row (:51), the per-slot
 * partner softmax without k_limit (:164-168), the slot context (:169-170), the
 * slot mix (:172-177) and the residual gate (:178).  The MLP's two Linears run
 * before it (rlm_relation_hidden_cached_seq over the S*K rows of each query,
 * then rlm_linear).
 *   raw [B,Tq,S*K,D] (row s*K + k; f32/bf16/f16), partner_scores f32
 *   [B,Tq,S,K] (-inf marks an inactive partner), norm_weight / norm_bias [D],
 *   slot_mix_logits [S], residual_gate 0-d, hidden [B,Tq,D] (the block input),
 *   positions [Tq] or [B,Tq] (slot s is active iff s <= t).
 *   S*K <= 64; D a multiple of 4, at most 2048.
 * Outputs: out [B,Tq,D] in hidden's dtype = hidden + sigmoid(gate) * context;
 *          context f32 [B,Tq,D] (the block's relation_context), or NULL.
 * raw_bias [D] or NULL: added to every raw row as it is loaded (fp32), so
 * the second Linear that produces raw may run without its bias.
 */
hipError_t rlm_multi_relation_reduce_seq(
    const rlm_tensor* raw, const rlm_tensor* partner_scores, const rlm_tensor* norm_weight,
    const rlm_tensor* norm_bias, const rlm_tensor* slot_mix_logits,
    const rlm_tensor* residual_gate, const rlm_tensor* hidden, const rlm_tensor* positions,
    double norm_eps, const rlm_tensor* out, const rlm_tensor* context,
    const rlm_tensor* raw_bias, hipStream_t stream);

/*
 * Replaces nn.LayerNorm over the last dimension: the block's input_norm and
 * the stack's final_norm (multi_relation_blocks.py:39, :111, :198, :207).
 *   input [..., D] (1-4 dims, f32/bf16/f16), weight / bias [D].  D a multiple
 *   of 4, at most 2048.  Statistics in fp32.
 * Output: out, input's shape and dtype.
 */
hipError_t rlm_layer_norm(const rlm_tensor* input, const rlm_tensor* weight,
                          const rlm_tensor* bias, double eps, const rlm_tensor* out,
                          hipStream_t stream);

/*
 * Replaces DistilledBlockRouter.block_statistics
 *   (src/relation_lm/routing/block_router.py:54-68): mean and biased std of
 * the router keys over each block of block_size positions, per channel.
 *   keys [B,T,C] (f32/bf16/f16), T a multiple of block_size.
 * Outputs: out_mean, out_std f32 [B,T/block_size,C] (the [B,NB,H,HD] block
 * statistics of the selection ops with C = H*HD).
 */
hipError_t rlm_block_statistics(const rlm_tensor* keys, int64_t block_size,
                                const rlm_tensor* out_mean, const rlm_tensor* out_std,
                                hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RELATION_LM_HIP_H */
