#!/usr/bin/env python3
"""Throughput of the routed relation path on one MI355X.

Step = one pass of the cfg2 prefill workload (B=8, T=512, d=512, block 32,
local 64, top 4, K=8, bf16 activations / fp32 scores, relation hidden 512):
    relation_select (all 4096 queries) || expanded-cache projection
    -> fused relation reduce (hidden -> second linear -> LayerNorm / softmax /
       partner sum in one kernel).
The selection and the projection are independent.  Two schedules of the step
are measured over the same K steps -- eager launches on one stream, and one HIP
graph in which the selection runs on a second stream beside the projection
(checked bit-equal to the eager step) -- and `value` is the faster one's
queries per second, with every input resident in HBM.

Before the first timed window the serial step runs for at least SETTLE_S
seconds (reported as `settle`).

Also reported:
  * every schedule's time (forked graph, serial eager, serial graph);
  * the same step through the reference's unfused op sequence
    (relation_hidden_cached -> linear -> relation_norm_reduce);
  * per-kernel average duration (HIP events on the launch stream) and the
    roofline fraction of the dominant kernel (HBM bytes at the operator
    contract, or matrix-core FLOPs for the fused reduce);
  * decode-step latency (cfg3: packed 576->512 projection, router cache update,
    cache-row writes, select, reduce, output-head preparation) at B=1 and B=8,
    eager and replayed from a HIP graph; the same step at position 4095 over 512-row ring-buffer caches;
  * routed multi-anchor selection at cfg5 (B=4, T=4096, 4 anchor slots x K=6,
    block 64, local 128, top 8): one layer's selection over all 16384 queries,
    and the 4-layer RelationBlockStack;
  * the reference's published microbenchmark policy (context 512, block 8,
    local 16, top 2, K 8, fp32): relation_select_packed, the two-op path and
    the packed projection at B=1 and B=8, beside the reference's figures;
  * the CPU baseline: the path restated in eager fp32 torch (oracle/eager.py),
    timed on all of this host's affinity threads at cfg1, cfg2 and the cfg3
    decode step.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "relation-lm_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
CALIBRATION_BYTES = 256 << 20  # plain copy whose counter readings scale FETCH/WRITE_SIZE
RING_POSITION = 4095            # decode position of the ring-buffer step (512-row caches)
MALL_BYTES = 256 * 2**20        # MI355X last-level (Infinity) cache
SETTLE_S = 3.0                  # seconds of headline steps before the first timed window
CPU_WARMUP = 3                  # CPU baseline: warm-up calls per shape
CPU_SAMPLES = 9                 # CPU baseline: timed calls per shape (median)
# Kernel-name prefixes (as rocprofv3 reports them) of the timed kernels.
KERNEL_SYMBOLS = {
    "expanded_projection": "smallk_kernel<rlm::bf16, rlm::bf16, rlm::bf16",
    "relation_select": "select_tile_kernel<float, false>",
    "relation_select_expand": "select_tile_kernel<float, true>",
    "relation_reduce_fused": "fused_reduce_kernel<",
    "relation_hidden": "hidden_tile_kernel<",
    "second_linear": "tile_kernel<float, rlm::bf16, float",
    "norm_reduce": "norm_reduce_vec_kernel<",
    "multi_anchor_select": "multi_tile_kernel<",
}


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--kernel-repeats", type=int, default=50)
    ap.add_argument("--decode-steps", type=int, default=200)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only-chain", action="store_true",
                    help="run only the timed chain (for profiler runs)")
    ap.add_argument("--decode-only", action="store_true",
                    help="time only the cfg3 decode step (B=1 and B=8) and exit")
    ap.add_argument("--policy-only", action="store_true",
                    help="time only the reference's published routing policy (block 8, local 16, "
                         "top 2, K 8, fp32)")
    ap.add_argument("--multi-only", action="store_true",
                    help="time only the cfg5 routed multi-anchor selection and exit")
    ap.add_argument("--gemm-only", action="store_true",
                    help="time only the hand-written GEMM on the second-Linear shapes and exit")
    ap.add_argument("--reduce-only", action="store_true",
                    help="time only the cfg4 fused reduce in isolation and exit")
    ap.add_argument("--profile-kernels", type=int, default=0, metavar="N",
                    help="run a 256 MiB calibration copy, then each timed kernel N times, and "
                         "exit (the command profiled by rocprofv3 --kernel-trace / --pmc)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="turn two rocprofv3 --pmc counter_collection.csv files (FETCH_SIZE, "
                         "WRITE_SIZE) of a --profile-kernels run into profiles/cfg2_traffic.json")
    return ap.parse_args()


def algorithmic_bytes(cfg):
    """Operator-contract bytes per launch (inputs at unique footprint + outputs)."""
    b, t, e, k = cfg.batch, cfg.context, cfg.exact_dim, cfg.k_out
    rd = cfg.heads * cfg.head_dim
    r, h, d = cfg.relation_dim, cfg.hidden_dim, cfg.d_model
    q = b * t
    s = 2  # bf16 activations
    nb = cfg.blocks
    out = {
        "expanded_projection": q * r * s + 2 * h * r * s + 2 * h * s + q * 2 * h * s,
        "relation_select": (q * (2 * e + 2 * rd) * s + b * (t * (3 * e + rd) * s + 4 * nb * rd * 4)
                            + q * (8 + 8 * k)),
        "relation_hidden": b * t * (2 * h + r) * s + h * r * s + q * k * h * 4 + q * (1 + k) * 4,
        "second_linear": q * k * h * 4 + d * h * s + d * s + q * k * d * 4,
        "norm_reduce": q * k * d * 4 + q * k * 4 + 2 * d * s + q * d * 4,
        "relation_reduce_fused": (b * t * (2 * h + r) * s + h * r * s + d * h * s + d * s
                                  + q * (1 + k) * 4 + q * k * 4 + 2 * d * s + q * d * 4),
    }
    # The selection launch that also projects the expanded cache: both contracts.
    out["relation_select_expand"] = out["relation_select"] + out["expanded_projection"]
    return out


def multi_select_bytes(cfg):
    """Operator-contract bytes of one multi-anchor selection launch: query-side
    rows, every key/cache row once, block statistics, outputs."""
    b, t, e, s_, k = cfg.batch, cfg.context, cfg.exact_dim, cfg.slots, cfg.k_out
    rd = cfg.heads * cfg.head_dim
    q = b * t
    a = 2  # bf16 activations
    query_side = q * (s_ * e + rd + s_ * (e + rd)) * a
    memory_side = b * t * s_ * (e + e + (e + rd)) * a + 2 * 2 * b * cfg.blocks * rd * 4
    outputs = q * s_ * (4 + 4) + q * s_ * k * (4 + 4)
    return query_side + memory_side + outputs


def multi_select_candidate_bytes(cfg):
    """Key bytes of the candidate vectors the queries score (each slot's vector of
    every candidate, anchor and partner side).  A per-query kernel streams all of
    them; the tile kernel reads each 16-row tile once for the 16 queries of a
    workgroup, so this is an effective figure, not its traffic."""
    cap = cfg.local_window + cfg.top_blocks * cfg.block_size
    return cfg.batch * cfg.context * 2 * cfg.slots * cap * cfg.exact_dim * 2


def algorithmic_flops(cfg):
    """Matrix-core FLOPs per launch at the operator contract (each product counted once)."""
    q, k = cfg.batch * cfg.context, cfg.k_out
    r, h, d = cfg.relation_dim, cfg.hidden_dim, cfg.d_model
    return {
        "expanded_projection": 2 * q * r * 2 * h,
        "relation_hidden": 2 * q * k * r * h,
        "second_linear": 2 * q * k * h * d,
        "relation_reduce_fused": 2 * q * k * (r * h + h * d),
    }


def main() -> int:
    args = parse_args()
    if args.summarize_pmc:
        return summarize_pmc(*args.summarize_pmc)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the routed relation path is batch-separable; "
              f"see DESIGN.md for the sharding plan); got --gpus {args.gpus}", file=sys.stderr)
        return 2

    import torch

    from relation_lm.kernels.relation_reduce import (
        mfma_fragments,
        relation_hidden_cached_seq,
        relation_linear,
        relation_norm_reduce_seq,
        relation_reduce_fused_seq,
    )
    from relation_lm.kernels.relation_select import (
        multi_relation_select_seq,
        relation_select_packed_seq,
        relation_select_packed_seq_expand,
    )
    from relation_lm.workloads import (
        CONFIGS,
        MULTI_CONFIGS,
        RelationConfig,
        causal_partner_indices,
        decode_state,
        multi_select_args,
        multi_selection_inputs,
        reduce_inputs,
        select_args,
        selection_inputs,
    )
    from relation_lm.workloads import ONE_ROUND_WORKGROUPS
    from relation_lm.workloads import decode_step as workload_decode_step

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)

    def windowed_us(fn, steps, windows=10):
        """Per-step microseconds of `fn`: the median over `windows` back-to-back
        windows of steps/windows calls each, so that one host-side stall in a
        window (an eager step launches about ten kernels from Python) does not
        move the figure."""
        per = max(1, steps // windows)
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(windows + 1)]
        torch.cuda.synchronize()
        marks[0].record()
        for w in range(windows):
            for _ in range(per):
                fn()
            marks[w + 1].record()
        torch.cuda.synchronize()
        return statistics.median(marks[w].elapsed_time(marks[w + 1]) * 1e3 / per
                                 for w in range(windows))

    def run_decode(ring_position=None):
        """Decode-step latency (cfg3) at B=1 and B=8, eager and from a HIP graph.

        ring_position: decode at that absolute position over ring-buffer caches of
        the cfg3 length (the *_ring ops; rows written at position mod length)."""
        decode = {}
        for batch in (1, 8):
            dcfg = RelationConfig(**{**CONFIGS["cfg3"].__dict__, "batch": batch})
            state = decode_state(dcfg, device=device, position=ring_position)

            def decode_step(state=state, dcfg=dcfg):
                # projection + cache rows + router update; selection with the
                # token's expanded-cache row; the relation tail (cached hidden,
                # second linear, norm-reduce with the output-head preparation)
                return workload_decode_step(state, dcfg)[-1]

            for _ in range(20):
                decode_step()
            torch.cuda.synchronize()
            eager_us = windowed_us(decode_step, args.decode_steps)
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                decode_step()
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                decode_step()
            for _ in range(10):
                graph.replay()
            torch.cuda.synchronize()
            graph_us = windowed_us(graph.replay, args.decode_steps)
            # Four steps per replay: the host's per-replay launch cost (about the
            # GPU time of one step once the step is three launches) paid once per
            # four steps; the GPU work per step is the same.
            graph4 = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph4):
                for _ in range(4):
                    decode_step()
            for _ in range(5):
                graph4.replay()
            torch.cuda.synchronize()
            graph4_us = windowed_us(graph4.replay, max(10, args.decode_steps // 4)) / 4
            one_launch_tail = batch * (dcfg.hidden_dim // 64) <= ONE_ROUND_WORKGROUPS
            decode[f"B{batch}"] = {"eager_us": round(eager_us, 2), "graph_us": round(graph_us, 2),
                                   "graph_x4_us": round(graph4_us, 2),
                                   "launches": 3 if one_launch_tail else 5}

        return decode

    def run_multi(repeats=20):
        """cfg5 routed multi-anchor selection: one layer's selection, every query."""
        mcfg = MULTI_CONFIGS["cfg5"]
        minp = multi_selection_inputs(mcfg, device=device)
        margs = multi_select_args(minp, mcfg)
        for _ in range(3):
            multi_relation_select_seq(*margs)
        torch.cuda.synchronize()
        start.record()
        for _ in range(repeats):
            multi_relation_select_seq(*margs)
        end.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(end) * 1e3 / repeats
        nbytes = multi_select_bytes(mcfg)
        scored = multi_select_candidate_bytes(mcfg)
        return {
            "workload": "cfg5 one layer: B=4 T=4096 4 anchor slots x K=6, block 64, local 128, "
                        "top 8, bf16, every position a query",
            "us": round(us, 1),
            "queries_per_s": round(mcfg.queries / (us * 1e-6), 1),
            "algorithmic_bytes": nbytes,
            "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "candidate_vector_bytes": scored,
            "candidate_vector_GBps_effective": round(scored / (us * 1e-6) / 1e9, 1),
            "stack": run_stack(mcfg),
        }

    def run_stack(mcfg, repeats=3):
        """The cfg5 RelationBlockStack (4 routed multi-anchor blocks + final norm) on
        the HIP path, random-init bf16 weights, synthetic N(0,1) hidden / memory:
        the whole forward timed, and one block split into its selection half
        (input norm, projections, router statistics, routed selection) and its
        relation half (MLP hidden, second linear, LayerNorm / softmax / slot mix)."""
        from relation_lm.models import MultiRelationBlockConfig, RelationBlockStack

        bcfg = MultiRelationBlockConfig(
            d_model=mcfg.d_model, gate_dim=mcfg.exact_dim, relation_dim=128, ff_mult=4,
            anchors_per_block=mcfg.slots, partners_per_anchor=mcfg.k_out,
            block_size=mcfg.block_size, local_window=mcfg.local_window,
            top_blocks=mcfg.top_blocks, router_heads=mcfg.heads, router_head_dim=mcfg.head_dim,
            rel_buckets=mcfg.rel_buckets)
        torch.manual_seed(mcfg.seed)
        stack = RelationBlockStack(bcfg, mcfg.layers).to(device=device, dtype=torch.bfloat16)
        g = torch.Generator().manual_seed(mcfg.seed + 1)
        shape = (mcfg.batch, mcfg.context, mcfg.d_model)
        hidden = torch.randn(shape, generator=g).to(device=device, dtype=torch.bfloat16)
        memory = torch.randn(shape, generator=g).to(device=device, dtype=torch.bfloat16)
        block = stack.blocks[0]
        with torch.no_grad():
            for _ in range(2):
                stack(hidden, memory)
            torch.cuda.synchronize()
            start.record()
            for _ in range(repeats):
                stack(hidden, memory)
            end.record()
            torch.cuda.synchronize()
            stack_ms = start.elapsed_time(end) / repeats
            marks = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
            marks[0].record()
            sel = block.select(hidden, memory)
            marks[1].record()
            block.relate(hidden, sel)
            marks[2].record()
            torch.cuda.synchronize()
        layer_flops = 2 * mcfg.queries * mcfg.slots * mcfg.k_out * (
            bcfg.relation_dim * bcfg.ff_mult * bcfg.d_model
            + bcfg.ff_mult * bcfg.d_model * bcfg.d_model)
        return {
            "workload": (f"cfg5 RelationBlockStack: {mcfg.layers} routed multi-anchor blocks + "
                         f"final norm, B={mcfg.batch} T={mcfg.context} d={mcfg.d_model}, "
                         f"{mcfg.slots} slots x K={mcfg.k_out}, relation dim 128, MLP hidden "
                         f"{bcfg.ff_mult * bcfg.d_model}, bf16, random-init weights"),
            "stack_ms": round(stack_ms, 3),
            "tokens_per_s": round(mcfg.queries / (stack_ms * 1e-3), 1),
            "layer0_select_ms": round(marks[0].elapsed_time(marks[1]), 3),
            "layer0_relate_ms": round(marks[1].elapsed_time(marks[2]), 3),
            "relation_mlp_tflop_per_layer": round(layer_flops / 1e12, 3),
        }

    def run_reduce_cfg4(repeats=20):
        """cfg4: the fused reduce in isolation (B=8, T=2048, d 512, hidden 1024, K=8),
        partners uniform over the causal history, against the unfused three-op chain."""
        rcfg = CONFIGS["cfg4"]
        rred = reduce_inputs(rcfg, device=device)
        rexp = relation_linear(rred["operand_cache"], rred["expanded_weight"],
                               rred["expanded_bias"])
        ra, rp, rs, rpos = (x.to(device) for x in causal_partner_indices(rcfg, seed=41))
        rw2 = mfma_fragments(rred["second_weight"])   # packed once, like the model's weights

        def fused_once():
            return relation_reduce_fused_seq(rexp, rred["operand_cache"], ra, rp,
                                             rred["product_weight"], rw2,
                                             rred["second_bias"], rs, rred["norm_weight"],
                                             rred["norm_bias"], rpos, 1e-5)

        def unfused_once():
            hid = relation_hidden_cached_seq(rexp, rred["operand_cache"], ra, rp,
                                             rred["product_weight"])
            raw = relation_linear(hid, rred["second_weight"], rred["second_bias"],
                                  out_dtype=torch.float32)
            return relation_norm_reduce_seq(raw, rs, rred["norm_weight"], rred["norm_bias"],
                                            rpos, 1e-5)

        out = {}
        for name, fn in (("fused", fused_once), ("unfused", unfused_once)):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            start.record()
            for _ in range(repeats):
                fn()
            end.record()
            torch.cuda.synchronize()
            out[name] = start.elapsed_time(end) * 1e3 / repeats
        flops = algorithmic_flops(rcfg)["relation_reduce_fused"]
        nbytes = algorithmic_bytes(rcfg)["relation_reduce_fused"]
        return {
            "workload": "cfg4 fused reduce in isolation: B=8 T=2048 d=512 hidden 1024 K=8 bf16, "
                        "partners uniform over the causal history",
            "us": round(out["fused"], 1),
            "unfused_us": round(out["unfused"], 1),
            "queries_per_s": round(rcfg.queries / (out["fused"] * 1e-6), 1),
            "algorithmic_flops": flops,
            "tflops": round(flops / (out["fused"] * 1e-6) / 1e12, 1),
            "mfma_frac": round(flops / (out["fused"] * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            "algorithmic_bytes": nbytes,
        }

    def run_gemm(repeats=20):
        """The hand-written MFMA GEMM (relation_linear, fp32 output with bias) on the
        second-Linear shapes of the path: cfg5's relation MLP (one batch row's
        [T*S*K, 4d] x [d, 4d]^T, bf16) and cfg2's second linear ([Q*K, H] x [D, H]^T,
        bf16 hidden as the fused reduce sees it, and the unfused chain's fp32 hidden)."""
        g = torch.Generator(device="cpu").manual_seed(7)
        shapes = {
            "cfg5_mlp_second_linear": (98304, 3072, 768, torch.bfloat16),
            "cfg5_mlp_second_linear_2rows": (196608, 3072, 768, torch.bfloat16),
            "cfg2_second_linear_bf16": (32768, 512, 512, torch.bfloat16),
            "cfg2_second_linear_fp32_hidden": (32768, 512, 512, torch.float32),
        }
        out = {}
        for name, (m, k, n, adt) in shapes.items():
            a = torch.randn(m, k, generator=g).to(device=device, dtype=adt)
            w = (torch.randn(n, k, generator=g) * k ** -0.5).to(device=device,
                                                               dtype=torch.bfloat16)
            bias = torch.randn(n, generator=g).to(device=device, dtype=torch.bfloat16)
            for _ in range(3):
                relation_linear(a, w, bias, out_dtype=torch.float32)
            torch.cuda.synchronize()
            start.record()
            for _ in range(repeats):
                relation_linear(a, w, bias, out_dtype=torch.float32)
            end.record()
            torch.cuda.synchronize()
            us = start.elapsed_time(end) * 1e3 / repeats
            flops = 2 * m * k * n
            tf = flops / (us * 1e-6) / 1e12
            out[name] = {"shape": f"[{m},{k}] x [{n},{k}]^T, A {str(adt)[6:]}, W bf16, fp32 out",
                         "us": round(us, 2), "tflops": round(tf, 1),
                         "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)}
            del a, w, bias
        out["cfg5_relation_mlp"] = run_relation_mlp(repeats)
        return out

    def run_relation_mlp(repeats=20):
        """cfg5's relation MLP for one batch row (T=4096, 4 slots x K=6 = 98304 rows,
        relation dim 128, hidden 3072, d_model 768, bf16): the fused kernel
        (relation_hidden_linear_seq_out, hidden on chip) against the two launches it
        replaces (relation_hidden_cached_seq_out into bf16, then relation_linear).
        Indices uniform over the batch row's 4096 positions."""
        from relation_lm.kernels.relation_reduce import (mfma_fragments,
                                                         relation_hidden_cached_seq_out,
                                                         relation_hidden_linear_seq_out)
        g = torch.Generator(device="cpu").manual_seed(11)
        t, q, k, r, h, d = 4096, 4096 * 4, 6, 128, 3072, 768
        expanded = (torch.randn(1, t, 2 * h, generator=g) * 0.5).to(device, torch.bfloat16)
        operand = torch.randn(1, t, r, generator=g).to(device, torch.bfloat16)
        anchor = torch.randint(0, t, (1, q), generator=g).to(device)
        partner = torch.randint(0, t, (1, q, k), generator=g).to(device)
        wm = (torch.randn(h, r, generator=g) * r ** -0.5).to(device, torch.bfloat16)
        w2 = (torch.randn(d, h, generator=g) * h ** -0.5).to(device, torch.bfloat16)
        raw = torch.empty((1, q, k, d), device=device)
        hidden = torch.empty((1, q, k, h), device=device, dtype=torch.bfloat16)

        wm_frags, w2_frags = mfma_fragments(wm), mfma_fragments(w2)

        def fused():
            relation_hidden_linear_seq_out(expanded, operand, anchor, partner, wm_frags, w2_frags,
                                           raw)

        def two_ops():
            relation_hidden_cached_seq_out(expanded, operand, anchor, partner, wm, hidden)
            relation_linear(hidden.view(q * k, h), w2, None, out_dtype=torch.float32)

        res = {}
        for name, fn in (("fused", fused), ("two_ops", two_ops)):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            start.record()
            for _ in range(repeats):
                fn()
            end.record()
            torch.cuda.synchronize()
            res[f"{name}_us"] = round(start.elapsed_time(end) * 1e3 / repeats, 2)
        rows = q * k
        flops = 2 * rows * h * (2 * r) + 2 * rows * h * d   # hi/lo product MFMAs + second Linear
        res.update({"rows": rows, "workload": "cfg5 relation MLP, one batch row: 98304 rows, "
                    "relation dim 128 -> hidden 3072 (GELU, bf16) -> d_model 768, fp32 out",
                    "mfma_tflop": round(flops / 1e12, 4),
                    "fused_tflops": round(flops / (res["fused_us"] * 1e-6) / 1e12, 1)})
        del expanded, operand, raw, hidden
        return res

    def run_published_policy(repeats=100, samples=9):
        """The only routing policy the reference publishes numbers for
        (benchmarks/benchmark_relation_select.py:14-57, results in
        benchmarks/results/relation_select_microbenchmark.json; packed projection:
        benchmarks/benchmark_packed_cache.py:13-47, packed_cache_microbenchmark.json):
        context 512, block 8 (64 blocks), local 16, top 2, K 8, fp32 inputs with
        the reference's distributions (randn, std = rand; projection weights
        0.02 randn), B=1 and B=8.  Each figure is the median of `samples`
        windows of `repeats` eager calls (event-timed), after 50 warm-up calls.
        The reference's numbers are from an unnamed NVIDIA GPU."""
        from relation_lm.inference import pack_sparse_cache_projection_weights
        from relation_lm.kernels.relation_select import relation_select_packed
        from relation_lm.kernels.triton_select import anchor_select, partner_topk

        reference_ms = {
            "B1": {"relation_select_packed": 0.14487551689147948, "two_op": 0.34379776000976564,
                   "packed_projection": 0.03127978642781575},
            "B8": {"relation_select_packed": 0.14664704322814942, "two_op": 0.3483852767944336,
                   "packed_projection": 0.03799040158589681},
        }

        def median_ms(fn):
            for _ in range(50):
                fn()
            torch.cuda.synchronize()
            marks = [torch.cuda.Event(enable_timing=True) for _ in range(samples + 1)]
            marks[0].record()
            for i in range(samples):
                for _ in range(repeats):
                    fn()
                marks[i + 1].record()
            torch.cuda.synchronize()
            return statistics.median(marks[i].elapsed_time(marks[i + 1]) / repeats
                                     for i in range(samples))

        out = {"policy": "context 512, block 8, local 16, top 2, K 8, fp32 (the reference's "
                         "published microbenchmark policy)",
               "reference_hardware": "unnamed NVIDIA GPU (reference's committed results)"}
        for batch in (1, 8):
            g = torch.Generator().manual_seed(17)
            ctx, blocks = 512, 64
            r = lambda *shape: torch.randn(*shape, generator=g)
            u = lambda *shape: torch.rand(*shape, generator=g)
            inp = {"aq": r(batch, 64), "ak": r(batch, ctx, 64), "arq": r(batch, 64),
                   "am": r(batch, blocks, 4, 16), "as": u(batch, blocks, 4, 16), "ag": r(4),
                   "ab": r(4, 16), "pb": r(batch, 128), "pc": r(batch, ctx, 128),
                   "pk": r(batch, ctx, 64), "pm": r(batch, blocks, 4, 16),
                   "ps": u(batch, blocks, 4, 16), "pg": r(4), "pbias": r(4, 16)}
            inp = {k: v.to(device) for k, v in inp.items()}
            position = torch.tensor(ctx - 1, dtype=torch.int64, device=device)

            def packed(inp=inp, position=position):
                return relation_select_packed(
                    inp["aq"], inp["ak"], inp["arq"], inp["am"], inp["as"], inp["ag"], inp["ab"],
                    inp["pb"], inp["pc"], inp["pk"], inp["pm"], inp["ps"], inp["pg"],
                    inp["pbias"], position, 16, 2, 8, False)

            def two_op(inp=inp, position=position):
                anchor, anchor_score = anchor_select(inp["aq"], inp["ak"], inp["arq"], inp["am"],
                                                     inp["as"], inp["ag"], inp["ab"], position,
                                                     16, 2, False)
                rows = torch.arange(anchor.size(0), device=anchor.device)
                contribution = inp["pc"][rows, anchor.long()]
                exact = inp["pb"][:, :64] + contribution[:, :64]
                router = inp["pb"][:, 64:] + contribution[:, 64:]
                partner, partner_score = partner_topk(
                    exact.contiguous(), inp["pk"], router.contiguous(), inp["pm"], inp["ps"],
                    inp["pg"], inp["pbias"], position, anchor, 16, 2, 8, False)
                return anchor, anchor_score, partner, partner_score

            ref, got = two_op(), packed()
            torch.cuda.synchronize()
            index_equal = bool(torch.equal(ref[0], got[0]) and torch.equal(ref[2], got[2]))
            gp = torch.Generator().manual_seed(20260822)
            memory = torch.randn(batch, 576, generator=gp).to(device)
            weights = [(torch.randn(w, 576, generator=gp) * 0.02).to(device)
                       for w in (64, 64, 128, 128, 64, 64)]
            projection = pack_sparse_cache_projection_weights(weights)
            packed_ms = median_ms(packed)
            two_ms = median_ms(two_op)
            proj_ms = median_ms(lambda projection=projection, memory=memory:
                                projection.project(memory))
            refs = reference_ms[f"B{batch}"]
            out[f"B{batch}"] = {
                "relation_select_packed_ms": round(packed_ms, 5),
                "two_op_ms": round(two_ms, 5),
                "packed_projection_ms": round(proj_ms, 5),
                "index_equal_packed_vs_two_op": index_equal,
                "reference_ms": refs,
                "speedup_vs_reference": {
                    "relation_select_packed": round(refs["relation_select_packed"] / packed_ms, 2),
                    "two_op": round(refs["two_op"] / two_ms, 2),
                    "packed_projection": round(refs["packed_projection"] / proj_ms, 2)},
            }
        return out

    if args.policy_only:
        print(json.dumps({"published_policy": run_published_policy()}), flush=True)
        return 0
    if args.multi_only:
        print(json.dumps({"multi_anchor_select": run_multi()}), flush=True)
        return 0
    if args.gemm_only:
        print(json.dumps({"gemm": run_gemm()}), flush=True)
        return 0
    if args.reduce_only:
        print(json.dumps({"fused_reduce_cfg4": run_reduce_cfg4()}), flush=True)
        return 0

    if args.decode_only:
        print(json.dumps({"decode_step_us": run_decode(),
                          "ring_decode_step_us": run_decode(RING_POSITION)}), flush=True)
        return 0

    cfg = CONFIGS["cfg2"]
    sel = selection_inputs(cfg, device=device)
    red = reduce_inputs(cfg, device=device)
    sargs = select_args(sel, cfg)
    positions = sel["positions"]
    operand = red["operand_cache"]

    def run_expanded():
        return relation_linear(operand, red["expanded_weight"], red["expanded_bias"])

    def run_select():
        return relation_select_packed_seq(*sargs)

    def run_hidden(expanded, a, p):
        return relation_hidden_cached_seq(expanded, operand, a, p, red["product_weight"])

    def run_second(hidden):
        return relation_linear(hidden, red["second_weight"], red["second_bias"],
                               out_dtype=torch.float32)

    def run_norm(raw, ps):
        return relation_norm_reduce_seq(raw, ps, red["norm_weight"], red["norm_bias"], positions,
                                        1e-5)

    # The second Linear's weight in MFMA fragment order, packed once (a weight
    # layout, like the reference's packed sparse-cache weights): the fused kernel
    # then reads each weight fragment as one contiguous 1 KiB, same result bits.
    second_frags = mfma_fragments(red["second_weight"])

    def run_fused(expanded, a, p, ps):
        return relation_reduce_fused_seq(expanded, operand, a, p, red["product_weight"],
                                         second_frags, red["second_bias"], ps,
                                         red["norm_weight"], red["norm_bias"], positions, 1e-5)

    def step():
        expanded = run_expanded()
        a, s, p, ps = run_select()
        return run_fused(expanded, a, p, ps)

    # The selection launch also projecting the whole expanded cache
    # (relation_select_packed_seq_expand: the same cache bits as relation_linear).
    expanded_buf = torch.empty(cfg.batch, cfg.context, red["expanded_weight"].shape[0],
                               dtype=red["operand_cache"].dtype, device=device)

    def run_select_expand():
        return relation_select_packed_seq_expand(*sargs, operand, red["expanded_weight"],
                                                 red["expanded_bias"], expanded_buf)

    def step_xp():
        a, s, p, ps = run_select_expand()
        return run_fused(expanded_buf, a, p, ps)

    # The headline schedule: the selection and the expanded projection do not
    # depend on each other, so the selection runs on a second stream beside the
    # projection and the fused reduce waits for both (replayed as one HIP graph;
    # every stream at the default priority).
    select_stream = torch.cuda.Stream()

    def step_forked():
        main = torch.cuda.current_stream()
        select_stream.wait_stream(main)
        with torch.cuda.stream(select_stream):
            a, s, p, ps = run_select()
        expanded = run_expanded()
        main.wait_stream(select_stream)
        for t in (a, p, ps):
            t.record_stream(main)
        return run_fused(expanded, a, p, ps)

    def step_unfused():
        expanded = run_expanded()
        a, s, p, ps = run_select()
        hidden = run_hidden(expanded, a, p)
        raw = run_second(hidden)
        return run_norm(raw, ps)

    for _ in range(args.warmup):
        step()
        step_xp()
        step_unfused()
    torch.cuda.synchronize()
    expanded = run_expanded()
    a, s, p, ps = run_select()
    hidden = run_hidden(expanded, a, p)
    raw = run_second(hidden)
    kernels = {
        "expanded_projection": run_expanded,
        "relation_select": run_select,
        "relation_select_expand": run_select_expand,
        "relation_reduce_fused": lambda: run_fused(expanded, a, p, ps),
        "relation_hidden": lambda: run_hidden(expanded, a, p),
        "second_linear": lambda: run_second(hidden),
        "norm_reduce": lambda: run_norm(raw, ps),
    }
    if args.profile_kernels:
        src = torch.empty(CALIBRATION_BYTES // 4, dtype=torch.float32, device=device).normal_()
        dst = torch.empty_like(src)
        for _ in range(2):
            dst.copy_(src)
        for fn in kernels.values():
            for _ in range(args.profile_kernels):
                fn()
        torch.cuda.synchronize()
        print(json.dumps({"profile_kernels": args.profile_kernels, "kernels": list(kernels)}),
              flush=True)
        return 0
    if args.only_chain:
        for _ in range(args.steps):
            step()
            step_unfused()
        torch.cuda.synchronize()
        print(json.dumps({"only_chain": True, "steps": args.steps}), flush=True)
        return 0

    def timed(fn, count):
        torch.cuda.synchronize()
        start.record()
        for _ in range(count):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / count

    # Warm-up floor: the serial step for at least SETTLE_S seconds (and at least
    # `warmup` steps) before any window is timed, so that short driver runs
    # (--steps 20 --warmup 5) measure settled clocks too.
    settle_start = time.perf_counter()
    settle_steps = 0
    while settle_steps < args.warmup or time.perf_counter() - settle_start < SETTLE_S:
        step()
        settle_steps += 1
        if settle_steps % 256 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    settle_s = time.perf_counter() - settle_start
    ms_unfused = timed(step_unfused, args.steps)

    def capture(fn):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = fn()
        return graph, out

    # The forked step as one HIP graph; it must reproduce the eager serial
    # step's output bit for bit.  Every schedule is warmed up before timing
    # (graph replays reach steady state only after some hundreds of replays).
    reference_out = step().clone()
    serial_graph, _ = capture(step)
    for _ in range(args.warmup):
        serial_graph.replay()
        step_forked()
    torch.cuda.synchronize()
    step_graph, graph_out = capture(step_forked)
    for _ in range(args.warmup):
        step_graph.replay()
    torch.cuda.synchronize()
    if not torch.equal(graph_out, reference_out):
        print("forked graph step differs from the eager step", file=sys.stderr)
        return 1
    if not torch.equal(step_xp(), reference_out):
        print("the one-launch projection step differs from the eager step", file=sys.stderr)
        return 1
    ms_forked_graph = timed(step_graph.replay, args.steps)
    ms_serial_graph = timed(serial_graph.replay, args.steps)
    ms_serial = timed(step, args.steps)
    ms_xp = timed(step_xp, args.steps)
    # The step's schedule is picked by measurement, as a kernel variant would
    # be: the forked graph when it is faster, else the serial eager launches
    # (both measured above over the same K steps; same output bits).
    schedules = {
        "forked_graph": ("HIP graph: select on a second stream beside the expanded projection, "
                         "fused reduce after both", ms_forked_graph),
        "serial_eager": ("eager launches on one stream: expanded projection, select, fused "
                         "reduce", ms_serial),
        "serial_eager_projection_in_select": (
            "eager launches on one stream: select with the expanded projection in the same "
            "launch (relation_select_packed_seq_expand), fused reduce", ms_xp),
    }
    chosen = min(schedules, key=lambda k: schedules[k][1])
    ms_per_step = schedules[chosen][1]
    queries = cfg.queries
    value = queries / (ms_per_step / 1e3)

    # The same serial step over rotating copies of every input (and fresh
    # outputs), together at least twice the 256 MiB MALL, so that no step finds
    # its inputs in the last-level cache: the HBM-resident figure beside the
    # cache-resident one above (the inputs above are reused every step).
    def nbytes_of(d):
        return sum(v.numel() * v.element_size() for v in d.values() if torch.is_tensor(v))

    set_bytes = nbytes_of(sel) + nbytes_of(red) + expanded.numel() * expanded.element_size()
    n_rot = max(2, -(-2 * MALL_BYTES // set_bytes))
    rot_sets = [({k: v.clone() for k, v in sel.items()}, {k: v.clone() for k, v in red.items()})
                for _ in range(n_rot)]
    for _, rr in rot_sets:
        rr["second_frags"] = mfma_fragments(rr["second_weight"])
    rot_state = {"i": 0}

    def step_rotated():
        rs, rr = rot_sets[rot_state["i"] % n_rot]
        rot_state["i"] += 1
        rexp = relation_linear(rr["operand_cache"], rr["expanded_weight"], rr["expanded_bias"])
        ra, _, rp, rps = relation_select_packed_seq(*select_args(rs, cfg))
        return relation_reduce_fused_seq(rexp, rr["operand_cache"], ra, rp, rr["product_weight"],
                                         rr["second_frags"], rr["second_bias"], rps,
                                         rr["norm_weight"], rr["norm_bias"], rs["positions"], 1e-5)

    for _ in range(2 * n_rot):
        step_rotated()
    ms_rotated = timed(step_rotated, max(args.steps, 2 * n_rot))
    del rot_sets

    # Per-kernel average duration on the launch stream (torch's current stream).
    per_kernel_us = {}
    for name, fn in kernels.items():
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        start.record()
        for _ in range(args.kernel_repeats):
            fn()
        end.record()
        torch.cuda.synchronize()
        per_kernel_us[name] = start.elapsed_time(end) * 1e3 / args.kernel_repeats
    # The same kernels inside the serial step (events between the launches on
    # the launch stream): each kernel starts with the previous one's outputs
    # in another XCD's L2, so these run longer than the loops above.  The
    # dominant kernel is the longest one here.
    headline = ("expanded_projection", "relation_select", "relation_reduce_fused")
    marks = [[torch.cuda.Event(enable_timing=True) for _ in range(4)]
             for _ in range(args.kernel_repeats)]
    torch.cuda.synchronize()
    for ev in marks:
        ev[0].record()
        expanded = run_expanded()
        ev[1].record()
        a, s, p, ps = run_select()
        ev[2].record()
        run_fused(expanded, a, p, ps)
        ev[3].record()
    torch.cuda.synchronize()
    in_step_us = {name: statistics.median(ev[i].elapsed_time(ev[i + 1]) * 1e3 for ev in marks)
                  for i, name in enumerate(headline)}
    marks_xp = [[torch.cuda.Event(enable_timing=True) for _ in range(3)]
                for _ in range(args.kernel_repeats)]
    torch.cuda.synchronize()
    for ev in marks_xp:
        ev[0].record()
        xa, _, xp, xps = run_select_expand()
        ev[1].record()
        run_fused(expanded_buf, xa, xp, xps)
        ev[2].record()
    torch.cuda.synchronize()
    in_step_xp_us = {name: statistics.median(ev[i].elapsed_time(ev[i + 1]) * 1e3
                                             for ev in marks_xp)
                     for i, name in enumerate(("relation_select_expand", "relation_reduce_fused"))}
    nbytes = algorithmic_bytes(cfg)
    nflops = algorithmic_flops(cfg)
    dominant = max(headline, key=in_step_us.get)

    def roofline_of(name):
        """Roofline entry of one headline kernel: the fused reduce against the
        bf16 MFMA peak, the others against HBM (algorithmic bytes at the op
        contract); `achieved` from the isolated loop above."""
        if name == "relation_reduce_fused":
            achieved = nflops[name] / (per_kernel_us[name] * 1e-6) / 1e12
            entry = {"bound": "mfma", "kernel": name, "achieved": round(achieved, 1),
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                     "algorithmic_flops": nflops[name]}
        else:
            achieved = nbytes[name] / (per_kernel_us[name] * 1e-6) / 1e9
            entry = {"bound": "hbm", "kernel": name, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "algorithmic_bytes": nbytes[name]}
        entry["traffic"] = measured_traffic(name)
        entry["residency"] = "cache-resident inputs (HBM-resident step: rotated_inputs)"
        return entry

    roof = roofline_of(dominant)
    rooflines = {name: roofline_of(name) for name in headline + ("relation_select_expand",)}
    trio = ("relation_select", "relation_hidden", "norm_reduce")
    trio_bytes = sum(nbytes[k] for k in trio)
    trio_us = sum(per_kernel_us[k] for k in trio)
    unfused_bytes = sum(nbytes[k] for k in ("expanded_projection", "relation_select",
                                            "relation_hidden", "second_linear", "norm_reduce"))
    fused_bytes = sum(nbytes[k] for k in headline)

    decode = run_decode()
    ring_decode = run_decode(RING_POSITION)
    multi = run_multi()
    reduce4 = run_reduce_cfg4()
    policy = run_published_policy()
    gemm = run_gemm()

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(torch)

    result = {
        "metric": "relation_select+reduce queries/s @B8 ctx512; decode-step us; % HBM roofline",
        "value": round(value, 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations/caches, N(0,1/fan_in) weights)",
        "config": {
            "workload": "cfg2 prefill: B=8 T=512 d=512 block32 local64 top4 K=8 hidden512 "
                        "(expanded projection + select + fused hidden/linear2/norm-reduce)",
            "batch": cfg.batch, "context": cfg.context, "d_model": cfg.d_model,
            "queries_per_step": queries, "parallelism": "single GPU",
        },
        "roofline": roof,
        "rooflines": rooflines,
        "per_kernel_in_step_us": {k: round(v, 2) for k, v in in_step_us.items()},
        "per_kernel_in_step_us_projection_in_select": {k: round(v, 2)
                                                       for k, v in in_step_xp_us.items()},
        "per_kernel_us": {k: round(v, 2) for k, v in per_kernel_us.items()},
        "settle": {"seconds": round(settle_s, 2), "steps": settle_steps,
                   "floor_s": SETTLE_S},
        "schedule": schedules[chosen][0],
        "schedules_ms_per_step": {"forked_graph": round(ms_forked_graph, 5),
                                  "serial_eager": round(ms_serial, 5),
                                  "serial_eager_projection_in_select": round(ms_xp, 5),
                                  "serial_graph": round(ms_serial_graph, 5)},
        "hbm_frac_fused_chain": round(fused_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "residency": (f"value, roofline and hbm_frac_* are cache-resident: the same "
                      f"{set_bytes / 2**20:.0f} MiB of inputs every step (< 256 MiB MALL); "
                      f"rotated_inputs repeats the serial eager step over {n_rot} copies"),
        "rotated_inputs": {
            "sets": n_rot,
            "bytes_per_set": set_bytes,
            "ms_per_step": round(ms_rotated, 5),
            "value": round(queries / (ms_rotated / 1e3), 1),
            "hbm_frac_fused_chain": round(fused_bytes / (ms_rotated * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        },
        "unfused_chain": {
            "ms_per_step": round(ms_unfused, 5),
            "value": round(queries / (ms_unfused / 1e3), 1),
            "hbm_frac_chain": round(unfused_bytes / (ms_unfused * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "hbm_frac_select_hidden_norm": round(
                trio_bytes / (trio_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        },
        "decode_step_us": decode,
        "ring_decode_step_us": {"position": RING_POSITION, "cache_rows": 512, **ring_decode},
        "multi_anchor_select": multi,
        "fused_reduce_cfg4": reduce4,
        "published_policy": policy,
        "gemm": gemm,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


def summarize_pmc(fetch_csv, write_csv):
    """Per-launch HBM bytes of each timed kernel from rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE (KiB per dispatch), each scaled by what the same counter reads for the
    plain calibration copy of CALIBRATION_BYTES (which reads and writes that many bytes)."""
    import csv
    import statistics

    def per_kernel(path, counter):
        values = {}
        with open(path) as f:
            for row in csv.DictReader(f):
                if row["Counter_Name"] != counter:
                    continue
                values.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
        return values

    out = {"calibration_bytes": CALIBRATION_BYTES, "kernels": {}}
    scale = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        values = per_kernel(path, counter)
        copy = [v for name, vs in values.items() if "copyBuffer" in name for v in vs]
        kib = max(copy)  # the calibration copy is the largest copyBuffer dispatch
        scale[counter] = CALIBRATION_BYTES / (kib * 1024.0)
        out[f"{counter.lower()}_copy_kib"] = kib
        out[f"{counter.lower()}_scale"] = round(scale[counter], 4)
        for key, prefix in KERNEL_SYMBOLS.items():
            vs = [v for name, vv in values.items() if prefix in name for v in vv]
            if vs:
                entry = out["kernels"].setdefault(key, {})
                entry[f"{counter.lower()}_kib"] = statistics.median(vs)
                entry[f"{counter.lower()}_bytes"] = round(
                    statistics.median(vs) * 1024.0 * scale[counter])
    for entry in out["kernels"].values():
        if "fetch_size_bytes" in entry and "write_size_bytes" in entry:
            entry["hbm_bytes_per_launch"] = entry["fetch_size_bytes"] + entry["write_size_bytes"]
    path = os.path.join(ROOT, "profiles", "cfg2_traffic.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=2, sort_keys=True)
        f.write("\n")
    print(json.dumps(out, sort_keys=True), flush=True)
    return 0


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` measured with rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, calibrated against a copy kernel), read from the committed summary
    profiles/cfg2_traffic.json; None when that kernel was not measured."""
    path = os.path.join(ROOT, "profiles", "cfg2_traffic.json")
    try:
        with open(path) as f:
            table = json.load(f)
    except (OSError, ValueError):
        return None
    entry = table.get("kernels", {}).get(kernel)
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def cpu_model_name():
    """The host CPU's model name (lscpu, else /proc/cpuinfo)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(torch):
    """The eager fp32 torch restatement of the path (oracle/eager.py) on this host's
    cores: torch.set_num_threads(len(sched_getaffinity)), 3 warm-up calls, then the
    median of 9 timed calls (time.perf_counter), per shape: cfg1 (the primary CPU
    shape), cfg2 (the GPU headline's workload, which `value` is quoted on) and the
    cfg3 decode step at B=1 and B=8.  Inputs are the GPU run's seeded tensors
    generated on the CPU (same bits), in fp32."""
    from oracle import eager
    from relation_lm.workloads import CONFIGS, RelationConfig, packed_projection_inputs
    from relation_lm.workloads import reduce_inputs, selection_inputs

    threads = len(os.sched_getaffinity(0))
    previous = torch.get_num_threads()
    torch.set_num_threads(threads)

    def fp32(d):
        return {k: (v.float() if v.dtype.is_floating_point else v) for k, v in d.items()}

    def median_s(fn):
        for _ in range(CPU_WARMUP):
            fn()
        samples = []
        for _ in range(CPU_SAMPLES):
            t0 = time.perf_counter()
            fn()
            samples.append(time.perf_counter() - t0)
        return statistics.median(samples)

    shapes = {}
    try:
        with torch.no_grad():
            for name in ("cfg1", "cfg2"):
                cfg = CONFIGS[name]
                sel = fp32(selection_inputs(cfg))
                red = fp32(reduce_inputs(cfg))
                sec = median_s(lambda: eager.relation_chain_seq(sel, red, cfg))
                shapes[name] = {"queries": cfg.queries, "s_per_call": round(sec, 5),
                                "queries_per_s": round(cfg.queries / sec, 1)}
            for batch in (1, 8):
                cfg = RelationConfig(**{**CONFIGS["cfg3"].__dict__, "batch": batch})
                sel = fp32(selection_inputs(cfg, queries=1))
                red = fp32(reduce_inputs(cfg))
                memory, weights = packed_projection_inputs(cfg)
                memory = memory.float()
                packed = torch.cat([w.float() for w in weights], dim=0)
                expanded = eager.expanded_cache(red)  # decode state, not per-step work
                sec = median_s(lambda: eager.relation_decode_step(sel, red, expanded, memory,
                                                                  packed, cfg))
                shapes[f"cfg3_decode_b{batch}"] = {"step_us": round(sec * 1e6, 1)}
    finally:
        torch.set_num_threads(previous)
    return {
        "value": shapes["cfg2"]["queries_per_s"],
        "unit": "queries/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"eager fp32 torch restatement of the path (oracle/eager.py) on "
                   f"{threads} threads, median of {CPU_SAMPLES} calls after {CPU_WARMUP} "
                   f"warm-ups; value = cfg2 (expanded projection, select, hidden, linear2, "
                   f"norm-reduce over all {CONFIGS['cfg2'].queries} queries); cfg1 is the "
                   f"primary CPU shape of the plan"),
        "primary_cfg1_queries_per_s": shapes["cfg1"]["queries_per_s"],
        "shapes": shapes,
        "threads": threads,
        "host_cpus": os.cpu_count(),
        "cpu_model": cpu_model_name(),
    }


if __name__ == "__main__":
    sys.exit(main())
