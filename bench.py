"""Benchmark: ESA varlen attention forward + backward on one MI355X.

Workload (the benchmark definition's configuration 1): 32 protein-like graphs
(node counts U{64..512}, 3.8 A random-walk chains, radius 8 A, at most 16
neighbours), one edge token per directed edge, packed with cu_seqlens; 16
heads of head_dim 16 (dim 256); q, k, v, dO ~ N(0, 1) in bf16; causal=False;
softmax scale 1/4.  A step is one forward and one backward over the batch,
with inputs already resident in HBM.

Prints one JSON line: throughput in edge-tokens/s, MFMA utilisation of the
dense-bf16 peak, the roofline of the dominant kernel and a CPU baseline (the
reference's padded attention path restated in oracle/ -- torch's
scaled_dot_product_attention over sets padded to N, the fallback of
esa/mha_flash_varlen.py:81-126 -- on the whole batch, on this host's cores).
Beside the headline the same line carries the edge-masked attention of
configuration 2 ("masked") and the gather / segment sum of configuration 3
("gather"), each with its own roofline and CPU baseline.  Step times come
from timed regions without instrumentation; the per-kernel durations of the
rooflines come from a second region of as many steps with HIP events around
every library launch (its step time is reported as ms_per_step_profiled).
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
HEADS, HEAD_DIM = 16, 16
DIM = HEADS * HEAD_DIM

# Algorithmic FLOPs per (query, key) pair per unit of model dim D = H*hd:
# forward 4D (QK^T, PV); backward 10D (QK^T recompute, dP, dV, dK, dQ).
# The dK/dV kernel is credited with QK^T, dP, dV, dK (8D); the dQ kernel with
# dQ only (2D): its own QK^T / dP recomputation is not algorithmic work.
FLOPS_PER_PAIR = {"attn_fwd": 4 * DIM, "attn_bwd_dkdv": 8 * DIM, "attn_bwd_dq": 2 * DIM}


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-sample-graphs", type=int, default=8,
                    help="graphs of the configuration-2 batch timed on the CPU for the masked baseline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="skip configuration 0's HIP-graph leg (for profiler runs that time eager launches only)")
    ap.add_argument("--no-sub", action="store_true",
                    help="headline only: skip the masked (configuration 2), gather (configuration 3), node, wide, "
                         "dropout, block (configuration 0) and stack (configuration 4) sub-objects")
    ap.add_argument("--config", choices=["varlen", "masked", "gather", "node", "block", "stack", "wide", "dropout"],
                    default="varlen",
                    help="varlen: configuration 1 (default, the headline metric); masked: configuration 2 "
                         "(edge-masked MAB attention fwd+bwd); gather: configuration 3 (edge gather + CSR "
                         "segment sum, HBM-bound); node: node-mode (CSR adjacency) attention fwd+bwd on a "
                         "65,536-node batch; block: configuration 0 (fp32 ESA block forward on small "
                         "molecules); stack: configuration 4 (bf16 ESA encoder stack train step); wide: dense "
                         "attention at head dims 64 and 32 (D = 512) on configuration 1's graphs; dropout: "
                         "step time without and with attention dropout (configuration 1 dense, rna-shaped node "
                         "mode)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy three times (HBM counter calibration)")
    return ap.parse_args()


def copy_calibration():
    """A copy of known size: 1 GiB read + 1 GiB written per launch, for scaling FETCH_SIZE / WRITE_SIZE."""
    import torch

    n = 1 << 28   # fp32 elements = 1 GiB
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": 4 * n, "copy_bytes_written": 4 * n, "launches": 3}), flush=True)


def _median_time(step, warmup: int = 2, runs: int = 5) -> tuple[float, int]:
    """Median wall time of `runs` calls after `warmup` untimed ones (perf_counter, the CPU baselines' method)."""
    for _ in range(warmup):
        step()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_baseline(gb, seed: int) -> dict:
    """The reference's padded attention path on the host cores, fp32, forward + backward on the whole batch.

    oracle.attention.padded_sdpa restates MABFlashVarlen._forward_padded (esa/mha_flash_varlen.py:81-126):
    every graph padded to N = nearest_multiple_of_8(max L + 1) positions and torch's
    scaled_dot_product_attention with the key-padding mask, backward by autograd.  Timed with all the
    process's cores, then with one thread (the reference's own setting, core/train_pretrain.py:850) on the
    median-length graph alone."""
    import torch

    from oracle import attention as oracle_attention
    from oracle.packing import nearest_multiple_of_8

    cores = len(os.sched_getaffinity(0))
    cu = gb.cu_seqlens.astype(np.int64)
    t = int(cu[-1])
    n = nearest_multiple_of_8(gb.max_seqlen + 1)
    g = torch.Generator().manual_seed(seed + 99)
    q, k, v, go = (torch.randn(t, HEADS, HEAD_DIM, generator=g) for _ in range(4))

    def make_step(qq, kk, vv, gg, cuq, nn):
        def step():
            qd, kd, vd = (x.detach().requires_grad_(True) for x in (qq, kk, vv))
            out = oracle_attention.padded_sdpa(qd, kd, vd, cuq, cuq, nn, 1.0 / HEAD_DIM ** 0.5)
            out.backward(gg)
        return step

    torch.set_num_threads(cores)
    med, runs = _median_time(make_step(q, k, v, go, cu, n))
    b = int(np.argsort(gb.edge_counts)[len(gb.edge_counts) // 2])
    s0, e0 = int(cu[b]), int(cu[b + 1])
    sub = np.array([0, e0 - s0])
    torch.set_num_threads(1)
    med1, runs1 = _median_time(make_step(q[s0:e0], k[s0:e0], v[s0:e0], go[s0:e0], sub, n), warmup=1, runs=3)
    torch.set_num_threads(cores)
    return {"value": t / med, "unit": "edge-tokens/s", "cores": cores, "kind": "port",
            "sample": (f"the whole batch ({t} edge tokens, {gb.num_graphs} graphs padded to N = {n}): the reference's "
                       f"padded path (esa/mha_flash_varlen.py:81-126) restated in oracle.attention.padded_sdpa, "
                       f"torch scaled_dot_product_attention fp32 forward + autograd backward on {cores} threads, "
                       f"median of {runs} runs after 2 warm-ups"),
            "one_thread": {"value": (e0 - s0) / med1, "unit": "edge-tokens/s", "cores": 1,
                           "sample": f"the median-length graph ({e0 - s0} edge tokens, padded to {n}), median of "
                                     f"{runs1} runs after 1 warm-up (padding to N makes shorter graphs cost as "
                                     f"much as the longest, so the batch runs slower per token)"}}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "The ESA attention batch shards by whole graphs with no exchange; run one process per GPU.",
              file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        copy_calibration()
        return
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.config == "varlen":
        result = bench_varlen(args)
        if not args.no_sub:
            result["masked"] = bench_masked(args, sub=True)
            result["gather"] = bench_gather(args, sub=True)
            result["node"] = bench_node(args, sub=True)
            result["block"] = bench_block(args, sub=True)
            result["stack"] = bench_stack(args, sub=True)
            # the heavy wide / dropout lines last: configuration 0's launch-bound step measured 2.5x slower when
            # it followed them in one process
            result["wide"] = bench_wide(args)
            result["dropout"] = bench_dropout(args)
        print(json.dumps(result), flush=True)
        return
    if args.config == "wide":
        print(json.dumps({"metric": "edge-tokens/sec through ESA attn fwd+bwd at head dims 64 / 32",
                          "value": None, "unit": "edge-tokens/s", **bench_wide(args)}), flush=True)
        return
    if args.config == "dropout":
        print(json.dumps({"metric": "ESA attn fwd+bwd step time without / with attention dropout", "value": None,
                          "unit": "ms", **bench_dropout(args)}), flush=True)
        return
    {"masked": bench_masked, "gather": bench_gather, "node": bench_node, "block": bench_block,
     "stack": bench_stack}[args.config](args)


def timed(step, steps: int, warmup: int, profile: bool = True):
    """Warm-up steps, then `steps` timed steps without instrumentation: (ms per step by HIP events, wall ms per
    step, per-kernel records, profiled ms per step).  With `profile`, a second region of `steps` steps runs with
    the library's per-kernel hook, which records a HIP event pair around every library kernel launch on the
    launch's own stream; its per-kernel average durations fill the records (empty without `profile`) and its
    step time, which includes the event records between launches, is the fourth value (None without
    `profile`)."""
    import torch

    from mind_amd import _lib

    def region():
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        gc.collect()
        gc.disable()   # as timeit does: no collector pauses inside the timed host loop
        try:
            torch.cuda.synchronize()
            wall0 = time.perf_counter()
            ev0.record()
            for _ in range(steps):
                step()
            ev1.record()
            torch.cuda.synchronize()
        finally:
            gc.enable()
        return ev0.elapsed_time(ev1) / steps, 1e3 * (time.perf_counter() - wall0) / steps

    for _ in range(warmup):
        step()
    ms, wall = region()
    if not profile:
        return ms, wall, {}, None
    _lib.profile_enable(True)
    ms_prof, _ = region()
    _lib.profile_enable(False)
    kern = {name: {"avg_us": 1e3 * t / n, "launches": n} for name, (t, n) in _lib.profile_collect().items() if n}
    return ms, wall, kern, ms_prof


def bench_varlen(args):
    import numpy as np
    import torch

    from mind_amd import _lib, generators
    from mind_amd.esa import attention

    dev = torch.device("cuda", 0)
    gb = generators.protein_like(seed=args.seed)
    cu_np = gb.cu_seqlens
    t = int(cu_np[-1])
    pairs = gb.sum_sq
    g = torch.Generator().manual_seed(args.seed)
    q, k, v, go = (torch.randn(t, HEADS, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev) for _ in range(4))
    cu = torch.as_tensor(cu_np).to(dev)
    maxlen = gb.max_seqlen
    scale = 1.0 / HEAD_DIM ** 0.5

    def step():
        out, lse = attention.attn_fwd(q, k, v, cu, cu, maxlen, maxlen, scale)
        attention.attn_bwd(go, q, k, v, out, lse, cu, cu, maxlen, maxlen, scale)

    ms_per_step, wall_ms, per_kernel, ms_prof = timed(step, args.steps, args.warmup)
    tokens_per_s = t / (ms_per_step * 1e-3)
    total_flops = 14 * DIM * pairs
    tflops = total_flops / (ms_per_step * 1e-3) / 1e12
    dom = max((n for n in FLOPS_PER_PAIR if n in per_kernel), key=lambda n: per_kernel[n]["avg_us"])
    dom_flops = FLOPS_PER_PAIR[dom] * pairs
    dom_avg_s = per_kernel[dom]["avg_us"] * 1e-6
    achieved = dom_flops / dom_avg_s / 1e12
    for name, rec in per_kernel.items():
        if name in FLOPS_PER_PAIR:
            rec["algorithmic_tflops"] = FLOPS_PER_PAIR[name] * pairs / (rec["avg_us"] * 1e-6) / 1e12

    traffic = None
    tfile = ROOT / "profiles" / f"{dom}_config1_traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")

    result = {
        "metric": "edge-tokens/sec through ESA attn fwd+bwd; MFMA util % of bf16 peak",
        "value": tokens_per_s,
        "unit": "edge-tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded protein-like radius graphs; q, k, v, dO ~ N(0,1))",
        "config": {
            "workload": "config1: varlen flash attention fwd+bwd over packed edge sets",
            "graphs": gb.num_graphs, "edge_tokens": t, "max_seqlen": maxlen, "sum_L2": pairs,
            "heads": HEADS, "head_dim": HEAD_DIM, "dim": DIM, "causal": False, "seed": args.seed,
        },
        "mfma_util_pct": 100.0 * tflops / PEAK_BF16_TFLOPS,
        "achieved_tflops": tflops,
        "algorithmic_flops_per_step": total_flops,
        "wall_ms_per_step": wall_ms, "ms_per_step_profiled": ms_prof,
        "kernels": per_kernel,
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": achieved, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / PEAK_BF16_TFLOPS, "traffic": traffic},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(gb, args.seed)
    return result


def bench_wide(args) -> dict:
    """Dense varlen attention fwd+bwd at the wide head dims of MIND's larger configurations (D = 512: 8 heads of
    64 in core/pretraining_config_qm9.yaml:27-28 / unimol / lba, 16 heads of 32 in pretraining_config_coconut.yaml:
    21-22) on configuration 1's batch (the same graphs and token counts as the headline), bf16; the MFMA kernels of
    esa_attn_wide.hip.  Per head dim: step time, edge-tokens/s, the step's fraction of dense-bf16 peak on 14 D per
    pair, and the dominant kernel's roofline (the kernel FLOPs of the headline: forward 4 D, dK/dV 8 D, dQ 2 D
    per pair)."""
    import torch

    from mind_amd import generators
    from mind_amd.esa import attention

    dev = torch.device("cuda", 0)
    gb = generators.protein_like(seed=args.seed)
    t, pairs, maxlen = int(gb.cu_seqlens[-1]), gb.sum_sq, gb.max_seqlen
    cu = torch.as_tensor(gb.cu_seqlens).to(dev)
    out = {"workload": "config1 graphs, dense varlen attention fwd+bwd at D = 512 (head dims 64 and 32), bf16",
           "graphs": gb.num_graphs, "edge_tokens": t, "sum_L2": pairs, "dim": 512}
    for hd in (64, 32):
        heads = 512 // hd
        d = heads * hd
        g = torch.Generator().manual_seed(args.seed + hd)
        q, k, v, go = (torch.randn(t, heads, hd, generator=g).to(torch.bfloat16).to(dev) for _ in range(4))
        scale = 1.0 / hd ** 0.5

        def step():
            o, lse = attention.attn_fwd(q, k, v, cu, cu, maxlen, maxlen, scale)
            attention.attn_bwd(go, q, k, v, o, lse, cu, cu, maxlen, maxlen, scale)

        ms, wall_ms, kern, ms_prof = timed(step, args.steps, args.warmup)
        per_pair = {"attn_fwd": 4 * d, "attn_bwd_dkdv": 8 * d, "attn_bwd_dq": 2 * d}
        for name, rec in kern.items():
            if name in per_pair:
                rec["algorithmic_tflops"] = per_pair[name] * pairs / (rec["avg_us"] * 1e-6) / 1e12
        dom = max((n for n in per_pair if n in kern), key=lambda n: kern[n]["avg_us"])
        achieved = kern[dom]["algorithmic_tflops"]
        tflops = 14 * d * pairs / (ms * 1e-3) / 1e12
        traffic = None   # HBM bytes per launch of the dominant kernel (rocprofv3 FETCH_SIZE + WRITE_SIZE)
        tfile = ROOT / "profiles" / "attn_bwd_dkdv_wide_traffic.json"
        if dom == "attn_bwd_dkdv" and tfile.exists():
            traffic = json.loads(tfile.read_text()).get(f"hd{hd}", {}).get("hbm_bytes_per_launch")
        out[f"hd{hd}"] = {"heads": heads, "head_dim": hd, "ms_per_step": ms, "wall_ms_per_step": wall_ms,
                          "edge_tokens_per_s": t / (ms * 1e-3), "achieved_tflops": tflops,
                          "mfma_util_pct": 100.0 * tflops / PEAK_BF16_TFLOPS, "ms_per_step_profiled": ms_prof,
                          "kernels": kern,
                          "roofline": {"bound": "mfma", "kernel": dom, "achieved": achieved,
                                       "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                                       "frac": achieved / PEAK_BF16_TFLOPS, "traffic": traffic}}
        del q, k, v, go
    # node mode at the same widths (the qm9 / unimol / lba M layers: node mode, 8 heads of 64; coconut: 16 of 32)
    from mind_amd.esa.packing import NodeAdjacency
    gn = generators.protein_budget(seed=args.seed, token_budget=65536, count="nodes")
    na = NodeAdjacency.from_edge_index(torch.as_tensor(gn.edge_index).to(dev), torch.as_tensor(gn.batch).to(dev),
                                       gn.num_graphs, int(gn.node_counts.max()))
    tn, ip, ix, cun = int(gn.node_counts.sum()), na.indptr, na.indices, na.cu_seqlens
    plan = attention.node_plan(ip, ix, cun)
    for hd in (64, 32):
        heads = 512 // hd
        g = torch.Generator().manual_seed(args.seed + hd)
        q, k, v, go = (torch.randn(tn, heads, hd, generator=g).to(torch.bfloat16).to(dev) for _ in range(4))

        def step():
            o, lse = attention.attn_fwd(q, k, v, cun, cun, 0, 0, hd ** -0.5, adj_indptr=ip, adj_indices=ix,
                                        adj_plan=plan)
            attention.attn_bwd(go, q, k, v, o, lse, cun, cun, 0, 0, hd ** -0.5, adj_indptr=ip, adj_indices=ix,
                               adj_plan=plan)

        ms, _, kern, _ = timed(step, args.steps, args.warmup)
        by = node_bytes(tn, int(ix.numel()), heads, hd)
        for name, rec in kern.items():
            if name in by:
                rec["algorithmic_bytes"] = by[name]
                rec["achieved_gbs"] = by[name] / (rec["avg_us"] * 1e-6) / 1e9
        dom = max((n for n in by if n in kern), key=lambda n: kern[n]["avg_us"])
        out[f"node_hd{hd}"] = {"workload": "node-mode attention fwd+bwd over a 65,536-node budget batch, node plan "
                                           "prebuilt (once per batch)",
                               "node_tokens": tn, "mask_nnz": int(ix.numel()), "heads": heads, "head_dim": hd,
                               "ms_per_step": ms, "node_tokens_per_s": tn / (ms * 1e-3), "kernels": kern,
                               "roofline": {"bound": "hbm", "kernel": dom, "achieved": kern[dom]["achieved_gbs"],
                                            "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                            "frac": kern[dom]["achieved_gbs"] / PEAK_HBM_GBS}}
        del q, k, v, go
    return out


def bench_dropout(args) -> dict:
    """The cost of attention dropout (the reference's training-time p, esa/mha.py:76,82; MIND's rna YAML trains
    with 0.08, core/pretraining_config_rna.yaml:76-78) on two workloads, each timed without and with dropout:
    configuration 1's dense fwd+bwd at 16 heads of 16 (with dropout the MFMA kernels of esa_attn_wide.hip take
    the call: they evaluate the keep mask per score), the same graphs at the rna YAML's 8 heads of 24 (its S
    layers; the wide kernels with and without dropout), and node-mode fwd+bwd at 8 heads of 24 over a
    65,536-node budget batch with its node plan (the gather kernels; its M layers)."""
    import torch

    from mind_amd import generators
    from mind_amd.esa import attention
    from mind_amd.esa.packing import NodeAdjacency

    dev = torch.device("cuda", 0)
    out = {"workload": "attention fwd+bwd without and with dropout p = 0.08 (seeded hashed keep mask)"}
    gb = generators.protein_like(seed=args.seed)
    t, maxlen = int(gb.cu_seqlens[-1]), gb.max_seqlen
    cu = torch.as_tensor(gb.cu_seqlens).to(dev)
    g = torch.Generator().manual_seed(args.seed)
    q, k, v, go = (torch.randn(t, HEADS, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev) for _ in range(4))
    rec = {"edge_tokens": t, "heads": HEADS, "head_dim": HEAD_DIM}
    for p in (0.0, 0.08):
        def step():
            o, lse = attention.attn_fwd(q, k, v, cu, cu, maxlen, maxlen, 0.25, dropout_p=p, dropout_seed=1)
            attention.attn_bwd(go, q, k, v, o, lse, cu, cu, maxlen, maxlen, 0.25, dropout_p=p, dropout_seed=1)
        ms, _, kern, _ = timed(step, args.steps, args.warmup)
        rec[f"p{p:g}"] = {"ms_per_step": ms, "edge_tokens_per_s": t / (ms * 1e-3),
                          "kernels": {n: r["avg_us"] for n, r in kern.items()}}
    rec["slowdown"] = rec["p0.08"]["ms_per_step"] / rec["p0"]["ms_per_step"]
    out["dense_config1"] = rec
    del q, k, v, go
    # the rna YAML's S layers: dense self-attention at 8 heads of 24 (dim 192) with dropout 0.08
    q, k, v, go = (torch.randn(t, 8, 24, generator=g).to(torch.bfloat16).to(dev) for _ in range(4))
    rec = {"edge_tokens": t, "heads": 8, "head_dim": 24}
    for p in (0.0, 0.08):
        def step():
            o, lse = attention.attn_fwd(q, k, v, cu, cu, maxlen, maxlen, 24 ** -0.5, dropout_p=p, dropout_seed=1)
            attention.attn_bwd(go, q, k, v, o, lse, cu, cu, maxlen, maxlen, 24 ** -0.5, dropout_p=p, dropout_seed=1)
        ms, _, kern, _ = timed(step, args.steps, args.warmup)
        rec[f"p{p:g}"] = {"ms_per_step": ms, "edge_tokens_per_s": t / (ms * 1e-3),
                          "kernels": {n: r["avg_us"] for n, r in kern.items()}}
    rec["slowdown"] = rec["p0.08"]["ms_per_step"] / rec["p0"]["ms_per_step"]
    out["dense_rna_shape"] = rec
    del q, k, v, go
    gn = generators.protein_budget(seed=args.seed, token_budget=65536, count="nodes")
    na = NodeAdjacency.from_edge_index(torch.as_tensor(gn.edge_index).to(dev), torch.as_tensor(gn.batch).to(dev),
                                       gn.num_graphs, int(gn.node_counts.max()))
    tn = int(gn.node_counts.sum())
    q, k, v, go = (torch.randn(tn, 8, 24, generator=g).to(torch.bfloat16).to(dev) for _ in range(4))
    ip, ix, cun = na.indptr, na.indices, na.cu_seqlens
    plan = attention.node_plan(ip, ix, cun)
    rec = {"node_tokens": tn, "mask_nnz": int(ix.numel()), "heads": 8, "head_dim": 24}
    for p in (0.0, 0.08):
        def step():
            o, lse = attention.attn_fwd(q, k, v, cun, cun, 0, 0, 24 ** -0.5, adj_indptr=ip, adj_indices=ix,
                                        adj_plan=plan, dropout_p=p, dropout_seed=1)
            attention.attn_bwd(go, q, k, v, o, lse, cun, cun, 0, 0, 24 ** -0.5, adj_indptr=ip, adj_indices=ix,
                               adj_plan=plan, dropout_p=p, dropout_seed=1)
        ms, _, kern, _ = timed(step, args.steps, args.warmup)
        rec[f"p{p:g}"] = {"ms_per_step": ms, "node_tokens_per_s": tn / (ms * 1e-3),
                          "kernels": {n: r["avg_us"] for n, r in kern.items()}}
    rec["slowdown"] = rec["p0.08"]["ms_per_step"] / rec["p0"]["ms_per_step"]
    out["node_rna_shape"] = rec
    return out


def edge_mask_stats(src: np.ndarray, dst: np.ndarray, cu: np.ndarray, tile: int = 32) -> dict:
    """Exact pair count of the share-an-endpoint mask, its 32x32 tile occupancy per graph, and the work the
    key-list kernels execute.

    nnz = #{(i, j): i != j, {s_i, d_i} and {s_j, d_j} intersect}; tiles count the (query tile, key tile)
    blocks of each graph with at least one such pair.  The list kernels visit, per 32-token tile of the
    packed token order, ceil(u / 32) compact tiles of 32 x 32 score slots, u the size of the union of the
    tile's tokens' partners (the edge-mask plan's list of the tile): compact_tiles sums those, list_entries
    the u.
    """
    nnz = tiles_any = tiles_all = 0
    pair_tile, pair_col = [], []
    for b in range(len(cu) - 1):
        s, e = int(cu[b]), int(cu[b + 1])
        if e == s:
            continue
        a, c = src[s:e], dst[s:e]
        m = ((a[:, None] == a[None, :]) | (c[:, None] == c[None, :]) |
             (a[:, None] == c[None, :]) | (c[:, None] == a[None, :]))
        np.fill_diagonal(m, False)
        nnz += int(m.sum())
        nt = -(-(e - s) // tile)
        pad = np.zeros((nt * tile, nt * tile), dtype=bool)
        pad[: e - s, : e - s] = m
        tiles_any += int(pad.reshape(nt, tile, nt, tile).any(axis=(1, 3)).sum())
        tiles_all += nt * nt
        i, j = np.nonzero(m)
        pair_tile.append((i + s) // tile)
        pair_col.append(j + s)
    if pair_tile:
        key = np.unique(np.concatenate(pair_tile).astype(np.int64) * (int(cu[-1]) + 1) + np.concatenate(pair_col))
        union = np.bincount(key // (int(cu[-1]) + 1))
    else:
        union = np.zeros(0, np.int64)
    return {"nnz": nnz, "tiles_nonempty": tiles_any, "tiles_total": tiles_all,
            "list_entries": int(union.sum()), "compact_tiles": int(((union + tile - 1) // tile).sum())}


def masked_bytes(t: int, compact_tiles: int, heads: int = HEADS) -> dict:
    """Compulsory HBM bytes per launch of the key-list kernels (bf16 [T, H, 16] tensors of T*H*32 bytes, the
    fp32 LSE [H, T], the dK/dV pass's 8-byte row statistics per (head, query), and per compact tile 32 list
    ids and 32 mask words of 4 bytes): forward reads Q, K, V and writes O and the LSE; dQ reads Q, K, V, O,
    dO and the LSE and writes dQ and the row statistics; dK/dV reads K, V, Q, dO and the row statistics and
    writes dK and dV.  Each gathered row counted once."""
    row = t * heads * HEAD_DIM * 2
    lists = compact_tiles * 32 * 8
    return {"attn_fwd_masked": 4 * row + heads * t * 4 + lists,
            "attn_bwd_dq_masked": 6 * row + heads * t * (4 + 8) + lists,
            "attn_bwd_dkdv_masked": 6 * row + heads * t * 8 + lists}


def cpu_baseline_masked(gb, seed: int, n_graphs: int) -> dict:
    """The reference's masked MAB attention on the host cores, fp32 forward + backward, on a bounded sample.

    The reference adds the edge bias (0 where two edges share a node, else -99999;
    esa/masked_layers.py:217-268) to the scores of every graph padded to N (esa/mha.py:73-77); on the CPU its
    attention call is torch's scaled_dot_product_attention with that additive bias (oracle.attention.
    padded_sdpa with a per-graph pair bias).  The bias of each graph is built per graph (the entries of the
    global E x E comparison, without its E^2 temporaries).  Sample: graphs spread over the length
    distribution, padded to the batch's N."""
    import torch

    from oracle import attention as oracle_attention
    from oracle import mask as oracle_mask
    from oracle.packing import nearest_multiple_of_8

    cores = len(os.sched_getaffinity(0))
    order = np.argsort(gb.edge_counts)
    pick = sorted(set(int(order[int(i)]) for i in np.linspace(0, len(order) - 1, n_graphs)))
    cu_all = gb.cu_seqlens.astype(np.int64)
    idx = np.concatenate([np.arange(cu_all[b], cu_all[b + 1]) for b in pick])
    lens = gb.edge_counts[pick]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    src, dst = gb.edge_index[0][idx], gb.edge_index[1][idx]
    t = int(cu[-1])
    n = nearest_multiple_of_8(gb.max_seqlen + 1)
    biases = [torch.where(torch.as_tensor(oracle_mask.edge_adjacency_segment(src, dst, int(cu[b]), int(cu[b + 1]))),
                          0.0, oracle_mask.MASK_FILL) for b in range(len(pick))]
    g = torch.Generator().manual_seed(seed + 99)
    q, k, v, go = (torch.randn(t, HEADS, HEAD_DIM, generator=g) for _ in range(4))

    def step():
        qd, kd, vd = (x.detach().requires_grad_(True) for x in (q, k, v))
        out = oracle_attention.padded_sdpa(qd, kd, vd, cu, cu, n, 1.0 / HEAD_DIM ** 0.5, pair_bias=lambda b: biases[b])
        out.backward(go)

    torch.set_num_threads(cores)
    med, runs = _median_time(step)
    return {"value": t / med, "unit": "edge-tokens/s", "cores": cores, "kind": "port",
            "sample": (f"{len(pick)} graphs of the batch spread over its lengths ({t} edge tokens, lengths "
                       f"{lens.tolist()}, padded to N = {n}): torch scaled_dot_product_attention fp32 with the "
                       f"reference's additive edge bias (oracle.attention.padded_sdpa), forward + autograd "
                       f"backward on {cores} threads, median of {runs} runs after 2 warm-ups")}


def node_bytes(t: int, nnz: int, heads: int = HEADS, head_dim: int = HEAD_DIM) -> dict:
    """Compulsory HBM bytes per launch of the node-mode kernels (bf16 [T, H, hd] tensors of T*H*hd*2 bytes,
    fp32 [H, T] row statistics, int32 CSR): forward reads Q, K, V and writes O and the LSE; dQ reads Q, K, V, O,
    dO and the LSE and writes dQ and D; dK/dV reads K, V, Q, dO, the LSE and D and the transposed CSR and
    writes dK and dV.  Each gathered row counted once (the rows of a graph are reused from cache)."""
    row = t * heads * head_dim * 2
    stat = heads * t * 4
    csr = 4 * (t + 1) + 4 * nnz
    return {"graph_attn_fwd": 4 * row + stat + csr, "graph_attn_bwd_dq": 6 * row + 2 * stat + csr,
            "graph_attn_bwd_dkdv": 6 * row + 2 * stat + csr}


def cpu_baseline_node(gb, seed: int, n_graphs: int) -> dict:
    """The reference's node-mode attention on the host cores, fp32 forward + backward, on a bounded sample: the
    node bias (0 at (src, dst) of every edge, else -99999; get_adj_mask_from_edge_index_node,
    esa/masked_layers.py:79-118) added to the scores of every graph padded to N (esa/mha.py:73-77), i.e.
    torch's scaled_dot_product_attention with that additive bias (oracle.attention.padded_sdpa).  Sample:
    graphs spread over the size distribution, padded to the batch's N."""
    import torch

    from oracle import attention as oracle_attention
    from oracle import mask as oracle_mask
    from oracle.packing import nearest_multiple_of_8

    cores = len(os.sched_getaffinity(0))
    order = np.argsort(gb.node_counts)
    pick = sorted(set(int(order[int(i)]) for i in np.linspace(0, len(order) - 1, n_graphs)))
    first = np.concatenate([[0], np.cumsum(gb.node_counts)]).astype(np.int64)
    lens = gb.node_counts[pick].astype(np.int64)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    # the sample's CSR over its own node numbering
    src, dst = gb.edge_index
    rows, cols = [], []
    for b, g in enumerate(pick):
        sel = (src >= first[g]) & (src < first[g + 1])
        rows.append(src[sel] - first[g] + cu[b])
        cols.append(dst[sel] - first[g] + cu[b])
    rows, cols = np.concatenate(rows), np.concatenate(cols)
    t = int(cu[-1])
    o = np.lexsort((cols, rows))
    indptr = np.searchsorted(rows[o], np.arange(t + 1))
    indices = cols[o]
    n = nearest_multiple_of_8(int(gb.node_counts.max()) + 1)
    biases = [torch.where(torch.as_tensor(oracle_mask.node_adjacency_segment(indptr, indices, int(cu[b]),
                                                                             int(cu[b + 1]), int(cu[b]),
                                                                             int(cu[b + 1]))),
                          0.0, oracle_mask.MASK_FILL) for b in range(len(pick))]
    g = torch.Generator().manual_seed(seed + 97)
    q, k, v, go = (torch.randn(t, HEADS, HEAD_DIM, generator=g) for _ in range(4))

    def step():
        qd, kd, vd = (x.detach().requires_grad_(True) for x in (q, k, v))
        out = oracle_attention.padded_sdpa(qd, kd, vd, cu, cu, n, 1.0 / HEAD_DIM ** 0.5, pair_bias=lambda b: biases[b])
        out.backward(go)

    torch.set_num_threads(cores)
    med, runs = _median_time(step)
    return {"value": t / med, "unit": "node-tokens/s", "cores": cores, "kind": "port",
            "sample": (f"{len(pick)} graphs of the batch spread over its sizes ({t} nodes, sizes {lens.tolist()}, "
                       f"padded to N = {n}): torch scaled_dot_product_attention fp32 with the reference's additive "
                       f"node bias (oracle.attention.padded_sdpa), forward + autograd backward on {cores} threads, "
                       f"median of {runs} runs after 2 warm-ups")}


def bench_node(args, sub: bool = False):
    """Node-mode attention fwd+bwd (the mask every MIND YAML applies: query node src attends to key node dst per
    edge, esa/masked_layers.py:79-118) on a 65,536-node budget batch of protein-like graphs (radius 8 A, at most
    16 neighbours), 16 heads x 16.  The timed step builds the batch's node plan from the CSR (once per batch,
    as the reference builds its node bias) and runs the attention forward and backward over it."""
    import torch

    from mind_amd import generators
    from mind_amd.esa import attention
    from mind_amd.esa.packing import NodeAdjacency

    dev = torch.device("cuda", 0)
    gb = generators.protein_budget(seed=args.seed, token_budget=65536, count="nodes")
    ei = torch.as_tensor(gb.edge_index).to(dev)
    bm = torch.as_tensor(gb.batch).to(dev)
    na = NodeAdjacency.from_edge_index(ei, bm, gb.num_graphs, int(gb.node_counts.max()))
    t, nnz = int(gb.node_counts.sum()), int(na.indices.numel())
    g = torch.Generator().manual_seed(args.seed)
    q, k, v, go = (torch.randn(t, HEADS, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev) for _ in range(4))
    cu, ip, ix = na.cu_seqlens, na.indptr, na.indices
    scale = 1.0 / HEAD_DIM ** 0.5

    def step():
        plan = attention.node_plan(ip, ix, cu)
        out, lse = attention.attn_fwd(q, k, v, cu, cu, 0, 0, scale, adj_indptr=ip, adj_indices=ix, adj_plan=plan)
        attention.attn_bwd(go, q, k, v, out, lse, cu, cu, 0, 0, scale, adj_indptr=ip, adj_indices=ix, adj_plan=plan)

    ms_per_step, wall_ms, per_kernel, ms_prof = timed(step, args.steps, args.warmup)
    by = node_bytes(t, nnz)
    for name, rec in per_kernel.items():
        if name in by:
            rec["algorithmic_bytes"] = by[name]
            rec["achieved_gbs"] = by[name] / (rec["avg_us"] * 1e-6) / 1e9
    dom = max((n for n in by if n in per_kernel), key=lambda n: per_kernel[n]["avg_us"])
    achieved = per_kernel[dom]["achieved_gbs"]
    traffic = None
    tfile = ROOT / "profiles" / f"{dom}_node_traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
    roofline = {"bound": "hbm", "kernel": dom, "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": achieved / PEAK_HBM_GBS, "traffic": traffic,
                "bytes": "compulsory: every tensor row and CSR entry once (node_bytes)"}
    out = {"workload": "node-mode attention fwd+bwd over a 65,536-node budget batch (node plan built each step)",
           "graphs": gb.num_graphs, "node_tokens": t, "mask_nnz": nnz, "heads": HEADS, "head_dim": HEAD_DIM,
           "ms_per_step": ms_per_step, "wall_ms_per_step": wall_ms, "node_tokens_per_s": t / (ms_per_step * 1e-3),
           "ms_per_step_profiled": ms_prof, "kernels": per_kernel, "roofline": roofline}
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_node(gb, args.seed, args.cpu_sample_graphs)
    if sub:
        return out
    result = {"metric": "node-tokens/sec through node-mode ESA attn fwd+bwd", "value": t / (ms_per_step * 1e-3),
              "unit": "node-tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
              "ms_per_step": ms_per_step, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
              "dtype": "bf16", "data": "synthetic (seeded protein-like radius graphs; q, k, v, dO ~ N(0,1))",
              "config": {"workload": out["workload"], "graphs": gb.num_graphs, "node_tokens": t, "mask_nnz": nnz,
                         "heads": HEADS, "head_dim": HEAD_DIM, "seed": args.seed}}
    result.update({k: v for k, v in out.items() if k not in ("workload", "graphs", "node_tokens", "mask_nnz")})
    print(json.dumps(result), flush=True)


def bench_masked(args, sub: bool = False):
    """Configuration 2: edge-masked attention fwd+bwd on a 65,536-edge-token budget batch.

    The timed step builds the batch's edge-mask plan from src/dst (the mask is
    built once per batch, as the reference builds its adjacency mask) and runs
    the attention forward and backward over it; the full SAB block
    (projections, attention, fc_o + mish) fwd+bwd on the same batch is timed
    after it and reported beside.
    """
    import torch

    from mind_amd import generators
    from mind_amd.esa import attention
    from mind_amd.esa.mha import SAB
    from mind_amd.esa.packing import EdgeAdjacency, nearest_multiple_of_8

    dev = torch.device("cuda", 0)
    gb = generators.protein_budget(seed=args.seed, token_budget=65536)
    cu_np = gb.cu_seqlens
    t = int(cu_np[-1])
    src_np, dst_np = gb.edge_index[0].astype(np.int32), gb.edge_index[1].astype(np.int32)
    stats = edge_mask_stats(src_np, dst_np, cu_np)
    g = torch.Generator().manual_seed(args.seed)
    q, k, v, go = (torch.randn(t, HEADS, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev) for _ in range(4))
    cu = torch.as_tensor(cu_np).to(dev)
    src, dst = torch.as_tensor(src_np).to(dev), torch.as_tensor(dst_np).to(dev)
    maxlen = gb.max_seqlen
    scale = 1.0 / HEAD_DIM ** 0.5

    def step():
        plan = attention.edge_plan(src, dst, cu)
        out, lse = attention.attn_fwd(q, k, v, cu, cu, maxlen, maxlen, scale, edge_plan=plan)
        attention.attn_bwd(go, q, k, v, out, lse, cu, cu, maxlen, maxlen, scale, edge_plan=plan)

    ms_per_step, wall_ms, per_kernel, ms_prof = timed(step, args.steps, args.warmup)
    eff_flops = 14 * DIM * stats["nnz"]
    # score slots the list kernels compute: every compact tile is 32 x 32 (query and key tiles' lists are one
    # list when the mask is symmetric, as here)
    exec_flops = 14 * DIM * stats["compact_tiles"] * 32 * 32
    tflops = eff_flops / (ms_per_step * 1e-3) / 1e12
    masked = {n + "_masked": f for n, f in FLOPS_PER_PAIR.items()}
    by = masked_bytes(t, stats["compact_tiles"])
    for name, rec in per_kernel.items():
        if name in masked:
            rec["effective_tflops"] = masked[name] * stats["nnz"] / (rec["avg_us"] * 1e-6) / 1e12
            rec["executed_tflops"] = masked[name] * stats["compact_tiles"] * 1024 / (rec["avg_us"] * 1e-6) / 1e12
            rec["algorithmic_bytes"] = by[name]
            rec["achieved_gbs"] = by[name] / (rec["avg_us"] * 1e-6) / 1e9
    dom = max((n for n in masked if n in per_kernel), key=lambda n: per_kernel[n]["avg_us"])
    achieved = per_kernel[dom]["effective_tflops"]
    traffic = None
    tfile = ROOT / "profiles" / f"{dom}_config2_traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
    roofline = {"bound": "mfma", "kernel": dom, "achieved": achieved, "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": achieved / PEAK_BF16_TFLOPS, "traffic": traffic,
                "flops": "effective (nnz of the mask)",
                "executed_frac": per_kernel[dom]["executed_tflops"] / PEAK_BF16_TFLOPS}
    roofline_hbm = {"bound": "hbm", "kernel": dom, "achieved": per_kernel[dom]["achieved_gbs"],
                    "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": per_kernel[dom]["achieved_gbs"] / PEAK_HBM_GBS,
                    "traffic": traffic, "bytes": "compulsory: every tensor row, statistic and list word once "
                                                 "(masked_bytes)"}
    if sub:
        out = {"workload": "config2: edge-masked attention fwd+bwd (edge-mask plan built from src/dst each step)",
               "graphs": gb.num_graphs, "edge_tokens": t, "mask_nnz": stats["nnz"],
               "mask_density": stats["nnz"] / gb.sum_sq, "tiles_nonempty": stats["tiles_nonempty"],
               "compact_tiles": stats["compact_tiles"], "list_entries": stats["list_entries"],
               "compact_tile_fill": stats["nnz"] / (stats["compact_tiles"] * 1024),
               "ms_per_step": ms_per_step, "edge_tokens_per_s": t / (ms_per_step * 1e-3),
               "achieved_tflops_effective": tflops,
               "achieved_tflops_executed": exec_flops / (ms_per_step * 1e-3) / 1e12,
               "ms_per_step_profiled": ms_prof, "kernels": per_kernel, "roofline": roofline,
               "roofline_hbm": roofline_hbm}
        if not args.no_cpu_baseline:
            out["cpu_baseline"] = cpu_baseline_masked(gb, args.seed, args.cpu_sample_graphs)
        return out

    # the SAB block on the same batch: padded [B, N, 256] input, EdgeAdjacency mask
    n_max = nearest_multiple_of_8(maxlen)
    ei = torch.as_tensor(gb.edge_index).to(dev)
    bm = torch.as_tensor(gb.batch).to(dev)
    adj = EdgeAdjacency.from_edge_index(ei, bm, gb.num_graphs, n_max)
    torch.manual_seed(args.seed)
    sab = SAB(DIM, DIM, HEADS, 0.0, "hip").to(dev)
    x = torch.zeros(gb.num_graphs * n_max, DIM, device=dev)
    x[adj.padded_index] = torch.randn(t, DIM, device=dev)
    x = x.view(gb.num_graphs, n_max, DIM).requires_grad_(True)
    gy = torch.randn(gb.num_graphs, n_max, DIM, device=dev)

    def block_step():
        y = sab(x, adj)
        y.backward(gy)

    block_ms, _, _, _ = timed(block_step, max(5, args.steps // 5), max(2, args.warmup // 5), profile=False)

    result = {
        "metric": "edge-tokens/sec through ESA attn fwd+bwd; MFMA util % of bf16 peak",
        "value": t / (ms_per_step * 1e-3),
        "unit": "edge-tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded lognormal protein-like graphs packed to a 65,536 edge-token budget; "
                "q, k, v, dO ~ N(0,1))",
        "config": {
            "workload": "config2: edge-masked attention fwd+bwd (edge-mask plan built from src/dst each step)",
            "graphs": gb.num_graphs, "edge_tokens": t, "max_seqlen": maxlen, "sum_L2": gb.sum_sq,
            "mask_nnz": stats["nnz"], "mask_density": stats["nnz"] / gb.sum_sq,
            "tiles_nonempty": stats["tiles_nonempty"], "tiles_total": stats["tiles_total"],
            "compact_tiles": stats["compact_tiles"], "list_entries": stats["list_entries"],
            "heads": HEADS, "head_dim": HEAD_DIM, "dim": DIM, "seed": args.seed,
        },
        "mfma_util_pct": 100.0 * tflops / PEAK_BF16_TFLOPS,
        "achieved_tflops_effective": tflops,
        "achieved_tflops_executed": exec_flops / (ms_per_step * 1e-3) / 1e12,
        "compact_tile_fill": stats["nnz"] / (stats["compact_tiles"] * 1024),
        "wall_ms_per_step": wall_ms, "ms_per_step_profiled": ms_prof,
        "kernels": per_kernel,
        "roofline": roofline,
        "roofline_hbm": roofline_hbm,
        "sab_block": {"ms_per_step": block_ms, "edge_tokens_per_s": t / (block_ms * 1e-3),
                      "what": "SAB(256, 256, 16 heads, 'hip') fwd+bwd incl. projections, fc_o + mish, padded "
                              f"[{gb.num_graphs}, {n_max}, {DIM}] fp32 input"},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_masked(gb, args.seed, args.cpu_sample_graphs)
    print(json.dumps(result), flush=True)


GATHER_N, GATHER_E, GATHER_F, GATHER_BLOCK = 1 << 21, 1 << 25, 256, 512


def gather_bytes(e: int, n: int, f: int, s: int) -> dict:
    """Compulsory HBM bytes: gather writes E*2F, reads each node row once and both index arrays;
    the segment sum reads E*F and indptr, writes N*F."""
    return {"edge_gather": e * 2 * f * s + n * f * s + 8 * e,
            "segment_sum": e * f * s + n * f * s + 4 * (n + 1)}


def cpu_baseline_gather(src, dst, seed: int, slice_edges: int) -> dict:
    """The reference's gather and edge->node sum on the host cores (torch, fp32) on a dst-sorted slice.

    oracle.edges.edge_gather_torch is the reference's own torch.cat((x[src], x[dst]), 1)
    (core/pretraining_model.py:153-155) and oracle.edges.scatter_sum_torch its scatter_add
    (core/molecular_encoder.py:241-242) as index_add_; both run multi-threaded in torch.  The first
    `slice_edges` dst-sorted edges; GB/s of the same algorithmic bytes, so the full-size time scales
    linearly."""
    import torch

    from oracle import edges as oracle_edges

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(seed + 7)
    s = torch.as_tensor(src[:slice_edges].astype(np.int64))
    d = torch.as_tensor(dst[:slice_edges].astype(np.int64))
    lo, hi = int(d[0]), int(d[-1]) + 1
    nodes = hi - lo
    x = torch.randn(int(max(int(s.max()), int(d.max()))) + 1, GATHER_F, generator=g)
    y = torch.randn(slice_edges, GATHER_F, generator=g)
    dl = d - lo
    by = gather_bytes(slice_edges, nodes, GATHER_F, 4)
    total = by["edge_gather"] + by["segment_sum"]

    def step():
        oracle_edges.edge_gather_torch(x, s, d)
        oracle_edges.scatter_sum_torch(y, dl, nodes)

    med, runs = _median_time(step)
    return {"value": total / med / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": (f"torch.cat((x[src], x[dst]), 1) + index_add_ by dst (the reference's expressions, "
                       f"oracle.edges.*_torch) on the first {slice_edges} dst-sorted edges ({nodes} nodes), fp32, "
                       f"{cores} threads, median of {runs} runs after 2 warm-ups; GB/s of the same algorithmic bytes")}


def minmax_bytes(e: int, n: int) -> int:
    """Compulsory HBM bytes of a 1-D segmented minimum with argument: the CSR permutation and one fp32 value
    per edge, indptr, one fp32 value and one int64 argument per node."""
    return 8 * e + 4 * (n + 1) + 12 * n


def bench_encoder_min(args, dev, src) -> dict:
    """The encoder's closest-neighbour reduction (core/molecular_encoder.py:214, scatter_min of a per-edge
    distance by edge_src) over configuration 3's graph: fp32 distances in [0.5, 3) on 2^25 edges to 2^21
    nodes, edges in the canonical dst-sorted order, so each node's edges are scattered; the CSR by src is
    built once outside the timed steps (csr_build_ms times that build).  Beside it: torch's scatter_reduce
    ('amin', the atomic library form of the same reduction) on the same GPU, and on the host cores over a
    2^21-edge slice."""
    import torch

    from mind_amd.edges import CSR, segment_minmax_csr

    csr_src = CSR.build(src, GATHER_N)
    g = torch.Generator(device=dev).manual_seed(args.seed + 3)
    dist = (torch.rand(GATHER_E, 1, device=dev, generator=g) * 2.5 + 0.5).contiguous()
    ms, _, kern, _ = timed(lambda: segment_minmax_csr(dist, csr_src.indptr, csr_src.perm),
                           max(5, args.steps // 2), 2)
    by = minmax_bytes(GATHER_E, GATHER_N)
    rec = kern.get("segment_minmax", {})
    if rec:
        rec["algorithmic_bytes"] = by
        rec["achieved_gbs"] = by / (rec["avg_us"] * 1e-6) / 1e9
    flat, src_l = dist.view(-1), src.long()
    base = torch.zeros(GATHER_N, device=dev)
    t_ms, _, _, _ = timed(lambda: base.clone().scatter_reduce_(0, src_l, flat, "amin", include_self=False),
                          max(5, args.steps // 2), 2, profile=False)
    out = {"workload": "scatter_min(dist, edge_src, dim=0, dim_size=N) over configuration 3's graph (fp32, 1-D)",
           "ms_per_step": ms, "algorithmic_bytes": by, "gb_per_s": by / (ms * 1e-3) / 1e9,
           "edges_per_s": GATHER_E / (ms * 1e-3), "kernels": kern, "csr_build_ms": None,
           "torch_scatter_reduce_gpu_ms": t_ms}
    if not args.no_cpu_baseline:
        from oracle import edges as oracle_edges

        k = 1 << 21
        d_cpu, s_cpu = flat[:k].cpu(), src_l[:k].cpu()
        oracle_edges.scatter_min_torch(d_cpu, s_cpu, GATHER_N)
        t0 = time.perf_counter()
        for _ in range(3):
            oracle_edges.scatter_min_torch(d_cpu, s_cpu, GATHER_N)
        cpu_ms = (time.perf_counter() - t0) / 3 * 1e3
        out["cpu_baseline"] = {"value": k / (cpu_ms * 1e-3), "unit": "edges/s", "cores": torch.get_num_threads(),
                               "kind": "port", "sample": (f"oracle.edges.scatter_min_torch (torch scatter_reduce "
                                                          f"amin) on the host over the first {k} edges of the batch")}
    t1 = torch.cuda.Event(enable_timing=True)
    t2 = torch.cuda.Event(enable_timing=True)
    t1.record()
    CSR.build(src, GATHER_N)
    t2.record()
    torch.cuda.synchronize()
    out["csr_build_ms"] = t1.elapsed_time(t2)
    del dist, csr_src, base
    torch.cuda.empty_cache()
    return out


def bench_gather(args, sub: bool = False):
    """Configuration 3: edge-token gather and CSR segment sum at 2^21 nodes x 2^25 edges x 256 features."""
    import torch

    from mind_amd import generators
    from mind_amd.edges import CSR, _gather_raw, segment_sum_csr

    dev = torch.device("cuda", 0)
    src_np, dst_np = generators.block_local_edges(seed=args.seed, num_nodes=GATHER_N, num_edges=GATHER_E,
                                                  block=GATHER_BLOCK)
    src_gen, dst_gen = torch.as_tensor(src_np).to(dev), torch.as_tensor(dst_np).to(dev)
    del src_np, dst_np
    # canonical order: edges sorted by dst (the CSR order); the sort itself is timed separately
    csr = CSR.build(dst_gen, GATHER_N)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(5):
        CSR.build(dst_gen, GATHER_N)
    ev1.record()
    torch.cuda.synchronize()
    csr_ms = ev0.elapsed_time(ev1) / 5
    src = src_gen.index_select(0, csr.perm.long()).contiguous()
    dst = dst_gen.index_select(0, csr.perm.long()).contiguous()
    indptr = csr.indptr

    results = {}
    for dtype, name in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
        s = torch.tensor([], dtype=dtype).element_size()
        g = torch.Generator(device=dev).manual_seed(args.seed)
        x = torch.randn(GATHER_N, GATHER_F, device=dev, generator=g).to(dtype)
        y = torch.randn(GATHER_E, GATHER_F, device=dev, generator=g).to(dtype)
        out = torch.empty(GATHER_E, 2 * GATHER_F, device=dev, dtype=dtype)
        agg = torch.empty(GATHER_N, GATHER_F, device=dev, dtype=dtype)

        def step():
            _gather_raw(x, src, dst, out)
            segment_sum_csr(y, indptr, out=agg)

        ms, wall_ms, kern, ms_prof = timed(step, args.steps, args.warmup)
        by = gather_bytes(GATHER_E, GATHER_N, GATHER_F, s)
        for kname, b in by.items():
            if kname in kern:
                kern[kname]["algorithmic_bytes"] = b
                kern[kname]["achieved_gbs"] = b / (kern[kname]["avg_us"] * 1e-6) / 1e9
        # generation order: gather with the unsorted indices, segment sum through perm

        def step_gen():
            _gather_raw(x, src_gen, dst_gen, out)
            segment_sum_csr(y, indptr, csr.perm, out=agg)

        ms_gen, _, kern_gen, _ = timed(step_gen, max(5, args.steps // 2), 2)
        results[name] = {"ms_per_step": ms, "wall_ms_per_step": wall_ms, "ms_per_step_profiled": ms_prof,
                         "kernels": kern,
                         "gb_per_s": (by["edge_gather"] + by["segment_sum"]) / (ms * 1e-3) / 1e9,
                         "generation_order": {"ms_per_step": ms_gen, "kernels": kern_gen}}
        del x, y, out, agg
        torch.cuda.empty_cache()

    encoder_min = bench_encoder_min(args, dev, src)

    # in-process reference: a plain device-to-device copy (torch) of the fp32 edge-output size, the practical
    # streaming rate of this allocation on this box
    a = torch.empty(GATHER_E, GATHER_F, device=dev)
    b = torch.empty_like(a)
    copy_ms, _, _, _ = timed(lambda: b.copy_(a), 5, 2, profile=False)
    copy_gbs = 2 * a.numel() * 4 / (copy_ms * 1e-3) / 1e9
    del a, b
    torch.cuda.empty_cache()

    f32 = results["f32"]
    dom = max(("edge_gather", "segment_sum"), key=lambda n: f32["kernels"][n]["avg_us"])
    achieved = f32["kernels"][dom]["achieved_gbs"]
    traffic = None
    tfile = ROOT / "profiles" / f"{dom}_config3_traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
    roofline = {"bound": "hbm", "kernel": dom, "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": achieved / PEAK_HBM_GBS, "traffic": traffic}
    hbm_frac = {f"{name}.{k}": v["achieved_gbs"] / PEAK_HBM_GBS
                for name in ("f32", "bf16") for k, v in results[name]["kernels"].items() if "achieved_gbs" in v}
    if sub:
        out = {"workload": "config3: edge gather [x[src] || x[dst]] + deterministic CSR segment sum to dst",
               "nodes": GATHER_N, "edges": GATHER_E, "features": GATHER_F, "order": "dst-sorted (CSR)",
               "ms_per_step_f32": f32["ms_per_step"], "gb_per_s_f32": f32["gb_per_s"],
               "ms_per_step_bf16": results["bf16"]["ms_per_step"], "gb_per_s_bf16": results["bf16"]["gb_per_s"],
               "kernels_f32": f32["kernels"], "kernels_bf16": results["bf16"]["kernels"],
               "hbm_frac": hbm_frac, "csr_build_ms": csr_ms, "reference_copy_gbs": copy_gbs,
               "roofline": roofline, "encoder_min": encoder_min}
        if not args.no_cpu_baseline:
            out["cpu_baseline"] = cpu_baseline_gather(src.cpu().numpy(), dst.cpu().numpy(), args.seed, 1 << 21)
        return out
    fused = bench_fused_projection(x_dtype=torch.float32, src=src, dst=dst, steps=max(3, args.steps // 2),
                                   warmup=2, seed=args.seed)
    result = {
        "metric": "GB/s of algorithmic HBM bytes through edge gather + CSR segment sum",
        "value": f32["gb_per_s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": f32["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded block-local edges; x, y ~ N(0,1))",
        "config": {
            "workload": "config3: edge gather [x[src] || x[dst]] + deterministic CSR segment sum to dst",
            "nodes": GATHER_N, "edges": GATHER_E, "features": GATHER_F, "block": GATHER_BLOCK,
            "order": "dst-sorted (CSR); generation order reported beside", "seed": args.seed,
        },
        "csr_build_ms": csr_ms,
        "reference_copy_gbs": copy_gbs,
        "fused_projection": fused,
        "encoder_min": encoder_min,
        "f32": f32,
        "bf16": results["bf16"],
        "hbm_frac": hbm_frac,
        "roofline": roofline,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_gather(src.cpu().numpy(), dst.cpu().numpy(), args.seed, 1 << 21)
    print(json.dumps(result), flush=True)


def bench_fused_projection(x_dtype, src, dst, steps: int, warmup: int, seed: int) -> dict:
    """The edge MLP's first Linear(2F -> F) over [x_src || x_dst] at configuration-3 sizes: the reference's form
    (gather the [E, 2F] edge tokens, then one [E, 2F] x [2F, F] GEMM) against the fused form (one node-level
    [N, F] x [F, 2F] GEMM, then the gather-add kernel writes out[e] = P[src e] + Q[dst e] + b)."""
    import torch

    from mind_amd.edges import _gather_raw, gather_add

    dev = src.device
    g = torch.Generator(device=dev).manual_seed(seed)
    n, f, e = GATHER_N, GATHER_F, src.numel()
    x = torch.randn(n, f, device=dev, generator=g).to(x_dtype)
    w = (torch.randn(f, 2 * f, device=dev, generator=g) / (2 * f) ** 0.5).to(x_dtype)
    b = torch.randn(f, device=dev, generator=g).to(x_dtype)
    w2 = torch.cat((w[:, :f], w[:, f:]), 0)
    out = torch.empty(e, f, device=dev, dtype=x_dtype)
    pq = torch.empty(n, 2 * f, device=dev, dtype=x_dtype)

    def fused():
        torch.mm(x, w2.t(), out=pq)
        gather_add(pq[:, :f], pq[:, f:], src, dst, b, out=out)

    ms_f, _, kern_f, _ = timed(fused, steps, warmup)
    fused_out = out[:4096].clone()
    del pq
    h = torch.empty(e, 2 * f, device=dev, dtype=x_dtype)

    def unfused():
        _gather_raw(x, src, dst, h)
        torch.addmm(b, h, w.t(), out=out)

    ms_u, _, _, _ = timed(unfused, steps, warmup, profile=False)
    diff = float((out[:4096] - fused_out).abs().max() / out[:4096].abs().max())
    del h, out, x
    torch.cuda.empty_cache()
    s = torch.tensor([], dtype=x_dtype).element_size()
    ga = kern_f.get("edge_gather_add", {})
    algo = e * f * s + 2 * n * f * s + 8 * e   # write out once, read each node row of P and Q once, indices
    return {"dtype": str(x_dtype).replace("torch.", ""), "fused_ms": ms_f, "unfused_ms": ms_u,
            "speedup": ms_u / ms_f, "gather_add_us": ga.get("avg_us"),
            "gather_add_algorithmic_gbs": algo / (ga["avg_us"] * 1e-6) / 1e9 if ga else None,
            "max_rel_diff_fused_vs_unfused": diff,
            "what": "Linear(2F->F) over [x_src || x_dst], F=256: fused = node GEMM + gather-add; "
                    "unfused = gather [E, 2F] + [E, 2F] x [2F, F] GEMM (the reference's form)"}


def _edge_tokens(gb, emb, proj, types_d, ei, bm):
    """Config-0 edge tokens from device-resident inputs (atom types, edge_index, batch mapping): one-hot atom
    types -> Linear(16, 128) -> [x_src || x_dst] -> Linear(256, 128), padded to [B, N, 128]
    (core/pretraining_model.py:152-211, esa/models.py:306-317)."""
    import torch

    from mind_amd.edges import edge_gather
    from mind_amd.esa.packing import EdgeAdjacency, nearest_multiple_of_8

    onehot = torch.nn.functional.one_hot(types_d, 16).float()
    n = nearest_multiple_of_8(gb.max_seqlen + 1)
    tok = proj(edge_gather(emb(onehot), ei[0].int(), ei[1].int()))
    adj = EdgeAdjacency.from_edge_index(ei, bm, gb.num_graphs, n)
    return adj.pad(tok), n


def bench_block(args, sub: bool = False):
    """Configuration 0: the ESA block forward in fp32 (edge tokens, masked MAB + SAB + PMA(1 seed), D=128, H=8).

    The batch's atom types, edge_index and batch mapping are in HBM before the timed region; a step computes
    the edge tokens from them and runs the block.  Timed twice: launched eagerly, and captured once into a HIP
    graph (mind_amd.esa.graphs.GraphedForward) whose replays take the same inputs (copied into the graph's
    input buffers each step); the replay's outputs are checked bit for bit against the eager step's.  The
    replay is the reported step (ms_per_step, value); the eager step is the `eager` sub-object."""
    import torch

    from mind_amd import generators
    from mind_amd.esa.graphs import GraphedForward
    from mind_amd.esa.masked_layers import ESA

    dev = torch.device("cuda", 0)
    gb, types = generators.small_molecules(seed=args.seed)
    torch.manual_seed(args.seed)
    d, h = 128, 8
    emb, proj = torch.nn.Linear(16, d).to(dev), torch.nn.Linear(2 * d, d).to(dev)
    model = ESA(num_outputs=1, dim_output=d, dim_hidden=[d, d, d], num_heads=[h, h, h], layer_types="MSP",
                xformers_or_torch_attn="hip", use_mlps=True, mlp_hidden_size=2 * d, num_mlp_layers=2,
                mlp_type="standard").to(dev).eval()
    t = gb.num_tokens
    types_d = torch.as_tensor(types).to(dev)
    ei = torch.as_tensor(gb.edge_index).to(dev)
    bm = torch.as_tensor(gb.batch).to(dev)

    def forward(types_in, ei_in, bm_in):
        with torch.no_grad():
            x, n = _edge_tokens(gb, emb, proj, types_in, ei_in, bm_in)
            return model(x, ei_in, bm_in, n)

    def step():
        forward(types_d, ei, bm)

    ms, wall_ms, kern, ms_prof = timed(step, args.steps, args.warmup)
    lib_ms = sum(k["avg_us"] * k["launches"] for k in kern.values()) / 1e3 / args.steps
    graph = None
    if not args.no_graph:
        ref = tuple(y.clone() for y in forward(types_d, ei, bm))
        gf = GraphedForward(forward, types_d, ei, bm)
        g_ms, g_wall, _, _ = timed(lambda: gf(types_d, ei, bm), args.steps, args.warmup, profile=False)
        got = gf(types_d, ei, bm)
        torch.cuda.synchronize()
        graph = {"ms_per_step": g_ms, "wall_ms_per_step": g_wall, "edge_tokens_per_s": t / (g_ms * 1e-3),
                 "bit_identical_to_eager": all(torch.equal(a, b) for a, b in zip(got, ref)),
                 "what": "the same step captured once into a HIP graph and replayed (inputs copied into the "
                         "graph's input buffers each step): one launch per step instead of about a hundred"}
    # The step as it runs: replayed as one HIP graph (every kernel of the step, inputs copied in each step);
    # the eager step (about a hundred host launches, host-bound) is reported beside it.  --no-graph: eager.
    p_ms, p_wall = (g_ms, g_wall) if graph else (ms, wall_ms)
    eager = {"ms_per_step": ms, "wall_ms_per_step": wall_ms, "edge_tokens_per_s": t / (ms * 1e-3),
             "ms_per_step_profiled": ms_prof, "library_kernel_ms_per_step": lib_ms, "other_ms_per_step": ms - lib_ms,
             "what": "the step launched eagerly from Python; kernels: this library's launches (HIP events per "
                     "launch); other: the rest of the step (torch GEMMs, embedding, gathers of the padded views, "
                     "launch gaps)"}
    mode = "HIP graph replay (mind_amd.esa.graphs.GraphedForward)" if graph else "eager launches"
    if sub:
        out = {"workload": "config0: edge tokens (embed, gather, project) + ESA block M-S-P(1 seed) forward, fp32",
               "graphs": gb.num_graphs, "edge_tokens": t, "dim": d, "heads": h, "ms_per_step": p_ms,
               "wall_ms_per_step": p_wall, "edge_tokens_per_s": t / (p_ms * 1e-3), "execution": mode,
               "kernels": kern, "eager": eager, "graph": graph}
        if not args.no_cpu_baseline:
            out["cpu_baseline"] = cpu_baseline_block(gb, types, emb, proj, model, h)
        return out
    result = {
        "metric": "edge-tokens/sec through the ESA block forward (fp32)",
        "value": t / (p_ms * 1e-3), "unit": "edge-tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": p_ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded small molecules: 64 graphs, 9-29 atoms, radius 5 A; random-init weights)",
        "config": {"workload": "config0: edge tokens (embed, gather, project) + ESA block M-S-P(1 seed) forward",
                   "graphs": gb.num_graphs, "edge_tokens": t, "max_seqlen": gb.max_seqlen, "dim": d, "heads": h,
                   "seed": args.seed},
        "wall_ms_per_step": p_wall, "execution": mode, "kernels": kern, "eager": eager, "graph": graph,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_block(gb, types, emb, proj, model, h)
    print(json.dumps(result), flush=True)


def cpu_baseline_block(gb, types, emb, proj, model, heads) -> dict:
    """The reference's padded path on the host cores in fp32: per-graph edge bias, M, S, PMA blocks.

    The oracle's block restatement (oracle/modules.py) runs with the model's weights in fp32 on the same
    inputs; the per-graph block-diagonal bias gives the global E x E mask's entries
    (esa/masked_layers.py:217-268) without the E x E temporaries.
    """
    import torch

    from mind_amd.esa.packing import nearest_multiple_of_8
    from oracle import mask as OM
    from oracle import modules as OMod

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    OMod.DT = torch.float32   # time the restatement in fp32, the reference modules' dtype
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    with torch.no_grad():
        e_sd = {"w": emb.weight.detach().cpu(), "b": emb.bias.detach().cpu()}
        p_sd = {"w": proj.weight.detach().cpu(), "b": proj.bias.detach().cpu()}
    n = nearest_multiple_of_8(gb.max_seqlen + 1)
    cu = gb.cu_seqlens
    gid = np.repeat(np.arange(gb.num_graphs), gb.edge_counts)

    def step():
        x = torch.nn.functional.one_hot(torch.as_tensor(types), 16).float() @ e_sd["w"].T + e_sd["b"]
        src, dst = torch.as_tensor(gb.edge_index[0]), torch.as_tensor(gb.edge_index[1])
        tok = torch.cat([x[src], x[dst]], 1) @ p_sd["w"].T + p_sd["b"]
        X = torch.zeros(gb.num_graphs * n, tok.shape[1])
        pos = torch.as_tensor(np.arange(gb.num_tokens) - np.repeat(cu[:-1], gb.edge_counts))
        X[torch.as_tensor(gid) * n + pos] = tok
        X = X.view(gb.num_graphs, n, -1)
        bias = torch.full((gb.num_graphs, 1, n, n), OM.MASK_FILL)
        for b in range(gb.num_graphs):
            s, e = int(cu[b]), int(cu[b + 1])
            blk = OM.edge_adjacency_segment(gb.edge_index[0], gb.edge_index[1], s, e)
            bias[b, 0, : e - s, : e - s][torch.as_tensor(blk)] = 0.0
        OMod.esa(sd, X, "MSP", heads, 2,
                 attn_m=lambda s_, p_, x_: OMod.mab_padded(s_, p_, x_, x_, heads, bias),
                 attn_s=lambda s_, p_, x_: OMod.mab_padded(s_, p_, x_, x_, heads),
                 pool=lambda s_, p_, x_: OMod.pma_complete(s_, p_, x_, heads, 2))

    try:
        med, runs = _median_time(step)
    finally:
        OMod.DT = torch.float64
    return {"value": gb.num_tokens / med, "unit": "edge-tokens/s", "cores": cores, "kind": "port",
            "sample": (f"the whole config-0 batch ({gb.num_tokens} edge tokens, {gb.num_graphs} graphs) through the "
                       f"oracle's fp32 restatement of the reference's padded path (torch CPU, {cores} threads: "
                       f"embedding, gather, per-graph edge bias, M + S + PMA blocks), median of {runs} runs after "
                       f"2 warm-ups")}


def count_gemm_flops(step) -> int:
    """FLOPs of the matrix products one call of `step` runs (forward and backward): every aten mm / addmm /
    bmm / baddbmm dispatched (in-place forms included), 2 m n k each (batch included), from its operands'
    shapes."""
    from torch.utils._python_dispatch import TorchDispatchMode

    class GemmCount(TorchDispatchMode):
        flops = 0

        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            name = func._overloadpacket.__name__.rstrip("_")
            if name in ("mm", "bmm"):
                a, b = args[0], args[1]
            elif name in ("addmm", "baddbmm"):
                a, b = args[1], args[2]
            else:
                a = b = None
            if a is not None:
                batch = a.shape[0] if a.dim() == 3 else 1
                GemmCount.flops += 2 * batch * a.shape[-2] * a.shape[-1] * b.shape[-1]
            return func(*args, **(kwargs or {}))

    with GemmCount():
        step()
    return GemmCount.flops


def stack_flops(step, gb, d: int, layers: str, k_seeds: int, mlp: int) -> dict:
    """Exact FLOPs of one configuration-4 train step: the GEMMs counted as they are dispatched over one step
    (projections, MLPs, weight and input gradients, each product with its real shape), plus the attention by
    pair counts, 14 D per (query, key) pair for forward + backward (QK^T and PV; QK^T recomputation, dP, dV,
    dK, dQ): the S layers' pairs are sum L^2, the masked M layers' the mask's nnz (effective), PMA's
    k_seeds * T.  gemm_analytic restates the GEMMs from the layer shapes (3x the forward products: forward,
    input and weight gradients) as a check of the count."""
    gemm = count_gemm_flops(step)
    stats = edge_mask_stats(gb.edge_index[0].astype(np.int64), gb.edge_index[1].astype(np.int64), gb.cu_seqlens)
    t, b = gb.num_tokens, gb.num_graphs
    n_enc = sum(1 for lt in layers[: layers.index("P")] if lt in "MS")
    enc = n_enc * (4 * 2 * t * d * d + 2 * 2 * t * d * mlp)                  # Q, K, V, O; MLP up and down
    pma = 2 * k_seeds * d * d + 2 * 2 * t * d * d + 2 * b * k_seeds * d * d   # seeds' Q; K, V over tokens; O
    pma += 2 * 2 * b * k_seeds * d * mlp + 2 * b * d * d                      # PMA MLP; decoder_linear
    attn = {"S": 14 * d * gb.sum_sq * layers.count("S"), "M": 14 * d * stats["nnz"] * layers.count("M"),
            "P": 14 * d * k_seeds * t * layers.count("P")}
    return {"gemm": gemm, "gemm_analytic": 3 * (enc + pma), "attention": attn, "total": gemm + sum(attn.values()),
            "mask_nnz": stats["nnz"], "sum_L2": gb.sum_sq}


def bench_stack(args, sub: bool = False):
    """Configuration 4: ESA encoder stack M-M-S-S-M-M-S-S-P(4 seeds), D=512, H=32, MLP 2048, bf16 train step.

    bf16-mixed as the reference trains (core/train_pretrain.py:753): fp32 parameters under
    torch.autocast(bfloat16), so projections and MLPs run bf16 GEMMs and attention the bf16 kernels; a step is
    forward, backward and an AdamW update.
    """
    import torch

    from mind_amd import generators
    from mind_amd.esa.masked_layers import ESA
    from mind_amd.esa.packing import EdgeAdjacency, nearest_multiple_of_8

    dev = torch.device("cuda", 0)
    gb = generators.protein_budget(seed=args.seed, token_budget=131072)
    d, h, layers = 512, 32, "MMSSMMSSP"
    torch.manual_seed(args.seed)
    model = ESA(num_outputs=4, dim_output=d, dim_hidden=[d] * len(layers), num_heads=[h] * len(layers),
                layer_types=layers, xformers_or_torch_attn="hip", use_mlps=True, mlp_hidden_size=2048,
                num_mlp_layers=2, mlp_type="standard").to(dev)
    with torch.no_grad():
        for name, prm in model.named_parameters():
            if name.endswith("weight") and prm.dim() >= 2 or name.endswith(".S"):
                prm.normal_(0.0, 0.02)
            elif name.endswith("bias"):
                prm.zero_()
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, fused=True)   # one fused update kernel per dtype group
    n = nearest_multiple_of_8(gb.max_seqlen + 1)
    ei = torch.as_tensor(gb.edge_index).to(dev)
    bm = torch.as_tensor(gb.batch).to(dev)
    adj = EdgeAdjacency.from_edge_index(ei, bm, gb.num_graphs, n)
    t = gb.num_tokens
    g = torch.Generator(device=dev).manual_seed(args.seed)
    x = adj.pad(torch.randn(t, d, device=dev, generator=g))

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            emb, _ = model(x, ei, bm, n)
        loss = emb.float().pow(2).mean()
        loss.backward()
        opt.step()
        opt.zero_grad(set_to_none=True)

    ms, wall_ms, kern, ms_prof = timed(step, args.steps, args.warmup)
    lib_ms = sum(k["avg_us"] * k["launches"] for k in kern.values()) / 1e3 / args.steps
    attn_ms = sum(k["avg_us"] * k["launches"] for n, k in kern.items() if n.startswith("attn")) / 1e3 / args.steps
    fl = stack_flops(step, gb, d, layers, 4, 2048)
    achieved = fl["total"] / (ms * 1e-3) / 1e12
    roofline = {"bound": "mfma", "kernel": "whole train step (GEMMs + attention)", "achieved": achieved,
                "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": achieved / PEAK_BF16_TFLOPS, "traffic": None,
                "flops": "exact: GEMMs counted as dispatched over one step, attention 14 D per pair "
                         "(S: sum L^2, M: mask nnz, P: seeds x tokens)"}
    split = {"library_kernels_ms": lib_ms, "attention_ms": attn_ms, "other_ms": ms - lib_ms,
             "what": "library_kernels: this library's launches by HIP events (attention, LayerNorm, Mish, column "
                     "sums, ...), attention_ms the attention kernels among them; other: hipBLASLt GEMMs, AdamW, "
                     "torch elementwise ops and gaps"}
    if sub:
        return {"workload": "config4: ESA encoder stack M-M-S-S-M-M-S-S-P(4 seeds) train step, bf16-mixed",
                "graphs": gb.num_graphs, "edge_tokens": t, "dim": d, "heads": h, "mlp_hidden": 2048,
                "ms_per_step": ms, "wall_ms_per_step": wall_ms, "edge_tokens_per_s": t / (ms * 1e-3),
                "ms_per_step_profiled": ms_prof, "flops_per_step": fl, "roofline": roofline, "split": split,
                "kernels": kern}
    result = {
        "metric": "edge-tokens/sec through the ESA encoder stack train step (fwd+bwd+AdamW, bf16-mixed)",
        "value": t / (ms * 1e-3), "unit": "edge-tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded lognormal protein-like graphs packed to a 131,072 edge-token budget; x ~ N(0,1); "
                "weights N(0, 0.02))",
        "config": {"workload": "config4: ESA encoder stack M-M-S-S-M-M-S-S-P(4 seeds) train step",
                   "graphs": gb.num_graphs, "edge_tokens": t, "max_seqlen": gb.max_seqlen, "padded_items": n,
                   "dim": d, "heads": h, "mlp_hidden": 2048, "seed": args.seed},
        "wall_ms_per_step": wall_ms, "ms_per_step_profiled": ms_prof, "kernels": kern,
        "flops_per_step": fl, "roofline": roofline, "split": split,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
