"""Benchmark: ESA varlen attention forward + backward on one MI355X.

Workload (the benchmark definition's configuration 1): 32 protein-like graphs
(node counts U{64..512}, 3.8 A random-walk chains, radius 8 A, at most 16
neighbours), one edge token per directed edge, packed with cu_seqlens; 16
heads of head_dim 16 (dim 256); q, k, v, dO ~ N(0, 1) in bf16; causal=False;
softmax scale 1/4.  A step is one forward and one backward over the batch,
with inputs already resident in HBM.

Prints one JSON line: throughput in edge-tokens/s, MFMA utilisation of the
dense-bf16 peak, the roofline of the dominant kernel (HIP events around every
launch in the timed region) and a CPU baseline (the oracle's per-graph fp32
attention forward + backward on a bounded sample of the same batch, on this
host's cores).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

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
    ap.add_argument("--cpu-sample-graphs", type=int, default=3,
                    help="graphs of the batch timed on the CPU for the baseline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
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


def cpu_baseline(gb, seed: int, n_graphs: int) -> dict:
    """Oracle per-graph attention fwd+bwd in fp32 on the host cores, bounded sample."""
    import numpy as np
    import torch

    from oracle import attention as oracle_attention

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    order = np.argsort(gb.edge_counts)
    # a sample spread over the length distribution: shortest, median, longest ...
    pick = sorted(set(int(order[int(i)]) for i in np.linspace(0, len(order) - 1, n_graphs)))
    lens = gb.edge_counts[pick]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    t = int(cu[-1])
    g = torch.Generator().manual_seed(seed + 99)
    q, k, v, go = (torch.randn(t, HEADS, HEAD_DIM, generator=g) for _ in range(4))

    def step():
        oracle_attention.varlen_attention(q, k, v, cu, cu, 0.25, dtype=torch.float32)
        oracle_attention.varlen_attention_bwd(go, q, k, v, cu, cu, 0.25, dtype=torch.float32)

    step()
    times = []
    budget = time.perf_counter() + 12.0
    while len(times) < 3 or (time.perf_counter() < budget and len(times) < 20):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {"value": t / med, "unit": "edge-tokens/s", "cores": cores, "kind": "port",
            "sample": (f"oracle fp32 per-graph attention fwd+bwd (torch CPU, {cores} threads) on {len(pick)} graphs "
                       f"of the batch ({t} tokens, lengths {lens.tolist()}), median of {len(times)} runs; the "
                       f"batch's throughput on the CPU would be lower (cost grows with the sum of squared lengths)")}


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

    import numpy as np
    import torch

    from mind_amd import _lib, generators
    from mind_amd.esa import attention

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
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

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    _lib.profile_enable(True)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    _lib.profile_enable(False)
    kern = _lib.profile_collect()
    ms_per_step = ev0.elapsed_time(ev1) / args.steps

    tokens_per_s = t / (ms_per_step * 1e-3)
    total_flops = 14 * DIM * pairs
    tflops = total_flops / (ms_per_step * 1e-3) / 1e12

    per_kernel = {}
    for name, (ms, n) in kern.items():
        if n:
            per_kernel[name] = {"avg_us": 1e3 * ms / n, "launches": n}
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
        "wall_ms_per_step": 1e3 * wall / args.steps,
        "kernels": per_kernel,
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": achieved, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / PEAK_BF16_TFLOPS, "traffic": traffic},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(gb, args.seed, args.cpu_sample_graphs)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
