#!/usr/bin/env python3
"""Throughput of raya's block-local attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--workload NAME]

A step is one launch of the fused fp32 attention kernel over one whole batch
whose Q, K, V (seeded N(0, 1)) are already resident in HBM.  The default
workload is B=32 sequences x 12 heads x L=2048 x D=64 with the BlockDiag(64)
mask and per-sequence valid lengths uniform in [512, 2048].  Prints one JSON
line: TFLOP/s on the algorithmic FLOP count (valid rows only), the kernel's
HBM roofline fraction (HIP events on the launch stream), and the reference's
Tiled CPU algorithm timed on this host on the same inputs.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_FP32_MFMA_TFLOPS = 157.3
METRIC = "fp32 block-local attn TFLOP/s + % roofline; encoder sequences/sec, 1 GPU"

WORKLOADS = {
    # name: (workload number for seeds, batch, heads, seq, head_dim, block, valid range, outliers)
    "attn_b32_h12_l2048_d64_blockdiag64": (2, 32, 12, 2048, 64, 64, (512, 2048), False),
    "attn_b1_h12_l512_d64_blockdiag64": (1, 1, 12, 512, 64, 64, (512, 512), False),
    "attn_b4_h12_l16384_d64_blockdiag128": (5, 4, 12, 16384, 64, 128, (8192, 16384), True),
}
DEFAULT = "attn_b32_h12_l2048_d64_blockdiag64"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic(valid, heads, head_dim, seq, block):
    """FLOP = 4 D H sum_b sum_{i<v_b} |keys(i)|; bytes = Q, K, V valid rows read once + all
    output rows written (fp32)."""
    keys = sum(block * block * (int(v) // block) + (int(v) % block) ** 2 for v in valid)
    flops = 4 * head_dim * heads * keys
    nbytes = 4 * (3 * heads * head_dim * int(sum(int(v) for v in valid))
                  + len(valid) * heads * seq * head_dim)
    return flops, nbytes


def make_inputs(wl):
    import numpy as np

    from raya_amd import synth

    c, b, h, s, d, block, (lo, hi), outliers = wl
    n = b * h * s * d
    qkv = []
    for i in range(3):
        x = synth.normal(synth.workload_seed(c, i), n).reshape(b, h, s, d)
        if outliers:
            synth.with_outliers(x, synth.workload_seed(c, 4) + 10 * i)
        qkv.append(x)
    valid = synth.integers(synth.workload_seed(c, 3), b, lo, hi).astype(np.int32)
    return qkv, valid


def cpu_baseline(qkv, valid, wl, budget_s: float):
    """The reference's Tiled algorithm (AVX2+FMA when present) on this host's cores."""
    import oracle

    c, b, h, s, d, block, _, _ = wl
    threads = min(16, len(os.sched_getaffinity(0)))
    q, k, v = qkv
    backend = 1 if oracle.cpu_has_avx2_fma() else 0
    flops, _ = algorithmic(valid, h, d, s, block)
    times = []
    out = None
    t_end = time.perf_counter() + budget_s
    while True:
        t0 = time.perf_counter()
        out, used = oracle.tiled_attend_batched(q, k, v, oracle.MASK_BLOCKDIAG, valid, 0.125,
                                                block=block, threads=threads, backend=backend,
                                                out=out)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end or len(times) >= 50:
            break
    med = statistics.median(times)
    # single-thread figure on the first sequences (the reference bench's t1 leg)
    n1 = max(1, min(b, 4))
    f1, _ = algorithmic(valid[:n1], h, d, s, block)
    t0 = time.perf_counter()
    oracle.tiled_attend_batched(q[:n1], k[:n1], v[:n1], oracle.MASK_BLOCKDIAG, valid[:n1], 0.125,
                                block=block, threads=1, backend=backend)
    t1 = time.perf_counter() - t0
    return out, {
        "value": flops / med / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"whole workload ({b} sequences), Tiled restatement "
                   f"({'avx2+fma' if used == 1 else 'portable'}), {threads} threads, "
                   f"median of {len(times)} runs ({med * 1e3:.1f} ms each)"),
        "t1_value": f1 / t1 / 1e12,
        "t1_sample": f"first {n1} sequences, 1 thread, {t1 * 1e3:.1f} ms",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default=DEFAULT, choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-seconds", type=float, default=5.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (got --gpus {args.gpus})",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import raya_amd as R

    wl = WORKLOADS[args.workload]
    c, b, h, s, d, block, (lo, hi), outliers = wl
    log(f"generating inputs for {args.workload}")
    qkv, valid = make_inputs(wl)
    dev = torch.device("cuda:0")
    q, k, v = (torch.from_numpy(x).to(dev) for x in qkv)
    vl = torch.from_numpy(valid).to(dev)
    out = torch.empty_like(q)
    kernel = R.HipAttention()
    mask = R.Mask.block_diag(block)
    stream = torch.cuda.current_stream(dev)
    flops, nbytes = algorithmic(valid, h, d, s, block)

    def step():
        kernel.attend_batched(q, k, v, out, vl, mask, stream=stream)

    log(f"warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # One event pair on the launch stream brackets the K back-to-back launches
    # (an event between launches costs ~10 us of idle queue per step), so the
    # average launch duration is the bracketed time over K.
    log(f"timing {args.steps} steps")
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    avg_kernel_s = start.elapsed_time(end) / 1e3 / args.steps
    ms_per_step = wall / args.steps * 1e3

    result = {
        "metric": METRIC,
        "value": flops / (ms_per_step / 1e3) / 1e12,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": args.workload, "batch": b, "heads": h, "seq": s, "head_dim": d,
                   "mask": f"block_diag({block})", "valid_len": f"uniform [{lo}, {hi}]",
                   "outliers": "1% x20" if outliers else "none", "flop_per_step": flops,
                   "bytes_per_step": nbytes},
        "kernel_ms": avg_kernel_s * 1e3,
        "kernel_tflops": flops / avg_kernel_s / 1e12,
        "mfma_frac": flops / avg_kernel_s / 1e12 / PEAK_FP32_MFMA_TFLOPS,
    }
    achieved = nbytes / avg_kernel_s / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"{args.workload}_traffic.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")
    result["roofline"] = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS,
                          "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS, "traffic": traffic}

    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu_out, cb = cpu_baseline(qkv, valid, wl, args.cpu_seconds)
        got = out.cpu().numpy()
        diff = 0.0
        for i in range(b):
            diff = max(diff, float(np.abs(got[i, :, : valid[i]] - cpu_out[i, :, : valid[i]]).max()))
        cb["gpu_vs_cpu_max_abs"] = diff
        result["cpu_baseline"] = cb
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
