#!/usr/bin/env python3
"""Throughput of raya's block-local attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 100] [--warmup 10] [--workload NAME] [--no-encoder]

A step is one launch of the fused fp32 attention kernel over one whole batch
whose Q, K, V (seeded N(0, 1)) are already resident in HBM.  The default
workload is B=32 sequences x 12 heads x L=2048 x D=64 with the BlockDiag(64)
mask and per-sequence valid lengths uniform in [512, 2048].  Prints one JSON
line: TFLOP/s on the algorithmic FLOP count (valid rows only), the kernel's
HBM roofline fraction (HIP events on the launch stream), and the reference's
Tiled CPU algorithm timed on this host on the same inputs.

With the default workload the line also carries "encoder": sequences/sec of the
full 12-layer ModernBERT-base decision-model forward (B=64, L=512, valid
lengths uniform in [128, 512], random N(0, 0.02) weights from a safetensors
checkpoint) and the oracle's CPU forward on the first sequences beside it, and
"encoder_layer": one block-local layer of that model on B=16 x L=1024 valid
tokens (BlockDiag(64) on the local layers), from the forward's own per-layer
event spans.
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

from raya_amd.workloads import (ATTENTION as WORKLOADS, DEFAULT_ATTENTION as DEFAULT, ENCODER,  # noqa: E402
                                ENCODER_WEIGHT_SEED, LAYER, REF_BLOCK, algorithmic, encoder_inputs,
                                mask_name)
from raya_amd.workloads import attention_inputs as make_inputs  # noqa: E402


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_cpu() -> dict:
    """CPU model and core counts of this host (the baseline's context)."""
    from raya_amd import meta

    return meta.host_cpu()


def cpu_baseline(qkv, valid, wl, budget_s: float):
    """The reference's Tiled algorithm (AVX2+FMA when present) on this host's cores."""
    import oracle

    b, h, s, d, mask = wl["batch"], wl["heads"], wl["seq"], wl["head_dim"], wl["mask"]
    kind = {"block_diag": oracle.MASK_BLOCKDIAG, "block3": oracle.MASK_BLOCK3,
            "window64": oracle.MASK_WINDOW64}[mask[0]]
    block = mask[1] if mask[0] == "block_diag" else REF_BLOCK
    threads = min(16, len(os.sched_getaffinity(0)))
    q, k, v = qkv
    backend = 1 if oracle.cpu_has_avx2_fma() else 0
    flops, _ = algorithmic(valid, h, d, s, mask)
    times = []
    out = None
    t_end = time.perf_counter() + budget_s
    while True:
        t0 = time.perf_counter()
        out, used = oracle.tiled_attend_batched(q, k, v, kind, valid, 0.125, block=block,
                                                threads=threads, backend=backend, out=out)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end or len(times) >= 50:
            break
    med = statistics.median(times)
    # single-thread figure on the first sequences (the reference bench's t1 leg)
    n1 = max(1, min(b, 4))
    f1, _ = algorithmic(valid[:n1], h, d, s, mask)
    t0 = time.perf_counter()
    oracle.tiled_attend_batched(q[:n1], k[:n1], v[:n1], kind, valid[:n1], 0.125, block=block,
                                threads=1, backend=backend)
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
        "host": host_cpu(),
    }


def encoder_flops(valid, d=768, inter=3072, heads=12, layers=12, global_every=3, window=64):
    """GEMM FLOP on valid tokens (2 d (3d + d + 2F + F) per token and layer, GeGLU Wi is
    [2F, d]) plus attention FLOP (4 D H per allowed (query, key) pair; Full on global layers,
    Sliding(window) on local layers)."""
    hd = d // heads
    gemm = sum(int(v) for v in valid) * 2 * d * (3 * d + d + 2 * inter + inter) * layers
    attn = 0
    for i in range(layers):
        for v in valid:
            v = int(v)
            if i % global_every == 0:
                pairs = v * v
            else:  # sum over i of |[i - w, i + w] ∩ [0, v)|
                pairs = sum(min(v, t + window + 1) - max(0, t - window) for t in range(v))
            attn += 4 * hd * heads * pairs
    return gemm, attn


def bench_encoder(steps: int, warmup: int, cpu_seconds: float, cpu: bool, layer: bool = True) -> dict:
    """Sequences/sec of the full forward (embed, 12 layers, final norm, scorer, act head) on a
    batch of 64; each step includes the input upload, every kernel, the output download and
    the stream synchronisation."""
    import shutil
    import tempfile

    import numpy as np

    from raya_amd import checkpoint, model as M

    spec = ENCODER
    tmp = tempfile.mkdtemp(prefix="raya_ckpt_")
    try:
        log("encoder: writing the synthetic checkpoint")
        checkpoint.write_synthetic(tmp, seed=ENCODER_WEIGHT_SEED)
        m = M.Model.load(tmp)
        ids, valid, pos, mask, qtype = encoder_inputs(spec)
        log(f"encoder: warmup {warmup}")
        for _ in range(warmup):
            out = m.forward_batch(ids, valid, pos, mask, qtype)
        log(f"encoder: timing {steps} forwards")
        t0 = time.perf_counter()
        for _ in range(steps):
            out = m.forward_batch(ids, valid, pos, mask, qtype)
        dt = (time.perf_counter() - t0) / steps
        gemm, attn = encoder_flops(valid)
        b = spec["batch"]
        res = {
            "workload": spec["workload"], "batch": b, "seq": spec["seq"],
            "valid_len": f"uniform [{spec['valid'][0]}, {spec['valid'][1]}]",
            "valid_tokens": int(valid.sum()), "sequences_per_s": b / dt, "ms_per_forward": dt * 1e3,
            "flop_per_forward_valid": gemm + attn, "tflops": (gemm + attn) / dt / 1e12,
            "mfma_frac": (gemm + attn) / dt / 1e12 / PEAK_FP32_MFMA_TFLOPS,
            "padding": "not computed (valid tokens are packed; padded rows cannot change valid rows)",
            "masks": "reference: Full on global layers, Sliding(64) on local layers",
            "weights": "N(0, 0.02), norms 1, safetensors under raya-weights names, loaded once",
            "steps": steps, "warmup": warmup,
            "act_logits_finite": bool(np.isfinite(out.act_logits).all()),
        }
        if layer:
            res["layer"] = bench_layer(m, steps, warmup)
        if cpu:
            log("encoder: cpu baseline")
            res["cpu_baseline"] = encoder_cpu_baseline(tmp, ids, valid, pos, mask, qtype, out,
                                                       cpu_seconds)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return res


GEMM_SHAPES = [
    # (name, n, k, epilogue) of the encoder's four projections, at the forward's M = 21,405
    # valid tokens (the mean of the encoder workload's packed batch)
    ("qkv_2304x768", 2304, 768, "none"),
    ("wo_768x768_residual", 768, 768, "residual"),
    ("geglu_wi_6144x768", 3072, 768, "geglu"),
    ("mlp_wo_768x3072_residual", 768, 3072, "residual"),
]
GEMM_M = 21405


def bench_gemms(steps: int, warmup: int) -> dict:
    """The encoder's four GEMM shapes alone, with their fused epilogues, inputs resident in
    HBM: K back-to-back launches per shape bracketed by one event pair on the launch stream.
    Every shape's warm-up launches run before any shape is timed, so the first one timed
    does not pay for the clock's ramp from idle."""
    import torch

    import raya_amd as R
    from raya_amd import _capi as C

    g = R.HipGemm()
    stream = torch.cuda.current_stream()
    gen = torch.Generator(device="cuda").manual_seed(1000 * 4 + 7)
    res = {"m": GEMM_M, "steps": steps, "warmup": warmup, "shapes": {}}
    steps_of = {}
    for name, n, k, epi in GEMM_SHAPES:
        rows = 2 * n if epi == "geglu" else n
        a = torch.randn(GEMM_M, k, device="cuda", generator=gen)
        b = 0.02 * torch.randn(rows, k, device="cuda", generator=gen)
        out = torch.randn(GEMM_M, n, device="cuda", generator=gen)
        act = C.RAYA_EPI_GEGLU if epi == "geglu" else C.RAYA_EPI_NONE
        resid = out if epi == "residual" else None
        steps_of[name] = (lambda a=a, b=b, out=out, act=act, resid=resid:
                          g.matmul_nt_device(out, a, b, activation=act, residual=resid, stream=stream))
    for _ in range(warmup):
        for step in steps_of.values():
            step()
    for name, n, k, epi in GEMM_SHAPES:
        step = steps_of[name]
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        flops = 2.0 * GEMM_M * (2 * n if epi == "geglu" else n) * k
        res["shapes"][name] = {"n_out": n, "k": k, "epilogue": epi, "ms": ms,
                               "tflops": flops / ms / 1e9,
                               "mfma_frac": flops / ms / 1e9 / PEAK_FP32_MFMA_TFLOPS}
    return res


def bench_layer(m, steps: int, warmup: int) -> dict:
    """One block-local encoder layer (pre-LN, QKV + RoPE, BlockDiag(64) attention, Wo + residual,
    LN, GeGLU, Wo + residual) on B=16 x L=1024 valid tokens: the per-layer event spans of the
    model's own forward (stage timing level 1), median over the local layers and steps; a level-2
    forward gives the per-kernel split."""
    import numpy as np

    from raya_amd import Mask

    spec = LAYER
    ids, valid, pos, mask, qtype = encoder_inputs(spec)
    info = m.info
    n_layers, every = info["num_hidden_layers"], info["global_attn_every_n_layers"]
    local = [i for i in range(n_layers) if i % every != 0]
    lm = Mask.block_diag(spec["block"])
    log(f"layer: warmup {warmup}, timing {steps} forwards (B={spec['batch']}, L={spec['seq']})")
    m.set_profiling(1)
    try:
        for _ in range(warmup):
            m.forward_batch(ids, valid, pos, mask, qtype, local_mask=lm)
        times = []
        for _ in range(steps):
            m.forward_batch(ids, valid, pos, mask, qtype, local_mask=lm)
            st = dict(m.stage_times())
            times += [st[f"encoder_layer_{i:02d}"] for i in local]
        m.set_profiling(2)
        m.forward_batch(ids, valid, pos, mask, qtype, local_mask=lm)
        st2 = m.stage_times()
    finally:
        m.set_profiling(0)
    ms = statistics.median(times)
    tokens = int(valid.sum())
    d, inter, heads = info["hidden_size"], info["intermediate_size"], info["num_attention_heads"]
    hd = d // heads
    gemm = tokens * 2 * d * (3 * d + d + 2 * inter + inter)
    b = spec["block"]
    attn = 4 * hd * heads * sum(b * b * (int(v) // b) + (int(v) % b) ** 2 for v in valid)
    ops = {}
    for name, t in st2:
        if "/" in name and int(name.split("/")[0].rsplit("_", 1)[1]) in local:
            ops.setdefault(name.split("/")[1], []).append(t)
    return {
        "workload": spec["workload"], "batch": spec["batch"], "seq": spec["seq"],
        "valid_tokens": tokens, "mask": f"block_diag({b}) (local layers)",
        "ms_per_layer": ms, "sequences_per_s": spec["batch"] / (ms / 1e3),
        "flop_per_layer": gemm + attn, "tflops": (gemm + attn) / (ms / 1e3) / 1e12,
        "mfma_frac": (gemm + attn) / (ms / 1e3) / 1e12 / PEAK_FP32_MFMA_TFLOPS,
        "timing": f"median of {len(times)} local-layer spans ({len(local)} layers x {steps} forwards)",
        "kernels_ms": {k: statistics.mean(v) for k, v in ops.items()},
        "layer_input": "normalised token embeddings of uniform random ids (unit variance rows)",
    }


def encoder_cpu_baseline(ckpt, ids, valid, pos, mask, qtype, gpu_out, budget_s: float) -> dict:
    """The oracle's restatement of Network::forward (sequential-f32 GEMMs on host threads,
    Naive attention) on the first sequences of the batch until the time budget is spent."""
    import numpy as np

    from oracle import forward as F

    cfg = F.load_config(ckpt)
    w = F.load_weights(os.path.join(ckpt, "model.safetensors"))
    threads = min(16, len(os.sched_getaffinity(0)))
    F.GEMM_THREADS = threads
    done, diff, t0 = 0, 0.0, time.perf_counter()
    while done < len(valid):
        v = int(valid[done])
        o = F.forward(cfg, w, ids[done, :v], v, pos[done], mask[done], int(qtype[done]))
        diff = max(diff, float(np.abs(o.act_logits - gpu_out.act_logits[done]).max()))
        done += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    return {"value": done / dt, "unit": "sequences/s", "cores": threads, "kind": "port",
            "host": host_cpu(),
            "sample": (f"first {done} sequences of the batch ({int(valid[:done].sum())} tokens), "
                       f"one at a time, {dt:.1f} s"),
            "gpu_vs_cpu_act_logits_max_abs": diff}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default=DEFAULT, choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-seconds", type=float, default=5.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-encoder", action="store_true", help="skip the encoder forward leg")
    ap.add_argument("--encoder-steps", type=int, default=10)
    ap.add_argument("--encoder-warmup", type=int, default=2)
    ap.add_argument("--gemm-only", action="store_true",
                    help="time only the encoder's four GEMM shapes and print their line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (got --gpus {args.gpus})",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import raya_amd as R

    if args.gemm_only:
        gm = bench_gemms(args.steps, args.warmup)
        # one layer's four projections: total FLOP over total time
        flop = sum(2.0 * GEMM_M * (2 * n if e == "geglu" else n) * k for _, n, k, e in GEMM_SHAPES)
        ms = sum(v["ms"] for v in gm["shapes"].values())
        print(json.dumps({"metric": "fp32 encoder GEMM TFLOP/s (one layer's four projections), 1 GPU",
                          "value": flop / ms / 1e9, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
                          "warmup": args.warmup, "higher_is_better": True, "dtype": "f32",
                          "data": "synthetic", "config": {"workload": "encoder_gemms_m21405"},
                          "gemms": gm}), flush=True)
        return 0

    wl = WORKLOADS[args.workload]
    b, h, s, d, mask_spec = wl["batch"], wl["heads"], wl["seq"], wl["head_dim"], wl["mask"]
    lo, hi = wl["valid"]
    log(f"generating inputs for {args.workload}")
    qkv, valid = make_inputs(wl)
    dev = torch.device("cuda:0")
    q, k, v = (torch.from_numpy(x).to(dev) for x in qkv)
    vl = torch.from_numpy(valid).to(dev)
    out = torch.empty_like(q)
    kernel = R.HipAttention()
    mask = {"block_diag": lambda: R.Mask.block_diag(mask_spec[1]), "block3": lambda: R.Mask.BLOCK3,
            "window64": lambda: R.Mask.WINDOW64}[mask_spec[0]]()
    stream = torch.cuda.current_stream(dev)
    flops, nbytes = algorithmic(valid, h, d, s, mask_spec)

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
                   "mask": mask_name(mask_spec),
                   "valid_len": f"uniform [{lo}, {hi}]" if lo != hi else f"{lo} (no padding)",
                   "inputs": ("xorshift U[-1, 1], seeds 42/43/44" if wl["data"] == "xorshift"
                              else "N(0, 1), SplitMix64 + Box-Muller"),
                   "outliers": "1% x20" if wl["outliers"] else "none", "flop_per_step": flops,
                   "bytes_per_step": nbytes},
        "kernel_ms": avg_kernel_s * 1e3,
        "kernel_tflops": flops / avg_kernel_s / 1e12,
        "mfma_frac": flops / avg_kernel_s / 1e12 / PEAK_FP32_MFMA_TFLOPS,
    }
    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"{args.workload}_traffic.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")
    # The bound is the one the arithmetic intensity reaches first.
    if flops / nbytes < PEAK_FP32_MFMA_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9):
        achieved = nbytes / avg_kernel_s / 1e9
        result["roofline"] = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS,
                              "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS, "traffic": traffic}
    else:
        achieved = flops / avg_kernel_s / 1e12
        result["roofline"] = {"bound": "mfma", "achieved": achieved, "peak": PEAK_FP32_MFMA_TFLOPS,
                              "unit": "TFLOP/s", "frac": achieved / PEAK_FP32_MFMA_TFLOPS,
                              "traffic": traffic}

    # One launch of the instrumented kernel after the timed region: where the
    # waves' cycles go (the reference's stage-timing split, tiled/stages.rs).
    st = kernel.attend_batched_stages(q, k, v, out, vl, mask, stream=stream)
    pct = st.percentages()
    waves = st.qk + st.softmax + st.pv + st.load_wait
    result["stage_split"] = {
        "qk_pct": pct[0], "softmax_pct": pct[1], "pv_pct": pct[2],
        "load_wait_of_wave_cycles_pct": 100.0 * st.load_wait / waves, "tiles": st.tiles,
        "source": "one instrumented launch after the timed region; shares of per-wave shader "
                  "clock cycles (qk/softmax/pv as in the reference's StageTimes::percentages)"}

    # BenchMetadata (crates/raya-kernels/src/meta.rs): host, GPU and build; threads is
    # the CPU baseline's worker count.
    from raya_amd import meta

    result["meta"] = meta.collect(threads=0 if args.no_cpu_baseline
                                  else min(16, len(os.sched_getaffinity(0))))

    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu_out, cb = cpu_baseline(qkv, valid, wl, args.cpu_seconds)
        got = out.cpu().numpy()
        diff = 0.0
        for i in range(b):
            diff = max(diff, float(np.abs(got[i, :, : valid[i]] - cpu_out[i, :, : valid[i]]).max()))
        cb["gpu_vs_cpu_max_abs"] = diff
        result["cpu_baseline"] = cb
    if args.workload == DEFAULT and not args.no_encoder:
        enc = bench_encoder(args.encoder_steps, args.encoder_warmup, args.cpu_seconds,
                            cpu=not args.no_cpu_baseline)
        layer = enc.pop("layer", None)
        result["encoder"] = enc
        if layer is not None:
            result["encoder_layer"] = layer
        log("encoder gemm shapes")
        result["encoder_gemms"] = bench_gemms(20, 3)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
