#!/usr/bin/env python3
"""Throughput of raya's block-local attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 100] [--warmup 10] [--workload NAME] [--no-encoder]
    python bench.py --refbench [--refbench-out PATH]
    python bench.py --predict [--predict-tokens 512,2048,4096] [--predict-repeats 20]

A step is one launch of the fused fp32 attention kernel over one whole batch
whose Q, K, V (seeded N(0, 1)) are already resident in HBM; successive steps
alternate between two copies of the inputs and outputs, so that no step finds the
previous step's bytes in the 256 MB memory-side cache in front of HBM.  The default
workload is B=32 sequences x 12 heads x L=2048 x D=64 with the BlockDiag(64)
mask and per-sequence valid lengths uniform in [512, 2048].  Prints one JSON
line: TFLOP/s on the algorithmic FLOP count (valid rows only), the kernel's
HBM roofline fraction (HIP events on the launch stream), and the reference's
Tiled CPU algorithm timed on this host on the same inputs.

Before the W warm-up steps every attention line runs its kernel back to back for
RAMP_MS of wall time ("ramp" in the line): from idle, the first ~150 launches of
the headline kernel run up to 25% slower while the GPU's power state rises, and
a handful of warm-up steps would time that transition instead of the kernel.

With the default workload the line also carries:
* "workloads": the other attention configurations, each with its own roofline
  and CPU baseline: one sequence of 12 x 512 (BlockDiag(64) and the reference's
  Block3; also the reference's Naive on one thread), 4 x 12 x 16384 with x20
  outliers (BlockDiag(128) and Block3), and the headline batch under Block3.
  Launches that take a few microseconds are timed as replays of a HIP graph of
  20 launches (the Python launch path alone takes ~8 us); their eager figure is
  reported beside it;
* "encoder": sequences/sec of the full 12-layer ModernBERT-base decision-model
  forward (B=64, L=512, valid lengths uniform in [128, 512], random N(0, 0.02)
  weights from a safetensors checkpoint) and the oracle's CPU forward on the
  first sequences beside it; "predict_latency" in it: p50/p90 of single-sequence
  predicts of 512, 2,048 and 4,096 tokens (end to end, host arrays in and out);
* "encoder_layer": one block-local layer of that model on B=16 x L=1024 valid
  tokens (BlockDiag(64) on the local layers), from the forward's own per-layer
  event spans;
* "encoder_gemms": the encoder's four GEMM shapes alone;
* "postln_layer": one post-LN encoder layer as BERT writes it (hidden 768 = 12 x 64,
  biases, erf-GELU feed-forward 3072, LayerNorm eps 1e-12 after each residual add)
  on B=16 x L=1024 tokens with BlockDiag(64) attention, N(0, 0.02) weights, zero
  biases, unit gains and N(0, 1) inputs, and the oracle's CPU layer on one sequence.

--refbench writes the reference bench's result document
(crates/raya-kernels/benches/local_attention.rs:89-172): label, metadata and one
row per kernel x mask x seq x threads with mean_ms, stddev_ms, samples and
stages, for this GPU beside the Tiled restatement (1 thread and all threads) and
Naive (1 thread) on 16 heads x L in {2048, 4096, 8192} x {Block3, Window64}.

--predict prints the predict-latency document that `raya bench` is specified to write
(specs/008-bench-harness/spec.md:19-31): one sequence of each token count through the
12-layer decision model, p50/p90 of the end-to-end call, the per-component split, the model's
load time and the peak RSS.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from raya_amd.workloads import (ATTENTION as WORKLOADS, DEFAULT_ATTENTION as DEFAULT, ENCODER,  # noqa: E402
                                ENCODER_WEIGHT_SEED, LAYER, POSTLN_LAYER, REF_BLOCK, algorithmic,
                                attention_inputs, encoder_inputs, mask_name, postln_flops, postln_inputs)

PEAK_HBM_GBS = 8000.0
PEAK_FP32_MFMA_TFLOPS = 157.3
METRIC = "fp32 block-local attn TFLOP/s + % roofline; encoder sequences/sec, 1 GPU"
RAMP_MS = 60.0
GRAPH_LAUNCHES = 20
# Copies of each attention workload's inputs and outputs, used in turn by successive launches.
INPUT_SETS = 2
# Launches shorter than this are timed from graph replays (eager launches are host-bound).
GRAPH_BELOW_MS = 0.05
# Ordered so that lines drawing the same inputs (same batch, another mask) follow each other.
SUBLINES = ["attn_b32_h12_l2048_d64_block3",
            "attn_b1_h12_l512_d64_blockdiag64", "attn_b1_h12_l512_d64_block3",
            "attn_b4_h12_l16384_d64_blockdiag128", "attn_b4_h12_l16384_d64_block3",
            "refbench_h16_l8192_d64_window64"]
# The trait's own path (host slices in and out, AttentionKernel::attend): the one-sequence
# workloads and the reference bench's smallest shape.
HOST_SLICE = ["attn_b1_h12_l512_d64_blockdiag64", "attn_b1_h12_l512_d64_block3", "refbench_h16_l2048_d64_block3"]
_INPUTS: dict = {}


def cached_inputs(wl):
    """attention_inputs(wl), reused by the next line that draws the same batch."""
    key = (wl["family"], wl["batch"], wl["heads"], wl["seq"], wl["valid"], wl["outliers"], wl["data"])
    if key not in _INPUTS:
        _INPUTS.clear()
        _INPUTS[key] = attention_inputs(wl)
    return _INPUTS[key]
NAIVE_T1 = {"attn_b1_h12_l512_d64_blockdiag64", "attn_b1_h12_l512_d64_block3"}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_cpu() -> dict:
    """CPU model and core counts of this host (the baseline's context)."""
    from raya_amd import meta

    return meta.host_cpu()


def cpu_threads() -> int:
    """The CPU baselines' worker count: RAYA_THREADS, else the physical cores this process may
    run on (the reference's default_threads, threads.rs:3-9)."""
    from raya_amd import meta

    return meta.default_threads()


def kernel_mask(spec):
    import raya_amd as R

    return {"block_diag": lambda: R.Mask.block_diag(spec[1]), "block3": lambda: R.Mask.BLOCK3,
            "window64": lambda: R.Mask.WINDOW64}[spec[0]]()


def oracle_mask(spec):
    import oracle

    kind = {"block_diag": oracle.MASK_BLOCKDIAG, "block3": oracle.MASK_BLOCK3,
            "window64": oracle.MASK_WINDOW64}[spec[0]]
    return kind, (spec[1] if spec[0] == "block_diag" else REF_BLOCK)


# --- GPU timing -------------------------------------------------------------------------------

def ramp(step, ms: float = RAMP_MS) -> int:
    """Back-to-back launches for `ms` of wall time (synchronising every 20); returns the count."""
    import torch

    n, t_end = 0, time.perf_counter() + ms / 1e3
    while time.perf_counter() < t_end:
        for _ in range(20):
            step()
        n += 20
        torch.cuda.synchronize()
    return n


def time_eager(step, steps: int, stream) -> tuple[float, float]:
    """(average kernel seconds from one event pair on the launch stream around `steps`
    back-to-back launches, host wall seconds per step)."""
    import torch

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    return e0.elapsed_time(e1) / 1e3 / steps, wall


def time_per_launch(step, steps: int, stream) -> list[float]:
    """Milliseconds of each of `steps` back-to-back launches: an event recorded on the launch
    stream before every launch and one after the last (for launches much longer than the
    host's launch path, so the stream never waits for the host)."""
    import torch

    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    for i in range(steps):
        ev[i].record(stream)
        step()
    ev[steps].record(stream)
    torch.cuda.synchronize()
    return [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]


def time_graph(launch_on, steps: int, stream) -> float:
    """Average seconds per launch over replays of a HIP graph holding GRAPH_LAUNCHES
    launches (captured on a side stream), one event pair around the replays."""
    import torch

    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            for _ in range(GRAPH_LAUNCHES):
                launch_on(side)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    reps = max(1, steps // GRAPH_LAUNCHES)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / (reps * GRAPH_LAUNCHES)


def traffic_for(workload: str) -> dict | None:
    """HBM bytes per launch measured by the rocprofv3 counter passes committed under
    profiles/ (not by this run), with where they came from and whether the attention
    source they were measured on is the one built now."""
    path = os.path.join(ROOT, "profiles", f"{workload}_traffic.json")
    if not os.path.exists(path):
        return None
    rec = json.load(open(path))
    src = os.path.join(ROOT, "raya_amd", "csrc", "attention.hip")
    sha = hashlib.sha256(open(src, "rb").read()).hexdigest()[:16]
    return {"bytes": rec.get("hbm_bytes_per_launch"),
            "source": f"profiles/{workload}_traffic.json (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)",
            "kernel_source_sha16": rec.get("attention_source_sha16"),
            "matches_this_build": rec.get("attention_source_sha16") == sha}


def roofline(flops: int, nbytes: int, seconds: float, workload: str) -> dict:
    """The bound the arithmetic intensity reaches first (ridge 157.3 TFLOP/s / 8 TB/s)."""
    t = traffic_for(workload)
    extra = {"traffic": t["bytes"] if t else None,
             "traffic_source": ({k: t[k] for k in ("source", "kernel_source_sha16", "matches_this_build")}
                                if t else None)}
    if flops / nbytes < PEAK_FP32_MFMA_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9):
        achieved = nbytes / seconds / 1e9
        return {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": achieved / PEAK_HBM_GBS, **extra}
    achieved = flops / seconds / 1e12
    return {"bound": "mfma", "achieved": achieved, "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s",
            "frac": achieved / PEAK_FP32_MFMA_TFLOPS, **extra}


# --- CPU baselines ------------------------------------------------------------------------------

def cpu_tiled(qkv, valid, wl, budget_s: float):
    """The reference's Tiled algorithm (AVX2+FMA when present) on this host's cores, whole
    workload, median of repeated runs; plus one thread on the first sequences."""
    import oracle

    b, h, s, d = wl["batch"], wl["heads"], wl["seq"], wl["head_dim"]
    kind, block = oracle_mask(wl["mask"])
    threads = cpu_threads()
    q, k, v = qkv
    backend = 1 if oracle.cpu_has_avx2_fma() else 0
    flops, _ = algorithmic(valid, h, d, s, wl["mask"])
    times, out, used = [], None, 0
    t_end = time.perf_counter() + budget_s
    while True:
        t0 = time.perf_counter()
        out, used = oracle.tiled_attend_batched(q, k, v, kind, valid, 0.125, block=block,
                                                threads=threads, backend=backend, out=out)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end or len(times) >= 50:
            break
    med = statistics.median(times)
    n1 = max(1, min(b, 4))
    f1, _ = algorithmic(valid[:n1], h, d, s, wl["mask"])
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


def cpu_naive_t1(qkv, valid, wl) -> dict:
    """The reference's Naive kernel (sequential f32, one thread) on the whole workload."""
    import oracle

    kind, block = oracle_mask(wl["mask"])
    flops, _ = algorithmic(valid, wl["heads"], wl["head_dim"], wl["seq"], wl["mask"])
    t0 = time.perf_counter()
    oracle.naive_attend_batched(*qkv, kind, valid, 0.125, block=block)
    dt = time.perf_counter() - t0
    return {"naive_t1_value": flops / dt / 1e12,
            "naive_t1_sample": f"whole workload, Naive restatement, 1 thread, {dt * 1e3:.1f} ms"}


def f64_errors(qkv, valid, wl, got, cpu_out) -> dict:
    """Distance of the GPU's and the CPU port's fp32 outputs from a float64 evaluation of the
    same attention (torch on the host), on the first sequence, max-abs and RMS.  On the x20
    outliers a score's fp32 rounding depends on the order its 64 products are summed in
    (one chain of 64 fused steps on the matrix core, 16 chains of 4 in the AVX2 kernel), and
    near-tied outlier scores turn that into max-abs differences of 1e-4 and more between any
    two fp32 evaluations; the RMS says how close each is overall.  Block masks only
    (BlockDiag(b) and Block3: each 128- or b-row query block against its key blocks)."""
    import numpy as np
    import torch

    q, k, v = (torch.from_numpy(x[0].astype(np.float64)) for x in qkv)
    vl = int(valid[0])
    kind = wl["mask"][0]
    blk = wl["mask"][1] if kind == "block_diag" else 128
    exact = np.zeros((q.shape[0], vl, q.shape[2]), np.float64)
    for q0 in range(0, vl, blk):
        q1 = min(q0 + blk, vl)
        lo, hi = (q0, q1) if kind == "block_diag" else (max(q0 - 128, 0), min(q0 + 256, vl))
        s_ = torch.bmm(q[:, q0:q1], k[:, lo:hi].transpose(1, 2).contiguous()) * 0.125
        exact[:, q0:q1] = torch.bmm(torch.softmax(s_, dim=-1), v[:, lo:hi]).numpy()
    e_gpu, e_cpu = np.abs(got[0, :, :vl] - exact), np.abs(cpu_out[0, :, :vl] - exact)
    return {"f64_sample": "sequence 0, every head, against torch float64 on the host",
            "gpu_vs_f64_max_abs": float(e_gpu.max()), "cpu_vs_f64_max_abs": float(e_cpu.max()),
            "gpu_vs_f64_rms": float(np.sqrt((e_gpu ** 2).mean())),
            "cpu_vs_f64_rms": float(np.sqrt((e_cpu ** 2).mean()))}


# --- one attention workload ---------------------------------------------------------------------

def attention_line(name: str, steps: int, warmup: int, cpu_seconds: float, cpu: bool) -> dict:
    """Times workload `name` on cuda:0 (and its CPU baseline); the keys of a bench line."""
    import numpy as np
    import torch

    import raya_amd as R

    wl = WORKLOADS[name]
    b, h, s, d = wl["batch"], wl["heads"], wl["seq"], wl["head_dim"]
    lo, hi = wl["valid"]
    log(f"{name}: inputs")
    qkv, valid = cached_inputs(wl)
    dev = torch.device("cuda:0")
    q, k, v = (torch.from_numpy(x).to(dev) for x in qkv)
    vl = torch.from_numpy(valid).to(dev)
    out = torch.empty_like(q)
    # Launches alternate between INPUT_SETS copies of the inputs and outputs, so no
    # launch finds the previous launch's bytes in the 256 MB memory-side cache in
    # front of HBM: every launch reads its inputs from HBM.
    sets = [(q, k, v, out)] + [(q.clone(), k.clone(), v.clone(), torch.empty_like(q))
                               for _ in range(INPUT_SETS - 1)]
    turn = [0]
    kernel = R.HipAttention()
    mask = kernel_mask(wl["mask"])
    stream = torch.cuda.current_stream(dev)
    flops, nbytes = algorithmic(valid, h, d, s, wl["mask"])

    def launch_on(st):
        qs, ks, vs, os_ = sets[turn[0] % INPUT_SETS]
        turn[0] += 1
        kernel.attend_batched(qs, ks, vs, os_, vl, mask, stream=st)

    def step():
        launch_on(stream)

    log(f"{name}: ramp {RAMP_MS:.0f} ms, warmup {warmup}, timing {steps} steps")
    ramped = ramp(step)
    for _ in range(warmup):
        step()
    kern_s, wall_s = time_eager(step, steps, stream)
    line = {
        "config": {"workload": name, "batch": b, "heads": h, "seq": s, "head_dim": d,
                   "mask": mask_name(wl["mask"]),
                   "valid_len": f"uniform [{lo}, {hi}]" if lo != hi else f"{lo} (no padding)",
                   "inputs": ("xorshift U[-1, 1], seeds 42/43/44" if wl["data"] == "xorshift"
                              else "N(0, 1), SplitMix64 + Box-Muller"),
                   "outliers": "1% x20" if wl["outliers"] else "none", "flop_per_step": flops,
                   "bytes_per_step": nbytes, "input_sets": INPUT_SETS},
        "ramp": {"ms": RAMP_MS, "launches": ramped},
        "ms_per_step": wall_s * 1e3,
        "kernel_ms": kern_s * 1e3,
        "timing": f"one event pair around {steps} back-to-back launches",
    }
    if kern_s * 1e3 >= GRAPH_BELOW_MS:
        per = sorted(time_per_launch(step, steps, stream))
        line["per_launch_ms"] = {"median": statistics.median(per), "p10": per[len(per) // 10],
                                 "p90": per[(9 * len(per)) // 10], "launches": len(per),
                                 "timing": "an event pair per launch, a second run after the one above; "
                                           "each launch also carries the marker between launches (~2 us)"}
    if kern_s * 1e3 < GRAPH_BELOW_MS:
        g_s = time_graph(launch_on, steps, stream)
        line["eager_kernel_ms"] = line["kernel_ms"]
        line["kernel_ms"] = g_s * 1e3
        line["timing"] = (f"replays of a HIP graph of {GRAPH_LAUNCHES} launches, one event pair; "
                          f"eager launches are host-bound ({wall_s * 1e6:.1f} us of host time per launch)")
        kern_s = g_s
    line["kernel_tflops"] = flops / kern_s / 1e12
    line["mfma_frac"] = line["kernel_tflops"] / PEAK_FP32_MFMA_TFLOPS
    line["roofline"] = roofline(flops, nbytes, kern_s, name)
    if cpu:
        log(f"{name}: cpu baseline")
        cpu_out, cb = cpu_tiled(qkv, valid, wl, cpu_seconds)
        if name in NAIVE_T1:
            cb.update(cpu_naive_t1(qkv, valid, wl))
        got = out.cpu().numpy()
        for other in sets[1:]:  # every copy received the same outputs
            if not torch.equal(other[3], out):
                raise RuntimeError(f"{name}: the input copies gave different outputs")
        cb["gpu_vs_cpu_max_abs"] = max(float(np.abs(got[i, :, : valid[i]] - cpu_out[i, :, : valid[i]]).max())
                                       for i in range(b))
        if wl["outliers"] and wl["mask"][0] in ("block_diag", "block3"):
            cb.update(f64_errors(qkv, valid, wl, got, cpu_out))
        line["cpu_baseline"] = cb
    line["_tensors"] = (q, k, v, out, vl, mask, stream)
    return line


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
            # one sequence per call, as raya predict runs: end-to-end latency
            res["predict_latency"] = [{k: r[k] for k in ("tokens", "p50_ms", "p90_ms", "calls")}
                                      for r in predict_rows(m, [512, 2048, 4096], 20, 3, 30.0)]
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
    HBM: K back-to-back launches per shape bracketed by one event pair on the launch stream,
    after RAMP_MS of back-to-back launches and every shape's warm-up launches."""
    import torch

    import raya_amd as R
    from raya_amd import _capi as C

    g = R.HipGemm()
    stream = torch.cuda.current_stream()
    gen = torch.Generator(device="cuda").manual_seed(1000 * 4 + 7)
    res = {"m": GEMM_M, "steps": steps, "warmup": warmup, "shapes": {}}
    steps_of, operands = {}, {}
    for name, n, k, epi in GEMM_SHAPES:
        rows = 2 * n if epi == "geglu" else n
        a = torch.randn(GEMM_M, k, device="cuda", generator=gen)
        b = 0.02 * torch.randn(rows, k, device="cuda", generator=gen)
        operands[name] = (a, b)
        out = torch.randn(GEMM_M, n, device="cuda", generator=gen)
        act = C.RAYA_EPI_GEGLU if epi == "geglu" else C.RAYA_EPI_NONE
        resid = out if epi == "residual" else None
        steps_of[name] = (lambda a=a, b=b, out=out, act=act, resid=resid:
                          g.matmul_nt_device(out, a, b, activation=act, residual=resid, stream=stream))
    # From idle (as with --gemm-only) the clock needs tens of milliseconds of work to rise.
    ramp(steps_of[GEMM_SHAPES[0][0]])
    for _ in range(warmup):
        for step in steps_of.values():
            step()

    def timed(step) -> float:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    for name, n, k, epi in GEMM_SHAPES:
        ms = timed(steps_of[name])
        flops = 2.0 * GEMM_M * (2 * n if epi == "geglu" else n) * k
        res["shapes"][name] = {"n_out": n, "k": k, "epilogue": epi, "ms": ms,
                               "tflops": flops / ms / 1e9,
                               "mfma_frac": flops / ms / 1e9 / PEAK_FP32_MFMA_TFLOPS}
    # The same products without epilogues, beside the vendor library's fp32 GEMM (torch.mm,
    # hipBLASLt / rocBLAS, TF32 off) on the same operands: a reference point, not a
    # component of any line.
    tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        plain = {}
        for name, n, k, epi in GEMM_SHAPES:
            rows = 2 * n if epi == "geglu" else n
            a, b = operands[name]
            out = torch.empty(GEMM_M, rows, device="cuda")
            ours = lambda a=a, b=b, out=out: g.matmul_nt_device(out, a, b, stream=stream)  # noqa: E731
            vendor = lambda a=a, b=b, out=out: torch.mm(a, b.t(), out=out)  # noqa: E731
            for _ in range(warmup):
                ours()
                vendor()
            flops = 2.0 * GEMM_M * rows * k
            # alternating, twice each, the faster of each pair
            t = [timed(ours), timed(vendor), timed(ours), timed(vendor)]
            t_ours, t_vendor = min(t[0], t[2]), min(t[1], t[3])
            plain[f"{rows}x{k}"] = {"ms": t_ours, "tflops": flops / t_ours / 1e9,
                                    "torch_mm_ms": t_vendor, "torch_mm_tflops": flops / t_vendor / 1e9}
        res["plain_vs_torch_mm"] = plain
    finally:
        torch.backends.cuda.matmul.allow_tf32 = tf32
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



def bench_postln(steps: int, warmup: int, cpu_seconds: float, cpu: bool) -> dict:
    """One post-LN layer (raya_postln_layer_forward: QKV GEMM + bias, attention reading the
    packed qkv, Wo GEMM + bias + residual, LayerNorm, W1 GEMM + bias + GELU, W2 GEMM + bias +
    residual, LayerNorm) on the whole batch with its inputs resident in HBM: K back-to-back
    forwards bracketed by one event pair on the launch stream."""
    import numpy as np
    import torch

    from raya_amd import Mask
    from raya_amd.layers import PostLNLayer

    spec = POSTLN_LAYER
    x, valid, w = postln_inputs(spec)
    layer = PostLNLayer({k: torch.from_numpy(v).cuda() for k, v in w.items()}, spec["heads"], spec["eps"],
                        Mask.block_diag(spec["block"]))
    xd, vd = torch.from_numpy(x).cuda(), torch.from_numpy(valid).cuda()
    out = torch.empty_like(xd)
    stream = torch.cuda.current_stream()
    log(f"post-LN layer: warmup {warmup}, timing {steps} forwards (B={spec['batch']}, L={spec['seq']})")
    # The inputs are generated on the host first, so the GPU starts this leg from idle:
    # ramp its clock like the attention lines before the warm-up forwards.
    n_ramp = ramp(lambda: layer.forward(xd, vd, out, stream=stream))
    for _ in range(warmup):
        layer.forward(xd, vd, out, stream=stream)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        layer.forward(xd, vd, out, stream=stream)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    gemm, attn = postln_flops(spec, valid)
    res = {
        "workload": spec["workload"], "batch": spec["batch"], "seq": spec["seq"], "hidden": spec["hidden"],
        "heads": spec["heads"], "ffn": spec["ffn"], "ln_eps": spec["eps"], "mask": f"block_diag({spec['block']})",
        "ms_per_layer": ms, "sequences_per_s": spec["batch"] / (ms / 1e3), "flop_per_layer": gemm + attn,
        "tflops": (gemm + attn) / (ms / 1e3) / 1e12,
        "mfma_frac": (gemm + attn) / (ms / 1e3) / 1e12 / PEAK_FP32_MFMA_TFLOPS,
        "timing": f"{steps} back-to-back forwards between two events on the launch stream, after "
                  f"{n_ramp} ramp and {warmup} warm-up forwards",
        "weights": "N(0, 0.02), zero biases, LayerNorm gain 1 and shift 0; x N(0, 1)",
    }
    if cpu:
        from oracle import forward as F

        import oracle

        got = out.cpu().numpy()
        F.GEMM_THREADS = cpu_threads()
        done, diff, t0 = 0, 0.0, time.perf_counter()
        while done < spec["batch"]:
            want = F.postln_layer(x[done], int(valid[done]), w, spec["heads"], spec["eps"], oracle.MASK_BLOCKDIAG,
                                  spec["block"])
            diff = max(diff, float(np.abs(got[done] - want).max()))
            done += 1
            if time.perf_counter() - t0 > cpu_seconds:
                break
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": done / dt, "unit": "sequences/s", "cores": F.GEMM_THREADS, "kind": "port",
                               "sample": f"first {done} sequences of the batch, one at a time, {dt:.1f} s",
                               "gpu_vs_cpu_max_abs": diff}
    return res


# --- the reference bench's document -------------------------------------------------------------

def refbench(out_path: str | None, samples: int, naive_samples: int, cpu: bool) -> dict:
    """benches/local_attention.rs:89-172 with this GPU's rows beside the CPU rows: 16 heads,
    D=64, L in {2048, 4096, 8192}, Block3 and Window64, xorshift inputs (seed 42); Naive on
    one thread, Tiled on one thread and on all threads; mean and standard deviation over
    `samples` timings (GPU: each the mean of back-to-back launches over >= 2 ms)."""
    import numpy as np
    import torch

    import oracle
    import raya_amd as R
    from raya_amd import meta

    threads = cpu_threads()
    backend = 1 if oracle.cpu_has_avx2_fma() else 0
    backend_name = "avx2" if backend == 1 else "portable"
    kernel = R.HipAttention()
    rows = []
    for seq in (2048, 4096, 8192):
        for m in ("block3", "window64"):
            name = f"refbench_h16_l{seq}_d64_{m}"
            wl = WORKLOADS[name]
            qkv, valid = attention_inputs(wl)
            dev = torch.device("cuda:0")
            q, k, v = (torch.from_numpy(x).to(dev) for x in qkv)
            vl = torch.from_numpy(valid).to(dev)
            out = torch.empty_like(q)
            mask = kernel_mask(wl["mask"])
            stream = torch.cuda.current_stream(dev)

            def step():
                kernel.attend_batched(q, k, v, out, vl, mask, stream=stream)

            ramp(step)
            per = max(10, int(2e-3 / max(time_eager(step, 10, stream)[0], 1e-7)))
            ts = [time_eager(step, per, stream)[0] * 1e3 for _ in range(samples)]
            st = kernel.attend_batched_stages(q, k, v, torch.empty_like(q), vl, mask, stream=stream)
            pct = st.percentages()
            base = {"mask": m, "seq": seq, "heads": 16, "head_dim": 64}
            rows.append({"kernel": "hip", **base, "backend": "gfx950", "threads": 0,
                         "device": torch.cuda.get_device_name(0),
                         "mean_ms": statistics.mean(ts), "stddev_ms": statistics.stdev(ts), "samples": samples,
                         "stages": {"qk_pct": pct[0], "softmax_pct": pct[1], "pv_pct": pct[2]}})
            log(f"refbench {name}: gpu {rows[-1]['mean_ms']:.4f} ms")
            if not cpu:
                continue
            kind, block = oracle_mask(wl["mask"])
            cq, ck, cv = qkv
            for t in sorted({1, threads}):
                tt = []
                for _ in range(samples):
                    t0 = time.perf_counter()
                    oracle.tiled_attend_batched(cq, ck, cv, kind, valid, 0.125, block=block, threads=t,
                                                backend=backend)
                    tt.append((time.perf_counter() - t0) * 1e3)
                rows.append({"kernel": "tiled", **base, "backend": backend_name, "threads": t,
                             "mean_ms": statistics.mean(tt), "stddev_ms": statistics.stdev(tt),
                             "samples": samples})
            tn = []
            for _ in range(naive_samples):
                t0 = time.perf_counter()
                oracle.naive_attend(cq[0], ck[0], cv[0], kind, int(valid[0]), 0.125, block=block)
                tn.append((time.perf_counter() - t0) * 1e3)
            rows.append({"kernel": "naive", **base, "backend": "scalar", "threads": 1,
                         "mean_ms": statistics.mean(tn),
                         "stddev_ms": statistics.stdev(tn) if len(tn) > 1 else 0.0, "samples": naive_samples})
            log(f"refbench {name}: cpu rows done")
            del q, k, v, out
            torch.cuda.empty_cache()
    md = meta.collect(threads=threads)
    md["backend"] = backend_name if cpu else md["backend"]
    doc = {"label": md["label"], "metadata": md, "results": rows}
    if out_path is None:
        out_path = os.path.join("results", "kernel-bench", md["timestamp"].replace(":", "-") + ".json")
    os.makedirs(os.path.dirname(os.path.abspath(out_path)), exist_ok=True)
    with open(out_path, "w") as f:
        json.dump(doc, f, indent=1)
    log(f"wrote {out_path}")
    return doc


def predict_rows(m, tokens: list[int], repeats: int, warmup: int, cap_s: float) -> list[dict]:
    """p50/p90 of end-to-end predicts of one sequence of each length on a loaded model (see
    predict_bench), with the forward's per-component split."""
    import numpy as np

    from raya_amd import synth

    info = m.info
    rows = []
    for n in tokens:
        if n > info["max_position_embeddings"]:
            rows.append({"tokens": n, "skipped": f"past max_position_embeddings "
                                                 f"{info['max_position_embeddings']}"})
            continue
        ids = (synth.uniform(synth.workload_seed(4, 20), n) * (info["vocab_size"] - 1)).astype(np.uint32)
        ids = ids.reshape(1, n)
        ids[0, 0] = 101  # the [CLS] id the encoder workload starts with
        valid = np.array([n], np.uint64)
        pos = np.array([[1, 2]], np.uint64)
        mask = np.ones((1, 2), np.uint8)
        qtype = np.zeros(1, np.uint64)
        log(f"predict: {n} tokens, warmup {warmup}, {repeats} calls")
        for _ in range(warmup):
            m.forward_batch(ids, valid, pos, mask, qtype)
        lat, capped, t_start = [], False, time.perf_counter()
        for _ in range(repeats):
            t1 = time.perf_counter()
            out = m.forward_batch(ids, valid, pos, mask, qtype)
            lat.append((time.perf_counter() - t1) * 1e3)
            if time.perf_counter() - t_start > cap_s:
                capped = True
                break
        m.set_profiling(1)
        try:
            m.forward_batch(ids, valid, pos, mask, qtype)
            parts = m.stage_times()
        finally:
            m.set_profiling(0)
        lat.sort()
        rows.append({
            "tokens": n, "calls": len(lat), "p50_ms": lat[len(lat) // 2],
            "p90_ms": lat[min(len(lat) - 1, (9 * len(lat)) // 10)], "mean_ms": statistics.mean(lat),
            "time_cap_hit": capped, "components_ms": {name: ms for name, ms in parts},
            "probabilities": [float(x) for x in out.probabilities[0]],
        })
    return rows


def predict_bench(tokens: list[int], repeats: int, warmup: int, cap_s: float) -> dict:
    """End-to-end predict latency of the decision model for one sequence of each length,
    as `raya bench` is specified (specs/008-bench-harness/spec.md:19-31, FR-001/FR-002): the
    bench's synthetic 12-layer checkpoint loaded once (load time reported apart), a fixed
    synthetic token input with one question (markers at positions 1 and 2, qtype 0), p50 and
    p90 over `repeats` calls after `warmup`, each call from host arrays to host outputs, the
    per-component split (embedding, each encoder layer, final norm, head) from the forward's
    own stage spans, peak RSS and whether the time cap cut a length short.  The reference's
    output-parity gate (FR-003) compares with saved Laya outputs, which this repository does
    not hold; the forward's parity is held by the test suite instead."""
    import resource
    import shutil
    import tempfile

    from raya_amd import checkpoint, model as M

    tmp = tempfile.mkdtemp(prefix="raya_ckpt_")
    rows = []
    try:
        log("predict: writing the synthetic checkpoint")
        checkpoint.write_synthetic(tmp, seed=ENCODER_WEIGHT_SEED)
        t0 = time.perf_counter()
        m = M.Model.load(tmp)
        load_ms = (time.perf_counter() - t0) * 1e3
        rows = predict_rows(m, tokens, repeats, warmup, cap_s)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return {
        "bench": "predict latency (raya bench, specs/008-bench-harness)", "model": "12-layer ModernBERT-base "
        "width synthetic checkpoint (N(0, 0.02) weights, vocab 30,522, max positions 4,096)",
        "model_load_ms": load_ms, "warmup": warmup, "repeats": repeats, "time_cap_s": cap_s,
        "peak_rss_mb": resource.getrusage(resource.RUSAGE_SELF).ru_maxrss / 1024.0,
        "attention_kernel": "hip-gfx950", "results": rows,
    }


def bench_host_slice(calls: int, warmup: int) -> dict:
    """raya_attend through HipAttention.attend on host (numpy) slices, as a Network holding
    the kernel would call it per layer (crates/raya-kernels/benches/local_attention.rs:102,
    :125 time the trait the same way): each call copies q, k, v to the device, launches and
    copies out back, then synchronises.  Median and p90 over `calls` calls, and the same
    launch on device-resident inputs (graph replays) beside it."""
    import numpy as np

    import raya_amd as R

    kernel = R.HipAttention()
    res = {}
    for name in HOST_SLICE:
        wl = WORKLOADS[name]
        (q, k, v), valid = attention_inputs(wl)
        h, s_, d = wl["heads"], wl["seq"], wl["head_dim"]
        q, k, v = (np.ascontiguousarray(x[0]).ravel() for x in (q, k, v))
        out = np.empty_like(q)
        shape = R.AttnShape(h, s_, d)
        params = R.AttnParams.new(kernel_mask(wl["mask"]), int(valid[0]), d)
        log(f"host-slice attend {name}: {calls} calls")
        for _ in range(warmup):
            kernel.attend(shape, params, q, k, v, out)
        t = []
        for _ in range(calls):
            t0 = time.perf_counter()
            kernel.attend(shape, params, q, k, v, out)
            t.append(time.perf_counter() - t0)
        t.sort()
        moved = 4 * 4 * q.size  # q, k, v to the device, out back
        res[name] = {"p50_ms": statistics.median(t) * 1e3, "p90_ms": t[(9 * len(t)) // 10] * 1e3,
                     "calls": calls, "bytes_moved": moved,
                     "host_link_gbs": moved / statistics.median(t) / 1e9}
    return res


def _r(x, digits: int = 4):
    """x rounded to `digits` significant digits (floats only)."""
    if isinstance(x, float):
        return float(f"{x:.{digits}g}")
    return x


def compact(result: dict) -> dict:
    """The line printed to stdout: the contract's keys, the headline's figures, and a `lines`
    map (one short entry per measured workload) last, small enough that a reader keeping the
    tail of stdout sees all of it.  The full document goes to --detail-out."""
    keep = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
            "scaling", "vs_baseline", "dtype", "data")
    out = {k: _r(result[k]) if k in ("value", "ms_per_step") else result[k] for k in keep}
    c = result["config"]
    out["config"] = {k: c[k] for k in ("workload", "batch", "heads", "seq", "head_dim", "mask", "valid_len",
                                       "flop_per_step", "bytes_per_step")}
    out["kernel_ms"] = _r(result["kernel_ms"])
    if "per_launch_ms" in result:
        out["per_launch_median_ms"] = _r(result["per_launch_ms"]["median"])
    out["kernel_tflops"] = _r(result["kernel_tflops"])
    out["mfma_frac"] = _r(result["mfma_frac"])
    rf = result["roofline"]
    out["roofline"] = {k: _r(rf[k]) for k in ("bound", "achieved", "peak", "unit", "frac", "traffic")}
    if "cpu_baseline" in result:
        cb = result["cpu_baseline"]
        out["cpu_baseline"] = {k: _r(cb[k]) for k in ("value", "unit", "cores", "kind", "sample", "t1_value",
                                                      "gpu_vs_cpu_max_abs") if k in cb}
    if "stage_split" in result:
        ss = result["stage_split"]
        out["stage_split_pct"] = {k.replace("_pct", "").replace("_of_wave_cycles", ""): _r(v, 3)
                                  for k, v in ss.items() if k.endswith("pct")}
    m = result.get("meta", {})
    out["meta"] = {"label": m.get("label"), "commit": str(m.get("git_commit", ""))[:12],
                   "cpu": m.get("cpu_model"), "threads": m.get("threads")}

    lines = {}
    for name, ln in result.get("workloads", {}).items():
        e = {"kernel_ms": _r(ln["kernel_ms"]), "tflops": _r(ln["kernel_tflops"]),
             "bound": ln["roofline"]["bound"], "frac": _r(ln["roofline"]["frac"], 3)}
        if "cpu_baseline" in ln:
            e["cpu_tflops"] = _r(ln["cpu_baseline"]["value"])
            e["max_abs"] = _r(ln["cpu_baseline"]["gpu_vs_cpu_max_abs"], 2)
            if "gpu_vs_f64_max_abs" in ln["cpu_baseline"]:  # [GPU, CPU port] against float64
                lb = ln["cpu_baseline"]
                e["f64_max_abs"] = [_r(lb["gpu_vs_f64_max_abs"], 2), _r(lb["cpu_vs_f64_max_abs"], 2)]
                e["f64_rms"] = [_r(lb["gpu_vs_f64_rms"], 2), _r(lb["cpu_vs_f64_rms"], 2)]
            if "naive_t1_value" in ln["cpu_baseline"]:
                e["cpu_naive_t1_tflops"] = _r(ln["cpu_baseline"]["naive_t1_value"])
        lines[name] = e
    enc = result.get("encoder")
    if enc:
        e = {"seq_per_s": _r(enc["sequences_per_s"]), "tflops": _r(enc["tflops"]),
             "mfma_frac": _r(enc["mfma_frac"], 3)}
        if "cpu_baseline" in enc:
            e["cpu_seq_per_s"] = _r(enc["cpu_baseline"]["value"])
            e["act_logits_max_abs"] = _r(enc["cpu_baseline"]["gpu_vs_cpu_act_logits_max_abs"], 2)
        lines[enc["workload"]] = e
        for r in enc.get("predict_latency", []):
            lines[f"predict_l{r['tokens']}"] = {"p50_ms": _r(r["p50_ms"]), "p90_ms": _r(r["p90_ms"])}
    lay = result.get("encoder_layer")
    if lay:
        lines[lay["workload"]] = {"seq_per_s": _r(lay["sequences_per_s"]), "tflops": _r(lay["tflops"]),
                                  "mfma_frac": _r(lay["mfma_frac"], 3)}
    pl = result.get("postln_layer")
    if pl:
        e = {"seq_per_s": _r(pl["sequences_per_s"]), "tflops": _r(pl["tflops"]), "mfma_frac": _r(pl["mfma_frac"], 3)}
        if "cpu_baseline" in pl:
            e["cpu_seq_per_s"] = _r(pl["cpu_baseline"]["value"])
            e["max_abs"] = _r(pl["cpu_baseline"]["gpu_vs_cpu_max_abs"], 2)
        lines[pl["workload"]] = e
    gm = result.get("encoder_gemms")
    if gm:
        for shp, v in gm.get("plain_vs_torch_mm", {}).items():
            lines[f"gemm_{shp}"] = {"tflops": _r(v["tflops"]), "torch_mm_tflops": _r(v["torch_mm_tflops"])}
    for name, v in result.get("host_slice_attend", {}).items():
        lines[f"host_slice_{name}"] = {"p50_ms": _r(v["p50_ms"]), "p90_ms": _r(v["p90_ms"])}
    out["lines"] = lines
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default=DEFAULT, choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-seconds", type=float, default=5.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-encoder", action="store_true", help="skip the encoder forward leg")
    ap.add_argument("--no-sublines", action="store_true", help="skip the other attention workloads")
    ap.add_argument("--encoder-steps", type=int, default=10)
    ap.add_argument("--encoder-warmup", type=int, default=2)
    ap.add_argument("--gemm-only", action="store_true",
                    help="time only the encoder's four GEMM shapes and print their line")
    ap.add_argument("--refbench", action="store_true",
                    help="write the reference bench's result document instead of the bench line")
    ap.add_argument("--refbench-out", default=None)
    ap.add_argument("--refbench-samples", type=int, default=10)
    ap.add_argument("--refbench-naive-samples", type=int, default=3)
    ap.add_argument("--predict", action="store_true",
                    help="print the predict-latency document (raya bench) instead of the bench line")
    ap.add_argument("--predict-tokens", default="512,2048,4096")
    ap.add_argument("--predict-repeats", type=int, default=20)
    ap.add_argument("--predict-warmup", type=int, default=3)
    ap.add_argument("--predict-cap-s", type=float, default=60.0)
    ap.add_argument("--detail-out", default=None,
                    help="also write the full bench document (every field of every leg) to this path")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (got --gpus {args.gpus})",
              file=sys.stderr)
        return 2

    import torch

    if args.refbench:
        doc = refbench(args.refbench_out, args.refbench_samples, args.refbench_naive_samples,
                       cpu=not args.no_cpu_baseline)
        print(json.dumps({"refbench_rows": len(doc["results"]), "label": doc["label"],
                          "gpu_rows": [{k: r[k] for k in ("mask", "seq", "mean_ms", "stddev_ms")}
                                       for r in doc["results"] if r["kernel"] == "hip"]}), flush=True)
        return 0

    if args.predict:
        doc = predict_bench([int(x) for x in args.predict_tokens.split(",")], args.predict_repeats,
                            args.predict_warmup, args.predict_cap_s)
        print(json.dumps(doc), flush=True)
        return 0

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

    head = attention_line(args.workload, args.steps, args.warmup, args.cpu_seconds,
                          cpu=not args.no_cpu_baseline)
    q, k, v, out, vl, mask, stream = head.pop("_tensors")
    flops = head["config"]["flop_per_step"]
    result = {
        "metric": METRIC,
        "value": flops / (head["ms_per_step"] / 1e3) / 1e12,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        **{key: head[key] for key in head if key not in ("ms_per_step",)},
    }

    # One launch of the instrumented kernel after the timed region: where the
    # waves' cycles go (the reference's stage-timing split, tiled/stages.rs).
    import raya_amd as R

    st = R.HipAttention().attend_batched_stages(q, k, v, out, vl, mask, stream=stream)
    pct = st.percentages()
    waves = st.qk + st.softmax + st.pv + st.load_wait
    result["stage_split"] = {
        "qk_pct": pct[0], "softmax_pct": pct[1], "pv_pct": pct[2],
        "load_wait_of_wave_cycles_pct": 100.0 * st.load_wait / waves, "tiles": st.tiles,
        "source": "one instrumented launch after the timed region; shares of per-wave shader "
                  "clock cycles (qk/softmax/pv as in the reference's StageTimes::percentages)"}
    del q, k, v, out
    torch.cuda.empty_cache()

    # BenchMetadata (crates/raya-kernels/src/meta.rs): host, GPU and build; threads is
    # the CPU baseline's worker count.
    from raya_amd import meta

    result["meta"] = meta.collect(threads=0 if args.no_cpu_baseline else cpu_threads())

    if args.workload == DEFAULT and not args.no_sublines:
        subs = {}
        for name in SUBLINES:
            line = attention_line(name, args.steps, args.warmup, min(args.cpu_seconds, 2.0),
                                  cpu=not args.no_cpu_baseline)
            line.pop("_tensors")
            subs[name] = line
            torch.cuda.empty_cache()
        result["workloads"] = subs
    if args.workload == DEFAULT and not args.no_encoder:
        enc = bench_encoder(args.encoder_steps, args.encoder_warmup, args.cpu_seconds,
                            cpu=not args.no_cpu_baseline)
        layer = enc.pop("layer", None)
        result["encoder"] = enc
        if layer is not None:
            result["encoder_layer"] = layer
        log("encoder gemm shapes")
        result["encoder_gemms"] = bench_gemms(20, 3)
        result["postln_layer"] = bench_postln(args.encoder_steps, args.encoder_warmup, min(args.cpu_seconds, 3.0),
                                              cpu=not args.no_cpu_baseline)
    if args.workload == DEFAULT and not args.no_sublines:
        result["host_slice_attend"] = bench_host_slice(50, 5)
    if args.detail_out:
        with open(args.detail_out, "w") as f:
            json.dump(result, f, indent=1)
    print(json.dumps(compact(result)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
