"""Machine and build description stored next to benchmark results: the fields of
BenchMetadata (crates/raya-kernels/src/meta.rs:12-104), with the GPU beside the host.

Same keys and label rule as the reference; where the reference names its Rust
toolchain, this build names its HIP one: ``build_flags`` holds the hipcc flags
(the reference's ``rustflags``) and ``compiler`` the hipcc version (``rustc``).
Both, and ``git_commit``, come from the library (``raya_build_info``), fixed when
it was built, as the reference's build.rs fixes them.
"""
from __future__ import annotations

import os
import time

from . import _capi as C

# meta.rs:5-10
LABEL_TARGET = "target machine"
LABEL_CLOUD = "cloud-agent hardware, indicative only"
LABEL_UNLABELED = "unlabeled machine, indicative only"

# The kernels the library holds (what is compiled in, as the reference's
# `features` lists cargo features): the plain attention kernel, its
# stage-timing copy, and the MFMA GEMM.
FEATURES = ["hip-gfx950", "stage-timing", "mfma-f32"]


def label_for(target_env: str | None) -> str:
    """RAYA_TARGET_MACHINE: "1" is the target machine, "cloud-agent" the cloud
    label, anything else (including unset) makes no claim (meta.rs:73-86)."""
    if target_env == "1":
        return LABEL_TARGET
    if target_env == "cloud-agent":
        return LABEL_CLOUD
    return LABEL_UNLABELED


def usable_physical_cores() -> int:
    """Physical cores among the CPUs this process may run on (0 when the topology is not
    readable)."""
    cores = set()
    for cpu in os.sched_getaffinity(0):
        base = f"/sys/devices/system/cpu/cpu{cpu}/topology/"
        try:
            pkg = open(base + "physical_package_id").read().strip()
            core = open(base + "core_id").read().strip()
        except OSError:
            return 0
        cores.add((pkg, core))
    return len(cores)


def default_threads(env: str | None = None, *, use_env: bool = True) -> int:
    """default_threads (crates/raya-kernels/src/threads.rs:3-9): RAYA_THREADS if it parses
    to a positive integer (Rust's usize grammar: optional '+', decimal digits, surrounding
    whitespace trimmed), else the physical cores this process may run on, at least 1."""
    if env is None and use_env:
        env = os.environ.get("RAYA_THREADS")
    if env is not None:
        t = env.strip()
        digits = t[1:] if t.startswith("+") else t
        if digits.isascii() and digits.isdigit() and int(digits) > 0:
            return int(digits)
    return max(1, usable_physical_cores() or len(os.sched_getaffinity(0)))


def host_cpu() -> dict:
    """CPU model and core counts of this host."""
    model, cores = "unknown", set()
    try:
        phys = core = None
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "model name" and model == "unknown":
                model = val
            elif key == "physical id":
                phys = val
            elif key == "core id":
                core = val
            elif not key and phys is not None and core is not None:
                cores.add((phys, core))
                phys = core = None
        if phys is not None and core is not None:
            cores.add((phys, core))
    except OSError:
        pass
    return {"model": model, "logical_cpus_usable": len(os.sched_getaffinity(0)),
            "logical_cpus": os.cpu_count(), "physical_cores": len(cores) or None}


def build_info() -> dict:
    """raya_build_info() as a dict (arch, compiler, commit, flags)."""
    text = C.lib().raya_build_info().decode()
    return dict(line.split("=", 1) for line in text.splitlines() if "=" in line)


def gpu_info() -> dict | None:
    """Name, architecture, compute units and memory of cuda:0, or None without a GPU."""
    import torch

    if not torch.cuda.is_available():
        return None
    p = torch.cuda.get_device_properties(0)
    return {"name": p.name, "arch": getattr(p, "gcnArchName", "unknown"),
            "compute_units": p.multi_processor_count, "memory_bytes": p.total_memory,
            "hip_runtime": getattr(torch.version, "hip", None)}


def collect(threads: int, target_env: str | None = None, *, use_env: bool = True) -> dict:
    """BenchMetadata::collect (meta.rs:73-104): `threads` is the CPU worker count of
    the run; the label follows RAYA_TARGET_MACHINE unless `target_env` is given
    with use_env=False."""
    env = os.environ.get("RAYA_TARGET_MACHINE") if use_env else target_env
    host = host_cpu()
    b = build_info()
    return {
        "label": label_for(env),
        "cpu_model": host["model"],
        "logical_cpus": host["logical_cpus"],
        "physical_cpus": host["physical_cores"],
        "threads": threads,
        "features": list(FEATURES),
        "backend": C.lib().raya_attention_name().decode(),
        "build_flags": b.get("flags", "unknown"),
        "compiler": b.get("compiler", "unknown"),
        "git_commit": b.get("commit", "unknown"),
        "timestamp": f"unix:{int(time.time())}",
        "gpu": gpu_info(),
    }
