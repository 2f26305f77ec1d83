"""Builds libraya_hip.so (the HIP kernels and the C ABI) in-tree for gfx950.

    python -m raya_amd.build

Each source compiles to an object under raya_amd/_build/ (in parallel), then
one link produces raya_amd/libraya_hip.so.  hipcc cross-compiles for gfx950
without a GPU.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libraya_hip.so")
SOURCES = ["attention.hip", "gemm.hip", "encoder.hip", "capi.cpp", "model.cpp", "postln.cpp"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP backend cannot be built")


def _flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        "-I", os.path.join(ROOT, "include"), "-I", CSRC,
        # Packed FP32 instructions stay off: hipcc -O3 would otherwise emit
        # v_pk_* f32 forms from ordinary float code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-function",
    ]


def _run(cmd: list[str]) -> str:
    """First line of a command's output, or "unknown" (as build.rs's run() does)."""
    try:
        r = subprocess.run(cmd, capture_output=True, text=True, cwd=ROOT, timeout=60)
    except (OSError, subprocess.SubprocessError):
        return "unknown"
    out = r.stdout.strip()
    return out.splitlines()[0] if r.returncode == 0 and out else "unknown"


def _c_string(x: str) -> str:
    return '"' + x.replace("\\", "\\\\").replace('"', '\\"') + '"'


def _stamp() -> list[str]:
    """What raya_build_info() reports, fixed at build time like the reference's
    RAYA_RUSTC_VERSION and RAYA_GIT_COMMIT (crates/raya-kernels/build.rs)."""
    flags = " ".join(f for f in _flags() if not f.startswith("-I") and not f.startswith(ROOT)
                     and f != "-I")
    return [f"-DRAYA_BUILD_COMPILER={_c_string(_run([hipcc(), '--version']))}",
            f"-DRAYA_BUILD_COMMIT={_c_string(_run(['git', 'rev-parse', 'HEAD']))}",
            f"-DRAYA_BUILD_FLAGS={_c_string(flags)}"]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *_flags(), "-c", os.path.join(CSRC, src), "-o", obj]
    if src == "capi.cpp":
        cmd[1:1] = _stamp()
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
