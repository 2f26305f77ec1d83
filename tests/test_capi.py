"""The C ABI on the CPU: the library loads, exports what include/*.h declares, and
rejects bad arguments with the reference's error variants before any GPU work."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

import oracle
import raya_amd as R
from raya_amd import _capi as C
from tests.conftest import ROOT


def declared_functions():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^[a-z_][\w\s\*]*?\b(raya_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_function():
    names = declared_functions()
    assert "raya_attend" in names and "raya_matmul_nt_device" in names
    lib = C.lib()
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(n for n, _, _ in C.SIGNATURES) == names


def test_names():
    assert R.HipAttention().name() == "hip-gfx950"
    assert R.HipGemm().name() == "hip-gfx950-mfma"


def _ok(shape):
    return np.zeros(shape.numel(), np.float32)


def test_bad_arguments_are_errors_not_panics():
    """crates/raya-kernels/tests/oracle.rs:34-78, through the C ABI."""
    k = R.HipAttention()
    shape = R.AttnShape(1, 4, 8)
    ok, out = _ok(shape), _ok(shape)
    p = R.AttnParams.new(R.Mask.BLOCK3, 4, 8)
    with pytest.raises(R.LengthError) as e:
        k.attend(shape, p, np.zeros(3, np.float32), ok, ok, out)
    assert e.value.name == "q" and e.value.got == 3 and e.value.expected == 32
    assert str(e.value) == "buffer `q` has length 3, expected 32"
    with pytest.raises(R.LengthError) as e:
        k.attend(shape, p, ok, ok, ok, np.zeros(3, np.float32))
    assert e.value.name == "out"
    bad = R.AttnShape(1, 4, 12)
    buf = _ok(bad)
    with pytest.raises(R.ShapeError):
        k.attend(bad, p, buf, buf, buf, _ok(bad))
    with pytest.raises(R.ShapeError):
        k.attend(shape, p.replace(valid_len=5), ok, ok, ok, out)
    with pytest.raises(R.UnsupportedError):
        k.attend(shape, p.replace(block=64), ok, ok, ok, out)
    with pytest.raises(R.ShapeError):
        k.attend(R.AttnShape(0, 4, 8), p, ok[:0], ok[:0], ok[:0], out[:0])


def test_hip_limits_are_unsupported_not_wrong():
    """head_dim 264 is past the widest instantiation (256): Unsupported, before any device work."""
    k = R.HipAttention()
    shape = R.AttnShape(1, 2, 264)
    buf = _ok(shape)
    with pytest.raises(R.UnsupportedError):
        k.attend(shape, R.AttnParams.new(R.Mask.WINDOW64, 2, 264), buf, buf, buf, _ok(shape))
    with pytest.raises(R.ShapeError):
        k.attend(R.AttnShape(1, 4, 8), R.AttnParams.new(R.Mask.block_diag(0), 4, 8),
                 *(_ok(R.AttnShape(1, 4, 8)) for _ in range(4)))


def test_empty_sequence_is_a_no_op():
    k = R.HipAttention()
    e = np.zeros(0, np.float32)
    k.attend(R.AttnShape(2, 0, 8), R.AttnParams.new(R.Mask.BLOCK3, 0, 8), e, e, e, e)


def test_gemm_length_checks_panic_like_the_reference():
    """gemm_reference.rs:24-31, gemm_edges.rs:4-24."""
    g = R.HipGemm()
    with pytest.raises(AssertionError, match="a must be"):
        g.matmul_nt(np.zeros(1, np.float32), np.ones(1, np.float32), np.ones(2, np.float32), 1, 1, 2)
    with pytest.raises(AssertionError, match="b must be"):
        g.matmul_nt(np.zeros(1, np.float32), np.ones(2, np.float32), np.ones(1, np.float32), 1, 1, 2)
    with pytest.raises(AssertionError, match="out must be"):
        g.matmul_nt(np.zeros(2, np.float32), np.ones(2, np.float32), np.ones(2, np.float32), 1, 1, 2)
    none = np.zeros(0, np.float32)
    g.matmul_nt(none, none, np.ones(2, np.float32), 0, 1, 2)
    g.matmul_nt(none, np.ones(2, np.float32), none, 1, 0, 2)
    g.matmul_nt(none, none, none, 0, 0, 0)


def test_gemm_empty_k_needs_no_gpu():
    out = np.full(6, 5.0, np.float32)
    R.HipGemm().matmul_nt(out, np.zeros(0, np.float32), np.zeros(0, np.float32), 2, 3, 0)
    assert (out == 0).all()


@pytest.mark.parametrize("mask,okind,block,window", [
    (R.Mask.BLOCK3, oracle.MASK_BLOCK3, 128, 0), (R.Mask.WINDOW64, oracle.MASK_WINDOW64, 128, 0),
    (R.Mask.FULL, oracle.MASK_FULL, 128, 0), (R.Mask.sliding(9), oracle.MASK_SLIDING, 128, 9),
    (R.Mask.block_diag(64), oracle.MASK_BLOCKDIAG, 64, 0)])
def test_host_mask_mirror_agrees_with_the_oracle(mask, okind, block, window):
    for valid in (0, 1, 130, 300):
        for i in range(0, 300, 7):
            r = mask.key_range(i, valid)
            assert (r.start, r.stop) == oracle.key_range(okind, i, valid, block=block, window=window)
            for j in range(0, 300, 13):
                assert mask.allows(i, j) == oracle.allows(okind, i, j, block=block, window=window)


def test_default_params():
    p = R.AttnParams.new(R.Mask.BLOCK3, 10, 40)
    assert p.block == 128 and p.valid_len == 10
    assert np.float32(p.scale) == np.float32(1.0) / np.sqrt(np.float32(40))


C_CLIENT = r"""
#include "raya_hip.h"
#include <stdio.h>
#include <string.h>

int main(void) {
    /* Shape errors come back as codes with the reference's text, before any GPU work. */
    raya_attn_shape shape = {0, 16, 8};
    raya_attn_params params;
    float buf[1] = {0.0f};
    int rc;
    memset(&params, 0, sizeof params);
    params.mask_kind = RAYA_MASK_FULL;
    params.scale = 1.0f;
    params.block = 128;
    rc = raya_attend(&shape, &params, buf, 0, buf, 0, buf, 0, buf, 0);
    printf("%s|%s|%d|%d|%s\n", raya_attention_name(), raya_gemm_name(), rc, raya_last_error()->code,
           raya_last_error()->message);
    return 0;
}
"""


def test_header_builds_a_plain_c_client(tmp_path):
    """include/raya_hip.h compiles as C99 and a C program links against libraya_hip.so
    (what a cgo / bindgen / build.rs consumer does)."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not found")
    src = tmp_path / "client.c"
    src.write_text(C_CLIENT)
    exe = tmp_path / "client"
    libdir = os.path.dirname(C.LIB_PATH)
    subprocess.run([gcc, "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), str(src),
                    "-L", libdir, "-lraya_hip", f"-Wl,-rpath,{libdir}", "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.strip()
    name, gemm, rc, code, msg = out.split("|", 4)
    assert (name, gemm) == ("hip-gfx950", "hip-gfx950-mfma")
    assert int(rc) == int(code) == C.RAYA_ERR_SHAPE
    assert msg.startswith("invalid shape")


def test_length_before_hip_limits():
    """validate() checks the buffer lengths right after the block (attention.rs:159-168),
    before anything the HIP kernel adds: head_dim 264 (past the kernel's 256) with a short
    `q` is a Length error, as the reference gives."""
    k = R.HipAttention()
    shape = R.AttnShape(1, 2, 264)
    buf = _ok(shape)
    with pytest.raises(R.LengthError) as e:
        k.attend(shape, R.AttnParams.new(R.Mask.WINDOW64, 2, 264), buf[:5], buf, buf, _ok(shape))
    assert (e.value.name, e.value.got, e.value.expected) == ("q", 5, 528)
    # the mask extension's own check also comes after the lengths
    s8 = R.AttnShape(1, 4, 8)
    with pytest.raises(R.LengthError):
        k.attend(s8, R.AttnParams.new(R.Mask.block_diag(0), 4, 8), _ok(s8), _ok(s8)[:1], _ok(s8), _ok(s8))


def test_numel_overflow_is_a_shape_error():
    """heads x seq x head_dim past 2^64 cannot match any buffer and must not wrap into one."""
    lib = C.lib()
    s = C.AttnShapeC(1 << 32, 1 << 16, 1 << 16)
    p = C.AttnParamsC(C.RAYA_MASK_FULL, 1.0, 0, 128, 0)
    buf = (ctypes.c_float * 1)()
    # the product is 2^64, which wraps to 0: zero-length buffers would "match" it
    rc = lib.raya_attend(ctypes.byref(s), ctypes.byref(p), buf, 0, buf, 0, buf, 0, buf, 0)
    assert rc == C.RAYA_ERR_SHAPE
    assert "overflows" in C.last_error().message.decode()
    assert C.last_error().code == rc


def test_gemm_device_arguments_are_checked_before_any_launch():
    """matmul_nt_device rejects another dtype, a short bias, a residual of the wrong shape
    and host tensors before a pointer reaches the C ABI."""
    import torch

    g = R.HipGemm()
    m, n, k = 4, 3, 8
    a, b, out = torch.zeros(m, k), torch.zeros(n, k), torch.zeros(m, n)
    with pytest.raises(TypeError, match="float32"):
        g.matmul_nt_device(out, a.double(), b)
    with pytest.raises(TypeError, match="float32"):
        g.matmul_nt_device(out, a, b.half())
    with pytest.raises(TypeError, match="float32"):
        g.matmul_nt_device(out, a, b, bias=torch.zeros(n, dtype=torch.float64))
    with pytest.raises(R.ShapeError, match="bias"):
        g.matmul_nt_device(out, a, b, bias=torch.zeros(n - 1))
    with pytest.raises(R.ShapeError, match="bias"):  # GeGLU needs 2n bias entries
        g.matmul_nt_device(out, a, torch.zeros(2 * n, k), bias=torch.zeros(n),
                           activation=C.RAYA_EPI_GEGLU)
    with pytest.raises(R.ShapeError, match="residual"):
        g.matmul_nt_device(out, a, b, residual=torch.zeros(m, n + 1))
    with pytest.raises(R.ShapeError, match="residual"):
        g.matmul_nt_device(out, a, b, residual=torch.zeros(n, m).t())
    with pytest.raises(TypeError, match="GPU"):  # host tensors never reach the library
        g.matmul_nt_device(out, a, b, bias=torch.zeros(n), residual=torch.zeros(m, n))


def test_attend_batched_layouts_must_stay_inside_their_tensors():
    """With explicit strides, a layout that reaches past a tensor's storage is a Shape
    error before any pointer reaches the library; one that fits gets past that check
    (here to the host-tensor check that follows it)."""
    import torch

    att = R.HipAttention()
    b, h, s, d = 2, 3, 5, 8
    # q, k, v interleaved per row as in a packed QKV projection: [b, s, 3, h, d].
    qkv = torch.zeros(b, s, 3, h, d)
    out = torch.zeros(b, h, s, d)
    strided = (s * 3 * h * d, d, 3 * h * d)
    lay = {"shape": (b, h, s, d), "q": strided, "k": strided, "v": strided, "out": (0, 0, 0)}
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    valid = torch.full((b,), s, dtype=torch.int32)
    with pytest.raises(R.ShapeError, match="valid_len"):  # fits: stops at the GPU checks
        att.attend_batched(q, k, v, out, valid, R.Mask.BLOCK3, layouts=lay)
    too_far = dict(lay, v=(s * 3 * h * d + 4, d, 3 * h * d))  # batch stride one chunk too long
    with pytest.raises(R.ShapeError, match="layout of `v`"):
        att.attend_batched(q, k, v, out, valid, R.Mask.BLOCK3, layouts=too_far)
    with pytest.raises(R.ShapeError, match="layout of `out`"):  # dense out one row short
        att.attend_batched(q, k, v, torch.zeros(b * h * s * d - d), valid, R.Mask.BLOCK3, layouts=lay)
    with pytest.raises(R.ShapeError, match="layout of `q`"):  # a longer shape than the buffer holds
        att.attend_batched(q, k, v, out, valid, R.Mask.BLOCK3, layouts=dict(lay, shape=(b, h, s + 1, d)))


def test_postln_layer_checks_before_any_gpu_work():
    """The post-LN layer rejects bad shapes and a short workspace without touching the GPU."""
    lib = C.lib()
    desc = C.PostLNLayerC(2, 16, 64, 2, 128, C.RAYA_MASK_BLOCKDIAG, 0, 16, 1e-5)
    for name in ("wqkv", "wo", "w1", "w2", "ln1_w", "ln2_w"):
        setattr(desc, name, 256)  # never dereferenced: the checks fail first
    need = lib.raya_postln_workspace_bytes(ctypes.byref(desc))
    assert need == 2 * 16 * (6 * 64 + 128) * 4
    rc = lib.raya_postln_layer_forward(ctypes.byref(desc), 256, 256, 256, 256, need - 4, None)
    assert rc == C.RAYA_ERR_SHAPE and "workspace" in C.last_error().message.decode()
    bad = C.PostLNLayerC(2, 16, 60, 4, 128, C.RAYA_MASK_BLOCKDIAG, 0, 16, 1e-5)  # head_dim 15
    assert lib.raya_postln_workspace_bytes(ctypes.byref(bad)) == 0
    assert lib.raya_postln_layer_forward(ctypes.byref(bad), 256, 256, 256, 256, 1 << 30, None) == C.RAYA_ERR_SHAPE
    odd = C.PostLNLayerC(2, 16, 64, 2, 128, 9, 0, 16, 1e-5)
    for name in ("wqkv", "wo", "w1", "w2", "ln1_w", "ln2_w"):
        setattr(odd, name, 256)
    assert lib.raya_postln_layer_forward(ctypes.byref(odd), 256, 256, 256, 256, 1 << 30, None) == C.RAYA_ERR_UNSUPPORTED


def test_postln_layer_rejects_a_bad_eps():
    lib = C.lib()
    for eps in (-1e-5, float("nan"), float("inf")):
        desc = C.PostLNLayerC(2, 16, 64, 2, 128, C.RAYA_MASK_BLOCKDIAG, 0, 16, eps)
        for name in ("wqkv", "wo", "w1", "w2", "ln1_w", "ln2_w"):
            setattr(desc, name, 256)
        assert lib.raya_postln_workspace_bytes(ctypes.byref(desc)) == 0
        assert "ln_eps" in C.last_error().message.decode()


def test_postln_layer_rejects_dimensions_past_its_indexing():
    """A batch past 2^31 is rejected before batch x seq is formed (no wraparound)."""
    lib = C.lib()
    desc = C.PostLNLayerC(1 << 40, (1 << 30) - 1, 64, 2, 128, C.RAYA_MASK_BLOCKDIAG, 0, 16, 1e-5)
    for name in ("wqkv", "wo", "w1", "w2", "ln1_w", "ln2_w"):
        setattr(desc, name, 256)
    assert lib.raya_postln_workspace_bytes(ctypes.byref(desc)) == 0
    assert "32-bit indexing" in C.last_error().message.decode()


def test_integration_notes_bind_every_declared_function():
    """The Rust binding in INTEGRATION.md declares every function include/*.h exports."""
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    missing = [n for n in declared_functions() if not re.search(r"pub fn " + n + r"\(", doc)]
    assert not missing, missing
