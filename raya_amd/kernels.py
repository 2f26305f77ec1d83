"""Host-side mirror of the reference's `raya-kernels` interface over libraya_hip.

The names, argument meanings and error behaviour follow
crates/raya-kernels/src/attention.rs and gemm.rs:

* ``Mask``, ``AttnShape``, ``AttnParams`` and ``KernelError`` (with ``Shape``,
  ``Length`` and ``Unsupported`` variants) as in attention.rs:8-106;
* ``AttentionKernel`` with ``name()`` and
  ``attend(shape, params, q, k, v, out)`` (attention.rs:113-125);
* ``GemmBackend`` with ``name()`` and ``matmul_nt(out, a, b, m, n, k)``
  (gemm.rs:2-11), which panics (raises ``AssertionError``) on bad lengths.

``HipAttention`` and ``HipGemm`` run on the GPU through the C ABI; there is no
CPU path in this package.  Device-resident entry points (``attend_batched``,
``matmul_nt_device``) take torch tensors already in HBM.
"""
from __future__ import annotations

import abc
import ctypes
import math
from dataclasses import dataclass

import numpy as np

from . import _capi as C

BLOCK = C.RAYA_BLOCK    # attention.rs:4
WINDOW = C.RAYA_WINDOW  # attention.rs:6


class KernelError(Exception):
    """KernelError (attention.rs:8-20)."""


class ShapeError(KernelError):
    """KernelError::Shape."""


class LengthError(KernelError):
    """KernelError::Length { name, got, expected }."""

    def __init__(self, message: str, name: str, got: int, expected: int):
        super().__init__(message)
        self.name, self.got, self.expected = name, got, expected


class UnsupportedError(KernelError):
    """KernelError::Unsupported."""


class DeviceError(KernelError):
    """A HIP runtime failure (no counterpart in the CPU-only reference)."""


def _raise_last(rc: int):
    e = C.last_error()
    msg = e.message.decode()
    if rc == C.RAYA_ERR_SHAPE:
        raise ShapeError(msg)
    if rc == C.RAYA_ERR_LENGTH:
        raise LengthError(msg, e.buffer.decode(), e.got, e.expected)
    if rc == C.RAYA_ERR_UNSUPPORTED:
        raise UnsupportedError(msg)
    raise DeviceError(msg)


@dataclass(frozen=True)
class Mask:
    """Mask (attention.rs:22-35) plus BlockDiag(b): query block i/b sees only its own block."""

    kind: int
    arg: int = 0

    @staticmethod
    def sliding(w: int) -> "Mask":
        return Mask(C.RAYA_MASK_SLIDING, w)

    @staticmethod
    def block_diag(b: int) -> "Mask":
        return Mask(C.RAYA_MASK_BLOCKDIAG, b)

    def name(self) -> str:
        return {C.RAYA_MASK_BLOCK3: "block3", C.RAYA_MASK_WINDOW64: "window64",
                C.RAYA_MASK_FULL: "full", C.RAYA_MASK_SLIDING: "sliding",
                C.RAYA_MASK_BLOCKDIAG: "block_diag"}[self.kind]

    def key_range(self, i: int, valid_len: int) -> range:
        """Keys row i may attend, clipped to valid_len (attention.rs:48-59)."""
        if self.kind == C.RAYA_MASK_BLOCK3:
            b = i // BLOCK
            lo, hi = max(b - 1, 0) * BLOCK, (b + 2) * BLOCK
        elif self.kind == C.RAYA_MASK_WINDOW64:
            lo, hi = max(i - WINDOW, 0), i + WINDOW + 1
        elif self.kind == C.RAYA_MASK_FULL:
            lo, hi = 0, valid_len
        elif self.kind == C.RAYA_MASK_SLIDING:
            lo, hi = max(i - self.arg, 0), i + self.arg + 1
        else:
            b = i // self.arg
            lo, hi = b * self.arg, (b + 1) * self.arg
        return range(min(lo, valid_len), min(hi, valid_len))

    def allows(self, i: int, j: int) -> bool:
        """Whether query i may attend key j, ignoring valid_len (attention.rs:62-69)."""
        if self.kind == C.RAYA_MASK_BLOCK3:
            return abs(i // BLOCK - j // BLOCK) <= 1
        if self.kind == C.RAYA_MASK_WINDOW64:
            return abs(i - j) <= WINDOW
        if self.kind == C.RAYA_MASK_FULL:
            return True
        if self.kind == C.RAYA_MASK_SLIDING:
            return abs(i - j) <= self.arg
        return i // self.arg == j // self.arg


Mask.BLOCK3 = Mask(C.RAYA_MASK_BLOCK3)
Mask.WINDOW64 = Mask(C.RAYA_MASK_WINDOW64)
Mask.FULL = Mask(C.RAYA_MASK_FULL)


@dataclass(frozen=True)
class AttnShape:
    """AttnShape (attention.rs:72-84): buffers are [heads][seq][head_dim]."""

    heads: int
    seq: int
    head_dim: int

    def numel(self) -> int:
        return self.heads * self.seq * self.head_dim


@dataclass(frozen=True)
class AttnParams:
    """AttnParams (attention.rs:86-106)."""

    mask: Mask
    block: int
    valid_len: int
    scale: float

    @staticmethod
    def new(mask: Mask, valid_len: int, head_dim: int) -> "AttnParams":
        """Block 128 and scale 1/sqrt(head_dim) computed in f32 (attention.rs:98-105)."""
        scale = np.float32(1.0) / np.sqrt(np.float32(head_dim))
        return AttnParams(mask, BLOCK, valid_len, float(scale))

    def replace(self, **kw) -> "AttnParams":
        d = dict(mask=self.mask, block=self.block, valid_len=self.valid_len, scale=self.scale)
        d.update(kw)
        return AttnParams(**d)


@dataclass
class StageTimes:
    """StageTimes (crates/raya-kernels/src/tiled/stages.rs:3-31), counted in
    shader clock cycles summed over waves rather than nanoseconds summed over
    threads; ``load_wait`` (load issue, waits and barriers) has no reference
    counterpart and stays out of the percentages, as the reference's stages hold
    no separate load time."""

    qk: int = 0
    softmax: int = 0
    pv: int = 0
    load_wait: int = 0
    tiles: int = 0

    def merge(self, other: "StageTimes") -> None:
        self.qk += other.qk
        self.softmax += other.softmax
        self.pv += other.pv
        self.load_wait += other.load_wait
        self.tiles += other.tiles

    def percentages(self):
        """(qk, softmax, pv) as percentages of their sum, or None if nothing was timed."""
        total = float(self.qk + self.softmax + self.pv)
        if total <= 0.0:
            return None
        return (100.0 * self.qk / total, 100.0 * self.softmax / total, 100.0 * self.pv / total)

    @staticmethod
    def _from_c(c) -> "StageTimes":
        return StageTimes(int(c.qk), int(c.softmax), int(c.pv), int(c.load_wait), int(c.tiles))


class AttentionKernel(abc.ABC):
    """AttentionKernel (attention.rs:113-125)."""

    @abc.abstractmethod
    def name(self) -> str: ...

    @abc.abstractmethod
    def attend(self, shape: AttnShape, params: AttnParams, q, k, v, out) -> None: ...


class GemmBackend(abc.ABC):
    """GemmBackend (gemm.rs:2-11)."""

    @abc.abstractmethod
    def name(self) -> str: ...

    @abc.abstractmethod
    def matmul_nt(self, out, a, b, m: int, n: int, k: int) -> None: ...


def _host_f32(x, name: str):
    """(pointer, length) of a contiguous float32 host buffer."""
    if not isinstance(x, np.ndarray) or x.dtype != np.float32 or not x.flags.c_contiguous:
        raise TypeError(f"`{name}` must be a contiguous numpy float32 array")
    return ctypes.c_void_p(x.ctypes.data), x.size


def _dev_ptr(t, name: str) -> ctypes.c_void_p:
    import torch

    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"`{name}` must be a torch tensor on the GPU")
    return ctypes.c_void_p(t.data_ptr())


def _layout_reach(strides, b: int, h: int, s: int, d: int) -> int:
    """One past the last float a [b, h, s, d] operand with (batch, head, row)
    strides touches (all zero: the dense layout).  Negative strides are left
    to the library, which rejects them."""
    bs, hs, rs = strides
    if bs == 0 and hs == 0 and rs == 0:
        return b * h * s * d
    if min(b, h, s, d) <= 0 or min(bs, hs, rs) < 0:
        return 0
    return (b - 1) * bs + (h - 1) * hs + (s - 1) * rs + d


def _floats_from(t) -> int:
    """Floats between a tensor's pointer and the end of its storage."""
    st = t.untyped_storage()
    return (st.nbytes() - (t.data_ptr() - st.data_ptr())) // 4


def _stream_ptr(stream) -> ctypes.c_void_p:
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


class HipAttention(AttentionKernel):
    """The fused HIP block-local attention kernel (gfx950) as an AttentionKernel."""

    def name(self) -> str:
        return C.lib().raya_attention_name().decode()

    def attend(self, shape: AttnShape, params: AttnParams, q, k, v, out) -> None:
        """Host slices in, out overwritten; errors raise KernelError subclasses."""
        (qp, ql), (kp, kl), (vp, vl), (op, ol) = (
            _host_f32(q, "q"), _host_f32(k, "k"), _host_f32(v, "v"), _host_f32(out, "out"))
        if not out.flags.writeable:
            raise TypeError("`out` must be writeable")
        s = C.AttnShapeC(shape.heads, shape.seq, shape.head_dim)
        p = C.AttnParamsC(params.mask.kind, params.scale, params.mask.arg, params.block,
                          params.valid_len)
        rc = C.lib().raya_attend(ctypes.byref(s), ctypes.byref(p), qp, ql, kp, kl, vp, vl, op, ol)
        if rc:
            _raise_last(rc)

    def attend_with_stages(self, shape: AttnShape, params: AttnParams, q, k, v, out) -> StageTimes:
        """``attend`` through the instrumented kernel, returning its stage totals
        (Tiled::attend_with_stages, crates/raya-kernels/src/tiled/mod.rs:61-126).
        The outputs equal ``attend``'s."""
        (qp, ql), (kp, kl), (vp, vl), (op, ol) = (
            _host_f32(q, "q"), _host_f32(k, "k"), _host_f32(v, "v"), _host_f32(out, "out"))
        if not out.flags.writeable:
            raise TypeError("`out` must be writeable")
        s = C.AttnShapeC(shape.heads, shape.seq, shape.head_dim)
        p = C.AttnParamsC(params.mask.kind, params.scale, params.mask.arg, params.block,
                          params.valid_len)
        st = C.StageCyclesC()
        rc = C.lib().raya_attend_with_stages(ctypes.byref(s), ctypes.byref(p), qp, ql, kp, kl, vp, vl,
                                             op, ol, ctypes.byref(st))
        if rc:
            _raise_last(rc)
        return StageTimes._from_c(st)

    def attend_batched(self, q, k, v, out, valid_len, mask: Mask, scale: float | None = None,
                       block: int = BLOCK, layouts=None, stream=None, stages=None) -> None:
        """Batched device path: q/k/v/out are GPU tensors viewed as
        [batch][heads][seq][head_dim] (or with explicit ``layouts``: a dict of
        name -> (batch_stride, head_stride, row_stride) in floats, plus
        ``shape`` = (batch, heads, seq, head_dim)); valid_len is a GPU int32
        tensor [batch].  Asynchronous on ``stream`` (torch's current stream by
        default).  ``stages``, a GPU int64 tensor of 5 entries, selects the
        instrumented kernel, which adds (qk, softmax, pv, load_wait, tiles) to it."""
        import torch

        if layouts is None:
            if q.dim() != 4:
                raise ShapeError("invalid shape: q must be [batch, heads, seq, head_dim]")
            b, h, s_, d = q.shape
            for name, t in (("q", q), ("k", k), ("v", v), ("out", out)):
                if tuple(t.shape) != (b, h, s_, d) or not t.is_contiguous():
                    raise ShapeError(f"invalid shape: `{name}` must be a contiguous [b, h, s, d] tensor")
            lay = {n: (0, 0, 0) for n in ("q", "k", "v", "out")}
        else:
            b, h, s_, d = layouts["shape"]
            lay = {n: layouts[n] for n in ("q", "k", "v", "out")}
            # The library sees bare pointers: every element a layout reaches must lie
            # inside the tensor's storage, counted from the tensor's own pointer.
            for name, t in (("q", q), ("k", k), ("v", v), ("out", out)):
                reach = _layout_reach(lay[name], b, h, s_, d)
                have = _floats_from(t)
                if reach > have:
                    raise ShapeError(f"invalid shape: the layout of `{name}` reaches {reach} floats past its "
                                     f"pointer, which holds {have}")
        for name, t in (("q", q), ("k", k), ("v", v), ("out", out)):
            if t.dtype != torch.float32:
                raise TypeError(f"`{name}` must be float32")
        if valid_len.dtype != torch.int32 or not valid_len.is_cuda or valid_len.numel() != b:
            raise ShapeError("invalid shape: valid_len must be a GPU int32 tensor of batch entries")
        if scale is None:
            scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
        desc = C.AttnBatchC(b, h, s_, d, mask.kind, scale, mask.arg, block,
                            C.AttnLayoutC(*lay["q"]), C.AttnLayoutC(*lay["k"]),
                            C.AttnLayoutC(*lay["v"]), C.AttnLayoutC(*lay["out"]))
        ptrs = (_dev_ptr(valid_len, "valid_len"), _dev_ptr(q, "q"), _dev_ptr(k, "k"),
                _dev_ptr(v, "v"), _dev_ptr(out, "out"))
        if stages is None:
            rc = C.lib().raya_attend_batched(ctypes.byref(desc), *ptrs, _stream_ptr(stream))
        else:
            if stages.dtype != torch.int64 or not stages.is_cuda or stages.numel() < 5 \
                    or not stages.is_contiguous():
                raise ShapeError("invalid shape: stages must be a contiguous GPU int64 tensor of 5 entries")
            rc = C.lib().raya_attend_batched_stages(ctypes.byref(desc), *ptrs, _dev_ptr(stages, "stages"),
                                                    _stream_ptr(stream))
        if rc:
            _raise_last(rc)

    def attend_batched_stages(self, q, k, v, out, valid_len, mask: Mask, scale: float | None = None,
                              block: int = BLOCK, layouts=None, stream=None) -> StageTimes:
        """``attend_batched`` through the instrumented kernel; waits for the
        stream and returns the launch's stage totals."""
        import torch

        stages = torch.zeros(5, dtype=torch.int64, device=q.device)
        self.attend_batched(q, k, v, out, valid_len, mask, scale, block, layouts, stream, stages=stages)
        (stream if stream is not None else torch.cuda.current_stream()).synchronize()
        return StageTimes(*(int(x) for x in stages.cpu().tolist()))


class HipGemm(GemmBackend):
    """The MFMA fp32 GEMM (gfx950) as a GemmBackend."""

    def name(self) -> str:
        return C.lib().raya_gemm_name().decode()

    def matmul_nt(self, out, a, b, m: int, n: int, k: int) -> None:
        (op, ol), (ap, al), (bp, bl) = _host_f32(out, "out"), _host_f32(a, "a"), _host_f32(b, "b")
        rc = C.lib().raya_matmul_nt(op, ol, ap, al, bp, bl, m, n, k)
        if rc == C.RAYA_ERR_LENGTH:
            # Reference::matmul_nt panics on a length mismatch (gemm.rs:23-25).
            raise AssertionError(C.last_error().message.decode())
        if rc:
            _raise_last(rc)

    def matmul_nt_device(self, out, a, b, *, bias=None, activation: int = C.RAYA_EPI_NONE,
                         residual=None, out_row_stats=None, in_row_stats=None, in_weight_sums=None,
                         stream=None) -> None:
        """out[m, n] = act(a[m, k] @ b[n, k]^T + bias) + residual on GPU tensors.
        For GEGLU, b is [2n, k] and bias [2n].  Row strides are taken from the
        tensors (last dimension must be contiguous).

        out_row_stats ([m, n // 64, 4] float32): the chunk statistics of out for
        row_norm_stats.  in_row_stats ([m, 4], from row_norm_stats) with in_weight_sums
        (b's row sums, from weight_row_sums): a's rows are LayerNorm-ed before the
        product, b carrying the norm's gain in its columns."""
        import torch

        # Every operand is checked before anything reaches the device: another
        # dtype, a short bias or a host tensor would hand the kernel fewer bytes
        # than it reads, or a pointer it cannot read.  Shapes and dtypes first,
        # the device last.
        named = [("out", out), ("a", a), ("b", b)]
        named += [(n_, t) for n_, t in (("bias", bias), ("residual", residual),
                                        ("out_row_stats", out_row_stats), ("in_row_stats", in_row_stats),
                                        ("in_weight_sums", in_weight_sums))
                  if t is not None]
        for name, t in named:
            if not isinstance(t, torch.Tensor):
                raise TypeError(f"`{name}` must be a torch tensor")
            if t.dtype != torch.float32:
                raise TypeError(f"`{name}` must be float32")
        for name, t in (("out", out), ("a", a), ("b", b)):
            if t.dim() != 2 or t.stride(1) != 1:
                raise ShapeError(f"invalid shape: `{name}` must be 2-D with contiguous rows")
        m, k = a.shape
        n = out.shape[1]
        rows_b = 2 * n if activation == C.RAYA_EPI_GEGLU else n
        if tuple(b.shape) != (rows_b, k) or out.shape[0] != m:
            raise ShapeError("invalid shape: operands do not agree")
        if bias is not None and (bias.dim() != 1 or bias.numel() != rows_b or not bias.is_contiguous()):
            raise ShapeError(f"invalid shape: `bias` must be a contiguous vector of {rows_b} entries")
        if residual is not None and (residual.dim() != 2 or tuple(residual.shape) != (m, n)
                                     or residual.stride(1) != 1):
            raise ShapeError("invalid shape: `residual` must be [m, n] with contiguous rows")
        if out_row_stats is not None and (not out_row_stats.is_contiguous()
                                          or tuple(out_row_stats.shape) != (m, n // 64, 4)):
            raise ShapeError(f"invalid shape: `out_row_stats` must be a contiguous [{m}, {n // 64}, 4]")
        if in_row_stats is not None and (not in_row_stats.is_contiguous()
                                         or tuple(in_row_stats.shape) != (m, 4)):
            raise ShapeError(f"invalid shape: `in_row_stats` must be a contiguous [{m}, 4]")
        if in_weight_sums is not None and (in_weight_sums.dim() != 1 or in_weight_sums.numel() != rows_b
                                           or not in_weight_sums.is_contiguous()):
            raise ShapeError(f"invalid shape: `in_weight_sums` must be a contiguous vector of {rows_b} entries")
        for name, t in named:
            if not t.is_cuda:
                raise TypeError(f"`{name}` must be a torch tensor on the GPU")
        ep = C.GemmEpilogueC(activation, 0,
                             _dev_ptr(bias, "bias") if bias is not None else None,
                             _dev_ptr(residual, "residual") if residual is not None else None,
                             residual.stride(0) if residual is not None else 0,
                             _dev_ptr(out_row_stats, "out_row_stats") if out_row_stats is not None else None,
                             _dev_ptr(in_row_stats, "in_row_stats") if in_row_stats is not None else None,
                             _dev_ptr(in_weight_sums, "in_weight_sums") if in_weight_sums is not None else None)
        rc = C.lib().raya_matmul_nt_device(_dev_ptr(out, "out"), out.stride(0), _dev_ptr(a, "a"),
                                           a.stride(0), _dev_ptr(b, "b"), b.stride(0), m, n, k,
                                           ctypes.byref(ep), _stream_ptr(stream))
        if rc:
            _raise_last(rc)

    def weight_row_sums(self, b, sums, stream=None) -> None:
        """sums[j] = sum_t b[j, t] (f64, rounded once) on GPU tensors: the in_weight_sums of
        a folded weight b ([rows, k], contiguous rows)."""
        import torch

        for name, t in (("b", b), ("sums", sums)):
            if not isinstance(t, torch.Tensor) or t.dtype != torch.float32:
                raise TypeError(f"`{name}` must be a float32 torch tensor")
        if b.dim() != 2 or b.stride(1) != 1 or sums.dim() != 1 or sums.numel() != b.shape[0] \
                or not sums.is_contiguous():
            raise ShapeError("invalid shape: b [rows, k] with contiguous rows and sums [rows]")
        for name, t in (("b", b), ("sums", sums)):
            if not t.is_cuda:
                raise TypeError(f"`{name}` must be a torch tensor on the GPU")
        rc = C.lib().raya_weight_row_sums(_dev_ptr(b, "b"), b.stride(0), b.shape[0], b.shape[1],
                                          _dev_ptr(sums, "sums"), _stream_ptr(stream))
        if rc:
            _raise_last(rc)

    def row_norm_stats(self, chunk_stats, row_stats, eps: float, stream=None) -> None:
        """Each row's LayerNorm (mean, 1/sqrt(var + eps)) from a GEMM's out_row_stats
        ([m, n // 64, 4]) into row_stats ([m, 4]), for a later in_row_stats."""
        import torch

        for name, t in (("chunk_stats", chunk_stats), ("row_stats", row_stats)):
            if not isinstance(t, torch.Tensor) or t.dtype != torch.float32:
                raise TypeError(f"`{name}` must be a float32 torch tensor")
            if not t.is_contiguous():
                raise ShapeError(f"invalid shape: `{name}` must be contiguous")
        if chunk_stats.dim() != 3 or chunk_stats.shape[2] != 4 or tuple(row_stats.shape) != (chunk_stats.shape[0], 4):
            raise ShapeError("invalid shape: chunk_stats [m, n // 64, 4] and row_stats [m, 4]")
        for name, t in (("chunk_stats", chunk_stats), ("row_stats", row_stats)):
            if not t.is_cuda:
                raise TypeError(f"`{name}` must be a torch tensor on the GPU")
        m, chunks = chunk_stats.shape[0], chunk_stats.shape[1]
        rc = C.lib().raya_row_norm_stats(_dev_ptr(chunk_stats, "chunk_stats"), m, 64 * chunks, eps,
                                         _dev_ptr(row_stats, "row_stats"), _stream_ptr(stream))
        if rc:
            _raise_last(rc)


def default_scale(head_dim: int) -> float:
    return float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))


assert math.isclose(default_scale(64), 0.125)
