"""A post-LN encoder layer on the device: BERT's layer (nn.TransformerEncoderLayer with
norm_first=False, erf GELU, biases) built from the library's GEMM, attention and LayerNorm
kernels (``raya_postln_layer_forward`` in include/raya_hip.h).  The reference's own layer is
pre-LN (crates/raya-core/src/encoder.rs:96-152); this one is the block-local layer in its
classic form.
"""
from __future__ import annotations

import ctypes

from . import _capi as C
from .kernels import Mask, ShapeError, _dev_ptr, _raise_last, _stream_ptr

WEIGHTS = ("wqkv", "bqkv", "wo", "bo", "ln1_w", "ln1_b", "w1", "b1", "w2", "b2", "ln2_w", "ln2_b")
OPTIONAL = {"bqkv", "bo", "b1", "b2", "ln1_b", "ln2_b"}


class PostLNLayer:
    """y1 = LN1(x + Attn(x Wqkv^T + bqkv) Wo^T + bo); out = LN2(y1 + gelu(y1 W1^T + b1) W2^T + b2).

    `weights` maps the names of WEIGHTS to float32 GPU tensors in nn.Linear's [out, in] layout
    (biases may be missing or None); attention uses `mask` and the per-sequence valid lengths
    with scale 1/sqrt(head_dim)."""

    def __init__(self, weights: dict, heads: int, eps: float = 1e-12, mask: Mask | None = None):
        import torch

        wqkv = weights["wqkv"]
        if wqkv.dim() != 2 or wqkv.shape[0] != 3 * wqkv.shape[1]:
            raise ShapeError("invalid shape: wqkv must be [3 hidden, hidden]")
        self.hidden = int(wqkv.shape[1])
        self.ffn = int(weights["w1"].shape[0])
        d, f = self.hidden, self.ffn
        want = {"wqkv": (3 * d, d), "bqkv": (3 * d,), "wo": (d, d), "bo": (d,), "ln1_w": (d,), "ln1_b": (d,),
                "w1": (f, d), "b1": (f,), "w2": (d, f), "b2": (d,), "ln2_w": (d,), "ln2_b": (d,)}
        self.w = {}
        for name in WEIGHTS:
            t = weights.get(name)
            if t is None:
                if name not in OPTIONAL:
                    raise ShapeError(f"invalid shape: `{name}` is required")
                continue
            if not isinstance(t, torch.Tensor) or t.dtype != torch.float32:
                raise TypeError(f"`{name}` must be a float32 torch tensor")
            if tuple(t.shape) != want[name] or not t.is_contiguous():
                raise ShapeError(f"invalid shape: `{name}` must be a contiguous {list(want[name])} tensor")
            if not t.is_cuda:
                raise TypeError(f"`{name}` must be a torch tensor on the GPU")
            if t.device != wqkv.device:
                raise TypeError(f"`{name}` is on {t.device}, wqkv on {wqkv.device}")
            self.w[name] = t
        self.heads, self.eps = heads, eps
        self.mask = mask if mask is not None else Mask.block_diag(64)
        # One workspace per stream, allocated on that stream: the caching allocator then
        # orders its reuse, after a growth frees it, behind the launches on that stream, and
        # forwards on different streams never share the qkv / context / sum buffers.
        self._ws = {}

    def _desc(self, batch: int, seq: int):
        desc = C.PostLNLayerC(batch, seq, self.hidden, self.heads, self.ffn, self.mask.kind, 0, self.mask.arg,
                              self.eps)
        for name in WEIGHTS:
            t = self.w.get(name)
            setattr(desc, name, t.data_ptr() if t is not None else None)
        return desc

    def forward(self, x, valid_len, out=None, stream=None):
        """x: GPU float32 [batch, seq, hidden]; valid_len: GPU int32 [batch].  Returns out
        (allocated when not given).  Asynchronous on `stream` (torch's current by default)."""
        import torch

        if not isinstance(x, torch.Tensor) or x.dtype != torch.float32 or x.dim() != 3 \
                or x.shape[2] != self.hidden or not x.is_contiguous():
            raise ShapeError(f"invalid shape: x must be a contiguous float32 [batch, seq, {self.hidden}] tensor")
        b, s, _ = x.shape
        dev = self.w["wqkv"].device
        if x.device != dev:
            raise TypeError(f"x is on {x.device}, the layer's weights on {dev}")
        if not isinstance(valid_len, torch.Tensor) or valid_len.dtype != torch.int32 \
                or valid_len.numel() != b or not valid_len.is_cuda:
            raise ShapeError("invalid shape: valid_len must be a GPU int32 tensor of batch entries")
        if valid_len.device != dev:
            raise TypeError(f"valid_len is on {valid_len.device}, the layer's weights on {dev}")
        if out is None:
            out = torch.empty_like(x)
        elif out.shape != x.shape or out.dtype != torch.float32 or not out.is_contiguous():
            raise ShapeError("invalid shape: out must match x")
        desc = self._desc(b, s)
        need = C.lib().raya_postln_workspace_bytes(ctypes.byref(desc))
        if need == 0:
            _raise_last(C.last_error().code)
        st = stream if stream is not None else torch.cuda.current_stream(dev)
        ws = self._ws.get(st.cuda_stream)
        if ws is None or ws.numel() * 4 < need:
            with torch.cuda.stream(st):
                ws = torch.empty((need + 3) // 4, dtype=torch.float32, device=dev)
            self._ws[st.cuda_stream] = ws
        rc = C.lib().raya_postln_layer_forward(ctypes.byref(desc), _dev_ptr(valid_len, "valid_len"), _dev_ptr(x, "x"),
                                               _dev_ptr(out, "out"), _dev_ptr(ws, "workspace"), need,
                                               _stream_ptr(st))
        if rc:
            _raise_last(rc)
        return out
