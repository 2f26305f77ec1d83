"""Host-side mirror of raya-core's decision model over libraya_hip.

Follows crates/raya-core/src/model.rs and crates/raya-weights:

* ``Model.load(checkpoint_dir, weights=None)`` = ``ModelConfig::from_dir`` +
  ``raya_weights::load`` + ``Model::bind`` (model.rs:18-29, store.rs:66-151);
* ``Model.forward(ForwardInput, trace=None)`` = ``Network::forward``
  (model.rs:261-348) for one sequence, returning ``ForwardOutput``;
* ``Model.forward_batch(...)`` runs many sequences in one device pass;
* ``Trace`` records the stages under the golden names (trace.rs).

Errors are ``raya_core::Error``'s variants (error.rs:5-33): ``ConfigError``,
``UnimplementedError``, ``InputError``, ``KernelCallError``, ``WeightsError``.
Everything runs in libraya_hip.so; there is no CPU path.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _capi as C
from .kernels import DeviceError, Mask, _raise_last


class Error(Exception):
    """raya_core::Error."""


class ConfigError(Error):
    """Error::Config / Io / Json."""


class UnimplementedError(Error):
    """Error::Unimplemented."""


class InputError(Error):
    """Error::Input."""


class KernelCallError(Error):
    """Error::Kernel: the attention kernel rejected the call."""


class WeightsError(Error):
    """Error::Weights (the LoadReport text)."""


_ERRORS = {C.RAYA_ERR_CONFIG: ConfigError, C.RAYA_ERR_UNIMPLEMENTED: UnimplementedError,
           C.RAYA_ERR_INPUT: InputError, C.RAYA_ERR_KERNEL: KernelCallError,
           C.RAYA_ERR_WEIGHTS: WeightsError}


def _check(rc: int) -> None:
    if rc == C.RAYA_OK:
        return
    if rc in _ERRORS:
        raise _ERRORS[rc](C.last_error().message.decode())
    if rc == C.RAYA_ERR_DEVICE:
        raise DeviceError(C.last_error().message.decode())
    _raise_last(rc)


@dataclass
class ForwardInput:
    """ForwardInput (model.rs:90-100)."""

    input_ids: np.ndarray
    valid_len: int
    marker_pos: np.ndarray
    marker_mask: np.ndarray
    qtype: int


@dataclass
class ForwardOutput:
    """ForwardOutput (model.rs:102-112); batched outputs carry a leading batch axis."""

    logits: np.ndarray
    probabilities: np.ndarray
    act_logits: np.ndarray
    features: np.ndarray
    pooled: np.ndarray


@dataclass
class Trace:
    """Intermediate activations in execution order (trace.rs)."""

    entries: list = field(default_factory=list)

    def push(self, name, shape, data):
        self.entries.append((name, tuple(shape), data))

    def get(self, name):
        for n, s, d in self.entries:
            if n == name:
                return s, d
        return None

    def names(self):
        return [n for n, _, _ in self.entries]


class Model:
    """A bound decision model; weights go to the GPU on the first forward call."""

    def __init__(self, handle: int):
        self._h = ctypes.c_void_p(handle)

    @classmethod
    def load(cls, checkpoint_dir: str, weights: str | None = None) -> "Model":
        h = ctypes.c_void_p()
        _check(C.lib().raya_model_load(checkpoint_dir.encode(),
                                       weights.encode() if weights else None, ctypes.byref(h)))
        return cls(h.value)

    def __del__(self):
        if getattr(self, "_h", None) and self._h.value:
            C.lib().raya_model_free(self._h)
            self._h = ctypes.c_void_p()

    @property
    def info(self) -> dict:
        i = C.ModelInfoC()
        _check(C.lib().raya_model_get_info(self._h, ctypes.byref(i)))
        return {name: getattr(i, name) for name, _ in C.ModelInfoC._fields_}

    def set_profiling(self, level: int) -> None:
        """0: off; 1: an event pair around every stage (embedding, each layer, final norm,
        head layers, scorer + act head); 2: also around every kernel of an encoder layer."""
        _check(C.lib().raya_model_set_profiling(self._h, int(level)))

    def stage_times(self) -> list[tuple[str, float]]:
        """(name, milliseconds) of every span the last forward recorded, in order."""
        n = ctypes.c_uint64()
        _check(C.lib().raya_model_stage_times(self._h, None, 0, ctypes.byref(n)))
        buf = (C.StageTimeC * max(1, n.value))()
        _check(C.lib().raya_model_stage_times(self._h, buf, n.value, ctypes.byref(n)))
        return [(buf[i].name.decode(), buf[i].ms) for i in range(n.value)]

    def forward(self, inp: ForwardInput, trace: Trace | None = None,
                local_mask: Mask | None = None) -> ForwardOutput:
        """Network::forward on one sequence (the trace has the reference's [1, seq, …] shapes)."""
        out = self.forward_batch(np.asarray(inp.input_ids)[None], [inp.valid_len],
                                 np.asarray(inp.marker_pos)[None], np.asarray(inp.marker_mask)[None],
                                 [inp.qtype], trace=trace, local_mask=local_mask)
        return ForwardOutput(out.logits[0], out.probabilities[0], out.act_logits[0],
                             out.features[0], out.pooled[0])

    def forward_batch(self, input_ids, valid_len, marker_pos, marker_mask, qtype,
                      trace: Trace | None = None, local_mask: Mask | None = None,
                      stream=None) -> ForwardOutput:
        """Many sequences in one device pass: input_ids [B, L], valid_len [B],
        marker_pos / marker_mask [B, K], qtype [B]."""
        ids = np.ascontiguousarray(input_ids, dtype=np.uint32)
        if ids.ndim != 2:
            raise InputError("invalid input: input_ids must be [batch, seq]")
        b, s = ids.shape
        valid = np.ascontiguousarray(valid_len, dtype=np.uint64).reshape(b)
        pos = np.ascontiguousarray(marker_pos, dtype=np.uint64).reshape(b, -1)
        k = pos.shape[1]
        mask = np.ascontiguousarray(marker_mask, dtype=np.uint8).reshape(b, k)
        qt = np.ascontiguousarray(qtype, dtype=np.uint64).reshape(b)
        info = self.info
        d, nact = info["hidden_size"], info["n_act"]
        res = ForwardOutput(np.empty((b, k), np.float32), np.empty((b, k), np.float32),
                            np.empty((b, nact), np.float32), np.empty((b, 4), np.float32),
                            np.empty((b, d), np.float32))
        desc = C.ForwardBatchC(b, s, k, ids.ctypes.data, valid.ctypes.data, pos.ctypes.data,
                               mask.ctypes.data, qt.ctypes.data, 0, 0, 0)
        if local_mask is not None:
            desc.local_override, desc.local_mask_kind, desc.local_mask_arg = 1, local_mask.kind, local_mask.arg
        outs = C.ForwardOutputC(*(x.ctypes.data for x in (res.logits, res.probabilities,
                                                          res.act_logits, res.features, res.pooled)))
        if trace is not None:
            def record(_user, name, shape, ndim, data):
                shp = tuple(shape[i] for i in range(ndim))
                n = int(np.prod(shp))
                arr = np.ctypeslib.as_array(data, shape=(n,)).copy().reshape(shp)
                trace.push(name.decode(), shp, arr)
            cb = C.TRACE_FN(record)
        else:
            cb = ctypes.cast(None, C.TRACE_FN)
        st = None
        if stream is not None:
            st = ctypes.c_void_p(getattr(stream, "cuda_stream", stream))
        _check(C.lib().raya_model_forward(self._h, ctypes.byref(desc), ctypes.byref(outs), cb,
                                          None, st))
        return res
