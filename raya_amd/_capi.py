"""ctypes binding of libraya_hip.so (declarations of include/raya_hip.h).

Loading the library does not touch the GPU; the first compute call does.
A missing library is an error, never a silent fallback.
"""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libraya_hip.so")

RAYA_OK, RAYA_ERR_SHAPE, RAYA_ERR_LENGTH, RAYA_ERR_UNSUPPORTED, RAYA_ERR_DEVICE = 0, 1, 2, 3, 4
RAYA_MASK_BLOCK3, RAYA_MASK_WINDOW64, RAYA_MASK_FULL, RAYA_MASK_SLIDING, RAYA_MASK_BLOCKDIAG = range(5)
RAYA_BLOCK, RAYA_WINDOW = 128, 64
RAYA_STATIC_ATTEND_MAX_NUMEL = 4194304
RAYA_EPI_NONE, RAYA_EPI_GELU, RAYA_EPI_RELU, RAYA_EPI_GEGLU = 0, 1, 2, 3
RAYA_ERR_CONFIG, RAYA_ERR_UNIMPLEMENTED, RAYA_ERR_INPUT, RAYA_ERR_KERNEL, RAYA_ERR_WEIGHTS = 5, 6, 7, 8, 9


class AttnShapeC(ctypes.Structure):
    _fields_ = [("heads", ctypes.c_uint64), ("seq", ctypes.c_uint64), ("head_dim", ctypes.c_uint64)]


class AttnParamsC(ctypes.Structure):
    _fields_ = [("mask_kind", ctypes.c_int32), ("scale", ctypes.c_float),
                ("mask_arg", ctypes.c_uint64), ("block", ctypes.c_uint64),
                ("valid_len", ctypes.c_uint64)]


class ErrorC(ctypes.Structure):
    _fields_ = [("code", ctypes.c_int32), ("buffer", ctypes.c_char * 8),
                ("got", ctypes.c_uint64), ("expected", ctypes.c_uint64),
                ("message", ctypes.c_char * 512)]


class AttnLayoutC(ctypes.Structure):
    _fields_ = [("batch_stride", ctypes.c_int64), ("head_stride", ctypes.c_int64),
                ("row_stride", ctypes.c_int64)]


class AttnBatchC(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_uint64), ("heads", ctypes.c_uint64), ("seq", ctypes.c_uint64),
                ("head_dim", ctypes.c_uint64), ("mask_kind", ctypes.c_int32),
                ("scale", ctypes.c_float), ("mask_arg", ctypes.c_uint64),
                ("block", ctypes.c_uint64), ("q", AttnLayoutC), ("k", AttnLayoutC),
                ("v", AttnLayoutC), ("out", AttnLayoutC)]


class GemmEpilogueC(ctypes.Structure):
    _fields_ = [("activation", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("bias", ctypes.c_void_p), ("residual", ctypes.c_void_p), ("ldr", ctypes.c_int64),
                ("out_row_stats", ctypes.c_void_p), ("in_row_stats", ctypes.c_void_p),
                ("in_weight_sums", ctypes.c_void_p)]


class ParamEntryC(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 128), ("ndim", ctypes.c_uint32),
                ("shape", ctypes.c_uint64 * 4)]


class ModelInfoC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
        "global_attn_every_n_layers", "local_attention", "vocab_size", "max_position_embeddings")] + \
        [(n, ctypes.c_double) for n in ("global_rope_theta", "local_rope_theta", "norm_eps")] + \
        [(n, ctypes.c_uint64) for n in ("head_layers", "head_heads", "head_ffn", "n_act",
                                        "param_floats")]


class PostLNLayerC(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_uint64), ("seq", ctypes.c_uint64), ("hidden", ctypes.c_uint64),
                ("heads", ctypes.c_uint64), ("ffn", ctypes.c_uint64), ("mask_kind", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("mask_arg", ctypes.c_uint64), ("ln_eps", ctypes.c_float)]
    _fields_ += [(n, ctypes.c_void_p) for n in ("wqkv", "bqkv", "wo", "bo", "ln1_w", "ln1_b", "w1", "b1",
                                                 "w2", "b2", "ln2_w", "ln2_b")]


class ForwardBatchC(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_uint64), ("seq", ctypes.c_uint64), ("markers", ctypes.c_uint64),
                ("input_ids", ctypes.c_void_p), ("valid_len", ctypes.c_void_p),
                ("marker_pos", ctypes.c_void_p), ("marker_mask", ctypes.c_void_p),
                ("qtype", ctypes.c_void_p), ("local_override", ctypes.c_int32),
                ("local_mask_kind", ctypes.c_int32), ("local_mask_arg", ctypes.c_uint64)]


class ForwardOutputC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("logits", "probabilities", "act_logits", "features", "pooled")]


class StageCyclesC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("qk", "softmax", "pv", "load_wait", "tiles")]


class StageTimeC(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("ms", ctypes.c_double)]


TRACE_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_char_p,
                            ctypes.POINTER(ctypes.c_uint64), ctypes.c_uint32,
                            ctypes.POINTER(ctypes.c_float))

_fp = ctypes.POINTER(ctypes.c_float)
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_u64, _i64 = ctypes.c_uint64, ctypes.c_int64

# (name, restype, argtypes) of every exported function, in header order.
SIGNATURES = [
    ("raya_last_error", ctypes.POINTER(ErrorC), []),
    ("raya_attention_name", ctypes.c_char_p, []),
    ("raya_gemm_name", ctypes.c_char_p, []),
    ("raya_build_info", ctypes.c_char_p, []),
    ("raya_attend", ctypes.c_int, [ctypes.POINTER(AttnShapeC), ctypes.POINTER(AttnParamsC),
                                   _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz]),
    ("raya_attend_static", ctypes.c_int, [ctypes.POINTER(AttnShapeC), ctypes.POINTER(AttnParamsC),
                                          _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp]),
    ("raya_attend_with_stages", ctypes.c_int, [ctypes.POINTER(AttnShapeC), ctypes.POINTER(AttnParamsC),
                                               _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz,
                                               ctypes.POINTER(StageCyclesC)]),
    ("raya_attend_batched", ctypes.c_int, [ctypes.POINTER(AttnBatchC), _vp, _vp, _vp, _vp, _vp, _vp]),
    ("raya_attend_batched_stages", ctypes.c_int, [ctypes.POINTER(AttnBatchC), _vp, _vp, _vp, _vp, _vp,
                                                  _vp, _vp]),
    ("raya_matmul_nt", ctypes.c_int, [_vp, _sz, _vp, _sz, _vp, _sz, _u64, _u64, _u64]),
    ("raya_matmul_nt_device", ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _u64, _u64, _u64,
                                             ctypes.POINTER(GemmEpilogueC), _vp]),
    ("raya_row_norm_stats", ctypes.c_int, [_vp, _u64, _u64, ctypes.c_float, _vp, _vp]),
    ("raya_weight_row_sums", ctypes.c_int, [_vp, _i64, _u64, _u64, _vp, _vp]),
    ("raya_postln_workspace_bytes", ctypes.c_uint64, [ctypes.POINTER(PostLNLayerC)]),
    ("raya_postln_layer_forward", ctypes.c_int, [ctypes.POINTER(PostLNLayerC), _vp, _vp, _vp, _vp, _u64, _vp]),
    ("raya_model_load", ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    ("raya_model_free", None, [_vp]),
    ("raya_expected_params", ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ParamEntryC), _u64,
                                            ctypes.POINTER(_u64)]),
    ("raya_model_get_info", ctypes.c_int, [_vp, ctypes.POINTER(ModelInfoC)]),
    ("raya_model_forward", ctypes.c_int, [_vp, ctypes.POINTER(ForwardBatchC),
                                          ctypes.POINTER(ForwardOutputC), TRACE_FN, _vp, _vp]),
    ("raya_model_set_profiling", ctypes.c_int, [_vp, ctypes.c_int]),
    ("raya_model_stage_times", ctypes.c_int, [_vp, ctypes.POINTER(StageTimeC), _u64,
                                              ctypes.POINTER(_u64)]),
]

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build the HIP backend with `python -m raya_amd.build`")
        # torch ships its own HIP and HSA runtimes.  Loaded first, its HSA runtime
        # (soname libhsa-runtime64.so.1) also serves this library's HIP runtime; loaded
        # after this library, torch brings a second HSA runtime into the process and
        # whichever HIP runtime initialises second finds no device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def last_error() -> ErrorC:
    return lib().raya_last_error().contents
