"""ctypes declarations of include/aexq.h and the loader of libaexq.so.

This is the Python twin of the C# P/Invoke wrapper a host would write: every
entry point of the C ABI, its status codes mapped to the exception kinds the
reference throws (ArgumentException, NotSupportedException,
InvalidOperationException, InvalidDataException).  There is no fallback: if
the library is missing the import of a binding fails loudly.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libaexq.so")
HEADER = os.path.join(ROOT, "include", "aexq.h")

OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_UNSUPPORTED = 2
ERR_SHAPE = 3
ERR_DEVICE = 4
ERR_OUT_OF_MEMORY = 5
ERR_FORMAT = 6

DTYPE_F16 = 1
DTYPE_F32 = 2
NIBBLE_TWOS = 0
NIBBLE_OFFSET8 = 1
LAYOUT_LINEAR = 0
LAYOUT_PACK4_LINEAR = 1
LAYOUT_PACK4_TILED = 2
LAYOUT_HEAD_PACKED = 3
EPI_RMSNORM_IN = 0x1
EPI_SWIGLU_OUT = 0x2
EPI_RESIDUAL_ADD = 0x4
EPI_ARGMAX_F16 = 0x8
EPI_EXACT_DEQUANT = 0x10


class AexqError(RuntimeError):
    """Base class; `status` holds the aexq_status code."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class ArgumentError(AexqError, ValueError):
    pass


class NotSupportedError(AexqError):
    """Strict-plan rejection: no kernel exists and nothing falls back."""


class InvalidOperationError(AexqError):
    pass


class DeviceError(AexqError):
    pass


class InvalidDataError(AexqError):
    pass


_STATUS_EXC = {
    ERR_INVALID_ARGUMENT: ArgumentError,
    ERR_UNSUPPORTED: NotSupportedError,
    ERR_SHAPE: InvalidOperationError,
    ERR_DEVICE: DeviceError,
    ERR_OUT_OF_MEMORY: DeviceError,
    ERR_FORMAT: InvalidDataError,
}


class Shape(ctypes.Structure):
    _fields_ = [("dims", ctypes.c_int), ("w", ctypes.c_int), ("h", ctypes.c_int),
                ("d", ctypes.c_int), ("c", ctypes.c_int)]


class Tensor(ctypes.Structure):
    _fields_ = [("logical", Shape), ("storage", Shape), ("layout", ctypes.c_int),
                ("dtype", ctypes.c_int), ("data", ctypes.c_void_p), ("batch", ctypes.c_int),
                ("batch_stride", ctypes.c_int64)]


class LinearArgs(ctypes.Structure):
    _fields_ = [("alpha", ctypes.c_float), ("beta", ctypes.c_float),
                ("c", ctypes.c_void_p), ("broadcast_c", ctypes.c_int),
                ("rms_gamma", ctypes.c_void_p), ("rms_gamma_size", ctypes.c_int),
                ("rms_eps", ctypes.c_float), ("up", ctypes.c_void_p),
                ("residual", ctypes.POINTER(Tensor)), ("flags", ctypes.c_uint)]


class WeightInfo(ctypes.Structure):
    _fields_ = [("bits", ctypes.c_int), ("n", ctypes.c_int), ("k", ctypes.c_int),
                ("block", ctypes.c_int), ("scale_dtype", ctypes.c_int),
                ("nibble_code", ctypes.c_int), ("batch", ctypes.c_int),
                ("code_bytes", ctypes.c_int64), ("scale_bytes", ctypes.c_int64)]


class DecoderLayer(ctypes.Structure):
    _fields_ = [("q_proj", ctypes.c_void_p), ("k_proj", ctypes.c_void_p),
                ("v_proj", ctypes.c_void_p), ("o_proj", ctypes.c_void_p),
                ("gate_proj", ctypes.c_void_p), ("up_proj", ctypes.c_void_p),
                ("down_proj", ctypes.c_void_p), ("attn_norm", ctypes.c_void_p),
                ("mlp_norm", ctypes.c_void_p), ("k_cache", ctypes.c_void_p),
                ("v_cache", ctypes.c_void_p)]


class DecoderConfig(ctypes.Structure):
    _fields_ = [("heads_q", ctypes.c_int), ("heads_kv", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("capacity", ctypes.c_int), ("rms_eps", ctypes.c_float),
                ("attn_scale", ctypes.c_float), ("rope_cos", ctypes.c_void_p),
                ("rope_sin", ctypes.c_void_p), ("workgroups", ctypes.c_int)]


_lib = None


def header_functions() -> list[str]:
    """Names of every function include/aexq.h declares."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aexq_[a-z0-9_]+)\s*\(", text)))


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is missing: build the HIP library first (python -m aiimage_amd.build); "
            "the aexq path has no CPU fallback")
    lib = ctypes.CDLL(path)
    _declare(lib)
    _lib = lib
    return lib


def _declare(L):
    P, i32, u32, f32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint, ctypes.c_float, ctypes.c_size_t
    PP = ctypes.POINTER(ctypes.c_void_p)
    TP = ctypes.POINTER(Tensor)
    AP = ctypes.POINTER(LinearArgs)
    sig = {
        "aexq_abi_version": (i32, []),
        "aexq_last_error": (ctypes.c_char_p, []),
        "aexq_create": (i32, [i32, P, PP]),
        "aexq_destroy": (None, [P]),
        "aexq_set_stream": (i32, [P, P]),
        "aexq_synchronize": (i32, [P]),
        "aexq_weight_q8": (i32, [P, P, P, i32, i32, i32, i32, PP]),
        "aexq_weight_q4": (i32, [P, P, P, i32, i32, i32, i32, i32, PP]),
        "aexq_weight_q8_from_f32": (i32, [P, P, i32, i32, i32, PP]),
        "aexq_weight_q4_from_f32": (i32, [P, P, i32, i32, i32, PP]),
        "aexq_archive_header": (i32, [P, sz, ctypes.POINTER(i32), ctypes.POINTER(i32),
                                      ctypes.POINTER(i32)]),
        "aexq_weight_from_record": (i32, [P, i32, P, sz, i32, i32, PP, ctypes.POINTER(sz)]),
        "aexq_weight_replicate": (i32, [P, P, i32, PP]),
        "aexq_weight_alias": (i32, [P, P, PP]),
        "aexq_weight_release": (None, [P]),
        "aexq_weight_get_info": (i32, [P, ctypes.POINTER(WeightInfo)]),
        "aexq_plan_check": (i32, [P, P, TP, TP, AP, ctypes.c_char_p, sz]),
        "aexq_linear": (i32, [P, P, TP, TP, AP]),
        "aexq_linear_group": (i32, [P, i32, PP, TP, ctypes.POINTER(TP), AP]),
        "aexq_lmhead_argmax": (i32, [P, P, TP, TP, P, P]),
        "aexq_lmhead_argmax_noalloc": (i32, [P, P, TP, P, P]),
        "aexq_lmhead_argmax_ex": (i32, [P, P, TP, TP, AP, P, P]),
        "aexq_argmax": (i32, [P, TP, P, P]),
        "aexq_dequant": (i32, [P, P, P]),
        "aexq_rmsnorm": (i32, [P, TP, TP, P, i32, f32]),
        "aexq_embed_q8": (i32, [P, P, P, i32, P]),
        "aexq_rope_kv_append": (i32, [P, P, P, P, P, P, i32, i32, i32, i32, i32, P, P]),
        "aexq_attention_decode": (i32, [P, P, P, P, i32, i32, i32, i32, i32, f32, P]),
        "aexq_attention_decode_rope": (i32, [P, P, P, P, P, P, i32, i32, i32, i32, i32, P, P,
                                             f32, P]),
        "aexq_attention_decode_rope_at": (i32, [P, P, P, P, P, P, i32, i32, i32, i32, P, P, P,
                                                f32, P]),
        "aexq_decode_advance": (i32, [P, P, P, P, P, i32]),
        "aexq_decoder_create": (i32, [P, ctypes.POINTER(DecoderConfig), ctypes.POINTER(DecoderLayer),
                                      i32, P, PP]),
        "aexq_decoder_run": (i32, [P, P, P, P]),
        "aexq_decoder_error": (i32, [P, ctypes.POINTER(i32)]),
        "aexq_decoder_info": (i32, [P, ctypes.POINTER(i32), ctypes.POINTER(i32),
                                    ctypes.POINTER(i32)]),
        "aexq_decoder_release": (None, [P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def check(status: int, what: str = "") -> None:
    if status == OK:
        return
    msg = load().aexq_last_error().decode(errors="replace")
    exc = _STATUS_EXC.get(status, AexqError)
    raise exc(status, f"{what}: {msg}" if what else msg)


def last_error() -> str:
    return load().aexq_last_error().decode(errors="replace")
