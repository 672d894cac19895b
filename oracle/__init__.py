"""ctypes binding of the CPU oracle (oracle/aexq_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP library and the CPU
baseline timed by bench.py.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this module; the product package
(aiimage_amd) never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

SCALE_F16 = 1
SCALE_F32 = 2
NIBBLE_TWOS = 0
NIBBLE_OFFSET8 = 1
RECORD_Q8, RECORD_RAW, RECORD_Q4 = 1, 2, 3

_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc)."""
    args = ["make", "-s", "-C", HERE]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    P = ctypes.c_void_p
    i32, f32, sz, i64 = ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_int64
    sig = {
        "orc_half_to_float": (f32, [ctypes.c_uint16]),
        "orc_float_to_half": (ctypes.c_uint16, [f32]),
        "orc_round_to_int": (i32, [f32]),
        "orc_q8_pack_rows": (i32, [P, i32, i32, i32, P, P]),
        "orc_q4_pack_rows": (i32, [P, i32, i32, i32, P, P, P]),
        "orc_archive_header": (sz, [P, i32, i32, i32, i64]),
        "orc_record_write_q8": (sz, [P, i32, i32, P]),
        "orc_record_write_q4": (sz, [P, i32, i32, P]),
        "orc_record_write_raw_f32": (sz, [P, i32, P]),
        "orc_record_write_q4_from_q8_rows": (sz, [P, P, i32, i32, i32, P]),
        "orc_archive_parse_header": (i32, [P, sz, P, P, P]),
        "orc_record_read_array": (i32, [P, sz, i32, P, P]),
        "orc_record_read_q8_packed": (i32, [P, sz, i32, i32, P, P, P, P]),
        "orc_record_read_q4_packed": (i32, [P, sz, i32, i32, P, P, P, P]),
        "orc_dequant_q8": (i32, [P, P, i32, i32, i32, i32, P]),
        "orc_dequant_q4": (i32, [P, P, i32, i32, i32, i32, i32, P]),
        "orc_gemm_cpu": (None, [P, i32, i32, P, i32, i32, f32, f32, P, i32, P]),
        "orc_gemm_cpu_mt": (None, [P, i32, i32, P, i32, i32, f32, f32, P, i32, P, i32]),
        "orc_gemm_gpu_semantics": (None, [P, i32, i32, P, i32, f32, f32, P, i32, P]),
        "orc_rmsnorm": (None, [P, i32, i32, f32, P, i32, P]),
        "orc_swish": (f32, [f32]),
        "orc_swiglu": (None, [P, P, i32, P]),
        "orc_argmax_rows": (None, [P, i32, i32, i64, P]),
        "orc_rope_table": (None, [i32, i32, ctypes.c_double, P, P]),
        "orc_rope_rotate_half": (None, [P, i32, i32, P, P, P]),
        "orc_sdpa_decode": (None, [P, P, P, i32, i32, i32, i32, f32, P]),
        "orc_head_pack": (None, [P, i32, i32, i32, P]),
        "orc_head_unpack": (None, [P, i32, i32, i32, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- scalar helpers --------------------------------------------------------

def half_to_float(bits: int) -> float:
    return lib().orc_half_to_float(int(bits))


def float_to_half(v: float) -> int:
    return lib().orc_float_to_half(float(v))


def round_to_int(v: float) -> int:
    return lib().orc_round_to_int(float(v))


# ---- packers ---------------------------------------------------------------

def q8_pack_rows(data, rows: int, cols: int, contiguous: bool = True):
    d = _c(data, np.float32).ravel()
    packed = np.zeros(max(1, (rows * cols + 3) // 4), np.uint32)
    scales = np.zeros(rows, np.float32)
    rc = lib().orc_q8_pack_rows(_p(d), rows, cols, int(contiguous), _p(packed), _p(scales))
    if rc:
        raise ValueError(f"orc_q8_pack_rows rc={rc}")
    return packed, scales


def q4_pack_rows(data, rows: int, cols: int, contiguous: bool = True):
    d = _c(data, np.float32).ravel()
    packed = np.zeros(max(1, (rows * cols + 7) // 8), np.uint32)
    scales = np.zeros(rows, np.float32)
    blk = ctypes.c_int(0)
    rc = lib().orc_q4_pack_rows(_p(d), rows, cols, int(contiguous), _p(packed), _p(scales),
                                ctypes.byref(blk))
    if rc:
        raise ValueError(f"orc_q4_pack_rows rc={rc}")
    return packed, scales, blk.value


# ---- archive ---------------------------------------------------------------

def archive_header(quant_bits: int, default_block: int, record_count: int, source_bytes: int) -> bytes:
    buf = np.zeros(32, np.uint8)
    lib().orc_archive_header(_p(buf), quant_bits, default_block, record_count, source_bytes)
    return buf.tobytes()


def record_write_q8(values, block: int) -> bytes:
    v = _c(values, np.float32).ravel()
    size = lib().orc_record_write_q8(_p(v), v.size, block, None)
    buf = np.zeros(size, np.uint8)
    lib().orc_record_write_q8(_p(v), v.size, block, _p(buf))
    return buf.tobytes()


def record_write_q4(values, block: int) -> bytes:
    v = _c(values, np.float32).ravel()
    size = lib().orc_record_write_q4(_p(v), v.size, block, None)
    buf = np.zeros(size, np.uint8)
    lib().orc_record_write_q4(_p(v), v.size, block, _p(buf))
    return buf.tobytes()


def record_write_raw_f32(values) -> bytes:
    v = _c(values, np.float32).ravel()
    size = lib().orc_record_write_raw_f32(_p(v), v.size, None)
    buf = np.zeros(size, np.uint8)
    lib().orc_record_write_raw_f32(_p(v), v.size, _p(buf))
    return buf.tobytes()


def record_write_q4_from_q8_rows(q8_packed, q8_scales, rows: int, row_size: int, group: int) -> bytes:
    pk = _c(q8_packed, np.uint32)
    sc = _c(q8_scales, np.float32)
    size = lib().orc_record_write_q4_from_q8_rows(_p(pk), _p(sc), rows, row_size, group, None)
    if size == 0:
        raise ValueError("invalid Q8->Q4 row conversion arguments")
    buf = np.zeros(size, np.uint8)
    lib().orc_record_write_q4_from_q8_rows(_p(pk), _p(sc), rows, row_size, group, _p(buf))
    return buf.tobytes()


def archive_parse_header(buf: bytes):
    b = np.frombuffer(buf, np.uint8).copy()
    bits, blk, rec = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    rc = lib().orc_archive_parse_header(_p(b), b.size, ctypes.byref(bits), ctypes.byref(blk),
                                        ctypes.byref(rec))
    return rc, bits.value, blk.value, rec.value


def record_read_array(rec: bytes, expected_count: int):
    b = np.frombuffer(rec, np.uint8).copy()
    out = np.zeros(max(1, expected_count), np.float32)
    used = ctypes.c_size_t(0)
    rc = lib().orc_record_read_array(_p(b), b.size, expected_count, _p(out), ctypes.byref(used))
    return rc, out[:expected_count], used.value


def record_read_q8_packed(rec: bytes, expected_count: int, expected_block: int = 0):
    b = np.frombuffer(rec, np.uint8).copy()
    packed = np.zeros(max(1, (expected_count + 3) // 4), np.uint32)
    scales = np.zeros(max(1, expected_count), np.float32)
    blk, used = ctypes.c_int(0), ctypes.c_size_t(0)
    rc = lib().orc_record_read_q8_packed(_p(b), b.size, expected_count, expected_block, _p(packed),
                                         _p(scales), ctypes.byref(blk), ctypes.byref(used))
    nb = 0 if expected_count == 0 or blk.value <= 0 else -(-expected_count // blk.value)
    return rc, packed, scales[:nb], blk.value, used.value


def record_read_q4_packed(rec: bytes, expected_count: int, expected_block: int = 0):
    b = np.frombuffer(rec, np.uint8).copy()
    packed = np.zeros(max(1, (expected_count + 7) // 8), np.uint32)
    scales = np.zeros(max(1, expected_count), np.float32)
    blk, used = ctypes.c_int(0), ctypes.c_size_t(0)
    rc = lib().orc_record_read_q4_packed(_p(b), b.size, expected_count, expected_block, _p(packed),
                                         _p(scales), ctypes.byref(blk), ctypes.byref(used))
    nb = 0 if expected_count == 0 or blk.value <= 0 else -(-expected_count // blk.value)
    return rc, packed, scales[:nb], blk.value, used.value


# ---- dequant ---------------------------------------------------------------

def _scale_arr(scales, scale_dtype):
    return _c(scales, np.float16 if scale_dtype == SCALE_F16 else np.float32)


def dequant_q8(words, scales, n: int, k: int, scale_dtype: int = SCALE_F32, block: int = 0):
    w = _c(words, np.uint32)
    s = _scale_arr(scales, scale_dtype)
    out = np.empty((n, k), np.float32)
    rc = lib().orc_dequant_q8(_p(w), _p(s), scale_dtype, n, k, block, _p(out))
    if rc:
        raise ValueError(f"orc_dequant_q8 rc={rc}")
    return out


def dequant_q4(words, scales, n: int, k: int, block: int, nibble_code: int = NIBBLE_TWOS,
               scale_dtype: int = SCALE_F32):
    w = _c(words, np.uint32)
    s = _scale_arr(scales, scale_dtype)
    out = np.empty((n, k), np.float32)
    rc = lib().orc_dequant_q4(_p(w), _p(s), scale_dtype, n, k, block, nibble_code, _p(out))
    if rc:
        raise ValueError(f"orc_dequant_q4 rc={rc}")
    return out


# ---- gemm ------------------------------------------------------------------

def gemm_cpu(a, b, n: int, trans_b: bool = True, alpha: float = 1.0, beta: float = 1.0, c=None,
             broadcast_c: int = -1, threads: int = 1):
    """RunGemmCpu restatement; a is [m][k], b is [n][k] (trans_b) or [k][n]."""
    a = _c(a, np.float32)
    m, k = a.shape
    b = _c(b, np.float32)
    cc = None if c is None else _c(c, np.float32)
    out = np.empty((m, n), np.float32)
    if threads > 1:
        lib().orc_gemm_cpu_mt(_p(a), m, k, _p(b), n, int(trans_b), alpha, beta, _p(cc), broadcast_c,
                              _p(out), threads)
    else:
        lib().orc_gemm_cpu(_p(a), m, k, _p(b), n, int(trans_b), alpha, beta, _p(cc), broadcast_c,
                           _p(out))
    return out


def gemm_gpu_semantics(a, b, alpha: float = 1.0, beta: float = 1.0, c=None, broadcast_c: int = -1):
    """Pack4-linear Gemm semantics alpha*(beta*C + a.b^T) in float64; b is [n][k]."""
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    m, k = a.shape
    n = b.shape[0]
    cc = None if c is None else _c(c, np.float32)
    out = np.empty((m, n), np.float64)
    lib().orc_gemm_gpu_semantics(_p(a), m, k, _p(b), n, alpha, beta, _p(cc), broadcast_c, _p(out))
    return out


# ---- epilogues / argmax ----------------------------------------------------

def rmsnorm(x, eps: float, gamma=None):
    x = _c(x, np.float32)
    if x.ndim == 1:
        x = x[None, :]
    rows, width = x.shape
    g = None if gamma is None else _c(gamma, np.float32)
    out = np.empty_like(x)
    lib().orc_rmsnorm(_p(x), rows, width, eps, _p(g), 0 if g is None else g.size, _p(out))
    return out


def swish(x: float) -> float:
    return lib().orc_swish(float(x))


def swiglu(gate, up):
    g = _c(gate, np.float32).ravel()
    u = _c(up, np.float32).ravel()
    out = np.empty_like(g)
    lib().orc_swiglu(_p(g), _p(u), g.size, _p(out))
    return out


def argmax_rows(logits, width: int | None = None):
    x = _c(logits, np.float32)
    if x.ndim == 1:
        x = x[None, :]
    rows, stride = x.shape
    w = stride if width is None else width
    out = np.empty(rows, np.int32)
    lib().orc_argmax_rows(_p(x), rows, w, stride, _p(out))
    return out


# ---- decode step around the linears -----------------------------------------

def rope_table(position: int, head_dim: int, base: float):
    """(cos, sin) float32 [head_dim/2] of one position (rotate-half layout)."""
    c = np.empty(head_dim // 2, np.float32)
    s = np.empty(head_dim // 2, np.float32)
    lib().orc_rope_table(position, head_dim, base, _p(c), _p(s))
    return c, s


def rope_rotate_half(x, cos_t, sin_t):
    """x [heads][head_dim] rotated per PN:414-473 (non-interleaved)."""
    x = _c(x, np.float32)
    heads, d = x.shape
    out = np.empty_like(x)
    lib().orc_rope_rotate_half(_p(x), heads, d, _p(_c(cos_t, np.float32)), _p(_c(sin_t, np.float32)),
                               _p(out))
    return out


def sdpa_decode(q, k, v, scale: float):
    """One query row: q [hq][d], k/v [hkv][length][d] -> float64 [hq][d] (MM:420-544)."""
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    hq, d = q.shape
    hkv, length, _ = k.shape
    out = np.empty((hq, d), np.float64)
    lib().orc_sdpa_decode(_p(q), _p(k), _p(v), hq, hkv, d, length, scale, _p(out))
    return out


def head_pack(x, heads: int, head_dim: int):
    """[rows][heads*head_dim] -> the attention head-packed storage (MM:1192-1318),
    flat float32 of ceil(heads/4) * rows * head_dim * 4 values."""
    x = _c(x, np.float32)
    rows = x.shape[0]
    out = np.empty(((heads + 3) // 4) * rows * head_dim * 4, np.float32)
    lib().orc_head_pack(_p(x), rows, heads, head_dim, _p(out))
    return out


def head_unpack(buf, rows: int, heads: int, head_dim: int):
    """Head-packed storage -> [rows][heads*head_dim] (MM:1320-1389 reads)."""
    buf = _c(buf, np.float32)
    out = np.empty((rows, heads * head_dim), np.float32)
    lib().orc_head_unpack(_p(buf), rows, heads, head_dim, _p(out))
    return out
