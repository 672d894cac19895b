"""Host-side mirror of Aexis's quantized Gemm operator over the aexq C ABI.

Reference (paths relative to the reference root):
  GL  = Packages/com.aexis/Runtime/Execution/Layers/AexisGemmLayer.cs
  GS  = Packages/com.aexis/Runtime/Execution/Graph/AexisGraphSession.cs
  WR  = Packages/com.aexis/Runtime/Execution/Graph/AexisWeightReader.cs

The classes keep the reference's names and argument meaning so a caller of
AexisGemmLayer finds the same contract: ncnn Gemm parameter ids, direct Q4/Q8
records (AexisQuantizedTensor), Pack4 storage-shape rules, and exceptions for
unsupported combinations instead of a fallback.  Device memory and streams
come from torch (HIP); every computation runs in libaexq.so.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np
import torch

from . import _abi
from ._abi import (DTYPE_F16, DTYPE_F32, EPI_RESIDUAL_ADD, EPI_RMSNORM_IN, EPI_SWIGLU_OUT,
                   LAYOUT_HEAD_PACKED, LAYOUT_LINEAR, LAYOUT_PACK4_LINEAR, LAYOUT_PACK4_TILED,
                   NIBBLE_OFFSET8,
                   NIBBLE_TWOS, InvalidOperationError, NotSupportedError, check)

MAX_TEXTURE_SIZE = 16384      # SystemInfo.maxTextureSize of the desktop targets
TILE_WIDTH_LIMIT = 8192       # GS:10852 min(8192, maxTextureSize)


# ---------------------------------------------------------------- storage shapes

def pack4_linear_storage(rows: int, width: int) -> tuple:
    """ResolvePack4LinearMatStorageShape (GS:10836-10841): {3, ceil(w/4), h, 1, 4}."""
    return (3, -(-max(1, width) // 4), max(1, rows), 1, 4)


def pack4_tiled_storage(rows: int, width: int, max_texture: int = MAX_TEXTURE_SIZE) -> tuple:
    """ResolvePack4TiledLinearMatStorageShape (GS:10843-10852)."""
    packs = -(-max(1, width) // 4)
    tile_w = min(packs, max(1, min(TILE_WIDTH_LIMIT, max_texture)))
    tile_rows = -(-packs // tile_w)
    return (3, tile_w, max(1, rows) * tile_rows, 1, 4)


def head_packed_storage(rows: int, heads: int, head_dim: int) -> tuple:
    """BufferShape of the attention head-packed layout (GL:1003-1043): {3, head_dim,
    rows, 1, heads}, stored as ceil(heads/4) slices of rows x head_dim float4 texels."""
    return (3, head_dim, max(1, rows), 1, heads)


def tensor_elements(layout: int, rows: int, width: int, head_dim: int = 0) -> int:
    """Elements one [rows][width] tensor occupies in storage."""
    if layout == LAYOUT_HEAD_PACKED:
        if head_dim <= 0 or width % head_dim:
            raise InvalidOperationError(_abi.ERR_SHAPE, f"width {width} is not heads x head_dim {head_dim}")
        return -(-(width // head_dim) // 4) * max(1, rows) * head_dim * 4
    return storage_elements(layout, rows, width) * rows


def storage_elements(layout: int, rows: int, width: int) -> int:
    """Elements of one row as laid out in storage (row stride)."""
    if layout == LAYOUT_LINEAR:
        return width
    if layout == LAYOUT_PACK4_LINEAR:
        return pack4_linear_storage(rows, width)[1] * 4
    if layout == LAYOUT_PACK4_TILED:
        s = pack4_tiled_storage(rows, width)
        return s[1] * (s[2] // max(1, rows)) * 4
    raise NotSupportedError(_abi.ERR_UNSUPPORTED, f"layout {layout} has no storage rule here")


def output_layout_for(n: int, max_texture: int = MAX_TEXTURE_SIZE) -> int:
    """GL:515-525: tiled when ceil(n/4) exceeds the texture limit, else Pack4
    linear when n % 4 == 0, else LinearMat."""
    if -(-n // 4) > max_texture:
        return LAYOUT_PACK4_TILED
    return LAYOUT_PACK4_LINEAR if n % 4 == 0 else LAYOUT_LINEAR


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float16:
        return DTYPE_F16
    if t.dtype == torch.float32:
        return DTYPE_F32
    raise NotSupportedError(_abi.ERR_UNSUPPORTED, f"dtype {t.dtype} is not a texture format")


def describe(t: torch.Tensor, rows: int, width: int, layout: int = LAYOUT_LINEAR,
             batch: int = 1, batch_stride: int = 0, head_dim: int = 0) -> _abi.Tensor:
    """aexq_tensor for a device tensor holding `batch` [rows][width] matrices
    (`head_dim` for the attention head-packed layout)."""
    d = _abi.Tensor()
    d.logical = _abi.Shape(2, width, rows, 1, 1)
    if layout == LAYOUT_HEAD_PACKED:
        if head_dim <= 0 or width % head_dim:
            raise InvalidOperationError(_abi.ERR_SHAPE, f"width {width} is not heads x head_dim {head_dim}")
        d.storage = _abi.Shape(*head_packed_storage(rows, width // head_dim, head_dim))
    elif layout == LAYOUT_LINEAR:
        d.storage = _abi.Shape(2, width, rows, 1, 1)
    elif layout == LAYOUT_PACK4_LINEAR:
        d.storage = _abi.Shape(*pack4_linear_storage(rows, width))
    elif layout == LAYOUT_PACK4_TILED:
        d.storage = _abi.Shape(*pack4_tiled_storage(rows, width))
    else:
        raise NotSupportedError(_abi.ERR_UNSUPPORTED, f"layout {layout}")
    need = tensor_elements(layout, rows, width, head_dim) + (batch - 1) * batch_stride
    if t.numel() < need:
        raise InvalidOperationError(_abi.ERR_SHAPE,
                                    f"tensor holds {t.numel()} elements, layout needs {need}")
    d.layout = layout
    d.dtype = _dtype_code(t)
    d.data = t.data_ptr()
    d.batch = batch
    d.batch_stride = batch_stride
    d._keep = t   # the descriptor keeps its device buffer alive until launch
    return d


def new_activation(rows: int, width: int, dtype=torch.float16, layout: int = LAYOUT_LINEAR,
                   device: str = "cuda", batch: int = 1, head_dim: int = 0) -> torch.Tensor:
    """A zeroed device buffer with the storage of `layout` for [batch][rows][width]."""
    per = tensor_elements(layout, rows, width, head_dim)
    return torch.zeros(batch * per, dtype=dtype, device=device)


# ---------------------------------------------------------------- records

@dataclass
class QuantizedTensor:
    """AexisQuantizedTensor(ElementCount, BlockSize, PackedValues, Scales) (WR:30-44),
    plus the two properties the synthetic format varies: scale dtype and nibble code."""

    element_count: int
    block_size: int
    packed_values: np.ndarray   # uint32 words
    scales: np.ndarray          # float32 (reference) or float16 (synthetic)
    bits: int = 8
    nibble_code: int = NIBBLE_TWOS

    @property
    def scale_dtype(self) -> int:
        return DTYPE_F16 if self.scales.dtype == np.float16 else DTYPE_F32


# ---------------------------------------------------------------- context / weights

def _stream_handle(stream) -> ctypes.c_void_p:
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


class Context:
    """aexq_ctx: the per-thread dispatch state (replaces AexisOps, OPS:706-760)."""

    def __init__(self, device: int = 0, stream=None):
        self._lib = _abi.load()
        self.device = device
        self.stream = stream if stream is not None else torch.cuda.current_stream(device)
        h = ctypes.c_void_p()
        check(self._lib.aexq_create(device, _stream_handle(self.stream), ctypes.byref(h)),
              "aexq_create")
        self.handle = h

    def close(self):
        if self.handle:
            self._lib.aexq_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self):
        check(self._lib.aexq_synchronize(self.handle), "aexq_synchronize")

    def set_stream(self, stream):
        """Enqueue subsequent work on `stream` (a torch HIP stream)."""
        self.stream = stream
        check(self._lib.aexq_set_stream(self.handle, _stream_handle(stream)), "aexq_set_stream")

    # ---- weights
    def weight(self, qt: QuantizedTensor, n: int, k: int) -> "QuantWeight":
        """Direct upload of a packed record (GS:12887-12907 / GS:12966-12996)."""
        if qt.element_count != n * k:
            raise _abi.ArgumentError(_abi.ERR_INVALID_ARGUMENT,
                                     "Direct upload shape does not match Gemm output channels and K.")
        pk = np.ascontiguousarray(qt.packed_values, np.uint32)
        sc = np.ascontiguousarray(qt.scales)
        h = ctypes.c_void_p()
        if qt.bits == 8:
            if sc.size != n:
                raise _abi.ArgumentError(_abi.ERR_INVALID_ARGUMENT,
                                         "Direct Q8 upload must contain one scale per output channel.")
            st = self._lib.aexq_weight_q8(self.handle, pk.ctypes.data, sc.ctypes.data,
                                          qt.scale_dtype, n, k, qt.block_size, ctypes.byref(h))
        else:
            if qt.block_size <= 0 or k % qt.block_size != 0 or sc.size != n * k // qt.block_size:
                raise _abi.ArgumentError(_abi.ERR_INVALID_ARGUMENT,
                                         "Direct Q4 upload scale count does not match its group size.")
            st = self._lib.aexq_weight_q4(self.handle, pk.ctypes.data, sc.ctypes.data,
                                          qt.scale_dtype, n, k, qt.block_size, qt.nibble_code,
                                          ctypes.byref(h))
        check(st, "weight upload")
        return QuantWeight(self, h)

    def weight_from_float(self, data: np.ndarray, n: int, k: int, bits: int = 8,
                          trans_b: bool = True) -> "QuantWeight":
        """Float overloads of NewInt8/Int4WeightOnlyUpload (GS:12838-12885, 12912-12964)."""
        d = np.ascontiguousarray(data, np.float32)
        h = ctypes.c_void_p()
        fn = self._lib.aexq_weight_q8_from_f32 if bits == 8 else self._lib.aexq_weight_q4_from_f32
        check(fn(self.handle, d.ctypes.data, n, k, int(trans_b), ctypes.byref(h)), "weight_from_float")
        return QuantWeight(self, h)

    def weight_from_record(self, record: bytes, n: int, k: int, bits: int) -> tuple:
        """One AQSGET8 Gemm weight record into the device layout, as
        AexisGemmLayer.LoadLayer reads and uploads it (GL:60-141).  Returns
        (weight, bytes consumed)."""
        buf = np.frombuffer(record, np.uint8)
        h = ctypes.c_void_p()
        used = ctypes.c_size_t(0)
        check(self._lib.aexq_weight_from_record(self.handle, bits, buf.ctypes.data, buf.size, n, k,
                                                ctypes.byref(h), ctypes.byref(used)),
              "weight_from_record")
        return QuantWeight(self, h), used.value

    # ---- execution
    def linear(self, w: "QuantWeight", x: _abi.Tensor, y: _abi.Tensor, *, alpha: float = 1.0,
               beta: float = 1.0, c: Optional[torch.Tensor] = None, broadcast_c: int = -1,
               rms_gamma: Optional[torch.Tensor] = None, rms_eps: float = 1e-3,
               rmsnorm: bool = False, up: Optional["QuantWeight"] = None,
               residual: Optional[_abi.Tensor] = None, exact: bool = False):
        args = make_args(alpha, beta, c, broadcast_c, rms_gamma, rms_eps, rmsnorm, up, residual,
                         exact)
        check(self._lib.aexq_linear(self.handle, w.handle, ctypes.byref(x), ctypes.byref(y),
                                    ctypes.byref(args)), "aexq_linear")

    def linear_group(self, ws: Sequence["QuantWeight"], x: _abi.Tensor, ys: Sequence[_abi.Tensor],
                     **kw):
        args = make_args(**kw)
        n = len(ws)
        warr = (ctypes.c_void_p * n)(*[w.handle.value for w in ws])
        yptrs = (ctypes.POINTER(_abi.Tensor) * n)(*[ctypes.pointer(y) for y in ys])
        check(self._lib.aexq_linear_group(self.handle, n, warr, ctypes.byref(x), yptrs,
                                          ctypes.byref(args)), "aexq_linear_group")

    def plan_check(self, w: "QuantWeight", x: _abi.Tensor, y: _abi.Tensor, **kw) -> str:
        args = make_args(**kw)
        buf = ctypes.create_string_buffer(1024)
        st = self._lib.aexq_plan_check(self.handle, w.handle, ctypes.byref(x), ctypes.byref(y),
                                       ctypes.byref(args), buf, len(buf))
        check(st, "aexq_plan_check")
        return buf.value.decode()

    def lmhead_argmax(self, w: "QuantWeight", x: _abi.Tensor, logits: Optional[_abi.Tensor],
                      argmax: torch.Tensor, top2_gap: Optional[torch.Tensor] = None, *,
                      rms_gamma: Optional[torch.Tensor] = None, rms_eps: float = 1e-3,
                      rmsnorm: bool = False, argmax_f16: bool = False):
        """Greedy token of the LM head; with rmsnorm=True the final RMSNorm
        (gamma rms_gamma) is applied to x inside the same launch; with
        argmax_f16=True the argmax compares the logits rounded to fp16 (the
        reference's ARGBHalf logits texture, GL:383-396)."""
        gap = ctypes.c_void_p(top2_gap.data_ptr()) if top2_gap is not None else None
        lg = ctypes.byref(logits) if logits is not None else None
        if rmsnorm or argmax_f16:
            args = make_args(rms_gamma=rms_gamma, rms_eps=rms_eps, rmsnorm=rmsnorm)
            if argmax_f16:
                args.flags |= _abi.EPI_ARGMAX_F16
            check(self._lib.aexq_lmhead_argmax_ex(
                self.handle, w.handle, ctypes.byref(x), lg, ctypes.byref(args),
                ctypes.c_void_p(argmax.data_ptr()), gap), "aexq_lmhead_argmax_ex")
            return
        check(self._lib.aexq_lmhead_argmax(
            self.handle, w.handle, ctypes.byref(x), lg,
            ctypes.c_void_p(argmax.data_ptr()), gap), "aexq_lmhead_argmax")

    def lmhead_argmax_noalloc(self, w: "QuantWeight", x: _abi.Tensor, argmax: torch.Tensor,
                              top2_gap: Optional[torch.Tensor] = None):
        """lmhead_argmax that allocates nothing (a fixed device scratch)."""
        check(self._lib.aexq_lmhead_argmax_noalloc(
            self.handle, w.handle, ctypes.byref(x), ctypes.c_void_p(argmax.data_ptr()),
            ctypes.c_void_p(top2_gap.data_ptr()) if top2_gap is not None else None),
            "aexq_lmhead_argmax_noalloc")

    def argmax(self, logits: _abi.Tensor, argmax: torch.Tensor,
               top2_gap: Optional[torch.Tensor] = None):
        check(self._lib.aexq_argmax(self.handle, ctypes.byref(logits),
                                    ctypes.c_void_p(argmax.data_ptr()),
                                    ctypes.c_void_p(top2_gap.data_ptr()) if top2_gap is not None else None),
              "aexq_argmax")

    # ---- decode-step operators around the linears
    def rmsnorm(self, x: _abi.Tensor, y: _abi.Tensor, gamma: Optional[torch.Tensor] = None,
                eps: float = 1e-3):
        """AexisRMSNormLayer (RMS:24-46): y = fp16(x * rsqrt(mean x^2 + eps) * gamma)."""
        check(self._lib.aexq_rmsnorm(self.handle, ctypes.byref(x), ctypes.byref(y),
                                     ctypes.c_void_p(gamma.data_ptr()) if gamma is not None else None,
                                     gamma.numel() if gamma is not None else 0, eps), "aexq_rmsnorm")

    def embed_q8(self, table: "QuantWeight", tokens: torch.Tensor, out: torch.Tensor):
        """Tied Q8 embedding rows (Qwen35SharedTokenEmbeddingWeights.cs:185-198)."""
        check(self._lib.aexq_embed_q8(self.handle, table.handle, ctypes.c_void_p(tokens.data_ptr()),
                                      tokens.numel(), ctypes.c_void_p(out.data_ptr())),
              "aexq_embed_q8")

    def rope_kv_append(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       k_cache: torch.Tensor, v_cache: torch.Tensor, heads_q: int, heads_kv: int,
                       head_dim: int, capacity: int, position: int, cos_t: torch.Tensor,
                       sin_t: torch.Tensor):
        """RoPE (PN:414-473, rotate-half) on q in place and k into the cache; v appended."""
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        check(self._lib.aexq_rope_kv_append(self.handle, P(q), P(k), P(v), P(k_cache), P(v_cache),
                                            heads_q, heads_kv, head_dim, capacity, position,
                                            P(cos_t), P(sin_t)), "aexq_rope_kv_append")

    def attention_decode(self, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                         heads_q: int, heads_kv: int, head_dim: int, capacity: int, length: int,
                         scale: float, out: torch.Tensor):
        """GQA decode attention over the cache (MM:420-544)."""
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        check(self._lib.aexq_attention_decode(self.handle, P(q), P(k_cache), P(v_cache), heads_q,
                                              heads_kv, head_dim, capacity, length, scale, P(out)),
              "aexq_attention_decode")

    def attention_decode_rope(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                              k_cache: torch.Tensor, v_cache: torch.Tensor, heads_q: int,
                              heads_kv: int, head_dim: int, capacity: int, length: int,
                              cos_t: torch.Tensor, sin_t: torch.Tensor, scale: float,
                              out: torch.Tensor):
        """RoPE + K/V append at position length-1 + decode attention in one pass."""
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        check(self._lib.aexq_attention_decode_rope(self.handle, P(q), P(k), P(v), P(k_cache),
                                                   P(v_cache), heads_q, heads_kv, head_dim,
                                                   capacity, length, P(cos_t), P(sin_t), scale,
                                                   P(out)), "aexq_attention_decode_rope")

    def attention_decode_rope_at(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                 k_cache: torch.Tensor, v_cache: torch.Tensor, heads_q: int,
                                 heads_kv: int, head_dim: int, capacity: int,
                                 position: torch.Tensor, cos_table: torch.Tensor,
                                 sin_table: torch.Tensor, scale: float, out: torch.Tensor):
        """attention_decode_rope at the device-side position (int32 tensor of one
        element); cos/sin tables are [capacity][head_dim/2] fp32."""
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        check(self._lib.aexq_attention_decode_rope_at(self.handle, P(q), P(k), P(v), P(k_cache),
                                                      P(v_cache), heads_q, heads_kv, head_dim,
                                                      capacity, P(position), P(cos_table),
                                                      P(sin_table), scale, P(out)),
              "aexq_attention_decode_rope_at")

    def decode_advance(self, position: torch.Tensor, token: torch.Tensor, argmax: torch.Tensor,
                       tokens_out: Optional[torch.Tensor] = None):
        """Device-side end of a generated token (DEC:1160-1237)."""
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        check(self._lib.aexq_decode_advance(
            self.handle, P(position), P(token), P(argmax),
            P(tokens_out) if tokens_out is not None else None,
            tokens_out.numel() if tokens_out is not None else 0), "aexq_decode_advance")

    def decoder(self, layers, embedding: "QuantWeight", heads_q: int, heads_kv: int,
                head_dim: int, capacity: int, rms_eps: float, attn_scale: float,
                rope_cos: torch.Tensor, rope_sin: torch.Tensor, workgroups: int = 0) -> "Decoder":
        """The decoder layers of a decode step as one launch (aexq_decoder_create).
        `layers` is a sequence of dicts with the seven Q4 weights (q_proj ...
        down_proj), the two gammas (attn_norm, mlp_norm) and the fp16 caches."""
        return Decoder(self, layers, embedding, heads_q, heads_kv, head_dim, capacity, rms_eps,
                       attn_scale, rope_cos, rope_sin, workgroups)

    def dequant(self, w: "QuantWeight") -> torch.Tensor:
        info = w.info()
        out = torch.empty((info.n, info.k), dtype=torch.float32, device=f"cuda:{self.device}")
        check(self._lib.aexq_dequant(self.handle, w.handle, ctypes.c_void_p(out.data_ptr())),
              "aexq_dequant")
        return out


def archive_header(buf: bytes) -> tuple:
    """(quant_bits, default_block, record_count) of an AQSGET8 archive header
    (Q8A:277-293); raises InvalidDataError for a malformed one."""
    b = np.frombuffer(buf, np.uint8)
    bits, blk, rec = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    check(_abi.load().aexq_archive_header(b.ctypes.data, b.size, ctypes.byref(bits),
                                          ctypes.byref(blk), ctypes.byref(rec)),
          "archive_header")
    return bits.value, blk.value, rec.value


def make_args(alpha: float = 1.0, beta: float = 1.0, c: Optional[torch.Tensor] = None,
              broadcast_c: int = -1, rms_gamma: Optional[torch.Tensor] = None,
              rms_eps: float = 1e-3, rmsnorm: bool = False, up: Optional["QuantWeight"] = None,
              residual: Optional[_abi.Tensor] = None, exact: bool = False) -> _abi.LinearArgs:
    """aexq_linear_args; exact=True keeps Q4 dequantisation exact in the tiled
    GEMM (AEXQ_EPI_EXACT_DEQUANT) instead of fp16 weight tiles."""
    a = _abi.LinearArgs()
    a.alpha = alpha
    a.beta = beta
    a.c = c.data_ptr() if c is not None else None
    a.broadcast_c = broadcast_c
    a.rms_gamma = rms_gamma.data_ptr() if rms_gamma is not None else None
    a.rms_gamma_size = rms_gamma.numel() if rms_gamma is not None else 0
    a.rms_eps = rms_eps
    a.up = up.handle.value if up is not None else None
    a.residual = ctypes.pointer(residual) if residual is not None else None
    flags = 0
    if rmsnorm:
        flags |= EPI_RMSNORM_IN
    if up is not None:
        flags |= EPI_SWIGLU_OUT
    if residual is not None:
        flags |= EPI_RESIDUAL_ADD
    if exact:
        flags |= _abi.EPI_EXACT_DEQUANT
    a.flags = flags
    a._keep = (c, rms_gamma, up, residual)
    return a


class QuantWeight:
    """aexq_weight handle (library-owned device copy)."""

    def __init__(self, ctx: Context, handle: ctypes.c_void_p, owner: "QuantWeight" = None):
        self.ctx = ctx
        self.handle = handle
        self._owner = owner

    def info(self) -> _abi.WeightInfo:
        inf = _abi.WeightInfo()
        check(self.ctx._lib.aexq_weight_get_info(self.handle, ctypes.byref(inf)), "weight info")
        return inf

    def replicate(self, batch: int) -> "QuantWeight":
        h = ctypes.c_void_p()
        check(self.ctx._lib.aexq_weight_replicate(self.ctx.handle, self.handle, batch,
                                                  ctypes.byref(h)), "replicate")
        return QuantWeight(self.ctx, h)

    def alias(self) -> "QuantWeight":
        """Tied embedding / LM head share (GL:91-111, owns=false)."""
        h = ctypes.c_void_p()
        check(self.ctx._lib.aexq_weight_alias(self.ctx.handle, self.handle, ctypes.byref(h)),
              "alias")
        return QuantWeight(self.ctx, h, owner=self)

    def release(self):
        if self.handle:
            self.ctx._lib.aexq_weight_release(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


# ---------------------------------------------------------------- the operator

class HipGemmLayer:
    """Drop-in for AexisGemmLayer on the quantized path (GL:15-162, 280-601).

    `params` are ncnn Gemm params by id: 0 alpha, 1 beta, 2 transA, 3 transB,
    4 constantA, 5 constantB, 6 constantC, 7 M, 8 N, 9 K, 10 broadcastTypeC.
    """

    def __init__(self, ctx: Context, name: str = "gemm"):
        self.ctx = ctx
        self.name = name
        self.weight: Optional[QuantWeight] = None
        self.c: Optional[torch.Tensor] = None

    def load_layer(self, params: dict, weights, bias: Optional[np.ndarray] = None):
        """LoadLayer (GL:15-162): direct Q4/Q8 records or float weights."""
        self.alpha = float(params.get(0, 1.0))
        self.beta = float(params.get(1, 1.0))
        self.trans_a = int(params.get(2, 0)) != 0
        self.trans_b = int(params.get(3, 0)) != 0
        self.constant_a = int(params.get(4, 0)) != 0
        self.constant_b = int(params.get(5, 0)) != 0
        self.constant_c = int(params.get(6, 0)) != 0
        self.m = int(params.get(7, 0))
        self.n = int(params.get(8, 0))
        self.k = int(params.get(9, 0))
        self.broadcast_c = int(params.get(10, 0))
        if self.constant_a:
            raise InvalidOperationError(_abi.ERR_SHAPE,
                                        f"Gemm constantA is not supported in AexisGraphSession: {self.name}")
        if not self.constant_b:
            raise NotSupportedError(_abi.ERR_UNSUPPORTED,
                                    f"| layer={self.name} | rejectedFallback=runtime-B Gemm")
        if self.trans_a:
            raise NotSupportedError(_abi.ERR_UNSUPPORTED, f"| layer={self.name} | transA=1")
        if isinstance(weights, QuantizedTensor):
            if not self.trans_b:
                raise NotSupportedError(_abi.ERR_UNSUPPORTED,
                                        f"| layer={self.name} | direct quantized records need transB")
            self.weight = self.ctx.weight(weights, self.n, self.k)
        else:
            bits = int(params.get("bits", 8))
            self.weight = self.ctx.weight_from_float(np.asarray(weights, np.float32), self.n,
                                                     self.k, bits=bits, trans_b=self.trans_b)
        if self.constant_c and self.broadcast_c != -1 and bias is not None:
            if self.broadcast_c not in (0, 1, 2, 3, 4):
                raise InvalidOperationError(
                    _abi.ERR_SHAPE,
                    f"Gemm broadcast_type_C unsupported: {self.broadcast_c} | {self.name}")
            self.c = torch.as_tensor(np.asarray(bias, np.float32), device=f"cuda:{self.ctx.device}")
        return self

    def forward(self, x: torch.Tensor, rows: int, x_layout: int = LAYOUT_PACK4_LINEAR,
                out_dtype=torch.float16) -> tuple[torch.Tensor, int]:
        """ExecuteCommandBuffer-equivalent: returns (y storage tensor, y layout)."""
        y_layout = output_layout_for(self.n)
        y = new_activation(rows, self.n, out_dtype, y_layout, device=x.device)
        self.ctx.linear(self.weight, describe(x, rows, self.k, x_layout),
                        describe(y, rows, self.n, y_layout), alpha=self.alpha, beta=self.beta,
                        c=self.c, broadcast_c=self.broadcast_c if self.c is not None else -1)
        return y, y_layout


class Decoder:
    """aexq_decoder: every decoder layer of a decode step in one persistent
    launch (DecodeCore, DEC:463-585).  Keeps references to the tensors and
    weights it points at, which must outlive it."""

    _WEIGHTS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

    def __init__(self, ctx: Context, layers, embedding, heads_q, heads_kv, head_dim, capacity,
                 rms_eps, attn_scale, rope_cos, rope_sin, workgroups=0):
        self._lib = ctx._lib
        self.ctx = ctx
        self._keep = (list(layers), embedding, rope_cos, rope_sin)
        arr = (_abi.DecoderLayer * len(layers))()
        for i, L in enumerate(layers):
            for name in self._WEIGHTS:
                setattr(arr[i], name, L[name].handle)
            arr[i].attn_norm = L["attn_norm"].data_ptr()
            arr[i].mlp_norm = L["mlp_norm"].data_ptr()
            arr[i].k_cache = L["k_cache"].data_ptr()
            arr[i].v_cache = L["v_cache"].data_ptr()
        cfg = _abi.DecoderConfig(heads_q, heads_kv, head_dim, capacity, rms_eps, attn_scale,
                                 rope_cos.data_ptr(), rope_sin.data_ptr(), workgroups)
        h = ctypes.c_void_p()
        check(self._lib.aexq_decoder_create(ctx.handle, ctypes.byref(cfg), arr, len(layers),
                                            embedding.handle, ctypes.byref(h)),
              "aexq_decoder_create")
        self.handle = h

    def run(self, token: torch.Tensor, position: torch.Tensor, hidden_out: torch.Tensor):
        check(self._lib.aexq_decoder_run(self.handle, ctypes.c_void_p(token.data_ptr()),
                                         ctypes.c_void_p(position.data_ptr()),
                                         ctypes.c_void_p(hidden_out.data_ptr())),
              "aexq_decoder_run")

    def error(self) -> int:
        """Synchronizes; 1 when a run gave up a bounded wait since the last call."""
        f = ctypes.c_int(0)
        check(self._lib.aexq_decoder_error(self.handle, ctypes.byref(f)), "aexq_decoder_error")
        return f.value

    def info(self):
        g, s, sp = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        check(self._lib.aexq_decoder_info(self.handle, ctypes.byref(g), ctypes.byref(s),
                                          ctypes.byref(sp)), "aexq_decoder_info")
        return {"workgroups": g.value, "splits": s.value, "split_positions": sp.value}

    def close(self):
        if self.handle:
            self._lib.aexq_decoder_release(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
