"""Seeded synthetic inputs of the benchmark configurations (numpy PCG64).

Formats follow the benchmark definitions:
  Q8: int8 codes uniform in [-127, 127], row-major [N][K], one fp16 scale per
      output row = |N(0, 0.02)| / 127 (about 30% of them are fp16 subnormals).
  Q4: codes uniform in [-7, 7], two per byte, low nibble first, stored with
      zero-point 8 (offset-8), one fp16 scale per 32 consecutive K =
      |N(0, 0.02)| / 7.
  activations: fp16 N(0, 1); RMSNorm weights 1 + N(0, 0.02) (fp32).
The packed words are the reference's layout: byte (i & 3) of word i >> 2 for
Q8, nibble (i & 7) of word i >> 3 for Q4, i = row * K + col.
"""
from __future__ import annotations

import numpy as np

from ._abi import NIBBLE_OFFSET8, NIBBLE_TWOS

SEED_BASE = 0xAE0C0F10

# One decoder layer's linears (name, N, K) of the 0.8B-shaped model.
LAYER_LINEARS = (
    ("q_proj", 2048, 1024),
    ("k_proj", 512, 1024),
    ("v_proj", 512, 1024),
    ("o_proj", 1024, 2048),
    ("gate_proj", 3584, 1024),
    ("up_proj", 3584, 1024),
    ("down_proj", 1024, 3584),
)
HIDDEN = 1024
VOCAB = 151936


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def q8_weights(n: int, k: int, seed: int, scale_dtype=np.float16):
    """(packed uint32 words, scales[n], codes int8 [n][k])."""
    g = rng(seed)
    codes = g.integers(-127, 128, size=(n, k), dtype=np.int8)
    scales = (np.abs(g.standard_normal(n)) * 0.02 / 127.0).astype(scale_dtype)
    flat = codes.reshape(-1)
    pad = (-flat.size) % 4
    if pad:
        flat = np.concatenate([flat, np.zeros(pad, np.int8)])
    return flat.view(np.uint32).copy(), scales, codes


def pack_nibbles(q: np.ndarray, code: int) -> np.ndarray:
    """Signed Q4 codes [n][k] -> uint32 words, low nibble first."""
    flat = q.reshape(-1).astype(np.int16)
    nib = ((flat + 8) & 0xF) if code == NIBBLE_OFFSET8 else (flat & 0xF)
    nib = nib.astype(np.uint8)
    pad = (-nib.size) % 8
    if pad:
        fill = 8 if code == NIBBLE_OFFSET8 else 0
        nib = np.concatenate([nib, np.full(pad, fill, np.uint8)])
    byte = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
    return byte.view(np.uint32).copy()


def q4_weights(n: int, k: int, seed: int, group: int = 32, code: int = NIBBLE_OFFSET8,
               scale_dtype=np.float16):
    """(packed words, scales[n*k/group], codes int8 [n][k])."""
    g = rng(seed)
    codes = g.integers(-7, 8, size=(n, k), dtype=np.int8)
    scales = (np.abs(g.standard_normal(n * k // group)) * 0.02 / 7.0).astype(scale_dtype)
    return pack_nibbles(codes, code), scales, codes


def activations(m: int, k: int, seed: int) -> np.ndarray:
    return rng(seed).standard_normal((m, k)).astype(np.float16)


def rms_gamma(k: int, seed: int) -> np.ndarray:
    return (1.0 + 0.02 * rng(seed).standard_normal(k)).astype(np.float32)


__all__ = ["q8_weights", "q4_weights", "pack_nibbles", "activations", "rms_gamma",
           "LAYER_LINEARS", "HIDDEN", "VOCAB", "SEED_BASE", "NIBBLE_OFFSET8", "NIBBLE_TWOS"]
