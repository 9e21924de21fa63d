"""Symmetric group-wise INT4/INT8 weight quantization (host side).

sl-precision, which defines this format for StarLight (README.md:96, 164,
239-247; ARCH-0004 §3.3 `TensorEncoding::GroupwiseQuantized`), is not part of
the reference tree, so this module states the convention the backend adopts
(byte layout, rounding, zero groups are therefore unpinned against it):

  scale[n, g] = max |w[n, g*G : (g+1)*G]| / qmax      (qmax 7 INT4, 127 INT8)
  q           = clamp(round_half_away_from_zero(w / scale), -qmax, qmax),
                q = 0 where scale == 0
  INT8 payload: int8 codes, row-major
  INT4 payload: two's-complement nibbles, element k of a row in byte k // 2,
                even k in the low nibble; rows padded to whole bytes
  payload words: bytes padded to a multiple of 4, little-endian u32
  dequant: w' = f32(q) * scale   (one f32 multiply)
"""
from __future__ import annotations

import numpy as np

from .ir import QuantFormat

QMAX = {QuantFormat.INT4: 7, QuantFormat.INT8: 127}


def round_half_away(v: np.ndarray) -> np.ndarray:
    t = np.trunc(v)
    frac = v - t  # exact for |v| < 2**23
    return t + (frac >= 0.5) - (frac <= -0.5)


def quantize_codes(w: np.ndarray, group: int, fmt: QuantFormat):
    """Returns (codes int8 [n, k], scales float32 [n, k // group])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    if group <= 0 or k % group:
        raise ValueError("k must be a positive multiple of group_size")
    qmax = np.float32(QMAX[QuantFormat(fmt)])
    wg = w.reshape(n, k // group, group)
    scales = (np.abs(wg).max(axis=2) / qmax).astype(np.float32)
    safe = np.where(scales == 0, np.float32(1), scales)[..., None]
    ratio = (wg / safe).astype(np.float32)
    q = np.clip(round_half_away(ratio), -qmax, qmax)
    q = np.where(scales[..., None] == 0, 0, q)
    return q.astype(np.int8).reshape(n, k), scales


def pack_codes(codes: np.ndarray, fmt: QuantFormat) -> np.ndarray:
    """Packs int8 codes [n, k] into little-endian u32 payload words."""
    codes = np.asarray(codes, dtype=np.int8)
    n, k = codes.shape
    if QuantFormat(fmt) == QuantFormat.INT8:
        raw = codes.view(np.uint8).reshape(-1)
    else:
        nib = (codes.astype(np.int16) & 0xF).astype(np.uint8)
        if k % 2:
            nib = np.concatenate([nib, np.zeros((n, 1), np.uint8)], axis=1)
        raw = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8).reshape(-1)
    pad = (-raw.size) % 4
    if pad:
        raw = np.concatenate([raw, np.zeros(pad, np.uint8)])
    return raw.view("<u4").astype(np.uint32)


def unpack_codes(words: np.ndarray, n: int, k: int, fmt: QuantFormat) -> np.ndarray:
    raw = np.ascontiguousarray(words, dtype="<u4").view(np.uint8)
    if QuantFormat(fmt) == QuantFormat.INT8:
        return raw[: n * k].view(np.int8).reshape(n, k)
    row_bytes = (k + 1) // 2
    b = raw[: n * row_bytes].reshape(n, row_bytes)
    nib = np.empty((n, row_bytes * 2), np.int16)
    nib[:, 0::2] = b & 0xF
    nib[:, 1::2] = b >> 4
    nib = nib[:, :k]
    return np.where(nib >= 8, nib - 16, nib).astype(np.int8)


def quantize(w: np.ndarray, group: int, fmt: QuantFormat):
    """Returns (payload u32 words, scales float32 [n, k // group])."""
    codes, scales = quantize_codes(w, group, fmt)
    return pack_codes(codes, fmt), scales


def dequantize(words: np.ndarray, scales: np.ndarray, n: int, k: int, group: int,
               fmt: QuantFormat) -> np.ndarray:
    codes = unpack_codes(words, n, k, fmt).astype(np.float32)
    s = np.repeat(np.asarray(scales, np.float32).reshape(n, k // group), group, axis=1)
    return (codes * s).astype(np.float32)


def payload_words(fmt: QuantFormat, n: int, k: int) -> int:
    nbytes = n * ((k + 1) // 2) if QuantFormat(fmt) == QuantFormat.INT4 else n * k
    return (nbytes + 3) // 4
