"""Quantized checkpoints on disk: Safetensors files holding the group-wise
payload and scales as tensors, with the recovery information in the file's
`starlight.quantization` metadata, and their upload to a device.

The reference's sl-precision quantizer writes files of this kind (README.md:
239-247: the output stores the quantized payload and the scales as tensors
and records what is needed to restore them in `starlight.quantization`
metadata; ordinary loaders cannot read it as weights). Its source is not in
the reference tree, so the tensor names, dtypes and metadata fields below
are this backend's own, following the payload convention of `quant.py`:
parity unpinned against sl-precision.

  <name>           INT4: U8 [n, ceil(k / 2)], two's-complement nibbles,
                   element k of a row in byte k // 2, even k in the low nibble;
                   INT8: I8 [n, k]; row-major
  <name>.__scales  F32 [n, k / group_size] (the scale Param's role,
                   ARCH-0006:147)
  any other tensor F32, stored as given
  metadata["starlight.quantization"] = JSON
      {"version": 1,
       "tensors": {"<name>": {"format": "int4" | "int8", "group_size": G,
                              "shape": [n, k], "scale": "<name>.__scales"}}}

On upload, a quantized tensor becomes two Params: the u32 payload words the
device takes (the bytes, padded to a multiple of 4, little-endian) under the
weight's role and its f32 scales under `<role>.__scales`; the engine's build
binds the pair, and the device builds its private tile layout from them.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from typing import Dict, Mapping, Tuple

import numpy as np

from . import quant
from .graph import SCALES_SUFFIX, LlamaConfig, weight_specs
from .ir import QuantFormat

METADATA_KEY = "starlight.quantization"
VERSION = 1
_FORMAT_NAMES = {QuantFormat.INT4: "int4", QuantFormat.INT8: "int8"}
_FORMATS = {v: k for k, v in _FORMAT_NAMES.items()}


@dataclass
class QuantTensor:
    """One group-quantized weight [n, k]: payload bytes [n, row_bytes] and
    scales [n, k / group]."""

    fmt: QuantFormat
    group: int
    n: int
    k: int
    payload: np.ndarray  # uint8 [n, ceil(k / 2)] (INT4) or int8 [n, k] (INT8)
    scales: np.ndarray   # float32 [n, k // group]

    def words(self) -> np.ndarray:
        """The payload as the device's u32 words (bytes padded to 4)."""
        raw = np.ascontiguousarray(self.payload).view(np.uint8).ravel()
        pad = (-raw.size) % 4
        if pad:
            raw = np.concatenate([raw, np.zeros(pad, np.uint8)])
        return raw.view("<u4").astype(np.uint32)

    def dequantize(self) -> np.ndarray:
        return quant.dequantize(self.words(), self.scales, self.n, self.k, self.group, self.fmt)


def quantize_tensor(w: np.ndarray, fmt: QuantFormat, group: int) -> QuantTensor:
    """Quantizes one f32 [n, k] weight with the convention of `quant.py`."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    fmt = QuantFormat(fmt)
    words, scales = quant.quantize(w, group, fmt)
    row_bytes = (k + 1) // 2 if fmt == QuantFormat.INT4 else k
    raw = words.view(np.uint8)[: n * row_bytes].reshape(n, row_bytes)
    payload = raw.copy() if fmt == QuantFormat.INT4 else raw.view(np.int8).copy()
    return QuantTensor(fmt, group, n, k, payload, np.ascontiguousarray(scales, dtype=np.float32))


def save(path: str, dense: Mapping[str, np.ndarray], quantized: Mapping[str, QuantTensor]) -> None:
    """Writes a checkpoint: `dense` tensors as F32, `quantized` ones as
    payload + scale tensors described in the metadata."""
    from safetensors.numpy import save_file

    tensors: Dict[str, np.ndarray] = {}
    entries = {}
    for name, a in dense.items():
        tensors[name] = np.ascontiguousarray(a, dtype=np.float32)
    for name, q in quantized.items():
        scale_name = name + SCALES_SUFFIX
        if name in tensors or scale_name in tensors:
            raise ValueError(f"tensor name {name!r} is used twice")
        tensors[name] = np.ascontiguousarray(q.payload)
        tensors[scale_name] = np.ascontiguousarray(q.scales, dtype=np.float32)
        entries[name] = {"format": _FORMAT_NAMES[q.fmt], "group_size": int(q.group), "shape": [int(q.n), int(q.k)],
                         "scale": scale_name}
    save_file(tensors, path, metadata={METADATA_KEY: json.dumps({"version": VERSION, "tensors": entries},
                                                                sort_keys=True)})


def load(path: str) -> Tuple[Dict[str, np.ndarray], Dict[str, QuantTensor]]:
    """Reads a checkpoint written by `save` (no code runs from the file):
    returns (dense f32 tensors, quantized tensors). Raises ValueError on a
    malformed description."""
    from safetensors import safe_open

    with safe_open(path, framework="numpy") as f:
        meta = (f.metadata() or {}).get(METADATA_KEY)
        entries = {}
        if meta is not None:
            desc = json.loads(meta)
            if desc.get("version") != VERSION:
                raise ValueError(f"unsupported {METADATA_KEY} version {desc.get('version')!r}")
            entries = desc.get("tensors", {})
        names = set(f.keys())
        quantized: Dict[str, QuantTensor] = {}
        used = set()
        for name, e in entries.items():
            fmt = _FORMATS.get(e.get("format"))
            if fmt is None:
                raise ValueError(f"{name}: unknown format {e.get('format')!r}")
            n, k = (int(v) for v in e["shape"])
            group = int(e["group_size"])
            scale_name = e.get("scale", name + SCALES_SUFFIX)
            if name not in names or scale_name not in names:
                raise ValueError(f"{name}: payload or scale tensor missing")
            if group <= 0 or k % group:
                raise ValueError(f"{name}: k = {k} is not a multiple of group_size {group}")
            payload = f.get_tensor(name)
            scales = f.get_tensor(scale_name)
            want_payload = ((n, (k + 1) // 2), np.uint8) if fmt == QuantFormat.INT4 else ((n, k), np.int8)
            if payload.shape != want_payload[0] or payload.dtype != want_payload[1]:
                raise ValueError(f"{name}: payload {payload.dtype}{list(payload.shape)}, expected "
                                 f"{np.dtype(want_payload[1])}{list(want_payload[0])}")
            if scales.shape != (n, k // group) or scales.dtype != np.float32:
                raise ValueError(f"{name}: scales {scales.dtype}{list(scales.shape)}, expected float32"
                                 f"{[n, k // group]}")
            quantized[name] = QuantTensor(fmt, group, n, k, payload, scales)
            used.update((name, scale_name))
        dense = {}
        for name in names - used:
            a = f.get_tensor(name)
            if a.dtype != np.float32:
                raise ValueError(f"{name}: {a.dtype} tensor without a {METADATA_KEY} entry")
            dense[name] = a
    return dense, quantized


def quantize_model(cfg: LlamaConfig, weights: Mapping[str, np.ndarray]
                   ) -> Tuple[Dict[str, np.ndarray], Dict[str, QuantTensor]]:
    """Splits f32 model weights into the dense and quantized tensors `save`
    writes for `cfg` (its quantized linear weights quantized with cfg.quant /
    cfg.group)."""
    dense, quantized = {}, {}
    for spec in weight_specs(cfg):
        if spec.quantized:
            quantized[spec.name] = quantize_tensor(weights[spec.name], cfg.quant, cfg.group)
        else:
            dense[spec.name] = np.ascontiguousarray(weights[spec.name], dtype=np.float32)
    return dense, quantized


def upload(device, cfg: LlamaConfig, dense: Mapping[str, np.ndarray],
           quantized: Mapping[str, QuantTensor]) -> Dict[str, int]:
    """Uploads a loaded checkpoint for `cfg` and returns role -> BufferId
    (scale Params under `<role>.__scales`), as engine.upload_weights does for
    f32 weights: every quantized weight of cfg must be present with cfg's
    format, group and shape."""
    buffers: Dict[str, int] = {}
    for spec in weight_specs(cfg):
        if spec.quantized:
            q = quantized.get(spec.name)
            if q is None:
                raise ValueError(f"{spec.name}: quantized tensor missing")
            if q.fmt != cfg.quant or q.group != cfg.group or (q.n, q.k) != tuple(spec.shape):
                raise ValueError(f"{spec.name}: {_FORMAT_NAMES[q.fmt]} g{q.group} [{q.n}, {q.k}] does not match "
                                 f"the model ({_FORMAT_NAMES[cfg.quant]} g{cfg.group} {list(spec.shape)})")
            buffers[spec.name] = device.upload_new_u32(q.words())
            buffers[spec.scales] = device.upload_new_f32(q.scales)
        else:
            a = dense.get(spec.name)
            if a is None or tuple(a.shape) != tuple(spec.shape):
                raise ValueError(f"{spec.name}: dense tensor missing or of the wrong shape")
            buffers[spec.name] = device.upload_new_f32(a)
    return buffers
