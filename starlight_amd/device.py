"""HipDevice: Python view of the C-ABI `sl_device::Device` implementation.

Method names, argument meaning and errors mirror the Rust trait
(ARCH-0007 §3.1) and `CpuDevice` (crates/backends/backend-cpu/src/device.rs):
`allocate_f32/u32`, `upload_*`, `download_*`, `dispatch`, `synchronize`.
Errors raise `DeviceError`, whose variant and payload match
`sl_device::DeviceError`.

The shared library is built in-tree (`starlight_amd/lib/libstarlight_hip.so`);
there is no fallback: if it is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import glob
import os
import re
from typing import Optional, Sequence

import numpy as np

from . import ir

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libstarlight_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "starlight_hip.h")

STATUS_NAMES = {
    0: "Ok",
    1: "OutOfMemory",
    2: "InvalidBuffer",
    3: "InvalidRange",
    4: "UnsupportedOp",
    5: "ShapeOverflow",
    6: "Execution",
    7: "Unimplemented",
}


class DeviceError(Exception):
    """sl_device::DeviceError: `kind` is the variant name; the payload fields
    that variant carries are set, the others are None."""

    def __init__(self, kind: str, buffer=None, offset=None, len=None, requested=None, op=None,
                 message: Optional[str] = None):
        self.kind = kind
        self.buffer = buffer
        self.offset = offset
        self.len = len
        self.requested = requested
        self.op = op
        self.message = message
        super().__init__(self._describe())

    def _describe(self) -> str:
        if self.kind == "OutOfMemory":
            return f"OutOfMemory {{ requested: {self.requested} }}"
        if self.kind == "InvalidBuffer":
            return f"InvalidBuffer(BufferId({self.buffer}))"
        if self.kind == "InvalidRange":
            return f"InvalidRange {{ buffer: {self.buffer}, offset: {self.offset}, len: {self.len} }}"
        if self.kind == "UnsupportedOp":
            return f"UnsupportedOp({self.op})"
        if self.kind in ("Execution", "Unimplemented"):
            return f'{self.kind}("{self.message}")'
        return self.kind

    # Variant constructors, named like the Rust enum.
    @classmethod
    def execution(cls, message: str) -> "DeviceError":
        return cls("Execution", message=message)

    @classmethod
    def unimplemented(cls, message: str) -> "DeviceError":
        return cls("Unimplemented", message=message)

    @classmethod
    def invalid_buffer(cls, buffer: int) -> "DeviceError":
        return cls("InvalidBuffer", buffer=buffer)

    @classmethod
    def invalid_range(cls, buffer: int, offset: int, len: int) -> "DeviceError":
        return cls("InvalidRange", buffer=buffer, offset=offset, len=len)

    @classmethod
    def out_of_memory(cls, requested: int) -> "DeviceError":
        return cls("OutOfMemory", requested=requested)

    def __eq__(self, other) -> bool:
        if not isinstance(other, DeviceError):
            return NotImplemented
        return (self.kind, self.buffer, self.offset, self.len, self.requested, self.op, self.message) == (
            other.kind, other.buffer, other.offset, other.len, other.requested, other.op, other.message)

    def __hash__(self):
        return hash((self.kind, self.message))

    @classmethod
    def from_c(cls, e: ir.CError) -> "DeviceError":
        kind = STATUS_NAMES.get(e.status, f"Status{e.status}")
        msg = e.message.decode() if e.message else None
        if kind == "OutOfMemory":
            return cls(kind, requested=e.requested)
        if kind == "InvalidBuffer":
            return cls(kind, buffer=e.buffer)
        if kind == "InvalidRange":
            return cls(kind, buffer=e.buffer, offset=e.offset, len=e.len)
        if kind == "UnsupportedOp":
            return cls(kind, op=e.op)
        if kind in ("Execution", "Unimplemented"):
            return cls(kind, message=msg)
        return cls(kind)


_lib = None

OPT_FUSION = 1
OPT_GRAPHS = 2


class HipStats(ctypes.Structure):
    """sl_hip_stats: counters of the submission machinery."""
    _fields_ = [("submissions", ctypes.c_uint64), ("commands", ctypes.c_uint64),
                ("fused_commands", ctypes.c_uint64), ("graph_captures", ctypes.c_uint64),
                ("graph_replays", ctypes.c_uint64)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


def exported_symbols() -> list:
    """Every `sl_hip_*` / `sl_engine_*` function the public headers
    (include/*.h) declare."""
    names = set()
    for path in sorted(glob.glob(os.path.join(os.path.dirname(HEADER_PATH), "*.h"))):
        with open(path) as f:
            names |= set(re.findall(r"\b(sl_(?:hip|engine)_[a-z0-9_]+)\s*\(", f.read()))
    return sorted(names)


def load_library() -> ctypes.CDLL:
    """Loads the in-tree HIP library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
            "(make -C starlight_amd/csrc); there is no CPU fallback")
    lib = ctypes.CDLL(LIB_PATH)
    P = ctypes.c_void_p
    U32P = ctypes.POINTER(ctypes.c_uint32)
    sigs = {
        "sl_hip_abi_version": ([], ctypes.c_uint32),
        "sl_hip_device_create": ([ctypes.c_int, ctypes.POINTER(P)], ctypes.c_int),
        "sl_hip_device_destroy": ([P], None),
        "sl_hip_allocate_f32": ([P, ctypes.c_size_t, ctypes.c_size_t, U32P], ctypes.c_int),
        "sl_hip_allocate_u32": ([P, ctypes.c_size_t, ctypes.c_size_t, U32P], ctypes.c_int),
        "sl_hip_upload_f32": ([P, ctypes.c_uint32, P, ctypes.c_size_t], ctypes.c_int),
        "sl_hip_upload_u32": ([P, ctypes.c_uint32, P, ctypes.c_size_t], ctypes.c_int),
        "sl_hip_download_f32": ([P, ctypes.c_uint32, P, ctypes.c_size_t], ctypes.c_int),
        "sl_hip_download_u32": ([P, ctypes.c_uint32, P, ctypes.c_size_t], ctypes.c_int),
        "sl_hip_dispatch": ([P, ctypes.POINTER(ir.COp), ctypes.POINTER(ir.CBufferRef),
                             ctypes.POINTER(ir.CValue), ctypes.c_size_t, ctypes.POINTER(ir.CBufferRef),
                             ctypes.POINTER(ir.CValue), ctypes.c_size_t, U32P, ctypes.c_size_t],
                            ctypes.c_int),
        "sl_hip_dispatch_noalloc": ([P, ctypes.POINTER(ir.COp), ctypes.POINTER(ir.CBufferRef),
                                     ctypes.POINTER(ir.CValue), ctypes.c_size_t, ctypes.POINTER(ir.CBufferRef),
                                     ctypes.POINTER(ir.CValue), ctypes.c_size_t, U32P, ctypes.c_size_t],
                                    ctypes.c_int),
        "sl_hip_paged_attention": ([P, ctypes.POINTER(ir.COp), ctypes.POINTER(ir.CBufferRef),
                                    ctypes.POINTER(ir.CBufferRef), ctypes.POINTER(ir.CBufferRef),
                                    ctypes.POINTER(ir.CBufferRef), ctypes.c_uint32, ctypes.c_void_p], ctypes.c_int),
        "sl_hip_bind_paged_state": ([P, ctypes.c_uint32, ctypes.c_void_p], ctypes.c_int),
        "sl_hip_paged_store": ([P, ctypes.c_void_p] + [ctypes.c_uint32] * 7, ctypes.c_int),
        "sl_hip_synchronize": ([P], ctypes.c_int),
        "sl_hip_last_error": ([P, ctypes.POINTER(ir.CError)], None),
        "sl_hip_bind_quantized": ([P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                   ctypes.c_uint32, ctypes.c_uint32], ctypes.c_int),
        "sl_hip_validate_dispatch": ([ctypes.POINTER(ir.CBufferDesc), ctypes.c_size_t, ctypes.POINTER(ir.COp),
                                      ctypes.POINTER(ir.CBufferRef), ctypes.POINTER(ir.CValue),
                                      ctypes.c_size_t, ctypes.POINTER(ir.CBufferRef),
                                      ctypes.POINTER(ir.CValue), ctypes.c_size_t, U32P, ctypes.c_size_t,
                                      ctypes.POINTER(ir.CError)], ctypes.c_int),
        "sl_hip_capabilities": ([ctypes.POINTER(ir.CCapabilities)], None),
        "sl_hip_stream": ([P], ctypes.c_void_p),
        "sl_hip_submit": ([P], ctypes.c_int),
        "sl_hip_set_options": ([P, ctypes.c_uint32], ctypes.c_int),
        "sl_hip_get_stats": ([P, ctypes.POINTER(HipStats)], None),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def _port_arrays(refs: Sequence[ir.BufferRef], values: Sequence[ir.Value]):
    n = len(refs)
    c_refs = (ir.CBufferRef * max(n, 1))(*[r.to_c() for r in refs])
    c_vals = (ir.CValue * max(len(values), 1))(*[v.to_c() for v in values])
    return c_refs, c_vals


def _scalars(scalars: Sequence[int]):
    return (ctypes.c_uint32 * max(len(scalars), 1))(*[int(s) for s in scalars])


class HipDevice:
    """One MI355X (gfx950) device: the `sl_device::Device` contract."""

    def __init__(self, ordinal: int = 0):
        self._lib = load_library()
        handle = ctypes.c_void_p()
        status = self._lib.sl_hip_device_create(ordinal, ctypes.byref(handle))
        if status != 0:
            raise DeviceError(STATUS_NAMES.get(status, "Execution"),
                              message=f"could not open HIP device {ordinal}")
        self._h = handle

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.sl_hip_device_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    @property
    def stream(self) -> int:
        """The device's hipStream_t (for HIP event timing)."""
        return self._lib.sl_hip_stream(self._h)

    def _check(self, status: int) -> None:
        if status != 0:
            err = ir.CError()
            self._lib.sl_hip_last_error(self._h, ctypes.byref(err))
            raise DeviceError.from_c(err)

    # -- trait Device ------------------------------------------------------
    def allocate_f32(self, elements: int, align: int) -> int:
        out = ctypes.c_uint32()
        self._check(self._lib.sl_hip_allocate_f32(self._h, elements, align, ctypes.byref(out)))
        return out.value

    def allocate_u32(self, elements: int, align: int) -> int:
        out = ctypes.c_uint32()
        self._check(self._lib.sl_hip_allocate_u32(self._h, elements, align, ctypes.byref(out)))
        return out.value

    def upload_f32(self, buffer: int, data) -> None:
        a = np.ascontiguousarray(data, dtype=np.float32)
        self._check(self._lib.sl_hip_upload_f32(self._h, buffer, a.ctypes.data, a.size))

    def upload_u32(self, buffer: int, data) -> None:
        a = np.ascontiguousarray(data, dtype=np.uint32)
        self._check(self._lib.sl_hip_upload_u32(self._h, buffer, a.ctypes.data, a.size))

    def download_f32(self, buffer: int, out: np.ndarray) -> None:
        assert out.dtype == np.float32 and out.flags.c_contiguous
        self._check(self._lib.sl_hip_download_f32(self._h, buffer, out.ctypes.data, out.size))

    def download_u32(self, buffer: int, out: np.ndarray) -> None:
        assert out.dtype == np.uint32 and out.flags.c_contiguous
        self._check(self._lib.sl_hip_download_u32(self._h, buffer, out.ctypes.data, out.size))

    def dispatch(self, op: ir.Op, inputs: Sequence[ir.BufferRef], input_values: Sequence[ir.Value],
                 outputs: Sequence[ir.BufferRef], output_values: Sequence[ir.Value],
                 scalars: Sequence[int] = ()) -> None:
        if len(inputs) != len(input_values):
            raise DeviceError.execution("inputs and input_values have different lengths")
        if len(outputs) != len(output_values):
            raise DeviceError.execution("outputs and output_values have different lengths")
        c_op = op.to_c()
        in_refs, in_vals = _port_arrays(inputs, input_values)
        out_refs, out_vals = _port_arrays(outputs, output_values)
        sc = _scalars(scalars)
        self._check(self._lib.sl_hip_dispatch(self._h, ctypes.byref(c_op), in_refs, in_vals, len(inputs),
                                              out_refs, out_vals, len(outputs), sc, len(scalars)))

    def dispatch_noalloc(self, op: ir.Op, inputs: Sequence[ir.BufferRef], input_values: Sequence[ir.Value],
                         outputs: Sequence[ir.BufferRef], output_values: Sequence[ir.Value],
                         scalars: Sequence[int] = ()) -> None:
        """sl_hip_dispatch_noalloc: validate, then enqueue this command's
        kernels at once with the static per-GPU scratch (no allocation)."""
        if len(inputs) != len(input_values) or len(outputs) != len(output_values):
            raise DeviceError.execution("ports and values have different lengths")
        c_op = op.to_c()
        in_refs, in_vals = _port_arrays(inputs, input_values)
        out_refs, out_vals = _port_arrays(outputs, output_values)
        sc = _scalars(scalars)
        self._check(self._lib.sl_hip_dispatch_noalloc(self._h, ctypes.byref(c_op), in_refs, in_vals, len(inputs),
                                                      out_refs, out_vals, len(outputs), sc, len(scalars)))

    def paged_attention(self, op: ir.Op, q: ir.BufferRef, k_new: ir.BufferRef, v_new: ir.BufferRef,
                        out: ir.BufferRef, batch: int, paged_kv) -> None:
        """sl_hip_paged_attention (starlight_amd.paged): decode attention
        over a paged KV cache, one new token per row at its own length."""
        c_op = op.to_c()
        refs = [r.to_c() for r in (q, k_new, v_new, out)]
        self._check(self._lib.sl_hip_paged_attention(self._h, ctypes.byref(c_op), *[ctypes.byref(r) for r in refs],
                                                      batch, ctypes.addressof(paged_kv)))

    def bind_paged_state(self, state: int, paged_kv=None) -> None:
        """sl_hip_bind_paged_state: CausalAttention commands on the State
        buffer `state` read and append through the paged cache `paged_kv`
        (an sl_paged_kv structure; None removes the binding)."""
        self._check(self._lib.sl_hip_bind_paged_state(
            self._h, state, None if paged_kv is None else ctypes.addressof(paged_kv)))

    def paged_store(self, paged_kv, row: int, state: int, index: int, max_seq: int, kv_heads: int, head_dim: int,
                    length: int) -> None:
        """sl_hip_paged_store: positions [0, length) of batch index `index`
        of a contiguous KV State into row `row`'s pages."""
        self._check(self._lib.sl_hip_paged_store(self._h, ctypes.addressof(paged_kv), row, state, index, max_seq,
                                                 kv_heads, head_dim, length))

    def synchronize(self) -> None:
        self._check(self._lib.sl_hip_synchronize(self._h))

    # -- extension: submission of logged dispatches -----------------------
    def submit(self) -> None:
        """Enqueues the logged dispatches without waiting."""
        self._check(self._lib.sl_hip_submit(self._h))

    def set_options(self, fusion: bool = True, graphs: bool = True) -> None:
        self._check(self._lib.sl_hip_set_options(self._h, (OPT_FUSION if fusion else 0) |
                                                 (OPT_GRAPHS if graphs else 0)))

    def stats(self) -> dict:
        st = HipStats()
        self._lib.sl_hip_get_stats(self._h, ctypes.byref(st))
        return st.as_dict()

    # -- extension: group-quantized weights ------------------------------
    def bind_quantized(self, payload: int, scales: int, qformat: ir.QuantFormat, group_size: int, n: int,
                       k: int) -> None:
        self._check(self._lib.sl_hip_bind_quantized(self._h, payload, scales, int(qformat), group_size, n, k))

    # -- convenience -------------------------------------------------------
    def upload_new_f32(self, data, align: int = 256) -> int:
        a = np.ascontiguousarray(data, dtype=np.float32).ravel()
        buf = self.allocate_f32(a.size, align)
        self.upload_f32(buf, a)
        return buf

    def upload_new_u32(self, data, align: int = 256) -> int:
        a = np.ascontiguousarray(data, dtype=np.uint32).ravel()
        buf = self.allocate_u32(a.size, align)
        self.upload_u32(buf, a)
        return buf

    def read_f32(self, buffer: int, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        self.download_f32(buffer, out)
        return out


def capabilities() -> dict:
    """DeviceCapabilities of this backend (no GPU needed)."""
    lib = load_library()
    c = ir.CCapabilities()
    lib.sl_hip_capabilities(ctypes.byref(c))
    return {f: (getattr(c, f).decode() if f == "backend" else getattr(c, f)) for f, _ in c._fields_}


def validate_dispatch(buffers: Sequence[dict], op: ir.Op, inputs: Sequence[ir.BufferRef],
                      input_values: Sequence[ir.Value], outputs: Sequence[ir.BufferRef],
                      output_values: Sequence[ir.Value], scalars: Sequence[int] = ()) -> Optional[DeviceError]:
    """Runs the dispatch checks against a described buffer table without a
    GPU. Each buffer is {"kind": "f32"|"u32"|None, "elements": n} plus, for a
    bound quantized payload, {"quant": (qformat, group, n, k)}. Returns the
    DeviceError dispatch would raise, or None."""
    lib = load_library()
    table = (ir.CBufferDesc * max(len(buffers), 1))()
    kinds = {None: 0, "f32": 1, "u32": 2}
    for i, b in enumerate(buffers):
        table[i].kind = kinds[b.get("kind")]
        table[i].elements = b.get("elements", 0)
        if "quant" in b:
            fmt, group, qn, qk = b["quant"]
            table[i].quantized = 1
            table[i].qformat = int(fmt)
            table[i].group_size = group
            table[i].qn = qn
            table[i].qk = qk
    if len(inputs) != len(input_values):
        return DeviceError.execution("inputs and input_values have different lengths")
    if len(outputs) != len(output_values):
        return DeviceError.execution("outputs and output_values have different lengths")
    in_refs, in_vals = _port_arrays(inputs, input_values)
    out_refs, out_vals = _port_arrays(outputs, output_values)
    err = ir.CError()
    c_op = op.to_c()
    status = lib.sl_hip_validate_dispatch(table, len(buffers), ctypes.byref(c_op), in_refs, in_vals, len(inputs),
                                          out_refs, out_vals, len(outputs), _scalars(scalars), len(scalars),
                                          ctypes.byref(err))
    return None if status == 0 else DeviceError.from_c(err)
