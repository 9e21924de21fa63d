"""Engine: the restated sl-core step loop (ARCH-0007 §3.2) plus weight
upload, for driving a device with lowered llama-dense programs.

`NativeEngine` runs the step loop in C++ (libstarlight_hip.so,
include/starlight_engine.h) over the HIP device; `Engine` is the same loop in
Python over any object with the Device methods (the CPU oracle device in the
tests). Both bind the same CompiledPrograms.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence

import numpy as np

from . import ir, quant
from .device import DeviceError, HipDevice, load_library
from .graph import LlamaConfig, Lowered, weight_specs


@dataclass
class CompiledProgram:
    """sl_core::CompiledProgram (ARCH-0007 §3.2)."""

    lowered: Lowered
    weights: Dict[int, int]  # ValueId -> BufferId


def upload_weights(device, cfg: LlamaConfig, tensors: Dict[str, np.ndarray]) -> Dict[str, int]:
    """Uploads every weight of `cfg` (float32 arrays by name) and returns
    role -> BufferId. Linear weights marked quantized are quantized with the
    group-wise convention and uploaded as two Params: the u32 payload under
    the weight's role and the f32 scales under `<role>.__scales`
    (ARCH-0006:147); Engine build binds the pair."""
    buffers: Dict[str, int] = {}
    for spec in weight_specs(cfg):
        w = np.ascontiguousarray(tensors[spec.name], dtype=np.float32)
        assert w.shape == spec.shape, (spec.name, w.shape, spec.shape)
        if spec.quantized:
            words, scales = quant.quantize(w, cfg.group, cfg.quant)
            buffers[spec.name] = device.upload_new_u32(words)
            buffers[spec.scales] = device.upload_new_f32(scales)
        else:
            buffers[spec.name] = device.upload_new_f32(w)
    return buffers


def compile_program(lowered: Lowered, weight_buffers: Dict[str, int]) -> CompiledProgram:
    """Binds a compiled program's Params to uploaded buffers by role."""
    return CompiledProgram(lowered, {lowered.weights[name]: buf for name, buf in weight_buffers.items()
                                     if name in lowered.weights})


class BuildError(Exception):
    """A program the engine cannot build on its device (Engine::build)."""


def quantized_bindings(prog: CompiledProgram):
    """(payload BufferId, scales BufferId, qformat, group, n, k) for every
    group-quantized Param of the program; raises BuildError when a quantized
    Param or its scale Param has no buffer, or the scale Param's shape is
    not [n, k / group]."""
    cb = prog.lowered.ir
    out = []
    for vid, v in enumerate(cb.values):
        if v.encoding != ir.Encoding.GROUPWISE_QUANTIZED:
            continue
        if v.role != ir.ValueRole.PARAM or vid not in prog.weights:
            raise BuildError(f"quantized value {vid} is not a bound Param")
        sid = prog.lowered.quant_scales.get(vid)
        if sid is None or sid not in prog.weights:
            raise BuildError(f"quantized Param {vid} has no bound scale Param")
        n, k = v.shape
        if v.group_size <= 0 or k % v.group_size or cb.values[sid].shape != (n, k // v.group_size):
            raise BuildError(f"scale Param {sid} does not have shape [n, k / group] for Param {vid}")
        out.append((prog.weights[vid], prog.weights[sid], v.qformat, v.group_size, n, k))
    return out


# ------------------------------------------------------------ native ------


class CCommand(ctypes.Structure):
    _fields_ = [("op", ir.COp), ("n_inputs", ctypes.c_uint32), ("n_outputs", ctypes.c_uint32),
                ("inputs", ctypes.c_uint32 * 4), ("outputs", ctypes.c_uint32 * 1), ("effect", ctypes.c_uint32),
                ("state", ctypes.c_uint32)]


class CSlot(ctypes.Structure):
    _fields_ = [("value", ctypes.c_uint32), ("reserved", ctypes.c_uint32), ("offset", ctypes.c_uint64),
                ("bytes", ctypes.c_uint64)]


class CCommandBuffer(ctypes.Structure):
    _fields_ = [("ir_version", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
                ("values", ctypes.POINTER(ir.CValue)), ("n_values", ctypes.c_size_t),
                ("commands", ctypes.POINTER(CCommand)), ("n_commands", ctypes.c_size_t),
                ("scratchpad_bytes", ctypes.c_uint64), ("slots", ctypes.POINTER(CSlot)), ("n_slots", ctypes.c_size_t)]


class CCompiledProgram(ctypes.Structure):
    _fields_ = [("ir", CCommandBuffer), ("weight_values", ctypes.POINTER(ctypes.c_uint32)),
                ("weight_buffers", ctypes.POINTER(ctypes.c_uint32)), ("n_weights", ctypes.c_size_t),
                ("token_ids", ctypes.c_uint32), ("positions", ctypes.c_int32), ("seq_len", ctypes.c_uint32),
                ("past_len", ctypes.c_int32), ("logits", ctypes.c_uint32),
                ("quant_params", ctypes.POINTER(ctypes.c_uint32)), ("quant_scales", ctypes.POINTER(ctypes.c_uint32)),
                ("n_quant", ctypes.c_size_t)]


def _to_c_program(prog: CompiledProgram):
    """Builds the C structures; returns (struct, keepalive list)."""
    cb = prog.lowered.ir
    values = (ir.CValue * len(cb.values))(*[v.to_c() for v in cb.values])
    cmds = (CCommand * len(cb.commands))()
    for i, c in enumerate(cb.commands):
        cmds[i].op = c.op.to_c()
        cmds[i].n_inputs = len(c.inputs)
        cmds[i].n_outputs = len(c.outputs)
        for j, v in enumerate(c.inputs):
            cmds[i].inputs[j] = v
        for j, v in enumerate(c.outputs):
            cmds[i].outputs[j] = v
        cmds[i].effect = int(c.effect)
        cmds[i].state = c.state if c.state is not None else 0
    slots = (CSlot * max(len(cb.plan.slots), 1))()
    for i, s in enumerate(cb.plan.slots):
        slots[i].value, slots[i].offset, slots[i].bytes = s.value, s.offset, s.bytes
    wv = (ctypes.c_uint32 * max(len(prog.weights), 1))(*prog.weights.keys())
    wb = (ctypes.c_uint32 * max(len(prog.weights), 1))(*prog.weights.values())
    c = CCompiledProgram()
    c.ir.ir_version = cb.ir_version
    c.ir.values = values
    c.ir.n_values = len(cb.values)
    c.ir.commands = cmds
    c.ir.n_commands = len(cb.commands)
    c.ir.scratchpad_bytes = cb.plan.scratchpad_bytes
    c.ir.slots = slots
    c.ir.n_slots = len(cb.plan.slots)
    c.weight_values, c.weight_buffers, c.n_weights = wv, wb, len(prog.weights)
    lw = prog.lowered
    c.token_ids, c.positions, c.seq_len, c.past_len, c.logits = lw.token_ids, lw.positions, lw.seq_len, \
        lw.past_len, lw.logits
    qp = (ctypes.c_uint32 * max(len(lw.quant_scales), 1))(*lw.quant_scales.keys())
    qs = (ctypes.c_uint32 * max(len(lw.quant_scales), 1))(*lw.quant_scales.values())
    c.quant_params, c.quant_scales, c.n_quant = qp, qs, len(lw.quant_scales)
    return c, [values, cmds, slots, wv, wb, qp, qs]


def _declare_engine(lib):
    if getattr(lib, "_engine_declared", False):
        return
    P = ctypes.c_void_p
    U32P = ctypes.POINTER(ctypes.c_uint32)
    F32P = ctypes.POINTER(ctypes.c_float)
    lib.sl_engine_build.argtypes = [P, ctypes.POINTER(CCompiledProgram), ctypes.POINTER(CCompiledProgram),
                                    ctypes.c_uint32, ctypes.c_uint32, ctypes.POINTER(P)]
    lib.sl_engine_build.restype = ctypes.c_int
    lib.sl_engine_step.argtypes = [P, ctypes.c_uint32, U32P, ctypes.c_size_t, U32P, ctypes.c_size_t, ctypes.c_uint32,
                                   ctypes.c_uint32, F32P, ctypes.c_size_t]
    lib.sl_engine_step.restype = ctypes.c_int
    lib.sl_engine_generate.argtypes = [P, U32P, ctypes.c_size_t, ctypes.c_uint32, U32P, F32P, ctypes.c_size_t]
    lib.sl_engine_generate.restype = ctypes.c_int
    lib.sl_engine_decode.argtypes = [P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, U32P]
    lib.sl_engine_decode.restype = ctypes.c_int
    lib.sl_engine_decode_batch.argtypes = [P, U32P, ctypes.c_uint32, ctypes.c_uint32, U32P]
    lib.sl_engine_decode_batch.restype = ctypes.c_int
    lib.sl_engine_decode_rows.argtypes = [P, U32P, U32P, ctypes.c_uint32, ctypes.c_uint32, U32P]
    lib.sl_engine_decode_rows.restype = ctypes.c_int
    lib.sl_engine_state_buffer.argtypes = [P, ctypes.c_uint32]
    lib.sl_engine_state_buffer.restype = ctypes.c_uint32
    lib.sl_engine_destroy.argtypes = [P]
    lib.sl_engine_destroy.restype = None
    lib._engine_declared = True


def _u32p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))


def _f32p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


class NativeEngine:
    """sl-core Engine over the HIP device, step loop in C++."""

    PREFILL, DECODE = 0, 1

    def __init__(self, device: HipDevice, prefill: CompiledProgram, decode: CompiledProgram, max_batch: int,
                 max_context: int):
        self._lib = load_library()
        _declare_engine(self._lib)
        self.device = device
        self._cp, self._keep_p = _to_c_program(prefill)
        self._cd, self._keep_d = _to_c_program(decode)
        handle = ctypes.c_void_p()
        status = self._lib.sl_engine_build(device.handle, ctypes.byref(self._cp), ctypes.byref(self._cd), max_batch,
                                           max_context, ctypes.byref(handle))
        self._raise(status)
        self._h = handle
        self.prefill, self.decode_program = prefill, decode

    def _raise(self, status: int) -> None:
        if status != 0:
            err = ir.CError()
            self._lib.sl_hip_last_error(self.device.handle, ctypes.byref(err))
            if err.status == status:
                raise DeviceError.from_c(err)
            raise DeviceError("Execution", message=f"engine call failed with status {status}")

    def close(self):
        if getattr(self, "_h", None):
            self._lib.sl_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def step(self, mode: int, token_ids, positions, seq_len: int, past_len: int, out: np.ndarray) -> None:
        t = np.ascontiguousarray(token_ids, np.uint32).ravel()
        p = np.ascontiguousarray(positions, np.uint32).ravel()
        assert out.dtype == np.float32 and out.flags.c_contiguous
        self._raise(self._lib.sl_engine_step(self._h, mode, _u32p(t), t.size, _u32p(p), p.size, seq_len, past_len,
                                             _f32p(out), out.size))

    def generate(self, prompt: Sequence[int], steps: int, vocab: int, keep_logits: bool = True):
        pr = np.ascontiguousarray(prompt, np.uint32)
        tokens = np.zeros(steps + 1, np.uint32)
        logits = np.zeros((steps + 1, vocab), np.float32) if keep_logits else None
        self._raise(self._lib.sl_engine_generate(self._h, _u32p(pr), pr.size, steps, _u32p(tokens), _f32p(logits),
                                                 vocab))
        return tokens, logits

    def decode(self, token: int, past_len: int, steps: int) -> np.ndarray:
        tokens = np.zeros(max(steps, 1), np.uint32)
        self._raise(self._lib.sl_engine_decode(self._h, token, past_len, steps, _u32p(tokens)))
        return tokens[:steps]

    def decode_batch(self, tokens, past_len: int, steps: int) -> np.ndarray:
        """Greedy decode of the compiled batch: ids [steps, batch]."""
        first = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.zeros((max(steps, 1), first.size), np.uint32)
        self._raise(self._lib.sl_engine_decode_batch(self._h, _u32p(first), past_len, steps, _u32p(out)))
        return out[:steps]

    def decode_rows(self, tokens, positions, lengths_buffer: int, steps: int) -> np.ndarray:
        """Greedy decode of rows at their own positions (a decode program
        whose KV State is bound to a paged cache; `lengths_buffer` is the
        binding's seq_lens): ids [steps, batch]."""
        first = np.ascontiguousarray(tokens, dtype=np.uint32)
        pos = np.ascontiguousarray(positions, dtype=np.uint32)
        out = np.zeros((max(steps, 1), first.size), np.uint32)
        self._raise(self._lib.sl_engine_decode_rows(self._h, _u32p(first), _u32p(pos), lengths_buffer, steps,
                                                    _u32p(out)))
        return out[:steps]

    def state_buffer(self, value: int) -> int:
        return int(self._lib.sl_engine_state_buffer(self._h, value))


# ------------------------------------------------------------ python ------


class Engine:
    """The same build/step logic in Python, over any Device-like object."""

    PREFILL, DECODE = 0, 1

    def __init__(self, device, prefill: CompiledProgram, decode: CompiledProgram, max_batch: int, max_context: int):
        self.device = device
        self.max_context = max_context
        # Quantized Params: each payload bound to its scale Param, once.
        bound = {}
        for prog in (prefill, decode):
            for b in quantized_bindings(prog):
                if bound.get(b[0]) != b:
                    device.bind_quantized(*b)
                    bound[b[0]] = b
        scratch = max(prefill.lowered.ir.plan.scratchpad_bytes, decode.lowered.ir.plan.scratchpad_bytes)
        self.scratch = device.allocate_f32((scratch + 3) // 4, 256) if scratch else None
        self.states: Dict[int, int] = {}
        self.programs = [self._resolve(prefill), self._resolve(decode)]

    def _resolve(self, prog: CompiledProgram):
        cb = prog.lowered.ir
        refs: Dict[int, ir.BufferRef] = {}
        for vid, buf in prog.weights.items():
            v = cb.values[vid]
            n = quant.payload_words(v.qformat, *v.shape) if v.encoding == ir.Encoding.GROUPWISE_QUANTIZED \
                else v.element_count()
            refs[vid] = ir.BufferRef(buf, 0, n)
        for s in cb.plan.slots:
            refs[s.value] = ir.BufferRef(self.scratch, s.offset // 4, s.bytes // 4)
        lw = prog.lowered
        for vid, v in enumerate(cb.values):
            if vid in refs:
                continue
            if v.role == ir.ValueRole.STATE:
                if vid not in self.states:
                    self.states[vid] = self.device.allocate_f32(v.element_count(), 256)
                refs[vid] = ir.BufferRef(self.states[vid], 0, v.element_count())
            elif v.role == ir.ValueRole.INPUT and vid in (lw.token_ids, lw.positions) and vid >= 0:
                refs[vid] = ir.BufferRef(self.device.allocate_u32(v.element_count(), 256), 0, v.element_count())
            elif v.role == ir.ValueRole.OUTPUT:
                refs[vid] = ir.BufferRef(self.device.allocate_f32(v.element_count(), 256), 0, v.element_count())
        commands = []
        for c in cb.commands:
            ins, ivals, scal = [], [], []
            for vid in c.inputs:
                v = cb.values[vid]
                if v.role == ir.ValueRole.SCALAR:
                    scal.append("seq" if vid == lw.seq_len else "past")
                else:
                    ins.append(refs[vid])
                    ivals.append(v)
            if c.effect != ir.Effect.NONE:
                ins.append(refs[c.state])
                ivals.append(cb.values[c.state])
            commands.append((c.op, ins, ivals, [refs[v] for v in c.outputs], [cb.values[v] for v in c.outputs], scal))
        return {"commands": commands, "tokens": refs[lw.token_ids],
                "positions": refs[lw.positions] if lw.positions >= 0 else None,
                "logits": refs[lw.logits], "seq": cb.values[lw.token_ids].shape[-1]}

    def step(self, mode: int, token_ids, positions, seq_len: int, past_len: int, out: np.ndarray) -> None:
        p = self.programs[mode]
        if seq_len == 0 or seq_len > p["seq"] or past_len + seq_len > self.max_context:
            raise DeviceError.execution("step input exceeds the compiled capacity")
        self.device.upload_u32(p["tokens"].buffer, np.ascontiguousarray(token_ids, np.uint32).ravel())
        if p["positions"] is not None:
            self.device.upload_u32(p["positions"].buffer, np.ascontiguousarray(positions, np.uint32).ravel())
        for op, ins, ivals, outs, ovals, scal in p["commands"]:
            scalars = [seq_len if s == "seq" else past_len for s in scal]
            self.device.dispatch(op, ins, ivals, outs, ovals, scalars)
        self.device.synchronize()
        self.device.download_f32(p["logits"].buffer, out)

    def generate(self, prompt: Sequence[int], steps: int, vocab: int):
        prompt = np.asarray(prompt, np.uint32)
        s = prompt.size
        logits = np.zeros((steps + 1, vocab), np.float32)
        tokens = np.zeros(steps + 1, np.uint32)
        self.step(self.PREFILL, prompt, np.arange(s, dtype=np.uint32), s, 0, logits[0])
        tokens[0] = int(np.argmax(logits[0]))
        for i in range(steps):
            past = s + i
            self.step(self.DECODE, [tokens[i]], [past], 1, past, logits[i + 1])
            tokens[i + 1] = int(np.argmax(logits[i + 1]))
        return tokens, logits
