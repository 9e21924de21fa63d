"""ORACLE — test infrastructure only.

A restated CpuDevice (crates/backends/backend-cpu/src/device.rs:31-213,
run_op :773-1227): host buffers, one operator per dispatch, every kernel a
call into the C restatement of the reference kernels (liboracle.so). It takes
commands the engine has already shaped correctly and does not repeat the
device's port validation (that is the product's, checked in tests/test_abi.py
and tests/test_gpu_device.py); geometry decoding follows run_op.

Group-quantized weights are dequantized once at bind time and then used as
dense f32 matrices: the reference has no quantized kernel, so this is
matmul_nt(a, dequant(q, s)).
"""
from __future__ import annotations

import numpy as np

import oracle
from starlight_amd import quant
from starlight_amd.ir import Encoding, OpCode, RopeVariant, ValueRole


class OracleDevice:
    def __init__(self):
        self.f32 = []   # list of np.ndarray or None
        self.u32 = []
        self.dequant = {}  # payload buffer id -> dense [n, k] f32

    # -- Device trait -----------------------------------------------------
    def allocate_f32(self, elements, align):
        self.f32.append(np.zeros(elements, np.float32))
        self.u32.append(None)
        return len(self.f32) - 1

    def allocate_u32(self, elements, align):
        self.f32.append(None)
        self.u32.append(np.zeros(elements, np.uint32))
        return len(self.u32) - 1

    def upload_f32(self, buf, data):
        self.f32[buf][:] = np.asarray(data, np.float32).ravel()

    def upload_u32(self, buf, data):
        self.u32[buf][:] = np.asarray(data, np.uint32).ravel()

    def download_f32(self, buf, out):
        out[:] = self.f32[buf]

    def download_u32(self, buf, out):
        out[:] = self.u32[buf]

    def synchronize(self):
        pass

    def upload_new_f32(self, data, align=256):
        a = np.ascontiguousarray(data, np.float32).ravel()
        b = self.allocate_f32(a.size, align)
        self.upload_f32(b, a)
        return b

    def upload_new_u32(self, data, align=256):
        a = np.ascontiguousarray(data, np.uint32).ravel()
        b = self.allocate_u32(a.size, align)
        self.upload_u32(b, a)
        return b

    def bind_quantized(self, payload, scales, qformat, group, n, k):
        bits = 4 if quant.QuantFormat(qformat) == quant.QuantFormat.INT4 else 8
        self.dequant[payload] = oracle.dequantize_groupwise(self.u32[payload].view(np.uint8), self.f32[scales], n, k,
                                                            group, bits)

    # -- dispatch ------------------------------------------------------------
    def _in(self, ref, value):
        if value.encoding == Encoding.GROUPWISE_QUANTIZED:
            return self.dequant[ref.buffer].ravel()
        store = self.u32 if value.dtype == 3 else self.f32
        return store[ref.buffer][ref.offset:ref.offset + ref.len]

    def _write(self, ref, data):
        self.f32[ref.buffer][ref.offset:ref.offset + ref.len] = np.asarray(data, np.float32).ravel()

    def dispatch(self, op, inputs, input_values, outputs, output_values, scalars=()):
        code = op.code
        ins = [self._in(r, v) for r, v in zip(inputs, input_values)]
        shp = [v.shape for v in input_values]
        out = outputs[0] if outputs else None
        oshape = output_values[0].shape if output_values else None
        if code in (OpCode.MATMUL_NT, OpCode.MATMUL_NN):
            nt = code == OpCode.MATMUL_NT
            a, b = shp[0], shp[1]
            m, k = a[-2], a[-1]
            n = b[-2] if nt else b[-1]
            ba = int(np.prod(a[:-2])) if len(a) > 2 else 1
            bb = int(np.prod(b[:-2])) if len(b) > 2 else 1
            batch = max(ba, bb) if min(ba, bb) else 0
            fn = oracle.matmul_nt if nt else oracle.matmul_nn
            res = [fn(ins[0].reshape(ba, -1)[i if ba > 1 else 0], ins[1].reshape(bb, -1)[i if bb > 1 else 0],
                      1, m, k, n) for i in range(batch)]
            if res:
                self._write(out, np.concatenate(res))
        elif code == OpCode.SOFTMAX:
            self._write(out, oracle.softmax(ins[0], int(np.prod(shp[0][:-1])), shp[0][-1]))
        elif code == OpCode.SOFTMAX_CAUSAL:
            self._write(out, oracle.softmax_causal(ins[0], int(np.prod(shp[0][:-1])), shp[0][-1], scalars[0],
                                                   scalars[1]))
        elif code == OpCode.RMS_NORM:
            h = shp[0][-1]
            self._write(out, oracle.rms_norm(ins[0], ins[1], ins[0].size // h, h, op.eps))
        elif code == OpCode.ROPE:
            s = shp[0]
            b, heads, seq, d = (s[0], s[1], s[2], s[3]) if len(s) == 4 else (s[0], 1, s[1], s[2])
            variant = "neox" if op.rope_variant == RopeVariant.NEOX else "gptj"
            self._write(out, oracle.rope(ins[0], ins[1], b, heads, seq, d, op.theta, variant))
        elif code == OpCode.SILU:
            self._write(out, oracle.silu(ins[0]))
        elif code == OpCode.SCALE:
            self._write(out, oracle.scale(ins[0], op.factor))
        elif code == OpCode.MUL:
            self._write(out, oracle.mul(ins[0], ins[1], ins[0].size))
        elif code == OpCode.ADD:
            self._write(out, oracle.add(ins[0], ins[1], ins[0].size))
        elif code == OpCode.GATHER:
            vocab, hidden = shp[0]
            self._write(out, oracle.gather(ins[0], ins[1], vocab, hidden, ins[1].size))
        elif code == OpCode.LAST_TOKEN:
            b, seq, h = shp[0]
            self._write(out, oracle.last_token(ins[0], b, seq, h, scalars[0]))
        elif code == OpCode.SPLIT_HEADS:
            b, seq, _ = shp[0]
            self._write(out, oracle.split_heads(ins[0], b, seq, op.heads, op.head_dim))
        elif code == OpCode.MERGE_HEADS:
            b, _, seq, _ = shp[0]
            self._write(out, oracle.merge_heads(ins[0], b, seq, op.heads, op.head_dim))
        elif code in (OpCode.KV_APPEND, OpCode.CAUSAL_ATTENTION):
            si = [i for i, v in enumerate(input_values) if v.role == ValueRole.STATE][0]
            st = shp[si]
            cache_ref = inputs[si]
            cache = self.f32[cache_ref.buffer][cache_ref.offset:cache_ref.offset + cache_ref.len]
            layers, max_seq = st[1], st[3]
            if code == OpCode.KV_APPEND:
                b, hkv, seq, d = shp[0]
                new = oracle.kv_append(ins[0], ins[1], cache, b, layers, op.layer, hkv, d, max_seq, scalars[0], seq)
            else:
                b, h, seq, d = shp[0]
                res, new = oracle.causal_attention(ins[0], ins[1], ins[2], cache, b, layers, op.layer, op.heads,
                                                   op.kv_heads, seq, scalars[0], d, max_seq, op.scale)
                self._write(out, res)
            self.f32[cache_ref.buffer][cache_ref.offset:cache_ref.offset + cache_ref.len] = new
        elif code == OpCode.SWIGLU:
            hidden = shp[0][-1]
            inter = shp[1][0]
            self._write(out, oracle.swiglu(ins[0], ins[1], ins[2], ins[3], ins[0].size // hidden, hidden, inter))
        elif code == OpCode.RMS_NORM_MATMUL:
            hidden = shp[0][-1]
            self._write(out, oracle.rms_norm_matmul(ins[0], ins[1], ins[2], ins[0].size // hidden, hidden,
                                                    shp[2][0], op.eps))
        else:
            raise NotImplementedError(code)
