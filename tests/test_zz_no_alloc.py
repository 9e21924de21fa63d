"""sl_hip_dispatch_noalloc, the entry point that allocates nothing: through
the C ABI, each command gives what sl_hip_dispatch (logged, then
synchronized) gives on the same inputs, on two calls in a row, the second
with a smaller input. The commands are ones whose kernels use scratch
memory: decode attention (split partials), SwiGlu (the silu(g) * u
intermediate), a quantized MatMulNT with m * k above the fused GEMV's limit
(split-K partials), and RmsNormMatMul (the normalised rows)."""
import math

import numpy as np
import pytest

from conftest import assert_normwise
from starlight_amd import quant
from starlight_amd.device import DeviceError
from starlight_amd.ir import BufferRef, Op, QuantFormat, Value, ValueRole

pytestmark = pytest.mark.gpu


def run_both(hip, op, inputs, in_vals, out_len, out_val, scalars=(), state=None):
    """Runs the command once through each entry point from identical
    buffers; returns ((out, state) logged, (out, state) no-alloc)."""
    results = []
    for noalloc in (False, True):
        refs = []
        for a in inputs:
            if a.dtype == np.uint32:
                b = hip.upload_new_u32(a)
            else:
                b = hip.upload_new_f32(a)
            refs.append(BufferRef(b, 0, a.size))
        ob = hip.allocate_f32(out_len, 256)
        outs = [BufferRef(ob, 0, out_len)]
        if noalloc:
            hip.dispatch_noalloc(op, refs, in_vals, outs, [out_val], scalars)
        else:
            hip.dispatch(op, refs, in_vals, outs, [out_val], scalars)
        hip.synchronize()
        st = hip.read_f32(refs[state].buffer, inputs[state].size) if state is not None else None
        results.append((hip.read_f32(ob, out_len), st))
    return results


def attention_case(hip, H, Hkv, D, past, max_seq, seed):
    r = np.random.default_rng(seed)
    B, S = 1, 1
    q = r.uniform(-1, 1, B * H * S * D).astype(np.float32)
    k = r.uniform(-1, 1, B * Hkv * S * D).astype(np.float32)
    v = r.uniform(-1, 1, B * Hkv * S * D).astype(np.float32)
    cache = r.uniform(-1, 1, B * 1 * 2 * max_seq * Hkv * D).astype(np.float32)
    q4, k4 = Value.f32([B, H, S, D]), Value.f32([B, Hkv, S, D])
    vals = [q4, k4, k4, Value.f32([B, 1, 2, max_seq, Hkv, D], ValueRole.STATE)]
    op = Op.causal_attention(0, H, Hkv, D, float(np.float32(1.0 / math.sqrt(D))))
    (o1, c1), (o2, c2) = run_both(hip, op, [q, k, v, cache], vals, q.size, q4, [past], state=3)
    np.testing.assert_array_equal(o2, o1)
    np.testing.assert_array_equal(c2, c1)


def test_decode_attention_twice_second_smaller(hip):
    attention_case(hip, 32, 8, 128, 1000, 4096, 1)   # 8B decode shape, long cache
    attention_case(hip, 8, 2, 64, 37, 64, 2)         # smaller


def qweight(hip, n, k, fmt, seed):
    r = np.random.default_rng(seed)
    w = (r.standard_normal((n, k)) * 0.05).astype(np.float32)
    words, scales = quant.quantize(w, 128, fmt)
    pb, sb = hip.upload_new_u32(words), hip.upload_new_f32(scales)
    hip.bind_quantized(pb, sb, fmt, 128, n, k)
    return BufferRef(pb, 0, words.size), Value.quantized([n, k], fmt, 128)


def run_weighted(hip, op, x, x_val, weights, extra, out_len, out_val):
    outs = []
    for noalloc in (False, True):
        xb = hip.upload_new_f32(x)
        refs = [BufferRef(xb, 0, x.size)] + [BufferRef(hip.upload_new_f32(a), 0, a.size) for a in extra]
        refs += [w[0] for w in weights]
        vals = [x_val] + [Value.f32([a.size], ValueRole.PARAM) for a in extra] + [w[1] for w in weights]
        ob = hip.allocate_f32(out_len, 256)
        fn = hip.dispatch_noalloc if noalloc else hip.dispatch
        fn(op, refs, vals, [BufferRef(ob, 0, out_len)], [out_val])
        hip.synchronize()
        outs.append(hip.read_f32(ob, out_len))
    np.testing.assert_array_equal(outs[1], outs[0])
    return outs[0]


def test_swiglu_twice_second_smaller(hip):
    for rows, hidden, inter, fmt, seed in ((4, 1024, 2816, QuantFormat.INT4, 3), (1, 256, 512, QuantFormat.INT8, 4)):
        g, u, d = (qweight(hip, inter, hidden, fmt, seed), qweight(hip, inter, hidden, fmt, seed + 10),
                   qweight(hip, hidden, inter, fmt, seed + 20))
        x = np.random.default_rng(seed).uniform(-1, 1, rows * hidden).astype(np.float32)
        run_weighted(hip, Op.swiglu(), x, Value.f32([rows, hidden]), [g, u, d], [], rows * hidden,
                     Value.f32([rows, hidden]))


def test_split_k_gemv_twice_second_smaller(hip):
    # m * k above 32768: the split-K GEMV with its partials in scratch
    for m, n, k, seed in ((16, 512, 4096, 5), (12, 256, 4096, 6)):
        w = qweight(hip, n, k, QuantFormat.INT4, seed)
        x = np.random.default_rng(seed).standard_normal(m * k).astype(np.float32)
        run_weighted(hip, Op.matmul_nt(), x, Value.f32([1, m, k]), [w], [], m * n, Value.f32([1, m, n]))


def test_rms_norm_matmul_twice_second_smaller(hip):
    for rows, hidden, out_f, seed in ((5, 2048, 768, 7), (2, 512, 256, 8)):
        w = qweight(hip, out_f, hidden, QuantFormat.INT8, seed)
        x = np.random.default_rng(seed).uniform(-2, 2, rows * hidden).astype(np.float32)
        gamma = np.random.default_rng(seed + 1).uniform(0.5, 1.5, hidden).astype(np.float32)
        run_weighted(hip, Op.rms_norm_matmul(1e-5), x, Value.f32([rows, hidden]), [w], [gamma], rows * out_f,
                     Value.f32([rows, out_f]))


def test_rejects_logged_commands_and_oversized_scratch(hip):
    a = hip.upload_new_f32(np.ones(8, np.float32))
    o = hip.allocate_f32(8, 256)
    v = Value.f32([8])
    hip.dispatch(Op.silu(), [BufferRef(a, 0, 8)], [v], [BufferRef(o, 0, 8)], [v])  # logged, not submitted
    with pytest.raises(DeviceError) as e:
        hip.dispatch_noalloc(Op.silu(), [BufferRef(a, 0, 8)], [v], [BufferRef(o, 0, 8)], [v])
    assert e.value == DeviceError.execution("commands are still logged: submit them before sl_hip_dispatch_noalloc")
    hip.submit()
    # a SwiGlu whose intermediate exceeds the static array (2 * inter > 2M floats)
    inter = (1 << 20) + 1
    x = hip.upload_new_f32(np.ones(1, np.float32))
    wts = [hip.upload_new_f32(np.ones(inter, np.float32)) for _ in range(3)]
    out = hip.allocate_f32(1, 256)
    with pytest.raises(DeviceError) as e:
        hip.dispatch_noalloc(Op.swiglu(), [BufferRef(x, 0, 1)] + [BufferRef(w, 0, inter) for w in wts],
                             [Value.f32([1, 1]), Value.f32([inter, 1], ValueRole.PARAM),
                              Value.f32([inter, 1], ValueRole.PARAM), Value.f32([1, inter], ValueRole.PARAM)],
                             [BufferRef(out, 0, 1)], [Value.f32([1, 1])])
    assert e.value == DeviceError.unimplemented("swiglu inter size exceeds the device workspace")
    hip.synchronize()
