"""The reference's device-contract tests (crates/backends/backend-cpu/src/
device.rs:1508-2285), run against the HIP device.

The reference compares CpuDevice bit-for-bit with direct calls of its scalar
kernels. Here the kernels are the C oracle and the device is the GPU, so
copies, Add, Mul and Scale stay bit-exact; Silu and RoPE are held to 1e-6
relative per element; reductions, matmuls and attention to 1e-4 normwise.
"""
import math

import numpy as np
import pytest

import oracle
from conftest import assert_elementwise, assert_normwise
from starlight_amd.device import DeviceError
from starlight_amd.ir import BufferRef, Op, RopeVariant, Value, ValueRole

pytestmark = pytest.mark.gpu


def f32_value(shape, role=ValueRole.TEMP):
    return Value.f32(shape, role)


def u32_value(shape):
    return Value.u32(shape, ValueRole.INPUT)


def test_allocate_upload_and_download_round_trip(hip):
    """device.rs:1508-1526."""
    floats = hip.allocate_f32(4, 64)
    hip.upload_f32(floats, [1.0, -2.0, 3.5, 0.0])
    out = np.zeros(4, np.float32)
    hip.download_f32(floats, out)
    assert out.tolist() == [1.0, -2.0, 3.5, 0.0]
    integers = hip.allocate_u32(3, 64)
    hip.upload_u32(integers, [7, 8, 9])
    ids = np.zeros(3, np.uint32)
    hip.download_u32(integers, ids)
    assert ids.tolist() == [7, 8, 9]


def test_fresh_buffers_are_zero_filled(hip):
    """device.rs:64-69: allocation zero-fills."""
    b = hip.allocate_f32(1000, 256)
    assert np.all(hip.read_f32(b, 1000) == 0.0)


def test_rejects_unknown_buffers_and_ranges(hip):
    """device.rs:1528-1558."""
    with pytest.raises(DeviceError) as err:
        hip.upload_f32(100000, [1.0])
    assert err.value == DeviceError.invalid_buffer(100000)
    floats = hip.allocate_f32(2, 64)
    with pytest.raises(DeviceError) as err:
        hip.upload_f32(floats, [1.0, 2.0, 3.0])
    assert err.value == DeviceError.invalid_range(floats, 0, 3)
    with pytest.raises(DeviceError) as err:
        hip.download_f32(floats, np.zeros(1, np.float32))
    assert err.value == DeviceError.invalid_range(floats, 0, 1)
    with pytest.raises(DeviceError) as err:
        hip.allocate_f32(1, 3)
    assert err.value == DeviceError.execution("alignment must be a nonzero power of two")


def test_dispatches_gather_rms_norm_matmul_and_last_token(hip):
    """device.rs:1560-1699: the runtime fixture chain through one scratchpad
    buffer at offsets 0 / 16 / 32."""
    table_data = (np.arange(32, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    norm_data = np.array([1.0, 0.5, 1.5, 0.75], np.float32)
    matmul_data = ((np.arange(32) % 7).astype(np.float32) - 3.0) * np.float32(0.2)
    table = hip.upload_new_f32(table_data)
    norm = hip.upload_new_f32(norm_data)
    matmul = hip.upload_new_f32(matmul_data)
    scratch = hip.allocate_f32(48, 64)
    ids = hip.upload_new_u32([3, 5])
    logits = hip.allocate_f32(8, 64)

    token_value = u32_value([1, 2])
    table_value = Value.f32([8, 4], ValueRole.PARAM)
    gather_value = f32_value([1, 2, 4])
    norm_value = Value.f32([4], ValueRole.PARAM)
    norm_out = f32_value([1, 2, 4])
    matmul_value = Value.f32([8, 4], ValueRole.PARAM)
    matmul_out = f32_value([1, 2, 8])
    logits_value = Value.f32([1, 8], ValueRole.OUTPUT)
    gather_ref = BufferRef(scratch, 0, 8)
    norm_out_ref = BufferRef(scratch, 16, 8)
    matmul_out_ref = BufferRef(scratch, 32, 16)

    hip.dispatch(Op.gather(), [BufferRef(table, 0, 32), BufferRef(ids, 0, 2)], [table_value, token_value],
                 [gather_ref], [gather_value])
    hip.dispatch(Op.rms_norm(1e-5), [gather_ref, BufferRef(norm, 0, 4)], [gather_value, norm_value],
                 [norm_out_ref], [norm_out])
    hip.dispatch(Op.matmul_nt(), [norm_out_ref, BufferRef(matmul, 0, 32)], [norm_out, matmul_value],
                 [matmul_out_ref], [matmul_out])
    hip.dispatch(Op.last_token(), [matmul_out_ref], [matmul_out], [BufferRef(logits, 0, 8)], [logits_value],
                 [2])
    hip.synchronize()

    expected_gather = oracle.gather(table_data, [3, 5], 8, 4, 2)
    expected_norm = oracle.rms_norm(expected_gather, norm_data, 2, 4, 1e-5)
    expected_matmul = oracle.matmul_nt(expected_norm, matmul_data, 1, 2, 4, 8)
    expected = oracle.last_token(expected_matmul, 1, 2, 8, 2)
    everything = hip.read_f32(scratch, 48)
    assert np.array_equal(everything[0:8], expected_gather)
    assert np.all(everything[8:16] == 0) and np.all(everything[24:32] == 0)
    assert_normwise(everything[16:24], expected_norm)
    assert_normwise(hip.read_f32(logits, 8), expected)


def test_dispatches_elementwise_ops(hip):
    """device.rs:1701-1791."""
    a_data = np.array([0.5, -1.0, 2.0, 0.0, -0.5, 1.5], np.float32)
    b_data = np.array([-0.25, 3.0, 0.5, -2.0, 1.0, 0.75], np.float32)
    a = hip.upload_new_f32(a_data)
    b = hip.upload_new_f32(b_data)
    out = hip.allocate_f32(6, 64)
    av, bv, ov = f32_value([2, 3]), f32_value([2, 3]), f32_value([2, 3], ValueRole.OUTPUT)
    ar, br, orf = BufferRef(a, 0, 6), BufferRef(b, 0, 6), BufferRef(out, 0, 6)

    hip.dispatch(Op.silu(), [ar], [av], [orf], [ov])
    assert_elementwise(hip.read_f32(out, 6), oracle.silu(a_data))
    hip.dispatch(Op.mul(), [ar, br], [av, bv], [orf], [ov])
    assert np.array_equal(hip.read_f32(out, 6), oracle.mul(a_data, b_data, 6))
    hip.dispatch(Op.add(), [ar, br], [av, bv], [orf], [ov])
    assert np.array_equal(hip.read_f32(out, 6), oracle.add(a_data, b_data, 6))
    hip.dispatch(Op.scale_by(-1.5), [ar], [av], [orf], [ov])
    assert np.array_equal(hip.read_f32(out, 6), oracle.scale(a_data, -1.5))


def test_dispatches_softmax_rope_and_head_layouts(hip):
    """device.rs:1793-1944."""
    x_data = np.array([0.5, -1.0, 2.0, 0.0, -0.5, 1.5], np.float32)
    x = hip.upload_new_f32(x_data)
    out = hip.allocate_f32(6, 64)
    xv, ov = f32_value([2, 3]), f32_value([2, 3], ValueRole.OUTPUT)
    xr, orf = BufferRef(x, 0, 6), BufferRef(out, 0, 6)
    hip.dispatch(Op.softmax(), [xr], [xv], [orf], [ov])
    assert_normwise(hip.read_f32(out, 6), oracle.softmax(x_data, 2, 3))
    hip.dispatch(Op.softmax_causal(), [xr], [xv], [orf], [ov], [2, 1])
    got = hip.read_f32(out, 6)
    want = oracle.softmax_causal(x_data, 2, 3, 2, 1)
    assert_normwise(got, want)
    assert got[2] == 0.0  # masked column is exactly zero

    rope_data = ((np.arange(16) - 7.0) * 0.125).astype(np.float32)
    positions = np.array([0, 1], np.uint32)
    rin = hip.upload_new_f32(rope_data)
    rout = hip.allocate_f32(16, 64)
    pos = hip.upload_new_u32(positions)
    hip.dispatch(Op.rope(RopeVariant.NEOX, 10_000.0), [BufferRef(rin, 0, 16), BufferRef(pos, 0, 2)],
                 [f32_value([1, 2, 2, 4]), u32_value([1, 2])], [BufferRef(rout, 0, 16)],
                 [f32_value([1, 2, 2, 4], ValueRole.OUTPUT)])
    assert_elementwise(hip.read_f32(rout, 16), oracle.rope(rope_data, positions, 1, 2, 2, 4, 10_000.0))

    sin_ = hip.upload_new_f32(rope_data)
    sout = hip.allocate_f32(16, 64)
    mout = hip.allocate_f32(16, 64)
    hip.dispatch(Op.split_heads(2, 4), [BufferRef(sin_, 0, 16)], [f32_value([1, 2, 8])],
                 [BufferRef(sout, 0, 16)], [f32_value([1, 2, 2, 4])])
    assert np.array_equal(hip.read_f32(sout, 16), oracle.split_heads(rope_data, 1, 2, 2, 4))
    hip.dispatch(Op.merge_heads(2, 4), [BufferRef(sout, 0, 16)], [f32_value([1, 2, 2, 4])],
                 [BufferRef(mout, 0, 16)], [f32_value([1, 2, 8], ValueRole.OUTPUT)])
    assert np.array_equal(hip.read_f32(mout, 16), rope_data)


def test_dispatches_matmul_nn_and_fused_ops(hip):
    """device.rs:1946-2124."""
    a_data = ((np.arange(6) - 2.0) * 0.25).astype(np.float32)
    b_data = ((np.arange(12) - 5.0) * 0.125).astype(np.float32)
    a, b, out = hip.upload_new_f32(a_data), hip.upload_new_f32(b_data), hip.allocate_f32(8, 64)
    hip.dispatch(Op.matmul_nn(), [BufferRef(a, 0, 6), BufferRef(b, 0, 12)],
                 [f32_value([2, 3]), Value.f32([3, 4], ValueRole.PARAM)], [BufferRef(out, 0, 8)],
                 [f32_value([2, 4], ValueRole.OUTPUT)])
    assert_normwise(hip.read_f32(out, 8), oracle.matmul_nn(a_data, b_data, 1, 2, 3, 4))

    x_data = np.array([0.25, -0.5, 1.0, 0.75, -0.25, 0.5], np.float32)
    gate_data = ((np.arange(12) % 5 - 2.0) * 0.3).astype(np.float32)
    up_data = ((np.arange(12) % 3 - 1.0) * 0.4).astype(np.float32)
    down_data = ((np.arange(12) % 7 - 3.0) * 0.2).astype(np.float32)
    x, g, u, d = (hip.upload_new_f32(v) for v in (x_data, gate_data, up_data, down_data))
    sout = hip.allocate_f32(6, 64)
    hip.dispatch(Op.swiglu(), [BufferRef(x, 0, 6), BufferRef(g, 0, 12), BufferRef(u, 0, 12), BufferRef(d, 0, 12)],
                 [f32_value([2, 3]), Value.f32([4, 3], ValueRole.PARAM), Value.f32([4, 3], ValueRole.PARAM),
                  Value.f32([3, 4], ValueRole.PARAM)], [BufferRef(sout, 0, 6)],
                 [f32_value([2, 3], ValueRole.OUTPUT)])
    assert_normwise(hip.read_f32(sout, 6), oracle.swiglu(x_data, gate_data, up_data, down_data, 2, 3, 4))

    norm_data = np.array([1.0, 0.5, 1.5], np.float32)
    matrix_data = ((np.arange(12) - 4.0) * 0.2).astype(np.float32)
    norm, matrix, fout = hip.upload_new_f32(norm_data), hip.upload_new_f32(matrix_data), hip.allocate_f32(8, 64)
    x2 = hip.upload_new_f32(x_data)
    hip.dispatch(Op.rms_norm_matmul(1e-5), [BufferRef(x2, 0, 6), BufferRef(norm, 0, 3), BufferRef(matrix, 0, 12)],
                 [f32_value([2, 3]), Value.f32([3], ValueRole.PARAM), Value.f32([4, 3], ValueRole.PARAM)],
                 [BufferRef(fout, 0, 8)], [f32_value([2, 4], ValueRole.OUTPUT)])
    assert_normwise(hip.read_f32(fout, 8), oracle.rms_norm_matmul(x_data, norm_data, matrix_data, 2, 3, 4, 1e-5))


def test_dispatches_kv_append_and_causal_attention_with_mutable_state(hip):
    """device.rs:2126-2248."""
    q_data = np.array([0.1, -0.2, 0.3, 0.4], np.float32)
    k_data = np.array([0.5, -0.1, 0.2, 0.7], np.float32)
    v_data = np.array([0.9, -0.4, 0.6, 0.2], np.float32)
    q, k, v = hip.upload_new_f32(q_data), hip.upload_new_f32(k_data), hip.upload_new_f32(v_data)
    state_append = hip.allocate_f32(16, 64)
    state_attention = hip.allocate_f32(16, 64)
    out = hip.allocate_f32(4, 64)
    qv = kv = vv = f32_value([1, 1, 2, 2])
    ov = f32_value([1, 1, 2, 2], ValueRole.OUTPUT)
    sv = Value.f32([1, 1, 2, 4, 1, 2], ValueRole.STATE)

    hip.dispatch(Op.kv_append(0), [BufferRef(k, 0, 4), BufferRef(v, 0, 4), BufferRef(state_append, 0, 16)],
                 [kv, vv, sv], [], [], [0])
    expected_cache = oracle.kv_append(k_data, v_data, np.zeros(16), 1, 1, 0, 1, 2, 4, 0, 2)
    assert np.array_equal(hip.read_f32(state_append, 16), expected_cache)

    hip.dispatch(Op.causal_attention(0, 1, 1, 2, 0.5),
                 [BufferRef(q, 0, 4), BufferRef(k, 0, 4), BufferRef(v, 0, 4), BufferRef(state_attention, 0, 16)],
                 [qv, kv, vv, sv], [BufferRef(out, 0, 4)], [ov], [0])
    expected_out, expected_state = oracle.causal_attention(q_data, k_data, v_data, np.zeros(16), 1, 1, 0, 1, 1,
                                                           2, 0, 2, 4, 0.5)
    assert_normwise(hip.read_f32(out, 4), expected_out)
    assert np.array_equal(hip.read_f32(state_attention, 16), expected_state)


def test_rejects_overlapping_ranges(hip):
    """device.rs:2250-2285."""
    buffer = hip.allocate_f32(8, 64)
    value = f32_value([4])
    output = hip.allocate_f32(4, 64)
    with pytest.raises(DeviceError) as err:
        hip.dispatch(Op.add(), [BufferRef(buffer, 0, 4), BufferRef(buffer, 2, 4)], [value, value],
                     [BufferRef(output, 0, 4)], [value])
    assert err.value == DeviceError.execution("one command aliases overlapping input ranges")


def test_gather_rejects_out_of_range_id_before_writing(hip):
    """layout.rs:298-318 through the device: the output is left unchanged."""
    table = hip.upload_new_f32([1.0, 2.0, 3.0, 4.0])
    ids = hip.upload_new_u32([0, 4])
    out = hip.upload_new_f32([9.0, 9.0, 9.0, 9.0])
    with pytest.raises(DeviceError) as err:
        hip.dispatch(Op.gather(), [BufferRef(table, 0, 4), BufferRef(ids, 0, 2)],
                     [Value.f32([2, 2], ValueRole.PARAM), u32_value([2])], [BufferRef(out, 0, 4)],
                     [f32_value([2, 2])])
    assert err.value == DeviceError.execution("id out of range")
    assert hip.read_f32(out, 4).tolist() == [9.0] * 4


def test_attention_rejects_overflowing_cache_before_writing(hip):
    """attention.rs:54-59 via the device: past_len + seq > max_seq fails and the cache is untouched."""
    cache = hip.upload_new_f32(np.full(16, 7.0, np.float32))
    q, k, v = (hip.upload_new_f32(np.ones(4, np.float32)) for _ in range(3))
    out = hip.allocate_f32(4, 64)
    sv = Value.f32([1, 1, 2, 4, 1, 2], ValueRole.STATE)
    t = f32_value([1, 1, 2, 2])
    with pytest.raises(DeviceError) as err:
        hip.dispatch(Op.causal_attention(0, 1, 1, 2, 0.5),
                     [BufferRef(q, 0, 4), BufferRef(k, 0, 4), BufferRef(v, 0, 4), BufferRef(cache, 0, 16)],
                     [t, t, t, sv], [BufferRef(out, 0, 4)], [f32_value([1, 1, 2, 2], ValueRole.OUTPUT)], [3])
    assert err.value == DeviceError.execution("past_len + seq exceeds max_seq")
    assert np.all(hip.read_f32(cache, 16) == 7.0)
