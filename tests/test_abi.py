"""CPU-side checks of the C ABI: the library loads, exports every entry
point the public header declares, and its dispatch validation reproduces
CpuDevice's checks, order and error values (crates/backends/backend-cpu/src/
device.rs:224-377 and the per-op geometry of run_op, :773-1227) — exercised
through sl_hip_validate_dispatch, which needs no GPU.
"""
import ctypes

import pytest

from starlight_amd import device as dev
from starlight_amd.device import DeviceError, validate_dispatch
from starlight_amd.ir import BufferRef, Op, OpCode, QuantFormat, RopeVariant, Value, ValueRole


def test_library_exports_every_declared_symbol():
    lib = dev.load_library()
    declared = dev.exported_symbols()
    assert len(declared) >= 14
    for name in declared:
        assert hasattr(lib, name), f"{name} is declared in starlight_hip.h but not exported"
    assert lib.sl_hip_abi_version() == 2


def test_capabilities_declare_all_ops_and_composites():
    caps = dev.capabilities()
    assert caps["backend"] == "hip-gfx950"
    assert caps["ir_version"] == 2
    assert caps["core_ops"] == (1 << 18) - 1
    for code in (OpCode.CAUSAL_ATTENTION, OpCode.SWIGLU, OpCode.RMS_NORM_MATMUL):
        assert caps["composite_ops"] & (1 << code)
    assert caps["min_buffer_align"] >= 64


F32 = lambda n: {"kind": "f32", "elements": n}  # noqa: E731
U32 = lambda n: {"kind": "u32", "elements": n}  # noqa: E731


def v(shape, role=ValueRole.TEMP):
    return Value.f32(shape, role)


def check(buffers, op, ins, in_vals, outs, out_vals, scalars=()):
    return validate_dispatch(buffers, op, ins, in_vals, outs, out_vals, scalars)


def test_accepts_the_runtime_fixture_chain():
    """The four commands of device.rs:1629-1668 against their buffers."""
    bufs = [F32(32), F32(4), F32(32), F32(48), U32(2), F32(8)]
    assert check(bufs, Op.gather(), [BufferRef(0, 0, 32), BufferRef(4, 0, 2)],
                 [Value.f32([8, 4], ValueRole.PARAM), Value.u32([1, 2])], [BufferRef(3, 0, 8)], [v([1, 2, 4])]) is None
    assert check(bufs, Op.rms_norm(1e-5), [BufferRef(3, 0, 8), BufferRef(1, 0, 4)],
                 [v([1, 2, 4]), Value.f32([4], ValueRole.PARAM)], [BufferRef(3, 16, 8)], [v([1, 2, 4])]) is None
    assert check(bufs, Op.last_token(), [BufferRef(3, 32, 16)], [v([1, 2, 8])], [BufferRef(5, 0, 8)],
                 [v([1, 8], ValueRole.OUTPUT)], [2]) is None


def test_rejects_overlapping_ranges():
    """device.rs:2250-2285."""
    err = check([F32(8), F32(4)], Op.add(), [BufferRef(0, 0, 4), BufferRef(0, 2, 4)], [v([4]), v([4])],
                [BufferRef(1, 0, 4)], [v([4])])
    assert err == DeviceError.execution("one command aliases overlapping input ranges")
    err = check([F32(8), F32(4)], Op.add(), [BufferRef(0, 0, 4), BufferRef(1, 0, 4)], [v([4]), v([4])],
                [BufferRef(0, 3, 4)], [v([4])])
    assert err == DeviceError.execution("a command output aliases an overlapping input range")


@pytest.mark.parametrize("case,expected", [
    # validate_call (device.rs:224-286)
    (dict(op=Op.add(), ins=5), DeviceError.execution("too many command ports")),
    (dict(op=Op.add(), ins=1), DeviceError.execution("input buffer count does not match the operator signature")),
    (dict(op=Op.add(), outs=0), DeviceError.execution("output count does not match the operator signature")),
    (dict(op=Op.add(), scalars=[1]), DeviceError.execution("scalar count does not match the operator signature")),
    (dict(op=Op.add(), state=True), DeviceError.execution("stateless operator received a State input")),
    (dict(op=Op.kv_append(0), ins=2, outs=0, scalars=[0]),
     DeviceError.execution("stateful operator requires exactly one State input")),
    # validate_port (device.rs:288-324)
    (dict(op=Op.add(), in_len=3), DeviceError.execution("BufferRef length does not match the value element count")),
    (dict(op=Op.add(), in_buffer=9), DeviceError.invalid_buffer(9)),
    (dict(op=Op.add(), in_offset=6), DeviceError.invalid_range(0, 6, 4)),
    (dict(op=Op.add(), in_buffer=2), DeviceError.invalid_buffer(2)),          # u32 buffer used as f32
    (dict(op=Op.add(), scalar_role=True),
     DeviceError.execution("scalar operands must be passed through the scalars argument")),
    (dict(op=Op.add(), rank9=True), DeviceError("ShapeOverflow")),
    (dict(op=Op.add(), dtype_f16=True), DeviceError.unimplemented("dtype is not supported by HipDevice")),
])
def test_call_and_port_errors(case, expected):
    bufs = [F32(8), F32(8), U32(8)]
    n_in = case.get("ins", 2)
    ins = [BufferRef(case.get("in_buffer", 0), case.get("in_offset", 0), case.get("in_len", 4))] + \
          [BufferRef(1, 0, 4)] * (n_in - 1)
    vals = [v([4])] * n_in
    if case.get("state"):
        vals = [v([4]), Value.f32([4], ValueRole.STATE)]
    if case.get("scalar_role"):
        vals = [Value.f32([4], ValueRole.SCALAR), v([4])]
    if case.get("rank9"):
        vals = [Value.f32([1] * 8 + [4], ValueRole.TEMP), v([4])]
    if case.get("dtype_f16"):
        from starlight_amd.ir import DType
        vals = [Value(DType.F16, (4,), ValueRole.TEMP), v([4])]
    if case["op"].code == OpCode.KV_APPEND:
        vals = [v([1, 1, 2, 2])] * n_in
    n_out = case.get("outs", 1)
    outs = [BufferRef(1, 4, 4)] * n_out
    assert check(bufs, case["op"], ins[:n_in], vals[:n_in], outs, [v([4])] * n_out, case.get("scalars", [])) == expected


def test_integer_outputs_and_unknown_ops_are_rejected():
    err = check([U32(4), F32(4)], Op.silu(), [BufferRef(1, 0, 4)], [v([4])], [BufferRef(0, 0, 4)],
                [Value.u32([4], ValueRole.OUTPUT)])
    assert err == DeviceError.execution("integer command outputs are not supported")
    bogus = Op(OpCode.ADD)
    object.__setattr__(bogus, "code", 99)
    err = validate_dispatch([F32(4)], bogus, [], [], [], [])
    assert err.kind == "UnsupportedOp" and err.op == 99


@pytest.mark.parametrize("op,ins,outs,scalars,message", [
    (Op.matmul_nt(), [v([2, 3]), v([4, 5])], [v([2, 4])], [], "matmul reduction dimensions must match"),
    (Op.matmul_nt(), [v([2, 3]), v([4, 3])], [v([2, 5])], [], "matmul output shape must be m x n"),
    (Op.matmul_nt(), [v([2, 2, 3]), v([3, 4, 3])], [v([3, 2, 4])], [], "matmul batch dimensions are not broadcastable"),
    (Op.matmul_nt(), [v([3]), v([4, 3])], [v([4])], [], "matmul operands and output must have rank at least 2"),
    (Op.matmul_nt(), [v([2, 2, 3]), v([4, 3])], [v([3, 2, 4])], [], "matmul output batch must match the operands"),
    (Op.softmax(), [v([2, 3])], [v([3, 2])], [], "softmax output shape must match its input"),
    (Op.softmax(), [v([0, 3])], [v([0, 3])], [], "softmax requires nonzero rows and cols"),
    (Op.softmax_causal(), [v([2, 3])], [v([2, 3])], [2, 0], "softmax_causal requires cols == past_len + seq"),
    (Op.softmax_causal(), [v([3, 2])], [v([3, 2])], [2, 0], "softmax_causal requires rows to be a multiple of seq"),
    (Op.softmax_causal(), [v([2, 2])], [v([2, 2])], [0, 2], "softmax_causal requires a nonzero seq"),
    (Op.rms_norm(1e-5), [v([2, 4]), Value.f32([3], ValueRole.PARAM)], [v([2, 4])], [],
     "rms_norm weight shape must be [hidden]"),
    (Op.rms_norm(1e-5), [v([2, 0]), Value.f32([0], ValueRole.PARAM)], [v([2, 0])], [],
     "rms_norm requires a nonzero hidden size"),
    (Op.rope(RopeVariant.NEOX, 1e4), [v([1, 2, 3]), Value.u32([1, 2])], [v([1, 2, 3])], [],
     "head_dim must be a positive even number"),
    (Op.rope(RopeVariant.NEOX, 1e4), [v([1, 2, 4]), Value.u32([2, 1])], [v([1, 2, 4])], [],
     "rope positions shape must be [batch, seq]"),
    (Op.rope(RopeVariant.NEOX, 1e4), [v([4, 4]), Value.u32([4, 1])], [v([4, 4])], [],
     "rope input must have rank 3 or 4"),
    (Op.mul(), [v([2, 2]), v([4])], [v([2, 2])], [], "mul/add operands and output must have identical shapes"),
    (Op.gather(), [Value.f32([8], ValueRole.PARAM), Value.u32([2])], [v([2, 4])], [],
     "gather table must have shape [vocab, hidden]"),
    (Op.gather(), [Value.f32([8, 4], ValueRole.PARAM), Value.u32([2])], [v([2, 5])], [],
     "gather output width must equal hidden"),
    (Op.gather(), [Value.f32([8, 4], ValueRole.PARAM), Value.u32([1, 2])], [v([2, 4])], [],
     "gather output rank must be the id rank plus one"),
    (Op.last_token(), [v([1, 2, 4])], [v([1, 4])], [3], "last_token requires 1 <= seq_len <= seq"),
    (Op.last_token(), [v([2, 4])], [v([1, 4])], [1], "last_token shapes must be [B, M, H] -> [B, H]"),
    (Op.split_heads(2, 2), [v([1, 2, 5])], [v([1, 2, 2, 2])], [], "split_heads input width must equal heads * head_dim"),
    (Op.merge_heads(2, 2), [v([1, 3, 2, 2])], [v([1, 2, 4])], [],
     "merge_heads input does not match its heads/head_dim attributes"),
    (Op.swiglu(), [v([2, 3]), v([4, 3]), v([4, 3]), v([4, 3])], [v([2, 3])], [],
     "swiglu weight shapes must be [inter, hidden], [inter, hidden], [hidden, inter]"),
    (Op.rms_norm_matmul(1e-5), [v([2, 3]), v([3]), v([4, 2])], [v([2, 4])], [],
     "rms_norm_matmul matrix shape must be [out_features, hidden]"),
])
def test_geometry_errors(op, ins, outs, scalars, message):
    bufs = []
    refs = []
    for val in ins:
        n = val.element_count()
        bufs.append(U32(max(n, 1)) if val.dtype == 3 else F32(max(n, 1)))
        refs.append(BufferRef(len(bufs) - 1, 0, n))
    out_refs = []
    for val in outs:
        bufs.append(F32(max(val.element_count(), 1)))
        out_refs.append(BufferRef(len(bufs) - 1, 0, val.element_count()))
    assert check(bufs, op, refs, ins, out_refs, outs, scalars) == DeviceError.execution(message)


def _attention_case(heads=2, kv_heads=2, layer=0, past=1, state_shape=(1, 1, 2, 3, 2, 4), seq=2):
    q = v([1, heads, seq, 4])
    k = v([1, kv_heads, seq, 4])
    st = Value.f32(list(state_shape), ValueRole.STATE)
    n_state = 1
    for d in state_shape:
        n_state *= d
    bufs = [F32(max(q.element_count(), 1)), F32(max(k.element_count(), 1)), F32(max(k.element_count(), 1)),
            F32(n_state), F32(max(q.element_count(), 1))]
    refs = [BufferRef(0, 0, q.element_count()), BufferRef(1, 0, k.element_count()),
            BufferRef(2, 0, k.element_count()), BufferRef(3, 0, n_state)]
    return check(bufs, Op.causal_attention(layer, heads, kv_heads, 4, 0.5), refs, [q, k, k, st],
                 [BufferRef(4, 0, q.element_count())], [q], [past])


def test_attention_errors_follow_the_reference_order():
    """device.rs:1068-1143 then attention.rs:146-156 and kv_append's checks."""
    assert _attention_case() is None
    assert _attention_case(layer=1) == DeviceError.execution("attention layer is out of range")
    assert _attention_case(past=2) == DeviceError.execution("past_len + seq exceeds max_seq")
    assert _attention_case(state_shape=(1, 1, 2, 3, 1, 4)) == DeviceError.execution(
        "KV cache shape must be [batch, layers, 2, max_seq, kv_heads, head_dim]")
    assert _attention_case(heads=3, kv_heads=2, state_shape=(1, 1, 2, 3, 2, 4)) == DeviceError.execution(
        "heads must be a multiple of kv_heads")


def test_quantized_operand_rules():
    # payload u32 buffer 0 bound as INT4 [8, 128] g128 (8 * 64 bytes = 128 words), scales f32 buffer 1
    bound = {"kind": "u32", "elements": 128, "quant": (QuantFormat.INT4, 128, 8, 128)}
    bufs = [bound, F32(8), F32(2 * 128), F32(16)]
    wv = Value.quantized([8, 128], QuantFormat.INT4, 128)
    ok = check(bufs, Op.matmul_nt(), [BufferRef(2, 0, 256), BufferRef(0, 0, 128)], [v([2, 128]), wv],
               [BufferRef(3, 0, 16)], [v([2, 8])])
    assert ok is None
    err = check(bufs, Op.matmul_nt(), [BufferRef(2, 0, 256), BufferRef(0, 0, 127)], [v([2, 128]), wv],
                [BufferRef(3, 0, 16)], [v([2, 8])])
    assert err == DeviceError.execution("BufferRef length does not match the quantized payload size")
    wrong = Value.quantized([8, 128], QuantFormat.INT8, 128)
    err = check(bufs, Op.matmul_nt(), [BufferRef(2, 0, 256), BufferRef(0, 0, 128)], [v([2, 128]), wrong],
                [BufferRef(3, 0, 16)], [v([2, 8])])
    assert err == DeviceError.execution("quantized operand does not match its buffer binding")
    unbound = [U32(128), F32(8), F32(256), F32(16)]
    err = check(unbound, Op.matmul_nt(), [BufferRef(2, 0, 256), BufferRef(0, 0, 128)], [v([2, 128]), wv],
                [BufferRef(3, 0, 16)], [v([2, 8])])
    assert err == DeviceError.execution("quantized operand buffer has no bound scales")
    err = check(bufs, Op.matmul_nn(), [BufferRef(2, 0, 256), BufferRef(0, 0, 128)], [v([2, 128]), wv],
                [BufferRef(3, 0, 16)], [v([2, 8])])
    assert err == DeviceError.unimplemented("quantized operand is not supported on this port")
