"""Capability negotiation (the capability step of sl-graph's compile,
ARCH-0004 §8, §10, §11) and quantized Params with separate scale Params
(ARCH-0006:147), on the CPU.

 * A composite the device does not declare is decomposed (SwiGlu,
   RmsNormMatMul; §5.3) with bit-identical results on the oracle device;
   CausalAttention has no rule: UnsupportedOp.
 * A missing core op is UnsupportedOp { node, op }; a dtype outside the
   device's set is UnsupportedDType { value, dtype }; each violated shape
   constraint is CapabilityMismatch { constraint, limit, actual }; a plan
   beyond max_scratchpad_bytes is PlanOverflow; another ir_version is
   VersionMismatch.
 * Engine build binds every quantized Param to its `<role>.__scales` Param
   and rejects a program whose scale Param is missing.
"""
import numpy as np
import pytest

from oracle.cpu_device import OracleDevice
from starlight_amd import device as dev
from starlight_amd import engine, graph, synth
from starlight_amd.graph import CompileError, ConstraintKind, DeviceCapabilities, LlamaConfig, ShapeConstraints
from starlight_amd.ir import IR_VERSION, BufferRef, DType, Op, OpCode, QuantFormat, Value, ValueRole

ALL = DeviceCapabilities("test", IR_VERSION, frozenset(OpCode), frozenset(graph.COMPOSITES),
                         frozenset({DType.F32, DType.U32}), 256, 1 << 40, 1 << 40)
QCFG = LlamaConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=384, theta=500_000.0,
                   quant=QuantFormat.INT4)


def codes(lowered):
    return [c.op.code for c in lowered.ir.commands]


def test_hip_capabilities_compile_the_llama_programs_unchanged():
    caps = DeviceCapabilities.from_c(dev.capabilities())
    assert caps.backend == "hip-gfx950" and OpCode.SWIGLU in caps.composite_ops
    for cfg in (graph.TINY, QCFG):
        low = graph.lower_llama(cfg, 1, 4, 16)
        out = graph.compile_for(low, caps)
        assert codes(out) == codes(low)
        for s in out.ir.plan.slots:
            assert s.offset % 256 == 0


def run(cfg, lowered_pre, lowered_dec, prompt, steps, seed=3):
    d = OracleDevice()
    bufs = engine.upload_weights(d, cfg, synth.llama_weights(cfg, seed))
    eng = engine.Engine(d, engine.compile_program(lowered_pre, bufs), engine.compile_program(lowered_dec, bufs), 1,
                        16)
    return eng.generate(prompt, steps, cfg.vocab)


@pytest.mark.parametrize("cfg", [graph.TINY, QCFG])
def test_undeclared_swiglu_is_decomposed_with_identical_results(cfg):
    caps = ALL.replace(composite_ops=frozenset({OpCode.CAUSAL_ATTENTION}))
    pre, dec = graph.lower_llama(cfg, 1, 5, 16), graph.lower_llama(cfg, 1, 1, 16)
    cpre, cdec = graph.compile_for(pre, caps), graph.compile_for(dec, caps)
    assert OpCode.SWIGLU not in codes(cpre)
    per_layer = [OpCode.MATMUL_NT, OpCode.MATMUL_NT, OpCode.SILU, OpCode.MUL, OpCode.MATMUL_NT]
    c = codes(cpre)
    i = c.index(OpCode.SILU) - 2
    assert c[i:i + 5] == per_layer
    assert c.count(OpCode.SILU) == cfg.layers
    prompt = synth.prompt(cfg.vocab, 5, 3)
    t_ref, l_ref = run(cfg, pre, dec, prompt, 3)
    t_dec, l_dec = run(cfg, cpre, cdec, prompt, 3)
    np.testing.assert_array_equal(t_dec, t_ref)
    assert l_dec.tobytes() == l_ref.tobytes()


def test_undeclared_rms_norm_matmul_is_decomposed_with_identical_results():
    b = graph._Builder()
    x = b.value(Value.f32([1, 3, 64], ValueRole.INPUT))
    w = b.value(Value.f32([64], ValueRole.PARAM))
    m = b.value(Value.f32([40, 64], ValueRole.PARAM))
    out = b.value(Value.f32([1, 3, 40], ValueRole.OUTPUT))
    b.cmd(Op.rms_norm_matmul(1e-5), [x, w, m], [out])
    cb = graph.CommandBuffer(IR_VERSION, b.values, b.commands, graph.plan_memory(b.values, b.commands), [x], [out],
                             [])
    low = graph.Lowered(cb, {"w": w, "m": m}, x, -1, -1, -1, out, -1)
    dlow = graph.compile_for(low, ALL.replace(composite_ops=frozenset()))
    assert codes(dlow) == [OpCode.RMS_NORM, OpCode.MATMUL_NT]
    r = np.random.default_rng(0)
    data = {x: r.standard_normal(192).astype(np.float32), w: r.uniform(0.5, 1.5, 64).astype(np.float32),
            m: r.standard_normal(40 * 64).astype(np.float32)}

    def execute(lw):
        d = OracleDevice()
        refs = {v: BufferRef(d.upload_new_f32(a), 0, a.size) for v, a in data.items()}
        refs[out] = BufferRef(d.allocate_f32(120, 256), 0, 120)
        if lw.ir.plan.scratchpad_bytes:
            sp = d.allocate_f32(lw.ir.plan.scratchpad_bytes // 4, 256)
            for s in lw.ir.plan.slots:
                refs[s.value] = BufferRef(sp, s.offset // 4, s.bytes // 4)
        for c in lw.ir.commands:
            d.dispatch(c.op, [refs[v] for v in c.inputs], [lw.ir.values[v] for v in c.inputs],
                       [refs[v] for v in c.outputs], [lw.ir.values[v] for v in c.outputs])
        return d.f32[refs[out].buffer].copy()

    assert execute(dlow).tobytes() == execute(low).tobytes()


def test_causal_attention_without_the_composite_is_unsupported():
    low = graph.lower_llama(graph.TINY, 1, 4, 16)
    node = codes(low).index(OpCode.CAUSAL_ATTENTION)
    with pytest.raises(CompileError) as e:
        graph.compile_for(low, ALL.replace(composite_ops=frozenset({OpCode.SWIGLU})))
    assert e.value == CompileError("UnsupportedOp", node=node, op=OpCode.CAUSAL_ATTENTION)


def test_missing_core_op_is_unsupported():
    low = graph.lower_llama(graph.TINY, 1, 4, 16)
    node = codes(low).index(OpCode.ROPE)
    with pytest.raises(CompileError) as e:
        graph.compile_for(low, ALL.replace(core_ops=frozenset(OpCode) - {OpCode.ROPE}))
    assert e.value == CompileError("UnsupportedOp", node=node, op=OpCode.ROPE)
    # a decomposition that needs a missing core op fails too, at the composite's node
    node = codes(low).index(OpCode.SWIGLU)
    with pytest.raises(CompileError) as e:
        graph.compile_for(low, ALL.replace(core_ops=frozenset(OpCode) - {OpCode.SILU},
                                           composite_ops=frozenset({OpCode.CAUSAL_ATTENTION})))
    assert e.value == CompileError("UnsupportedOp", node=node, op=OpCode.SILU)


def test_dtype_outside_the_device_set():
    low = graph.lower_llama(graph.TINY, 1, 4, 16)
    with pytest.raises(CompileError) as e:
        graph.compile_for(low, ALL.replace(dtypes=frozenset({DType.F32})))
    assert e.value == CompileError("UnsupportedDType", value=low.token_ids, dtype=DType.U32)


@pytest.mark.parametrize("constraints,kind,limit,actual", [
    (ShapeConstraints(head_dim_multiple_of=128), ConstraintKind.HEAD_DIM_MULTIPLE_OF, 128, 64),
    (ShapeConstraints(max_heads=2), ConstraintKind.MAX_HEADS, 2, 4),
    (ShapeConstraints(matmul_k_multiple_of=512), ConstraintKind.MATMUL_K_MULTIPLE_OF, 512, 256),
])
def test_constraint_violations_name_constraint_limit_and_actual(constraints, kind, limit, actual):
    low = graph.lower_llama(graph.TINY, 1, 4, 16)
    with pytest.raises(CompileError) as e:
        graph.compile_for(low, ALL.replace(constraints=constraints))
    assert e.value == CompileError("CapabilityMismatch", constraint=kind, limit=limit, actual=actual)


def test_plan_overflow_and_version_mismatch():
    low = graph.lower_llama(graph.TINY, 1, 4, 16)
    need = graph.compile_for(low, ALL).ir.plan.scratchpad_bytes
    with pytest.raises(CompileError) as e:
        graph.compile_for(low, ALL.replace(max_scratchpad_bytes=need - 1))
    assert e.value == CompileError("PlanOverflow", required=need, limit=need - 1)
    with pytest.raises(CompileError) as e:
        graph.compile_for(low, ALL.replace(ir_version=IR_VERSION + 1))
    assert e.value == CompileError("VersionMismatch", device=IR_VERSION + 1, compiler=IR_VERSION)


def test_quantized_params_carry_separate_scale_params():
    low = graph.lower_llama(QCFG, 1, 1, 16)
    q = low.weights["layers.0.attn.q"]
    s = low.weights["layers.0.attn.q.__scales"]
    assert low.quant_scales[q] == s
    v, sv = low.ir.values[q], low.ir.values[s]
    assert v.shape == (256, 256) and sv.shape == (256, 2) and sv.role == ValueRole.PARAM and sv.dtype == DType.F32
    assert len(low.quant_scales) == 7 * QCFG.layers + 1  # q k v o gate up down per layer, and lm_head


def test_build_binds_scale_params_and_rejects_a_missing_one():
    d = OracleDevice()
    bufs = engine.upload_weights(d, QCFG, synth.llama_weights(QCFG, 1))
    assert "lm_head.__scales" in bufs
    low = graph.lower_llama(QCFG, 1, 1, 16)
    engine.Engine(d, engine.compile_program(low, bufs), engine.compile_program(low, bufs), 1, 16)
    assert len(d.dequant) == len(low.quant_scales)
    missing = {k: v for k, v in bufs.items() if k != "layers.1.mlp.up.__scales"}
    with pytest.raises(engine.BuildError, match="no bound scale Param"):
        engine.Engine(OracleDevice(), engine.compile_program(low, missing), engine.compile_program(low, missing), 1,
                      16)
