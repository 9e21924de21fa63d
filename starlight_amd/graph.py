"""llama-dense lowering and static memory planning — the thin slice of
sl-model-adapters and sl-graph the device needs to be driven end to end.

Neither crate is in the reference tree; this restates what its docs fix:
  * the per-layer op sequence and weight roles (ARCH-0006:159-198,
    ARCH-0004 §5.2-5.3; the runtime fixture's Gather -> RmsNorm -> MatMulNT ->
    LastToken order, distros/starlight-runtime/src/fixture.rs:98-123);
  * composites kept whole because the device declares them (ARCH-0004 §5.3);
  * NeoX RoPE on [B, H, S, D] with positions [B, S] (ARCH-0006:211);
  * the KV cache State [B, L, 2, max_seq, Hkv, D] (ARCH-0004 §9.1);
  * Temp values packed into one scratchpad by greedy interval colouring over
    [first_use, last_use], offsets aligned to 256 bytes (ARCH-0004 §7).
LastToken runs before the final RmsNorm and lm_head: both are row-wise, so the
last row's logits are identical and the prefill skips an [S, V] projection.
The exact op order of sl-model-adapters is not readable here (parity
unpinned); the engine's GPU-vs-oracle comparison runs one and the same
CommandBuffer on both devices.
"""
from __future__ import annotations

import dataclasses
import enum
import math
from dataclasses import dataclass, field
from typing import Dict, FrozenSet, List, Optional, Tuple

from .ir import (IR_VERSION, Command, CommandBuffer, DType, Effect, KvCacheDecl, MemoryPlan, Op, OpCode,
                 QuantFormat, RopeVariant, Slot, Value, ValueRole)

PLAN_ALIGN = 256


@dataclass(frozen=True)
class LlamaConfig:
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    eps: float = 1e-5
    theta: float = 10_000.0
    quant: Optional[QuantFormat] = None   # linear weights (q/k/v/o/gate/up/down)
    group: int = 128
    quant_lm_head: bool = True            # lm_head follows `quant` when set


# The configurations the benchmark and the tests run (synthetic weights).
TINY = LlamaConfig(layers=2, hidden=256, heads=4, kv_heads=4, head_dim=64, ffn=688, vocab=1024, eps=1e-5,
                   theta=10_000.0)
LLAMA_1B_INT4 = LlamaConfig(layers=16, hidden=2048, heads=32, kv_heads=8, head_dim=64, ffn=8192, vocab=32000,
                            eps=1e-5, theta=500_000.0, quant=QuantFormat.INT4)
LLAMA_8B_INT4 = LlamaConfig(layers=32, hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
                            eps=1e-5, theta=500_000.0, quant=QuantFormat.INT4)
LLAMA_8B_INT8 = LlamaConfig(layers=32, hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
                            eps=1e-5, theta=500_000.0, quant=QuantFormat.INT8)


@dataclass
class WeightSpec:
    name: str
    shape: Tuple[int, ...]
    quantized: bool  # stored group-quantized (payload + scales)
    kind: str        # "embed" | "norm" | "linear"
    # role of the separate f32 scale Param [n, k / group] of a quantized
    # weight (ARCH-0006:147: "<role>.__scales", not carried in the encoding)
    scales: Optional[str] = None


SCALES_SUFFIX = ".__scales"


def weight_specs(cfg: LlamaConfig) -> List[WeightSpec]:
    """Canonical weight roles of llama-dense (ARCH-0006:159-172), in a fixed order."""
    q = cfg.quant is not None
    H, D = cfg.hidden, cfg.head_dim
    specs = [WeightSpec("embed", (cfg.vocab, H), False, "embed")]
    for l in range(cfg.layers):
        p = f"layers.{l}."
        specs += [
            WeightSpec(p + "attn_norm", (H,), False, "norm"),
            WeightSpec(p + "attn.q", (cfg.heads * D, H), q, "linear"),
            WeightSpec(p + "attn.k", (cfg.kv_heads * D, H), q, "linear"),
            WeightSpec(p + "attn.v", (cfg.kv_heads * D, H), q, "linear"),
            WeightSpec(p + "attn.o", (H, cfg.heads * D), q, "linear"),
            WeightSpec(p + "mlp_norm", (H,), False, "norm"),
            WeightSpec(p + "mlp.gate", (cfg.ffn, H), q, "linear"),
            WeightSpec(p + "mlp.up", (cfg.ffn, H), q, "linear"),
            WeightSpec(p + "mlp.down", (H, cfg.ffn), q, "linear"),
        ]
    specs += [WeightSpec("final_norm", (H,), False, "norm"),
              WeightSpec("lm_head", (cfg.vocab, H), q and cfg.quant_lm_head, "linear")]
    for spec in specs:
        if spec.quantized:
            spec.scales = spec.name + SCALES_SUFFIX
    return specs


@dataclass
class Lowered:
    """One compiled program plus the ValueIds the engine binds (the
    CompiledProgram metadata of ARCH-0007 §3.2)."""

    ir: CommandBuffer
    weights: Dict[str, int]        # weight role (scale Params included) -> ValueId
    token_ids: int
    positions: int
    seq_len: int
    past_len: int
    logits: int
    kv_cache: int
    # quantized Param ValueId -> ValueId of its scale Param
    quant_scales: Dict[int, int] = field(default_factory=dict)


class _Builder:
    def __init__(self):
        self.values: List[Value] = []
        self.commands: List[Command] = []

    def value(self, v: Value) -> int:
        self.values.append(v)
        return len(self.values) - 1

    def temp(self, shape) -> int:
        return self.value(Value.f32(shape, ValueRole.TEMP))

    def cmd(self, op: Op, inputs, outputs, effect=Effect.NONE, state=None) -> None:
        self.commands.append(Command(op, list(inputs), list(outputs), effect, state))


def lower_llama(cfg: LlamaConfig, batch: int, seq: int, max_seq: int) -> Lowered:
    """Lowers llama-dense for one concrete (batch, seq) shape: seq = prompt
    length for prefill, 1 for decode (ARCH-0006:184-190)."""
    b = _Builder()
    H, D, Hq, Hkv = cfg.hidden, cfg.head_dim, cfg.heads, cfg.kv_heads
    token_ids = b.value(Value.u32([batch, seq], ValueRole.INPUT))
    positions = b.value(Value.u32([batch, seq], ValueRole.INPUT))
    seq_len = b.value(Value(DType.U32, (), ValueRole.SCALAR))
    past_len = b.value(Value(DType.U32, (), ValueRole.SCALAR))
    kv = b.value(Value.f32([batch, cfg.layers, 2, max_seq, Hkv, D], ValueRole.STATE))

    weights: Dict[str, int] = {}
    quant_scales: Dict[int, int] = {}
    for spec in weight_specs(cfg):
        if spec.quantized:
            weights[spec.name] = b.value(Value.quantized(spec.shape, cfg.quant, cfg.group))
            n, k = spec.shape
            weights[spec.scales] = b.value(Value.f32([n, k // cfg.group], ValueRole.PARAM))
            quant_scales[weights[spec.name]] = weights[spec.scales]
        else:
            weights[spec.name] = b.value(Value.f32(spec.shape, ValueRole.PARAM))

    h = b.temp([batch, seq, H])
    b.cmd(Op.gather(), [weights["embed"], token_ids], [h])
    scale = float(1.0 / math.sqrt(D))
    for l in range(cfg.layers):
        p = f"layers.{l}."
        x = b.temp([batch, seq, H])
        b.cmd(Op.rms_norm(cfg.eps), [h, weights[p + "attn_norm"]], [x])
        q, k, v = b.temp([batch, seq, Hq * D]), b.temp([batch, seq, Hkv * D]), b.temp([batch, seq, Hkv * D])
        b.cmd(Op.matmul_nt(), [x, weights[p + "attn.q"]], [q])
        b.cmd(Op.matmul_nt(), [x, weights[p + "attn.k"]], [k])
        b.cmd(Op.matmul_nt(), [x, weights[p + "attn.v"]], [v])
        qh, kh, vh = b.temp([batch, Hq, seq, D]), b.temp([batch, Hkv, seq, D]), b.temp([batch, Hkv, seq, D])
        b.cmd(Op.split_heads(Hq, D), [q], [qh])
        b.cmd(Op.split_heads(Hkv, D), [k], [kh])
        b.cmd(Op.split_heads(Hkv, D), [v], [vh])
        qr, kr = b.temp([batch, Hq, seq, D]), b.temp([batch, Hkv, seq, D])
        b.cmd(Op.rope(RopeVariant.NEOX, cfg.theta), [qh, positions], [qr])
        b.cmd(Op.rope(RopeVariant.NEOX, cfg.theta), [kh, positions], [kr])
        att = b.temp([batch, Hq, seq, D])
        b.cmd(Op.causal_attention(l, Hq, Hkv, D, scale), [qr, kr, vh, past_len], [att], Effect.WRITE_STATE, kv)
        merged = b.temp([batch, seq, Hq * D])
        b.cmd(Op.merge_heads(Hq, D), [att], [merged])
        o = b.temp([batch, seq, H])
        b.cmd(Op.matmul_nt(), [merged, weights[p + "attn.o"]], [o])
        h2 = b.temp([batch, seq, H])
        b.cmd(Op.add(), [h, o], [h2])
        x2 = b.temp([batch, seq, H])
        b.cmd(Op.rms_norm(cfg.eps), [h2, weights[p + "mlp_norm"]], [x2])
        f = b.temp([batch, seq, H])
        b.cmd(Op.swiglu(), [x2, weights[p + "mlp.gate"], weights[p + "mlp.up"], weights[p + "mlp.down"]], [f])
        h3 = b.temp([batch, seq, H])
        b.cmd(Op.add(), [h2, f], [h3])
        h = h3
    last = b.temp([batch, H])
    b.cmd(Op.last_token(), [h, seq_len], [last])
    normed = b.temp([batch, H])
    b.cmd(Op.rms_norm(cfg.eps), [last, weights["final_norm"]], [normed])
    logits = b.value(Value.f32([batch, cfg.vocab], ValueRole.OUTPUT))
    b.cmd(Op.matmul_nt(), [normed, weights["lm_head"]], [logits])

    plan = plan_memory(b.values, b.commands)
    ir = CommandBuffer(IR_VERSION, b.values, b.commands, plan, [token_ids, positions], [logits],
                       [KvCacheDecl(kv, batch, cfg.layers, Hkv, D, max_seq)])
    return Lowered(ir, weights, token_ids, positions, seq_len, past_len, logits, kv, quant_scales)


def plan_memory(values: List[Value], commands: List[Command], align: int = PLAN_ALIGN) -> MemoryPlan:
    """Greedy interval colouring of Temp values (ARCH-0004 §7): lifetimes are
    [first use, last use as an input]; values sorted by first use take the
    lowest aligned offset whose byte range is free of every overlapping live
    value. O(N log N) in the number of values for the sort, deterministic."""
    first: Dict[int, int] = {}
    last: Dict[int, int] = {}
    for i, c in enumerate(commands):
        for vid in list(c.inputs) + list(c.outputs):
            first.setdefault(vid, i)
            last[vid] = max(last.get(vid, i), i)
    temps = sorted((vid for vid in first if values[vid].role == ValueRole.TEMP), key=lambda v: (first[v], v))
    placed: List[Tuple[int, int, int, int]] = []  # (offset, end, first, last)
    slots: List[Slot] = []
    top = 0
    for vid in temps:
        size = values[vid].byte_size()
        need = (size + align - 1) // align * align
        live = sorted((o, e) for (o, e, f, l) in placed if not (l < first[vid] or f > last[vid]))
        offset = 0
        for o, e in live:
            if offset + need <= o:
                break
            offset = max(offset, (e + align - 1) // align * align)
        placed.append((offset, offset + need, first[vid], last[vid]))
        slots.append(Slot(vid, offset, size))
        top = max(top, offset + need)
    slots.sort(key=lambda s: s.value)
    return MemoryPlan(top, slots)


def validate_plan(values: List[Value], commands: List[Command], plan: MemoryPlan, align: int = PLAN_ALIGN) -> None:
    """MemoryPlan invariants of ARCH-0004 §7; raises AssertionError."""
    first: Dict[int, int] = {}
    last: Dict[int, int] = {}
    for i, c in enumerate(commands):
        for vid in list(c.inputs) + list(c.outputs):
            first.setdefault(vid, i)
            last[vid] = max(last.get(vid, i), i)
    seen = set()
    for s in plan.slots:
        assert values[s.value].role == ValueRole.TEMP, "only Temp values get slots"
        assert s.value not in seen, "a value appears twice"
        seen.add(s.value)
        assert s.offset % align == 0, "slot offset is not aligned"
        assert s.offset + s.bytes <= plan.scratchpad_bytes, "slot exceeds the scratchpad"
        assert s.bytes == values[s.value].byte_size(), "slot size differs from the value size"
    temps = {v for v in first if values[v].role == ValueRole.TEMP}
    assert temps == seen, "every Temp value needs exactly one slot"
    ss = sorted(plan.slots, key=lambda s: s.offset)
    for i, a in enumerate(ss):
        for bb in ss[i + 1:]:
            if bb.offset >= a.offset + a.bytes:
                break
            disjoint_life = last[a.value] < first[bb.value] or last[bb.value] < first[a.value]
            assert disjoint_life, f"values {a.value} and {bb.value} share bytes while both are live"


# Runtime fixture (distros/starlight-runtime/src/fixture.rs:26-36, 59-217):
# vocab 8, hidden 4, Gather -> RmsNorm(1e-5) -> MatMulNT(lm_head) -> LastToken.
FIXTURE_VOCAB, FIXTURE_HIDDEN = 8, 4


def fixture_weights():
    """fixture.rs:200-217: embed[i] = (i - 3) * 0.1, norm [1, .5, 1.5, .75],
    lm_head[i] = ((i % 5) - 2) * 0.1 — each computed in f32 like the Rust."""
    import numpy as np

    idx = np.arange(FIXTURE_VOCAB * FIXTURE_HIDDEN, dtype=np.float32)
    embed = ((idx - np.float32(3.0)) * np.float32(0.1)).astype(np.float32)
    lm = (((np.arange(FIXTURE_VOCAB * FIXTURE_HIDDEN) % 5).astype(np.float32) - np.float32(2.0)) *
          np.float32(0.1)).astype(np.float32)
    return {"embed": embed.reshape(FIXTURE_VOCAB, FIXTURE_HIDDEN), "norm": np.array([1.0, 0.5, 1.5, 0.75], np.float32),
            "lm_head": lm.reshape(FIXTURE_VOCAB, FIXTURE_HIDDEN)}


def lower_fixture(seq: int) -> Lowered:
    """The fixture program for one sequence length; the command order is the
    one rt/tests/fixture_compile.rs:35-48 asserts."""
    b = _Builder()
    token_ids = b.value(Value.u32([1, seq], ValueRole.INPUT))
    embed = b.value(Value.f32([FIXTURE_VOCAB, FIXTURE_HIDDEN], ValueRole.PARAM))
    gathered = b.temp([1, seq, FIXTURE_HIDDEN])
    norm = b.value(Value.f32([FIXTURE_HIDDEN], ValueRole.PARAM))
    rms = b.temp([1, seq, FIXTURE_HIDDEN])
    lm_head = b.value(Value.f32([FIXTURE_VOCAB, FIXTURE_HIDDEN], ValueRole.PARAM))
    matmul = b.temp([1, seq, FIXTURE_VOCAB])
    seq_len = b.value(Value(DType.U32, (), ValueRole.SCALAR))
    logits = b.value(Value.f32([1, FIXTURE_VOCAB], ValueRole.OUTPUT))
    b.cmd(Op.gather(), [embed, token_ids], [gathered])
    b.cmd(Op.rms_norm(1e-5), [gathered, norm], [rms])
    b.cmd(Op.matmul_nt(), [rms, lm_head], [matmul])
    b.cmd(Op.last_token(), [matmul, seq_len], [logits])
    plan = plan_memory(b.values, b.commands)
    ir = CommandBuffer(IR_VERSION, b.values, b.commands, plan, [token_ids], [logits], [])
    # The fixture has no RoPE or KV cache: positions/past_len are absent (-1).
    return Lowered(ir, {"embed": embed, "norm": norm, "lm_head": lm_head}, token_ids, -1, seq_len, -1, logits, -1)


# ------------------------------------------------- capability negotiation --
#
# The capability step of sl-graph's compile(program, shape_spec, caps)
# (ARCH-0004 §8, §10 step 3, §11 CompileError; §5.3 decomposition rules):
#  * a composite the device does not declare is decomposed when a rule
#    exists (SwiGlu, RmsNormMatMul), else UnsupportedOp { node, op };
#  * every remaining op must be a core op of the device (UnsupportedOp);
#  * every value's dtype must be in the device's set (UnsupportedDType);
#  * a violated shape constraint is CapabilityMismatch { constraint, limit,
#    actual };
#  * ir_version must equal the compiler's IR_VERSION (VersionMismatch);
#  * the plan is made after decomposition, with offsets aligned to
#    max(64, min_buffer_align) (ARCH-0004 §7), and must fit
#    max_scratchpad_bytes (PlanOverflow).

COMPOSITES = (OpCode.CAUSAL_ATTENTION, OpCode.SWIGLU, OpCode.RMS_NORM_MATMUL)


class ConstraintKind(enum.Enum):
    HEAD_DIM_MULTIPLE_OF = "head_dim_multiple_of"
    MATMUL_K_MULTIPLE_OF = "matmul_k_multiple_of"
    MAX_HEADS = "max_heads"


@dataclass(frozen=True)
class ShapeConstraints:
    head_dim_multiple_of: int = 1
    matmul_k_multiple_of: int = 1
    max_heads: int = 0xFFFFFFFF


@dataclass(frozen=True)
class DeviceCapabilities:
    """sl_ir::DeviceCapabilities (ARCH-0004 §8); op and dtype sets as frozensets."""

    backend: str
    ir_version: int
    core_ops: FrozenSet[OpCode]
    composite_ops: FrozenSet[OpCode]
    dtypes: FrozenSet[DType]
    min_buffer_align: int
    max_scratchpad_bytes: int
    max_value_bytes: int
    constraints: ShapeConstraints = ShapeConstraints()

    @staticmethod
    def from_c(c: dict) -> "DeviceCapabilities":
        """From the sl_capabilities struct a backend reports (bitsets over
        sl_opcode / sl_dtype), e.g. starlight_amd.device.capabilities()."""
        ops = lambda mask: frozenset(o for o in OpCode if mask >> int(o) & 1)  # noqa: E731
        return DeviceCapabilities(
            c["backend"], c["ir_version"], ops(c["core_ops"]), ops(c["composite_ops"]),
            frozenset(d for d in DType if c["dtypes"] >> int(d) & 1), c["min_buffer_align"],
            c["max_scratchpad_bytes"], c["max_value_bytes"],
            ShapeConstraints(c["head_dim_multiple_of"], c["matmul_k_multiple_of"], c["max_heads"]))

    def replace(self, **kw) -> "DeviceCapabilities":
        return dataclasses.replace(self, **kw)


class CompileError(Exception):
    """sl_graph::CompileError (ARCH-0004 §11): `kind` is the variant name,
    `fields` its payload."""

    def __init__(self, kind: str, **fields):
        self.kind = kind
        self.fields = fields
        super().__init__(f"{kind} {fields}")

    def __eq__(self, other):
        return isinstance(other, CompileError) and (self.kind, self.fields) == (other.kind, other.fields)

    __hash__ = Exception.__hash__


def _decompose(b: _Builder, c: Command, values: List[Value]) -> Optional[List[Command]]:
    """The §5.3 rules, or None when the composite has none. Each keeps the
    reference's arithmetic order, so results are bit-identical to the
    composite's (swiglu.rs:40-84: silu(dot(x, Wg_i)) * dot(x, Wu_i), then
    sum over i ascending of (g u)_i Wd[j, i]; fused.rs:41-90: ((x inv) w_i)
    W[c, i] summed left to right)."""
    if c.op.code == OpCode.SWIGLU:
        x, wg, wu, wd = c.inputs
        lead = values[x].shape[:-1]
        inter = values[wg].shape[0]
        g, u, sg, h = (b.temp(list(lead) + [inter]) for _ in range(4))
        return [Command(Op.matmul_nt(), [x, wg], [g]), Command(Op.matmul_nt(), [x, wu], [u]),
                Command(Op.silu(), [g], [sg]), Command(Op.mul(), [sg, u], [h]),
                Command(Op.matmul_nt(), [h, wd], c.outputs)]
    if c.op.code == OpCode.RMS_NORM_MATMUL:
        x, w, mat = c.inputs
        normed = b.temp(values[x].shape)
        return [Command(Op.rms_norm(c.op.eps), [x, w], [normed]), Command(Op.matmul_nt(), [normed, mat], c.outputs)]
    return None


def _check_constraints(node: int, c: Command, values: List[Value], k: ShapeConstraints) -> None:
    def mismatch(kind, limit, actual):
        raise CompileError("CapabilityMismatch", constraint=kind, limit=limit, actual=actual)

    code = c.op.code
    head_dim = None
    if code in (OpCode.SPLIT_HEADS, OpCode.MERGE_HEADS, OpCode.CAUSAL_ATTENTION):
        head_dim = c.op.head_dim
    elif code == OpCode.ROPE:
        head_dim = values[c.inputs[0]].shape[-1]
    if head_dim is not None and head_dim % max(1, k.head_dim_multiple_of):
        mismatch(ConstraintKind.HEAD_DIM_MULTIPLE_OF, k.head_dim_multiple_of, head_dim)
    if code in (OpCode.SPLIT_HEADS, OpCode.MERGE_HEADS, OpCode.CAUSAL_ATTENTION) and c.op.heads > k.max_heads:
        mismatch(ConstraintKind.MAX_HEADS, k.max_heads, c.op.heads)
    if code in (OpCode.MATMUL_NT, OpCode.MATMUL_NN, OpCode.RMS_NORM_MATMUL):
        kk = values[c.inputs[0]].shape[-1]
        if kk % max(1, k.matmul_k_multiple_of):
            mismatch(ConstraintKind.MATMUL_K_MULTIPLE_OF, k.matmul_k_multiple_of, kk)


def compile_for(lowered: Lowered, caps: DeviceCapabilities) -> Lowered:
    """The capability, plan and emit steps for one device: returns a Lowered
    whose CommandBuffer the device can run, or raises CompileError."""
    cb = lowered.ir
    if caps.ir_version != cb.ir_version:
        raise CompileError("VersionMismatch", device=caps.ir_version, compiler=cb.ir_version)
    b = _Builder()
    b.values = list(cb.values)
    for node, c in enumerate(cb.commands):
        emitted = [c]
        if c.op.code in COMPOSITES and c.op.code not in caps.composite_ops:
            emitted = _decompose(b, c, b.values)
            if emitted is None:
                raise CompileError("UnsupportedOp", node=node, op=c.op.code)
        for e in emitted:
            if e.op.code not in caps.core_ops and e.op.code not in caps.composite_ops:
                raise CompileError("UnsupportedOp", node=node, op=e.op.code)
            _check_constraints(node, e, b.values, caps.constraints)
            b.commands.append(e)
    used = set()
    for c in b.commands:
        used.update(c.inputs)
        used.update(c.outputs)
        if c.state is not None:
            used.add(c.state)
    used.update(lowered.quant_scales.values())
    for vid in sorted(used):
        if b.values[vid].dtype not in caps.dtypes:
            raise CompileError("UnsupportedDType", value=vid, dtype=b.values[vid].dtype)
    align = max(64, caps.min_buffer_align)
    plan = plan_memory(b.values, b.commands, align)
    if plan.scratchpad_bytes > caps.max_scratchpad_bytes:
        raise CompileError("PlanOverflow", required=plan.scratchpad_bytes, limit=caps.max_scratchpad_bytes)
    validate_plan(b.values, b.commands, plan, align)
    ir = CommandBuffer(cb.ir_version, b.values, b.commands, plan, list(cb.inputs), list(cb.outputs),
                       list(cb.states))
    return dataclasses.replace(lowered, ir=ir)
