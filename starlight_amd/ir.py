"""Python mirror of the sl-ir types that cross the device boundary.

Names and declaration orders follow sl-ir as specified in the reference's
docs (ARCH-0004 §3 types, §5.1 `OpCode`/`Op`, §6 `CommandBuffer`, §7
`MemoryPlan`) and `sl_device::BufferRef` (ARCH-0007 §3.1). The ctypes
structures match include/starlight_hip.h field for field.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Tuple

MAX_RANK = 8


class DType(enum.IntEnum):
    F32 = 0
    F16 = 1
    BF16 = 2
    U32 = 3
    I32 = 4
    U8 = 5
    I8 = 6


class ValueRole(enum.IntEnum):
    INPUT = 0
    SCALAR = 1
    OUTPUT = 2
    PARAM = 3
    STATE = 4
    TEMP = 5


class Encoding(enum.IntEnum):
    DENSE = 0
    GROUPWISE_QUANTIZED = 1
    OPAQUE_QUANTIZED = 2


class QuantFormat(enum.IntEnum):
    INT4 = 0
    INT8 = 1


class OpCode(enum.IntEnum):
    MATMUL_NT = 0
    MATMUL_NN = 1
    SOFTMAX = 2
    SOFTMAX_CAUSAL = 3
    RMS_NORM = 4
    ROPE = 5
    SILU = 6
    MUL = 7
    ADD = 8
    SCALE = 9
    GATHER = 10
    LAST_TOKEN = 11
    KV_APPEND = 12
    SPLIT_HEADS = 13
    MERGE_HEADS = 14
    CAUSAL_ATTENTION = 15
    SWIGLU = 16
    RMS_NORM_MATMUL = 17


class RopeVariant(enum.IntEnum):
    NEOX = 0
    GPTJ = 1


# ---------------------------------------------------------------- ctypes --


class CValue(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_uint32),
        ("role", ctypes.c_uint32),
        ("rank", ctypes.c_uint32),
        ("dims", ctypes.c_uint32 * MAX_RANK),
        ("encoding", ctypes.c_uint32),
        ("qformat", ctypes.c_uint32),
        ("group_size", ctypes.c_uint32),
    ]


class COp(ctypes.Structure):
    _fields_ = [
        ("code", ctypes.c_uint32),
        ("rope_variant", ctypes.c_uint32),
        ("eps", ctypes.c_float),
        ("theta", ctypes.c_float),
        ("factor", ctypes.c_float),
        ("scale", ctypes.c_float),
        ("layer", ctypes.c_uint32),
        ("heads", ctypes.c_uint32),
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
    ]


class CBufferRef(ctypes.Structure):
    _fields_ = [
        ("buffer", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("offset", ctypes.c_uint64),
        ("len", ctypes.c_uint64),
    ]


class CError(ctypes.Structure):
    _fields_ = [
        ("status", ctypes.c_int32),
        ("buffer", ctypes.c_uint32),
        ("offset", ctypes.c_uint64),
        ("len", ctypes.c_uint64),
        ("requested", ctypes.c_uint64),
        ("op", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("message", ctypes.c_char_p),
    ]


class CBufferDesc(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_uint32),
        ("quantized", ctypes.c_uint32),
        ("qformat", ctypes.c_uint32),
        ("group_size", ctypes.c_uint32),
        ("qn", ctypes.c_uint32),
        ("qk", ctypes.c_uint32),
        ("elements", ctypes.c_uint64),
    ]


class CCapabilities(ctypes.Structure):
    _fields_ = [
        ("backend", ctypes.c_char_p),
        ("ir_version", ctypes.c_uint32),
        ("core_ops", ctypes.c_uint32),
        ("composite_ops", ctypes.c_uint32),
        ("dtypes", ctypes.c_uint32),
        ("min_buffer_align", ctypes.c_uint32),
        ("max_scratchpad_bytes", ctypes.c_uint64),
        ("max_value_bytes", ctypes.c_uint64),
        ("head_dim_multiple_of", ctypes.c_uint32),
        ("matmul_k_multiple_of", ctypes.c_uint32),
        ("max_heads", ctypes.c_uint32),
    ]


# ------------------------------------------------------------- values ------


@dataclass(frozen=True)
class Value:
    """sl_ir::Value with concrete dims: dtype, shape, role, encoding."""

    dtype: DType
    shape: Tuple[int, ...]
    role: ValueRole
    encoding: Encoding = Encoding.DENSE
    qformat: QuantFormat = QuantFormat.INT4
    group_size: int = 0

    @staticmethod
    def f32(shape: Sequence[int], role: ValueRole = ValueRole.TEMP) -> "Value":
        return Value(DType.F32, tuple(int(d) for d in shape), role)

    @staticmethod
    def u32(shape: Sequence[int], role: ValueRole = ValueRole.INPUT) -> "Value":
        return Value(DType.U32, tuple(int(d) for d in shape), role)

    @staticmethod
    def quantized(shape: Sequence[int], qformat: QuantFormat, group_size: int) -> "Value":
        return Value(DType.F32, tuple(int(d) for d in shape), ValueRole.PARAM,
                     Encoding.GROUPWISE_QUANTIZED, QuantFormat(qformat), int(group_size))

    def element_count(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    def byte_size(self) -> int:
        return 4 * self.element_count()

    def to_c(self) -> CValue:
        v = CValue()
        v.dtype = int(self.dtype)
        v.role = int(self.role)
        v.rank = len(self.shape)
        for i, d in enumerate(self.shape[:MAX_RANK]):
            v.dims[i] = d
        v.encoding = int(self.encoding)
        v.qformat = int(self.qformat)
        v.group_size = self.group_size
        return v


@dataclass(frozen=True)
class Op:
    """sl_ir::Op: the opcode plus its attributes."""

    code: OpCode
    rope_variant: RopeVariant = RopeVariant.NEOX
    eps: float = 0.0
    theta: float = 0.0
    factor: float = 0.0
    scale: float = 0.0
    layer: int = 0
    heads: int = 0
    kv_heads: int = 0
    head_dim: int = 0

    # Constructors named after the Op variants (ARCH-0004 §5.1).
    @staticmethod
    def matmul_nt() -> "Op":
        return Op(OpCode.MATMUL_NT)

    @staticmethod
    def matmul_nn() -> "Op":
        return Op(OpCode.MATMUL_NN)

    @staticmethod
    def softmax() -> "Op":
        return Op(OpCode.SOFTMAX)

    @staticmethod
    def softmax_causal() -> "Op":
        return Op(OpCode.SOFTMAX_CAUSAL)

    @staticmethod
    def rms_norm(eps: float) -> "Op":
        return Op(OpCode.RMS_NORM, eps=eps)

    @staticmethod
    def rope(variant: RopeVariant, theta: float) -> "Op":
        return Op(OpCode.ROPE, rope_variant=RopeVariant(variant), theta=theta)

    @staticmethod
    def silu() -> "Op":
        return Op(OpCode.SILU)

    @staticmethod
    def mul() -> "Op":
        return Op(OpCode.MUL)

    @staticmethod
    def add() -> "Op":
        return Op(OpCode.ADD)

    @staticmethod
    def scale_by(factor: float) -> "Op":
        return Op(OpCode.SCALE, factor=factor)

    @staticmethod
    def gather() -> "Op":
        return Op(OpCode.GATHER)

    @staticmethod
    def last_token() -> "Op":
        return Op(OpCode.LAST_TOKEN)

    @staticmethod
    def kv_append(layer: int) -> "Op":
        return Op(OpCode.KV_APPEND, layer=layer)

    @staticmethod
    def split_heads(heads: int, head_dim: int) -> "Op":
        return Op(OpCode.SPLIT_HEADS, heads=heads, head_dim=head_dim)

    @staticmethod
    def merge_heads(heads: int, head_dim: int) -> "Op":
        return Op(OpCode.MERGE_HEADS, heads=heads, head_dim=head_dim)

    @staticmethod
    def causal_attention(layer: int, heads: int, kv_heads: int, head_dim: int, scale: float) -> "Op":
        return Op(OpCode.CAUSAL_ATTENTION, layer=layer, heads=heads, kv_heads=kv_heads,
                  head_dim=head_dim, scale=scale)

    @staticmethod
    def swiglu() -> "Op":
        return Op(OpCode.SWIGLU)

    @staticmethod
    def rms_norm_matmul(eps: float) -> "Op":
        return Op(OpCode.RMS_NORM_MATMUL, eps=eps)

    def to_c(self) -> COp:
        o = COp()
        o.code = int(self.code)
        o.rope_variant = int(self.rope_variant)
        o.eps = self.eps
        o.theta = self.theta
        o.factor = self.factor
        o.scale = self.scale
        o.layer = self.layer
        o.heads = self.heads
        o.kv_heads = self.kv_heads
        o.head_dim = self.head_dim
        return o


@dataclass(frozen=True)
class BufferRef:
    """sl_device::BufferRef: buffer id, element offset, element count."""

    buffer: int
    offset: int
    len: int

    def to_c(self) -> CBufferRef:
        r = CBufferRef()
        r.buffer = self.buffer
        r.offset = self.offset
        r.len = self.len
        return r


# --------------------------------------------------- CommandBuffer (§6/7) --


class Effect(enum.IntEnum):
    NONE = 0
    READ_STATE = 1
    WRITE_STATE = 2


@dataclass
class Command:
    op: Op
    inputs: List[int]
    outputs: List[int]
    effect: Effect = Effect.NONE
    state: Optional[int] = None  # ValueId of the state the effect targets


@dataclass
class Slot:
    value: int
    offset: int  # bytes
    bytes: int


@dataclass
class MemoryPlan:
    scratchpad_bytes: int
    slots: List[Slot] = field(default_factory=list)


@dataclass
class KvCacheDecl:
    value: int
    batch: int
    layers: int
    kv_heads: int
    head_dim: int
    max_seq: int


@dataclass
class CommandBuffer:
    ir_version: int
    values: List[Value]
    commands: List[Command]
    plan: MemoryPlan
    inputs: List[int]
    outputs: List[int]
    states: List[KvCacheDecl]


IR_VERSION = 2
