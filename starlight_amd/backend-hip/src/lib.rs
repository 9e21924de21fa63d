// SPDX-License-Identifier: MIT OR Apache-2.0
//! [`HipDevice`]: an [`sl_device::Device`] on one MI355X (gfx950) GPU, over
//! the C ABI of `include/starlight_hip.h` (`libstarlight_hip.so`, built by
//! `build.rs`).
//!
//! It replaces `CpuDevice` (crates/backends/backend-cpu/src/device.rs:114-213)
//! method for method: buffers are device allocations with dense `BufferId`s,
//! `dispatch` validates with the same checks, order and static messages as
//! `CpuDevice` and enqueues the command, and `synchronize` waits for the
//! device. The library submits logged commands before anything can observe
//! them (synchronize, upload, download), so `sl-core`'s `Engine::step` loop
//! runs unchanged.
//!
//! Types follow sl-ir as ARCH-0004 fixes them: `Op` (§5.1), `Value` with
//! `DType`, `Shape` of `Dim::{Const, Sym}`, `ValueRole` and `TensorEncoding`
//! (§3), and `DeviceCapabilities` (§8).

mod ffi;

use std::ffi::CStr;
use std::ptr;

use sl_device::{BufferRef, Device, DeviceError};
use sl_ir::{
    BackendTag, BufferId, DType, DTypeSet, DeviceCapabilities, Dim, Op, OpCode, OpSet, QuantizationFormat,
    RopeVariant, ShapeConstraints, TensorEncoding, Value, ValueRole, IR_VERSION,
};

/// A paged KV cache's device buffers and geometry: `pool` f32
/// [layer][page][K, V][slot][kv_head][head_dim], `block_table` u32
/// [batch][pages_per_seq] page ids, `seq_lens` u32 [batch] cached lengths.
#[derive(Clone, Copy, Debug)]
pub struct PagedKv {
    pub pool: BufferId,
    pub block_table: BufferId,
    pub seq_lens: BufferId,
    pub layers: u32,
    pub num_pages: u32,
    pub page_size: u32,
    pub pages_per_seq: u32,
}

/// The HIP device. Single owner: every method takes `&mut self`, as the
/// trait does, and the library is not called from two threads at once.
pub struct HipDevice {
    raw: *mut ffi::sl_hip_device,
}

// The handle is owned by this value and only used through `&mut self`.
unsafe impl Send for HipDevice {}

impl HipDevice {
    /// Opens GPU `ordinal` (0 on a one-GPU node): creates the device's
    /// stream and workspace (`CpuDevice::new`, device.rs:41-45).
    pub fn new(ordinal: i32) -> Result<Self, DeviceError> {
        if unsafe { ffi::sl_hip_abi_version() } != ffi::SL_HIP_ABI_VERSION {
            return Err(DeviceError::Execution("libstarlight_hip.so has another ABI version"));
        }
        let mut raw = ptr::null_mut();
        let status = unsafe { ffi::sl_hip_device_create(ordinal, &mut raw) };
        if status != ffi::SL_OK || raw.is_null() {
            return Err(match status {
                ffi::SL_ERR_OUT_OF_MEMORY => DeviceError::OutOfMemory { requested: 0 },
                _ => DeviceError::Execution("the HIP device could not be opened"),
            });
        }
        Ok(Self { raw })
    }

    /// Binds a group-wise quantized weight: `payload` holds the u32 words of
    /// the packed codes, `scales` the f32 [n, k / group_size] scales (a
    /// separate Param, ARCH-0006:147). Ports whose value has
    /// `TensorEncoding::GroupwiseQuantized` then read `payload` (MatMulNT B,
    /// SwiGlu gate/up/down, RmsNormMatMul matrix). No reference counterpart:
    /// the 18 operator signatures carry no scale port.
    pub fn bind_quantized(
        &mut self,
        payload: BufferId,
        scales: BufferId,
        format: QuantizationFormat,
        group_size: u32,
        n: u32,
        k: u32,
    ) -> Result<(), DeviceError> {
        let qformat = match format {
            QuantizationFormat::Int4 => ffi::SL_QFORMAT_INT4,
            QuantizationFormat::Int8 => ffi::SL_QFORMAT_INT8,
        };
        let status = unsafe { ffi::sl_hip_bind_quantized(self.raw, payload.0, scales.0, qformat, group_size, n, k) };
        self.check(status)
    }

    /// Enqueues the logged commands without waiting (for timing with events
    /// on [`HipDevice::stream`]).
    pub fn submit(&mut self) -> Result<(), DeviceError> {
        let status = unsafe { ffi::sl_hip_submit(self.raw) };
        self.check(status)
    }

    /// The `hipStream_t` all work runs on.
    pub fn stream(&self) -> *mut std::os::raw::c_void {
        unsafe { ffi::sl_hip_stream(self.raw) }
    }

    /// `sl_hip_dispatch_noalloc`: the command's kernels enqueued at once with
    /// the library's static per-GPU scratch array, no allocation (for callers
    /// under their own HIP graph capture). Requires no logged commands.
    pub fn dispatch_noalloc(
        &mut self,
        op: &Op,
        inputs: &[BufferRef],
        input_values: &[&Value],
        outputs: &[BufferRef],
        output_values: &[&Value],
        scalars: &[u32],
    ) -> Result<(), DeviceError> {
        let call = Call::new(op, inputs, input_values, outputs, output_values)?;
        let status = unsafe {
            ffi::sl_hip_dispatch_noalloc(
                self.raw,
                &call.op,
                call.inputs.as_ptr(),
                call.input_values.as_ptr(),
                call.n_inputs,
                call.outputs.as_ptr(),
                call.output_values.as_ptr(),
                call.n_outputs,
                scalars.as_ptr(),
                scalars.len(),
            )
        };
        self.check(status)
    }

    /// `sl_hip_paged_attention`: one decode step of CausalAttention for
    /// `batch` rows over a paged KV cache, each row at its own cached length
    /// (`seq_lens`), reading and appending through its block table. No
    /// reference counterpart (ARCH-0008:123-124, gaps G-17 and G-18).
    pub fn paged_attention(
        &mut self,
        op: &Op,
        q: &BufferRef,
        k_new: &BufferRef,
        v_new: &BufferRef,
        out: &BufferRef,
        batch: u32,
        kv: &PagedKv,
    ) -> Result<(), DeviceError> {
        let op = to_sl_op(op)?;
        let raw_kv = ffi::sl_paged_kv {
            pool: kv.pool.0,
            block_table: kv.block_table.0,
            seq_lens: kv.seq_lens.0,
            layers: kv.layers,
            num_pages: kv.num_pages,
            page_size: kv.page_size,
            pages_per_seq: kv.pages_per_seq,
            reserved: 0,
        };
        let (q, k, v, o) = (to_sl_buffer_ref(q), to_sl_buffer_ref(k_new), to_sl_buffer_ref(v_new), to_sl_buffer_ref(out));
        let status = unsafe { ffi::sl_hip_paged_attention(self.raw, &op, &q, &k, &v, &o, batch, &raw_kv) };
        self.check(status)
    }

    /// `sl_status` plus `sl_hip_last_error` -> `DeviceError`, variant for
    /// variant (the messages are the library's static strings).
    fn check(&self, status: ffi::sl_status) -> Result<(), DeviceError> {
        if status == ffi::SL_OK {
            return Ok(());
        }
        let mut e = ffi::sl_error {
            status: 0,
            buffer: 0,
            offset: 0,
            len: 0,
            requested: 0,
            op: 0,
            reserved: 0,
            message: ptr::null(),
        };
        unsafe { ffi::sl_hip_last_error(self.raw, &mut e) };
        let message: &'static str = if e.message.is_null() {
            ""
        } else {
            // SAFETY: the library's messages are string literals of the
            // loaded library, alive until the process ends.
            unsafe { CStr::from_ptr::<'static>(e.message) }.to_str().unwrap_or("")
        };
        Err(match status {
            ffi::SL_ERR_OUT_OF_MEMORY => DeviceError::OutOfMemory { requested: e.requested as usize },
            ffi::SL_ERR_INVALID_BUFFER => DeviceError::InvalidBuffer(BufferId(e.buffer)),
            ffi::SL_ERR_INVALID_RANGE => DeviceError::InvalidRange {
                buffer: BufferId(e.buffer),
                offset: e.offset as usize,
                len: e.len as usize,
            },
            ffi::SL_ERR_UNSUPPORTED_OP => match opcode_from_u32(e.op) {
                Some(op) => DeviceError::UnsupportedOp(op),
                // a code this binding does not know: the library is newer
                // than the binding, which must not guess an op
                None => DeviceError::Execution("HIP library reported UnsupportedOp with an op code unknown to this binding"),
            },
            ffi::SL_ERR_SHAPE_OVERFLOW => DeviceError::ShapeOverflow,
            ffi::SL_ERR_EXECUTION => DeviceError::Execution(message),
            _ => DeviceError::Unimplemented(message),
        })
    }
}

impl Drop for HipDevice {
    fn drop(&mut self) {
        unsafe { ffi::sl_hip_device_destroy(self.raw) }
    }
}

impl Device for HipDevice {
    fn allocate_f32(&mut self, elements: usize, align: usize) -> Result<BufferId, DeviceError> {
        let mut id = 0u32;
        let status = unsafe { ffi::sl_hip_allocate_f32(self.raw, elements, align, &mut id) };
        self.check(status).map(|()| BufferId(id))
    }

    fn allocate_u32(&mut self, elements: usize, align: usize) -> Result<BufferId, DeviceError> {
        let mut id = 0u32;
        let status = unsafe { ffi::sl_hip_allocate_u32(self.raw, elements, align, &mut id) };
        self.check(status).map(|()| BufferId(id))
    }

    fn upload_f32(&mut self, buffer: BufferId, data: &[f32]) -> Result<(), DeviceError> {
        let status = unsafe { ffi::sl_hip_upload_f32(self.raw, buffer.0, data.as_ptr(), data.len()) };
        self.check(status)
    }

    fn upload_u32(&mut self, buffer: BufferId, data: &[u32]) -> Result<(), DeviceError> {
        let status = unsafe { ffi::sl_hip_upload_u32(self.raw, buffer.0, data.as_ptr(), data.len()) };
        self.check(status)
    }

    fn download_f32(&mut self, buffer: BufferId, out: &mut [f32]) -> Result<(), DeviceError> {
        let status = unsafe { ffi::sl_hip_download_f32(self.raw, buffer.0, out.as_mut_ptr(), out.len()) };
        self.check(status)
    }

    fn download_u32(&mut self, buffer: BufferId, out: &mut [u32]) -> Result<(), DeviceError> {
        let status = unsafe { ffi::sl_hip_download_u32(self.raw, buffer.0, out.as_mut_ptr(), out.len()) };
        self.check(status)
    }

    fn dispatch(
        &mut self,
        op: &Op,
        inputs: &[BufferRef],
        input_values: &[&Value],
        outputs: &[BufferRef],
        output_values: &[&Value],
        scalars: &[u32],
    ) -> Result<(), DeviceError> {
        let call = Call::new(op, inputs, input_values, outputs, output_values)?;
        let status = unsafe {
            ffi::sl_hip_dispatch(
                self.raw,
                &call.op,
                call.inputs.as_ptr(),
                call.input_values.as_ptr(),
                call.n_inputs,
                call.outputs.as_ptr(),
                call.output_values.as_ptr(),
                call.n_outputs,
                scalars.as_ptr(),
                scalars.len(),
            )
        };
        self.check(status)
    }

    fn synchronize(&mut self) -> Result<(), DeviceError> {
        let status = unsafe { ffi::sl_hip_synchronize(self.raw) };
        self.check(status)
    }
}

/// One dispatch's arguments in the C layout, on the stack (dispatch must not
/// allocate, ARCH-0007 §3.1). The port-count checks come first, with the
/// reference's messages and order (device.rs:224-245); the library repeats
/// them and every other check.
struct Call {
    op: ffi::sl_op,
    inputs: [ffi::sl_buffer_ref; ffi::SL_MAX_INPUTS],
    input_values: [ffi::sl_value; ffi::SL_MAX_INPUTS],
    n_inputs: usize,
    outputs: [ffi::sl_buffer_ref; ffi::SL_MAX_OUTPUTS],
    output_values: [ffi::sl_value; ffi::SL_MAX_OUTPUTS],
    n_outputs: usize,
}

impl Call {
    fn new(
        op: &Op,
        inputs: &[BufferRef],
        input_values: &[&Value],
        outputs: &[BufferRef],
        output_values: &[&Value],
    ) -> Result<Self, DeviceError> {
        if inputs.len() != input_values.len() {
            return Err(DeviceError::Execution("inputs and input_values have different lengths"));
        }
        if outputs.len() != output_values.len() {
            return Err(DeviceError::Execution("outputs and output_values have different lengths"));
        }
        if inputs.len() > ffi::SL_MAX_INPUTS || outputs.len() > ffi::SL_MAX_OUTPUTS {
            return Err(DeviceError::Execution("too many command ports"));
        }
        let mut call = Call {
            op: to_sl_op(op)?,
            inputs: [ffi::sl_buffer_ref::default(); ffi::SL_MAX_INPUTS],
            input_values: [ffi::sl_value::default(); ffi::SL_MAX_INPUTS],
            n_inputs: inputs.len(),
            outputs: [ffi::sl_buffer_ref::default(); ffi::SL_MAX_OUTPUTS],
            output_values: [ffi::sl_value::default(); ffi::SL_MAX_OUTPUTS],
            n_outputs: outputs.len(),
        };
        for (i, (r, v)) in inputs.iter().zip(input_values).enumerate() {
            call.inputs[i] = to_sl_buffer_ref(r);
            call.input_values[i] = to_sl_value(v)?;
        }
        for (i, (r, v)) in outputs.iter().zip(output_values).enumerate() {
            call.outputs[i] = to_sl_buffer_ref(r);
            call.output_values[i] = to_sl_value(v)?;
        }
        Ok(call)
    }
}

fn to_sl_buffer_ref(r: &BufferRef) -> ffi::sl_buffer_ref {
    ffi::sl_buffer_ref { buffer: r.buffer.0, reserved: 0, offset: r.offset as u64, len: r.len as u64 }
}

/// sl_ir::Value -> sl_value. A symbolic dimension is rejected as CpuDevice
/// rejects it (device.rs:723-725); ranks above 8 are ShapeOverflow.
fn to_sl_value(v: &Value) -> Result<ffi::sl_value, DeviceError> {
    let shape = v.shape.as_slice();
    if shape.len() > ffi::SL_MAX_RANK {
        return Err(DeviceError::ShapeOverflow);
    }
    let mut out = ffi::sl_value {
        dtype: match v.dtype {
            DType::F32 => ffi::SL_DTYPE_F32,
            DType::F16 => ffi::SL_DTYPE_F16,
            DType::BF16 => ffi::SL_DTYPE_BF16,
            DType::U32 => ffi::SL_DTYPE_U32,
            DType::I32 => ffi::SL_DTYPE_I32,
            DType::U8 => ffi::SL_DTYPE_U8,
            DType::I8 => ffi::SL_DTYPE_I8,
        },
        role: match v.role {
            ValueRole::Input => ffi::SL_ROLE_INPUT,
            ValueRole::Scalar => ffi::SL_ROLE_SCALAR,
            ValueRole::Output => ffi::SL_ROLE_OUTPUT,
            ValueRole::Param => ffi::SL_ROLE_PARAM,
            ValueRole::State => ffi::SL_ROLE_STATE,
            ValueRole::Temp => ffi::SL_ROLE_TEMP,
        },
        rank: shape.len() as u32,
        ..ffi::sl_value::default()
    };
    for (i, dim) in shape.iter().enumerate() {
        out.dims[i] = match dim {
            Dim::Const(n) => *n,
            Dim::Sym(_) => {
                return Err(DeviceError::Execution("value shape still contains a symbolic dimension"));
            }
        };
    }
    match &v.encoding {
        TensorEncoding::Dense => out.encoding = ffi::SL_ENCODING_DENSE,
        TensorEncoding::GroupwiseQuantized { format, group_size } => {
            out.encoding = ffi::SL_ENCODING_GROUPWISE_QUANTIZED;
            out.qformat = match format {
                QuantizationFormat::Int4 => ffi::SL_QFORMAT_INT4,
                QuantizationFormat::Int8 => ffi::SL_QFORMAT_INT8,
            };
            out.group_size = *group_size;
        }
        TensorEncoding::OpaqueQuantized { .. } => out.encoding = ffi::SL_ENCODING_OPAQUE_QUANTIZED,
    }
    Ok(out)
}

/// sl_ir::Op -> sl_op (the C opcodes follow OpCode's declaration order).
/// A variant this backend does not know is UnsupportedOp (ARCH-0004 §12.4).
#[allow(unreachable_patterns)]
fn to_sl_op(op: &Op) -> Result<ffi::sl_op, DeviceError> {
    let mut c = ffi::sl_op::default();
    c.code = match op {
        Op::MatMulNT => ffi::SL_OP_MATMUL_NT,
        Op::MatMulNN => ffi::SL_OP_MATMUL_NN,
        Op::Softmax => ffi::SL_OP_SOFTMAX,
        Op::SoftmaxCausal => ffi::SL_OP_SOFTMAX_CAUSAL,
        Op::RmsNorm { eps } => {
            c.eps = *eps;
            ffi::SL_OP_RMS_NORM
        }
        Op::Rope { variant, theta } => {
            c.rope_variant = match variant {
                RopeVariant::Neox => ffi::SL_ROPE_NEOX,
                RopeVariant::GptJ => ffi::SL_ROPE_GPTJ,
            };
            c.theta = *theta;
            ffi::SL_OP_ROPE
        }
        Op::Silu => ffi::SL_OP_SILU,
        Op::Mul => ffi::SL_OP_MUL,
        Op::Add => ffi::SL_OP_ADD,
        Op::Scale { factor } => {
            c.factor = *factor;
            ffi::SL_OP_SCALE
        }
        Op::Gather => ffi::SL_OP_GATHER,
        Op::LastToken => ffi::SL_OP_LAST_TOKEN,
        Op::KvAppend { layer } => {
            c.layer = *layer;
            ffi::SL_OP_KV_APPEND
        }
        Op::SplitHeads { heads, head_dim } => {
            c.heads = *heads;
            c.head_dim = *head_dim;
            ffi::SL_OP_SPLIT_HEADS
        }
        Op::MergeHeads { heads, head_dim } => {
            c.heads = *heads;
            c.head_dim = *head_dim;
            ffi::SL_OP_MERGE_HEADS
        }
        Op::CausalAttention { layer, heads, kv_heads, head_dim, scale } => {
            c.layer = *layer;
            c.heads = *heads;
            c.kv_heads = *kv_heads;
            c.head_dim = *head_dim;
            c.scale = *scale;
            ffi::SL_OP_CAUSAL_ATTENTION
        }
        Op::SwiGlu => ffi::SL_OP_SWIGLU,
        Op::RmsNormMatMul { eps } => {
            c.eps = *eps;
            ffi::SL_OP_RMS_NORM_MATMUL
        }
        _ => return Err(DeviceError::UnsupportedOp(op.code())),
    };
    Ok(c)
}

/// The OpCodes in `sl_opcode` order.
const OPCODES: [OpCode; 18] = [
    OpCode::MatMulNT,
    OpCode::MatMulNN,
    OpCode::Softmax,
    OpCode::SoftmaxCausal,
    OpCode::RmsNorm,
    OpCode::Rope,
    OpCode::Silu,
    OpCode::Mul,
    OpCode::Add,
    OpCode::Scale,
    OpCode::Gather,
    OpCode::LastToken,
    OpCode::KvAppend,
    OpCode::SplitHeads,
    OpCode::MergeHeads,
    OpCode::CausalAttention,
    OpCode::SwiGlu,
    OpCode::RmsNormMatMul,
];

/// The OpCode of a C `sl_opcode` value (declaration order), or None for a
/// value past the known ops.
fn opcode_from_u32(code: u32) -> Option<OpCode> {
    OPCODES.get(code as usize).copied()
}

/// The backend's DeviceCapabilities (ARCH-0004 §8), from
/// `sl_hip_capabilities`: every core op, the three composites, F32/U32 data,
/// its alignment, scratchpad and shape limits.
pub fn hip_capabilities() -> DeviceCapabilities {
    let mut c = ffi::sl_capabilities {
        backend: ptr::null(),
        ir_version: 0,
        core_ops: 0,
        composite_ops: 0,
        dtypes: 0,
        min_buffer_align: 0,
        max_scratchpad_bytes: 0,
        max_value_bytes: 0,
        head_dim_multiple_of: 0,
        matmul_k_multiple_of: 0,
        max_heads: 0,
    };
    unsafe { ffi::sl_hip_capabilities(&mut c) };
    let ops = |mask: u32| {
        OPCODES.iter().enumerate().filter(|(i, _)| mask >> i & 1 == 1).map(|(_, op)| *op).collect::<Vec<_>>()
    };
    let mut dtypes = DTypeSet::ONLY_F32;
    if c.dtypes >> ffi::SL_DTYPE_U32 & 1 == 1 {
        dtypes = dtypes.union(DTypeSet::ONLY_U32);
    }
    debug_assert_eq!(c.ir_version, IR_VERSION);
    DeviceCapabilities {
        backend: BackendTag("hip-gfx950"),
        ir_version: c.ir_version,
        core_ops: OpSet::new(ops(c.core_ops)),
        composite_ops: OpSet::new(ops(c.composite_ops)),
        dtypes,
        min_buffer_align: c.min_buffer_align,
        max_scratchpad_bytes: c.max_scratchpad_bytes,
        max_value_bytes: c.max_value_bytes,
        constraints: ShapeConstraints {
            head_dim_multiple_of: c.head_dim_multiple_of,
            matmul_k_multiple_of: c.matmul_k_multiple_of,
            max_heads: c.max_heads,
        },
    }
}
