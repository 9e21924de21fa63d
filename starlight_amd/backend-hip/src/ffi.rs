//! The C ABI of `include/starlight_hip.h`, one to one: every struct is
//! `#[repr(C)]` with the header's field order and types, every enum a set of
//! `u32` constants with the header's values, every function an `extern "C"`
//! declaration with the header's parameters. (`tests/test_rust_binding.py`
//! checks the struct layouts against the header compiled by a C compiler, and
//! that each header function is declared here with the same parameter count.)
#![allow(non_camel_case_types, dead_code)]

use std::os::raw::{c_char, c_int, c_void};

pub const SL_HIP_ABI_VERSION: u32 = 2;
pub const SL_IR_VERSION: u32 = 2;
pub const SL_MAX_RANK: usize = 8;
pub const SL_MAX_INPUTS: usize = 4;
pub const SL_MAX_OUTPUTS: usize = 1;
pub const SL_HIP_STATIC_SCRATCH_BYTES: usize = 16 << 20;

/// `sl_status`: the `DeviceError` variants (ARCH-0007 §3.1), 1:1.
pub type sl_status = c_int;
pub const SL_OK: sl_status = 0;
pub const SL_ERR_OUT_OF_MEMORY: sl_status = 1;
pub const SL_ERR_INVALID_BUFFER: sl_status = 2;
pub const SL_ERR_INVALID_RANGE: sl_status = 3;
pub const SL_ERR_UNSUPPORTED_OP: sl_status = 4;
pub const SL_ERR_SHAPE_OVERFLOW: sl_status = 5;
pub const SL_ERR_EXECUTION: sl_status = 6;
pub const SL_ERR_UNIMPLEMENTED: sl_status = 7;

/// `sl_dtype` (sl_ir::DType declaration order).
pub const SL_DTYPE_F32: u32 = 0;
pub const SL_DTYPE_F16: u32 = 1;
pub const SL_DTYPE_BF16: u32 = 2;
pub const SL_DTYPE_U32: u32 = 3;
pub const SL_DTYPE_I32: u32 = 4;
pub const SL_DTYPE_U8: u32 = 5;
pub const SL_DTYPE_I8: u32 = 6;

/// `sl_value_role` (sl_ir::ValueRole declaration order).
pub const SL_ROLE_INPUT: u32 = 0;
pub const SL_ROLE_SCALAR: u32 = 1;
pub const SL_ROLE_OUTPUT: u32 = 2;
pub const SL_ROLE_PARAM: u32 = 3;
pub const SL_ROLE_STATE: u32 = 4;
pub const SL_ROLE_TEMP: u32 = 5;

/// `sl_encoding` (sl_ir::TensorEncoding).
pub const SL_ENCODING_DENSE: u32 = 0;
pub const SL_ENCODING_GROUPWISE_QUANTIZED: u32 = 1;
pub const SL_ENCODING_OPAQUE_QUANTIZED: u32 = 2;

/// `sl_qformat` (sl_ir::QuantizationFormat).
pub const SL_QFORMAT_INT4: u32 = 0;
pub const SL_QFORMAT_INT8: u32 = 1;

/// `sl_opcode` (sl_ir::OpCode declaration order, ARCH-0004 §5.1).
pub const SL_OP_MATMUL_NT: u32 = 0;
pub const SL_OP_MATMUL_NN: u32 = 1;
pub const SL_OP_SOFTMAX: u32 = 2;
pub const SL_OP_SOFTMAX_CAUSAL: u32 = 3;
pub const SL_OP_RMS_NORM: u32 = 4;
pub const SL_OP_ROPE: u32 = 5;
pub const SL_OP_SILU: u32 = 6;
pub const SL_OP_MUL: u32 = 7;
pub const SL_OP_ADD: u32 = 8;
pub const SL_OP_SCALE: u32 = 9;
pub const SL_OP_GATHER: u32 = 10;
pub const SL_OP_LAST_TOKEN: u32 = 11;
pub const SL_OP_KV_APPEND: u32 = 12;
pub const SL_OP_SPLIT_HEADS: u32 = 13;
pub const SL_OP_MERGE_HEADS: u32 = 14;
pub const SL_OP_CAUSAL_ATTENTION: u32 = 15;
pub const SL_OP_SWIGLU: u32 = 16;
pub const SL_OP_RMS_NORM_MATMUL: u32 = 17;

/// `sl_rope_variant`.
pub const SL_ROPE_NEOX: u32 = 0;
pub const SL_ROPE_GPTJ: u32 = 1;

/// `sl_buffer_kind`.
pub const SL_BUFFER_NONE: u32 = 0;
pub const SL_BUFFER_F32: u32 = 1;
pub const SL_BUFFER_U32: u32 = 2;

/// Submission options of `sl_hip_set_options`.
pub const SL_HIP_OPT_FUSION: u32 = 1;
pub const SL_HIP_OPT_GRAPHS: u32 = 2;

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct sl_error {
    pub status: i32,
    pub buffer: u32,
    pub offset: u64,
    pub len: u64,
    pub requested: u64,
    pub op: u32,
    pub reserved: u32,
    pub message: *const c_char,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct sl_value {
    pub dtype: u32,
    pub role: u32,
    pub rank: u32,
    pub dims: [u32; SL_MAX_RANK],
    pub encoding: u32,
    pub qformat: u32,
    pub group_size: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct sl_op {
    pub code: u32,
    pub rope_variant: u32,
    pub eps: f32,
    pub theta: f32,
    pub factor: f32,
    pub scale: f32,
    pub layer: u32,
    pub heads: u32,
    pub kv_heads: u32,
    pub head_dim: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct sl_buffer_ref {
    pub buffer: u32,
    pub reserved: u32,
    pub offset: u64,
    pub len: u64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct sl_buffer_desc {
    pub kind: u32,
    pub quantized: u32,
    pub qformat: u32,
    pub group_size: u32,
    pub qn: u32,
    pub qk: u32,
    pub elements: u64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct sl_capabilities {
    pub backend: *const c_char,
    pub ir_version: u32,
    pub core_ops: u32,
    pub composite_ops: u32,
    pub dtypes: u32,
    pub min_buffer_align: u32,
    pub max_scratchpad_bytes: u64,
    pub max_value_bytes: u64,
    pub head_dim_multiple_of: u32,
    pub matmul_k_multiple_of: u32,
    pub max_heads: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct sl_hip_stats {
    pub submissions: u64,
    pub commands: u64,
    pub fused_commands: u64,
    pub graph_captures: u64,
    pub graph_replays: u64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct sl_paged_kv {
    pub pool: u32,
    pub block_table: u32,
    pub seq_lens: u32,
    pub layers: u32,
    pub num_pages: u32,
    pub page_size: u32,
    pub pages_per_seq: u32,
    pub reserved: u32,
}

/// Opaque device handle.
#[repr(C)]
pub struct sl_hip_device {
    _private: [u8; 0],
}

extern "C" {
    pub fn sl_hip_abi_version() -> u32;
    pub fn sl_hip_device_create(ordinal: c_int, out: *mut *mut sl_hip_device) -> sl_status;
    pub fn sl_hip_device_destroy(device: *mut sl_hip_device);
    pub fn sl_hip_allocate_f32(device: *mut sl_hip_device, elements: usize, align: usize, out_id: *mut u32)
        -> sl_status;
    pub fn sl_hip_allocate_u32(device: *mut sl_hip_device, elements: usize, align: usize, out_id: *mut u32)
        -> sl_status;
    pub fn sl_hip_upload_f32(device: *mut sl_hip_device, buffer: u32, data: *const f32, len: usize) -> sl_status;
    pub fn sl_hip_upload_u32(device: *mut sl_hip_device, buffer: u32, data: *const u32, len: usize) -> sl_status;
    pub fn sl_hip_download_f32(device: *mut sl_hip_device, buffer: u32, out: *mut f32, len: usize) -> sl_status;
    pub fn sl_hip_download_u32(device: *mut sl_hip_device, buffer: u32, out: *mut u32, len: usize) -> sl_status;
    pub fn sl_hip_dispatch(
        device: *mut sl_hip_device,
        op: *const sl_op,
        inputs: *const sl_buffer_ref,
        input_values: *const sl_value,
        n_inputs: usize,
        outputs: *const sl_buffer_ref,
        output_values: *const sl_value,
        n_outputs: usize,
        scalars: *const u32,
        n_scalars: usize,
    ) -> sl_status;
    pub fn sl_hip_dispatch_noalloc(
        device: *mut sl_hip_device,
        op: *const sl_op,
        inputs: *const sl_buffer_ref,
        input_values: *const sl_value,
        n_inputs: usize,
        outputs: *const sl_buffer_ref,
        output_values: *const sl_value,
        n_outputs: usize,
        scalars: *const u32,
        n_scalars: usize,
    ) -> sl_status;
    pub fn sl_hip_synchronize(device: *mut sl_hip_device) -> sl_status;
    pub fn sl_hip_last_error(device: *const sl_hip_device, out: *mut sl_error);
    pub fn sl_hip_bind_quantized(
        device: *mut sl_hip_device,
        payload: u32,
        scales: u32,
        qformat: u32,
        group_size: u32,
        n: u32,
        k: u32,
    ) -> sl_status;
    pub fn sl_hip_paged_attention(
        device: *mut sl_hip_device,
        op: *const sl_op,
        q: *const sl_buffer_ref,
        k_new: *const sl_buffer_ref,
        v_new: *const sl_buffer_ref,
        out: *const sl_buffer_ref,
        batch: u32,
        kv: *const sl_paged_kv,
    ) -> sl_status;
    pub fn sl_hip_bind_paged_state(device: *mut sl_hip_device, state: u32, kv: *const sl_paged_kv) -> sl_status;
    pub fn sl_hip_paged_store(
        device: *mut sl_hip_device,
        kv: *const sl_paged_kv,
        row: u32,
        state: u32,
        index: u32,
        max_seq: u32,
        kv_heads: u32,
        head_dim: u32,
        length: u32,
    ) -> sl_status;
    pub fn sl_hip_validate_dispatch(
        buffers: *const sl_buffer_desc,
        n_buffers: usize,
        op: *const sl_op,
        inputs: *const sl_buffer_ref,
        input_values: *const sl_value,
        n_inputs: usize,
        outputs: *const sl_buffer_ref,
        output_values: *const sl_value,
        n_outputs: usize,
        scalars: *const u32,
        n_scalars: usize,
        err: *mut sl_error,
    ) -> sl_status;
    pub fn sl_hip_capabilities(out: *mut sl_capabilities);
    pub fn sl_hip_stream(device: *const sl_hip_device) -> *mut c_void;
    pub fn sl_hip_submit(device: *mut sl_hip_device) -> sl_status;
    pub fn sl_hip_set_options(device: *mut sl_hip_device, options: u32) -> sl_status;
    pub fn sl_hip_get_stats(device: *const sl_hip_device, out: *mut sl_hip_stats);
}
