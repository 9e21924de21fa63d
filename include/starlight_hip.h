/*
 * starlight_hip.h — C ABI of the MI355X (gfx950) StarLight compute backend.
 *
 * This is the drop-in boundary for StarLight's `sl_device::Device` contract
 * (docs ARCH-0007 §3.1, "sl-device"): buffer allocation, whole-buffer
 * upload/download, single-operator dispatch and synchronize. The reference
 * implementation of that trait is `CpuDevice`
 * (crates/backends/backend-cpu/src/device.rs:114-213); every entry point below
 * names the method it replaces. A Rust `backend-hip` crate binds these
 * symbols one-to-one through an `extern "C"` block.
 *
 * Conventions
 *  - All entry points return `sl_status`; SL_OK is 0. On failure the device
 *    keeps the full `DeviceError` payload, readable with sl_hip_last_error().
 *  - BufferRef offsets and lengths are ELEMENTS of the value's dtype, as in
 *    `sl_device::BufferRef` (ARCH-0007 §3.1).
 *  - A device is single-owner and not thread-safe, like `&mut self` methods of
 *    `trait Device: Send`.
 *  - dispatch() validates (every error a reference dispatch reports is
 *    reported by the same call) and logs the command; logged commands are
 *    enqueued on the device's stream, in order, before anything can observe
 *    them: synchronize(), upload_*(), download_*(), bind_quantized(),
 *    sl_hip_submit(). Results are visible to download_*() and after
 *    synchronize(); a kernel failure surfaces there as Execution. dispatch()
 *    performs no device allocation.
 */
#ifndef STARLIGHT_HIP_H
#define STARLIGHT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SL_HIP_ABI_VERSION 2u
/* sl-ir IR_VERSION this backend implements (ARCH-0004 §12). */
#define SL_IR_VERSION 2u
#define SL_MAX_RANK 8u
#define SL_MAX_INPUTS 4u
#define SL_MAX_OUTPUTS 1u

/* DeviceError variants (ARCH-0007 §3.1 `enum DeviceError`), 1:1. */
typedef enum sl_status {
    SL_OK = 0,
    SL_ERR_OUT_OF_MEMORY = 1,  /* OutOfMemory { requested }            */
    SL_ERR_INVALID_BUFFER = 2, /* InvalidBuffer(BufferId)              */
    SL_ERR_INVALID_RANGE = 3,  /* InvalidRange { buffer, offset, len } */
    SL_ERR_UNSUPPORTED_OP = 4, /* UnsupportedOp(OpCode)                */
    SL_ERR_SHAPE_OVERFLOW = 5, /* ShapeOverflow                        */
    SL_ERR_EXECUTION = 6,      /* Execution(&'static str)              */
    SL_ERR_UNIMPLEMENTED = 7   /* Unimplemented(&'static str)          */
} sl_status;

/* Full DeviceError payload. `message` is a static string (never freed). */
typedef struct sl_error {
    int32_t status;
    uint32_t buffer;    /* InvalidBuffer / InvalidRange */
    uint64_t offset;    /* InvalidRange */
    uint64_t len;       /* InvalidRange */
    uint64_t requested; /* OutOfMemory */
    uint32_t op;        /* UnsupportedOp: sl_opcode */
    uint32_t reserved;
    const char *message; /* Execution / Unimplemented reason; NULL otherwise */
} sl_error;

/* sl_ir::DType (ARCH-0004 §3.1), declaration order. */
typedef enum sl_dtype {
    SL_DTYPE_F32 = 0,
    SL_DTYPE_F16 = 1,
    SL_DTYPE_BF16 = 2,
    SL_DTYPE_U32 = 3,
    SL_DTYPE_I32 = 4,
    SL_DTYPE_U8 = 5,
    SL_DTYPE_I8 = 6
} sl_dtype;

/* sl_ir::ValueRole (ARCH-0004 §3.3), declaration order. */
typedef enum sl_value_role {
    SL_ROLE_INPUT = 0,
    SL_ROLE_SCALAR = 1,
    SL_ROLE_OUTPUT = 2,
    SL_ROLE_PARAM = 3,
    SL_ROLE_STATE = 4,
    SL_ROLE_TEMP = 5
} sl_value_role;

/* sl_ir::TensorEncoding (ARCH-0004 §3.3). */
typedef enum sl_encoding {
    SL_ENCODING_DENSE = 0,
    SL_ENCODING_GROUPWISE_QUANTIZED = 1,
    SL_ENCODING_OPAQUE_QUANTIZED = 2
} sl_encoding;

/* sl_ir::QuantizationFormat (ARCH-0004 §3.3). */
typedef enum sl_qformat { SL_QFORMAT_INT4 = 0, SL_QFORMAT_INT8 = 1 } sl_qformat;

/* sl_ir::Value with every Dim already concrete (a CommandBuffer holds no
 * Dim::Sym, ARCH-0004 §3.2; the binding layer rejects symbolic dims with
 * Execution("value shape still contains a symbolic dimension") before the
 * call, as device.rs:723-725 does). */
typedef struct sl_value {
    uint32_t dtype; /* sl_dtype */
    uint32_t role;  /* sl_value_role */
    uint32_t rank;  /* <= SL_MAX_RANK; larger ranks are ShapeOverflow */
    uint32_t dims[SL_MAX_RANK];
    uint32_t encoding;   /* sl_encoding */
    uint32_t qformat;    /* sl_qformat, when encoding is groupwise */
    uint32_t group_size; /* when encoding is groupwise */
} sl_value;

/* sl_ir::OpCode (ARCH-0004 §5.1), declaration order. */
typedef enum sl_opcode {
    SL_OP_MATMUL_NT = 0,
    SL_OP_MATMUL_NN = 1,
    SL_OP_SOFTMAX = 2,
    SL_OP_SOFTMAX_CAUSAL = 3,
    SL_OP_RMS_NORM = 4,
    SL_OP_ROPE = 5,
    SL_OP_SILU = 6,
    SL_OP_MUL = 7,
    SL_OP_ADD = 8,
    SL_OP_SCALE = 9,
    SL_OP_GATHER = 10,
    SL_OP_LAST_TOKEN = 11,
    SL_OP_KV_APPEND = 12,
    SL_OP_SPLIT_HEADS = 13,
    SL_OP_MERGE_HEADS = 14,
    SL_OP_CAUSAL_ATTENTION = 15,
    SL_OP_SWIGLU = 16,
    SL_OP_RMS_NORM_MATMUL = 17
} sl_opcode;

typedef enum sl_rope_variant { SL_ROPE_NEOX = 0, SL_ROPE_GPTJ = 1 } sl_rope_variant;

/* sl_ir::Op: the opcode plus the attributes its variant carries
 * (ARCH-0004 §5.1). Fields an op does not use are ignored. */
typedef struct sl_op {
    uint32_t code;         /* sl_opcode */
    uint32_t rope_variant; /* Rope */
    float eps;             /* RmsNorm, RmsNormMatMul */
    float theta;           /* Rope */
    float factor;          /* Scale */
    float scale;           /* CausalAttention */
    uint32_t layer;        /* KvAppend, CausalAttention */
    uint32_t heads;        /* SplitHeads, MergeHeads, CausalAttention */
    uint32_t kv_heads;     /* CausalAttention */
    uint32_t head_dim;     /* SplitHeads, MergeHeads, CausalAttention */
} sl_op;

/* sl_device::BufferRef (ARCH-0007 §3.1). */
typedef struct sl_buffer_ref {
    uint32_t buffer;
    uint32_t reserved;
    uint64_t offset; /* elements */
    uint64_t len;    /* elements (storage words for a quantized payload) */
} sl_buffer_ref;

typedef struct sl_hip_device sl_hip_device;

/* CpuDevice::new() (device.rs:41-45). Opens HIP device `ordinal`, creates the
 * device's stream and its fixed workspace (512 MiB, or the byte count in the
 * environment variable SL_HIP_WORKSPACE_BYTES, at least 64 KiB; fused
 * launches that do not fit a smaller workspace run unfused). */
sl_status sl_hip_device_create(int ordinal, sl_hip_device **out);
void sl_hip_device_destroy(sl_hip_device *device);

/* Device::allocate_f32 / allocate_u32 (device.rs:115-121, 55-83): a
 * zero-filled buffer of `elements`; `align` must be a nonzero power of two
 * (device.rs:215-222). Buffer ids are dense indices starting at 0. */
sl_status sl_hip_allocate_f32(sl_hip_device *device, size_t elements, size_t align, uint32_t *out_id);
sl_status sl_hip_allocate_u32(sl_hip_device *device, size_t elements, size_t align, uint32_t *out_id);

/* Device::upload_f32 / upload_u32 (device.rs:123-147): `len` must equal the
 * buffer's capacity, else InvalidRange { buffer, 0, len }. */
sl_status sl_hip_upload_f32(sl_hip_device *device, uint32_t buffer, const float *data, size_t len);
sl_status sl_hip_upload_u32(sl_hip_device *device, uint32_t buffer, const uint32_t *data, size_t len);

/* Device::download_f32 / download_u32 (device.rs:149-173). Orders after all
 * previously dispatched work and blocks until the copy is complete. */
sl_status sl_hip_download_f32(sl_hip_device *device, uint32_t buffer, float *out, size_t len);
sl_status sl_hip_download_u32(sl_hip_device *device, uint32_t buffer, uint32_t *out, size_t len);

/* Device::dispatch (device.rs:176-208; run_op device.rs:773-1227).
 * `input_values[i]` / `output_values[i]` describe port i. Validation and its
 * error precedence follow device.rs:224-377 and the per-op geometry checks;
 * a rejected call changes no buffer. */
sl_status sl_hip_dispatch(sl_hip_device *device, const sl_op *op, const sl_buffer_ref *inputs,
                          const sl_value *input_values, size_t n_inputs, const sl_buffer_ref *outputs,
                          const sl_value *output_values, size_t n_outputs, const uint32_t *scalars,
                          size_t n_scalars);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): sl_hip_dispatch without the log. It validates exactly
 * as sl_hip_dispatch does, then enqueues this one command's kernels on the
 * device's stream at once (no fusion, no graph, past_len taken from the
 * scalar), and calls no hipMalloc, hipFree or allocating routine. Its
 * scratch memory (attention partials, SwiGlu intermediates, split-K
 * partials) is a static array of SL_HIP_STATIC_SCRATCH_BYTES held by each
 * GPU the library runs on until the process ends, not the device workspace.
 * Errors: Execution when commands are still logged (call sl_hip_submit
 * first) or the array's address could not be found at device creation;
 * Unimplemented when the command needs more scratch than the array holds.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (several devices or streams on it) race. A Gather whose id buffer is
 * larger than 16 MiB checks its ids with a device-to-host copy and a stream
 * synchronize, which graph capture does not allow. */
#define SL_HIP_STATIC_SCRATCH_BYTES (16u << 20)
sl_status sl_hip_dispatch_noalloc(sl_hip_device *device, const sl_op *op, const sl_buffer_ref *inputs,
                                  const sl_value *input_values, size_t n_inputs, const sl_buffer_ref *outputs,
                                  const sl_value *output_values, size_t n_outputs, const uint32_t *scalars,
                                  size_t n_scalars);

/* Device::synchronize (device.rs:210-212): submits the logged commands,
 * blocks until all of them have finished and reports any execution failure. */
sl_status sl_hip_synchronize(sl_hip_device *device);

/* The DeviceError of the most recent failing call on `device`. */
void sl_hip_last_error(const sl_hip_device *device, sl_error *out);

/* Group-wise quantized weights (no reference counterpart: sl-ir v2 defines
 * TensorEncoding::GroupwiseQuantized, ARCH-0004 §3.3, but the 18 operator
 * signatures carry no scale port and sl-core rejects non-dense Params,
 * ARCH-0006:147). Associates an uploaded u32 payload buffer with its f32
 * scale buffer for a logical [n, k] weight:
 *   INT8: int8 codes, row-major, n*k bytes;
 *   INT4: two's-complement nibbles, element k of a row in byte k/2 with even
 *         k in the low nibble, n*ceil(k/2) bytes;
 *   payload words = ceil(bytes / 4), little-endian;
 *   scales: f32 [n, k / group_size], weight = code * scale.
 * After binding, a dispatch port whose value has encoding
 * SL_ENCODING_GROUPWISE_QUANTIZED (role Param, dtype F32, logical shape
 * [n, k]) reads the payload through a BufferRef { payload, 0, words }.
 * Ports that accept it: MatMulNT B, SwiGlu gate/up/down, RmsNormMatMul matrix.
 * The device repacks the codes into a private tile layout here; a later
 * upload_u32 to the payload buffer refreshes that copy. */
sl_status sl_hip_bind_quantized(sl_hip_device *device, uint32_t payload, uint32_t scales,
                                uint32_t qformat, uint32_t group_size, uint32_t n, uint32_t k);

/* Paged KV cache (no reference counterpart: gaps G-17 paged KV and G-18
 * per-request lengths, ARCH-0008:123-124). `pool` is an f32 buffer of
 * layers * num_pages * 2 * page_size * kv_heads * head_dim elements laid out
 * [layer][page][K, V][slot][kv_head][head_dim]; position j of batch row b is
 * slot j % page_size of page block_table[b * pages_per_seq + j / page_size];
 * `block_table` (u32, batch * pages_per_seq ids) and `seq_lens` (u32, batch
 * cached lengths) are u32 buffers of at most 16 MiB (the device checks their
 * contents on the host before launching). page_size is a multiple of 16. */
typedef struct sl_paged_kv {
    uint32_t pool;
    uint32_t block_table;
    uint32_t seq_lens;
    uint32_t layers;
    uint32_t num_pages;
    uint32_t page_size;
    uint32_t pages_per_seq;
    uint32_t reserved;
} sl_paged_kv;

/* Decode attention over a paged KV cache, one new token per batch row, each
 * row at its own length (continuous batching): for row b with
 * L = seq_lens[b], appends k_new / v_new [batch, kv_heads, 1, head_dim] at
 * position L of layer op->layer, then writes to `out` [batch, heads, 1,
 * head_dim] the CausalAttention of q [batch, heads, 1, head_dim] over
 * positions 0..L (reference/attention.rs:129-219 with the cache read
 * through the block table). `op` is a CausalAttention op (layer, heads,
 * kv_heads, head_dim, scale). Logged commands are submitted first; the
 * attention is enqueued at once (no fusion, no graph). Errors: Execution for
 * a length whose position L falls outside the row's table, a page id not
 * below num_pages, a row appending into a page another row reads (pages
 * only read may be shared, e.g. a common prefix), or shapes and buffers
 * that do not match; Unimplemented for head_dim not a multiple of 64 up to
 * 256, more than 16 query heads per KV head, or page_size not a multiple of
 * 16. seq_lens is not advanced: the caller adds 1 per row after the step. */
sl_status sl_hip_paged_attention(sl_hip_device *device, const sl_op *op, const sl_buffer_ref *q,
                                 const sl_buffer_ref *k_new, const sl_buffer_ref *v_new, const sl_buffer_ref *out,
                                 uint32_t batch, const sl_paged_kv *kv);

/* Continuous batching through a compiled decode program (no reference
 * counterpart: gaps G-17 / G-18, ARCH-0008:123-124). Binds the State buffer
 * `state` (the KV cache value [batch, layers, 2, max_seq, kv_heads,
 * head_dim] of a program) to the paged cache `kv`; kv == NULL removes the
 * binding. While bound, every CausalAttention command whose State port is
 * `state` reads and appends K/V through the block tables instead: row b
 * attends over its own seq_lens[b] cached positions plus its new token and
 * appends at position seq_lens[b]; the command's past_len scalar is not
 * read (pass 0). The lengths and tables are read when the work runs, so a
 * replayed submission serves every step; upload them before the step, and
 * advance seq_lens after it. dispatch() then fails with Unimplemented for a
 * CausalAttention on `state` with more than one token per row or a KvAppend
 * on it, and with Execution for the table checks of sl_hip_paged_attention
 * or a pool whose size does not match the command's layers, kv_heads and
 * head_dim. Logged commands are submitted first; cached graphs are dropped.
 * Errors: InvalidBuffer for a state that is not an f32 buffer or pool /
 * table / lengths buffers of the wrong kind; Unimplemented for tables or
 * lengths above 16 MiB or page_size not a multiple of 16. */
sl_status sl_hip_bind_paged_state(sl_hip_device *device, uint32_t state, const sl_paged_kv *kv);

/* Copies positions [0, length) of batch index `index` of a contiguous KV
 * State buffer `state` ([batch, layers, 2, max_seq, kv_heads, head_dim], as
 * a prefill program wrote it) into row `row` of the paged cache `kv`, every
 * layer's K and V, through the row's block table: how a sequence prefilled
 * on its own joins a paged decode batch. Logged commands are submitted
 * first; the copy is enqueued at once. Errors: Execution when a position
 * below `length` falls outside the row's table, a page id is not below
 * num_pages, length exceeds max_seq, or the buffer sizes do not match;
 * InvalidBuffer for buffers of the wrong kind. No reference counterpart. */
sl_status sl_hip_paged_store(sl_hip_device *device, const sl_paged_kv *kv, uint32_t row, uint32_t state,
                             uint32_t index, uint32_t max_seq, uint32_t kv_heads, uint32_t head_dim,
                             uint32_t length);

/* One entry of the buffer table sl_hip_validate_dispatch checks against. */
typedef enum sl_buffer_kind {
    SL_BUFFER_NONE = 0,
    SL_BUFFER_F32 = 1,
    SL_BUFFER_U32 = 2
} sl_buffer_kind;

typedef struct sl_buffer_desc {
    uint32_t kind;      /* sl_buffer_kind */
    uint32_t quantized; /* 1: a u32 payload bound by sl_hip_bind_quantized */
    uint32_t qformat;   /* binding: sl_qformat */
    uint32_t group_size;
    uint32_t qn, qk;   /* binding: logical [n, k] */
    uint64_t elements; /* capacity in elements */
} sl_buffer_desc;

/* Validation only, no GPU needed: runs exactly the checks sl_hip_dispatch
 * performs before it enqueues anything (port counts, value/BufferRef
 * agreement, dtypes, ranges, aliasing, per-op geometry and the kernels' own
 * shape checks) against a caller-described buffer table indexed by buffer
 * id, and reports the first failure into *err (status SL_OK when the call
 * would be accepted). U32 buffer contents are not part of the table, so the
 * data-dependent Gather id check is not made here. */
sl_status sl_hip_validate_dispatch(const sl_buffer_desc *buffers, size_t n_buffers, const sl_op *op,
                                   const sl_buffer_ref *inputs, const sl_value *input_values,
                                   size_t n_inputs, const sl_buffer_ref *outputs,
                                   const sl_value *output_values, size_t n_outputs,
                                   const uint32_t *scalars, size_t n_scalars, sl_error *err);

/* sl_ir::DeviceCapabilities (ARCH-0004 §8) for this backend; op masks are
 * bitsets over sl_opcode. Consumed by the graph compiler, not by dispatch. */
typedef struct sl_capabilities {
    const char *backend; /* "hip-gfx950" */
    uint32_t ir_version;
    uint32_t core_ops;      /* bit i set: sl_opcode i supported as a core op */
    uint32_t composite_ops; /* CausalAttention, SwiGlu, RmsNormMatMul */
    uint32_t dtypes;        /* bit i set: sl_dtype i */
    uint32_t min_buffer_align;
    uint64_t max_scratchpad_bytes;
    uint64_t max_value_bytes;
    uint32_t head_dim_multiple_of;
    uint32_t matmul_k_multiple_of;
    uint32_t max_heads;
} sl_capabilities;

void sl_hip_capabilities(sl_capabilities *out);

/* The hipStream_t the device enqueues all work on (as void*), so a caller
 * can record HIP events around its submissions for timing. No reference
 * counterpart (CpuDevice has no stream). */
void *sl_hip_stream(const sl_hip_device *device);

/* Submission of logged dispatches (no reference counterpart: CpuDevice
 * executes each dispatch at once). sl_hip_dispatch validates and logs;
 * logged commands are enqueued on the stream, in order, by sl_hip_submit and
 * before any call that can observe their effects (synchronize, upload,
 * download, bind_quantized, destroy). sl_hip_submit returns without waiting;
 * a kernel launch failure is reported by it or by the next synchronize. */
sl_status sl_hip_submit(sl_hip_device *device);

/* Submission options, all on by default:
 *   SL_HIP_OPT_FUSION: adjacent commands may run as one kernel (every
 *     command's outputs are still written);
 *   SL_HIP_OPT_GRAPHS: a submission identical to the previous one except for
 *     past_len values is captured as a HIP graph and later ones replay it. */
#define SL_HIP_OPT_FUSION 1u
#define SL_HIP_OPT_GRAPHS 2u
sl_status sl_hip_set_options(sl_hip_device *device, uint32_t options);

/* Counters of the submission machinery since the device was created. */
typedef struct sl_hip_stats {
    uint64_t submissions;    /* non-empty submissions */
    uint64_t commands;       /* commands submitted */
    uint64_t fused_commands; /* commands that ran inside a fused launch */
    uint64_t graph_captures; /* submissions captured as a graph */
    uint64_t graph_replays;  /* submissions run by replaying a graph */
} sl_hip_stats;
void sl_hip_get_stats(const sl_hip_device *device, sl_hip_stats *out);

/* ABI version of the loaded library (SL_HIP_ABI_VERSION). */
uint32_t sl_hip_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* STARLIGHT_HIP_H */
