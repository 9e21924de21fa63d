// Host-side validation and launch geometry shared by the HIP device and the
// GPU-free validation entry point. Nothing here touches the GPU.
#pragma once

#include <cstddef>
#include <cstdint>

#include "starlight_hip.h"

namespace slhip {

constexpr size_t kMaxInputs = 4;   // device.rs:26
constexpr size_t kMaxOutputs = 1;  // device.rs:27
constexpr size_t kMaxRank = 8;     // device.rs:29
constexpr uint32_t kOpCount = 18;  // sl_opcode values 0..17

// A DeviceError (ARCH-0007 §3.1) with its payload; `message` is static.
struct Error {
    sl_status status = SL_OK;
    uint32_t buffer = 0;
    uint64_t offset = 0;
    uint64_t len = 0;
    uint64_t requested = 0;
    uint32_t op = 0;
    const char* message = nullptr;

    bool ok() const { return status == SL_OK; }
    static Error execution(const char* why) { Error e; e.status = SL_ERR_EXECUTION; e.message = why; return e; }
    static Error unimplemented(const char* why) { Error e; e.status = SL_ERR_UNIMPLEMENTED; e.message = why; return e; }
    static Error overflow() { Error e; e.status = SL_ERR_SHAPE_OVERFLOW; return e; }
    static Error invalid_buffer(uint32_t b) { Error e; e.status = SL_ERR_INVALID_BUFFER; e.buffer = b; return e; }
    static Error invalid_range(uint32_t b, uint64_t off, uint64_t len) {
        Error e; e.status = SL_ERR_INVALID_RANGE; e.buffer = b; e.offset = off; e.len = len; return e;
    }
    static Error out_of_memory(uint64_t requested) {
        Error e; e.status = SL_ERR_OUT_OF_MEMORY; e.requested = requested; return e;
    }
    static Error unsupported_op(uint32_t op) { Error e; e.status = SL_ERR_UNSUPPORTED_OP; e.op = op; return e; }
};

// What validation needs to know about a buffer (the device's table, or the
// caller-described one of sl_hip_validate_dispatch).
struct BufferView {
    virtual ~BufferView() = default;
    virtual size_t count() const = 0;
    virtual const sl_buffer_desc* get(uint32_t id) const = 0;  // nullptr when unknown
};

// Logical description of a group-quantized weight operand.
struct QuantOperand {
    bool present = false;
    uint32_t format = 0;  // sl_qformat
    uint32_t group = 0;
    uint64_t n = 0, k = 0;
};

// Launch geometry decoded from the op and the port values; field meaning
// depends on `code`.
struct Plan {
    uint32_t code = 0;
    // generic row geometry (softmax, norm, swiglu, rms_norm_matmul)
    uint64_t rows = 0, cols = 0, hidden = 0;
    // matmul
    uint64_t batch = 0, batch_a = 0, batch_b = 0, m = 0, k = 0, n = 0;
    // attention / layout
    uint64_t heads = 0, kv_heads = 0, seq = 0, head_dim = 0, layers = 0, layer = 0, max_seq = 0;
    uint64_t past_len = 0, seq_len = 0, vocab = 0, inter = 0, out_features = 0, len = 0;
    float eps = 0.f, theta = 0.f, factor = 0.f, scale = 0.f;
    uint32_t rope_variant = 0;
    // quantized weight ports (MatMulNT B; SwiGlu gate/up/down; RmsNormMatMul matrix)
    QuantOperand quant[kMaxInputs];
    int state_index = -1;
};

// Runs every check CpuDevice::dispatch performs before touching data
// (device.rs:185-192 and the geometry/kernel checks of run_op), in the same
// order, and fills `plan`. Returns false with `err` set on the first failure.
bool validate_dispatch(const BufferView& buffers, const sl_op& op, const sl_buffer_ref* inputs,
                       const sl_value* input_values, size_t n_inputs, const sl_buffer_ref* outputs,
                       const sl_value* output_values, size_t n_outputs, const uint32_t* scalars,
                       size_t n_scalars, Plan* plan, Error* err);

// Payload storage words of a quantized [n, k] weight.
uint64_t quant_payload_words(uint32_t format, uint64_t n, uint64_t k);

}  // namespace slhip
