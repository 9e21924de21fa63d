// HipDevice: the MI355X implementation of StarLight's sl_device::Device
// contract (ARCH-0007 §3.1), exported through the C ABI in starlight_hip.h.
//
// It plays the role CpuDevice plays for backend-cpu
// (crates/backends/backend-cpu/src/device.rs:31-213):
//  * buffers are device allocations indexed by dense u32 ids, zero-filled at
//    allocation (device.rs:55-83);
//  * dispatch() validates exactly as CpuDevice does (validate.cpp), then
//    enqueues the op's kernels on the device's single stream and returns;
//  * synchronize() waits for the stream (CpuDevice's is a no-op because it is
//    synchronous).
// Ports that share a buffer (the sl-core scratchpad) are plain base + offset
// pointers; CpuDevice's take/restore staging (device.rs:379-706) has no GPU
// counterpart.
//
// U32 buffers are never written by a command (device.rs:311-316), only by
// upload_u32, so the device keeps a host copy of small ones and checks Gather
// ids before launching, like reference/layout.rs:207-213 checks them before
// its first write.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

#include "kernels/kernels.h"
#include "plan.h"
#include "starlight_hip.h"

namespace slhip {
namespace {

constexpr uint64_t kMirrorMaxElements = 1ull << 22;        // host copy of u32 buffers up to 16 MiB
constexpr uint64_t kWorkspaceBytes = 512ull << 20;          // split-K partials, SwiGlu intermediates
constexpr uint64_t kCounterWords = 1ull << 16;              // cross-block completion counters (kept at zero)
constexpr uint64_t kIdScratchElements = 1ull << 20;         // host scratch for unmirrored id checks

struct Buffer {
    sl_buffer_desc desc{};
    void* base = nullptr;  // allocation start
    void* ptr = nullptr;   // aligned data start
    std::vector<uint32_t> mirror;
    bool mirrored = false;
    // group-quantized binding
    uint32_t scales = 0;
    uint8_t* tiles = nullptr;
    QuantLayout layout = QuantLayout::RowMajor;
};

}  // namespace

struct Device : BufferView {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    std::vector<Buffer> buffers;
    float* workspace = nullptr;
    uint64_t workspace_floats = 0;
    uint32_t* counters = nullptr;
    std::vector<uint32_t> id_scratch;
    Error last;

    size_t count() const override { return buffers.size(); }
    const sl_buffer_desc* get(uint32_t id) const override {
        if (id >= buffers.size()) return nullptr;
        return &buffers[id].desc;
    }

    sl_status fail(const Error& e) {
        last = e;
        return e.status;
    }
    sl_status hip_fail(hipError_t e) { return fail(Error::execution(hipGetErrorString(e))); }
};

namespace {

float* fptr(Device* d, const sl_buffer_ref& r) {
    return static_cast<float*>(d->buffers[r.buffer].ptr) + r.offset;
}
const uint32_t* uptr(Device* d, const sl_buffer_ref& r) {
    return static_cast<const uint32_t*>(d->buffers[r.buffer].ptr) + r.offset;
}

// validate_alignment (device.rs:215-222).
bool valid_alignment(size_t align) { return align != 0 && (align & (align - 1)) == 0; }

sl_status allocate(Device* d, size_t elements, size_t align, uint32_t kind, uint32_t* out_id) {
    if (!valid_alignment(align)) return d->fail(Error::execution("alignment must be a nonzero power of two"));
    if (d->buffers.size() >= 0xffffffffull) return d->fail(Error::out_of_memory(d->buffers.size()));
    if (elements > (UINT64_MAX - 4096) / 4) return d->fail(Error::out_of_memory(elements));
    Buffer b;
    b.desc.kind = kind;
    b.desc.elements = elements;
    if (elements != 0) {
        const size_t bytes = elements * 4;
        const size_t extra = align > 256 ? align : 0;  // hipMalloc returns 256-byte aligned memory
        if (hipMalloc(&b.base, bytes + extra) != hipSuccess) {
            (void)hipGetLastError();
            return d->fail(Error::out_of_memory(elements));
        }
        uintptr_t p = reinterpret_cast<uintptr_t>(b.base);
        if (extra) p = (p + align - 1) & ~static_cast<uintptr_t>(align - 1);
        b.ptr = reinterpret_cast<void*>(p);
        hipError_t e = hipMemsetAsync(b.ptr, 0, bytes, d->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
        if (e != hipSuccess) {
            (void)hipFree(b.base);
            return d->hip_fail(e);
        }
    }
    if (kind == SL_BUFFER_U32 && elements <= kMirrorMaxElements) {
        b.mirror.assign(elements, 0u);
        b.mirrored = true;
    }
    *out_id = static_cast<uint32_t>(d->buffers.size());
    d->buffers.push_back(std::move(b));
    return SL_OK;
}

sl_status copy_in(Device* d, uint32_t id, const void* data, size_t len, uint32_t kind) {
    if (id >= d->buffers.size() || d->buffers[id].desc.kind != kind) return d->fail(Error::invalid_buffer(id));
    Buffer& b = d->buffers[id];
    if (b.desc.elements != len) return d->fail(Error::invalid_range(id, 0, len));
    if (len == 0) return SL_OK;
    hipError_t e = hipMemcpyAsync(b.ptr, data, len * 4, hipMemcpyHostToDevice, d->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) return d->hip_fail(e);
    if (b.mirrored) std::memcpy(b.mirror.data(), data, len * 4);
    if (b.tiles) {
        // A re-uploaded quantized payload refreshes the private tile copy.
        e = launch_quant_repack(static_cast<const uint8_t*>(b.ptr), b.tiles, b.desc.qformat, b.desc.qn, b.desc.qk,
                                b.layout, d->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
        if (e != hipSuccess) return d->hip_fail(e);
    }
    return SL_OK;
}

sl_status copy_out(Device* d, uint32_t id, void* out, size_t len, uint32_t kind) {
    if (id >= d->buffers.size() || d->buffers[id].desc.kind != kind) return d->fail(Error::invalid_buffer(id));
    Buffer& b = d->buffers[id];
    if (b.desc.elements != len) return d->fail(Error::invalid_range(id, 0, len));
    if (len == 0) return SL_OK;
    hipError_t e = hipMemcpyAsync(out, b.ptr, len * 4, hipMemcpyDeviceToHost, d->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) return d->hip_fail(e);
    return SL_OK;
}

// Gather ids must all be < vocab before anything is written
// (reference/layout.rs:207-213).
bool gather_ids_in_range(Device* d, const sl_buffer_ref& ids, uint64_t vocab, Error* err) {
    const Buffer& b = d->buffers[ids.buffer];
    const char* why = "id out of range";
    if (b.mirrored) {
        const uint32_t* v = b.mirror.data() + ids.offset;
        for (uint64_t i = 0; i < ids.len; ++i)
            if (v[i] >= vocab) {
                *err = Error::execution(why);
                return false;
            }
        return true;
    }
    for (uint64_t done = 0; done < ids.len; done += kIdScratchElements) {
        const uint64_t n = ids.len - done < kIdScratchElements ? ids.len - done : kIdScratchElements;
        hipError_t e = hipMemcpyAsync(d->id_scratch.data(), static_cast<const uint32_t*>(b.ptr) + ids.offset + done,
                                      n * 4, hipMemcpyDeviceToHost, d->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
        if (e != hipSuccess) {
            *err = Error::execution(hipGetErrorString(e));
            return false;
        }
        for (uint64_t i = 0; i < n; ++i)
            if (d->id_scratch[i] >= vocab) {
                *err = Error::execution(why);
                return false;
            }
    }
    return true;
}

WeightRef weight_ref(Device* d, const sl_buffer_ref& r, const QuantOperand& q) {
    WeightRef w{};
    if (!q.present) {
        w.dense = fptr(d, r);
        return w;
    }
    const Buffer& b = d->buffers[r.buffer];
    w.quant.tiles = b.tiles;
    w.quant.layout = b.layout;
    w.quant.scales = static_cast<const float*>(d->buffers[b.scales].ptr);
    w.quant.format = q.format;
    w.quant.group = q.group;
    w.quant.n = q.n;
    w.quant.k = q.k;
    return w;
}

// Enqueues the kernels of one validated command.
hipError_t launch(Device* d, const Plan& p, const sl_buffer_ref* in, const sl_buffer_ref* out) {
    hipStream_t s = d->stream;
    const Workspace ws{d->workspace, d->workspace_floats, d->counters, kCounterWords};
    switch (p.code) {
        case SL_OP_MATMUL_NT:
        case SL_OP_MATMUL_NN: {
            if (p.batch == 0) return hipSuccess;  // device.rs:1370-1372
            if (p.quant[1].present) {
                // [.., M, K] x quantized [N, K]: the batch folds into rows.
                return launch_qmatmul(fptr(d, in[0]), weight_ref(d, in[1], p.quant[1]).quant, fptr(d, out[0]),
                                      p.batch * p.m, ws, s);
            }
            return launch_matmul(fptr(d, in[0]), fptr(d, in[1]), fptr(d, out[0]), p.batch, p.batch_a, p.batch_b,
                                 p.m, p.k, p.n, p.code == SL_OP_MATMUL_NT, s);
        }
        case SL_OP_SOFTMAX:
            return launch_softmax(fptr(d, in[0]), fptr(d, out[0]), p.rows, p.cols, false, 0, 0, s);
        case SL_OP_SOFTMAX_CAUSAL:
            return launch_softmax(fptr(d, in[0]), fptr(d, out[0]), p.rows, p.cols, true, p.seq, p.past_len, s);
        case SL_OP_RMS_NORM:
            return launch_rms_norm(fptr(d, in[0]), fptr(d, in[1]), fptr(d, out[0]), p.rows, p.hidden, p.eps, s);
        case SL_OP_ROPE:
            return launch_rope(fptr(d, in[0]), uptr(d, in[1]), fptr(d, out[0]), p.batch, p.heads, p.seq, p.head_dim,
                               p.theta, p.rope_variant == SL_ROPE_GPTJ, s);
        case SL_OP_SILU:
            return launch_silu(fptr(d, in[0]), fptr(d, out[0]), p.len, s);
        case SL_OP_SCALE:
            return launch_scale(fptr(d, in[0]), fptr(d, out[0]), p.len, p.factor, s);
        case SL_OP_MUL:
            return launch_mul(fptr(d, in[0]), fptr(d, in[1]), fptr(d, out[0]), p.len, s);
        case SL_OP_ADD:
            return launch_add(fptr(d, in[0]), fptr(d, in[1]), fptr(d, out[0]), p.len, s);
        case SL_OP_GATHER:
            return launch_gather(fptr(d, in[0]), uptr(d, in[1]), fptr(d, out[0]), p.rows, p.hidden, s);
        case SL_OP_LAST_TOKEN:
            return launch_last_token(fptr(d, in[0]), fptr(d, out[0]), p.batch, p.seq, p.hidden, p.seq_len, s);
        case SL_OP_SPLIT_HEADS:
        case SL_OP_MERGE_HEADS:
            return launch_heads_permute(fptr(d, in[0]), fptr(d, out[0]), p.batch, p.seq, p.heads, p.head_dim,
                                        p.code == SL_OP_SPLIT_HEADS, s);
        case SL_OP_KV_APPEND:
            return launch_kv_append(fptr(d, in[0]), fptr(d, in[1]), fptr(d, in[p.state_index]), p.batch, p.layers,
                                    p.layer, p.kv_heads, p.head_dim, p.max_seq, p.past_len, p.seq, s);
        case SL_OP_CAUSAL_ATTENTION: {
            AttentionArgs a{fptr(d, in[0]), fptr(d, in[1]), fptr(d, in[2]), fptr(d, in[p.state_index]),
                            fptr(d, out[0]), p.batch, p.layers, p.layer, p.heads, p.kv_heads, p.seq,
                            p.past_len, p.head_dim, p.max_seq, p.scale};
            return launch_attention(a, ws, s);
        }
        case SL_OP_SWIGLU:
            return launch_swiglu(fptr(d, in[0]), weight_ref(d, in[1], p.quant[1]), weight_ref(d, in[2], p.quant[2]),
                                 weight_ref(d, in[3], p.quant[3]), fptr(d, out[0]), p.rows, p.hidden, p.inter, ws,
                                 s);
        case SL_OP_RMS_NORM_MATMUL:
            return launch_rms_norm_matmul(fptr(d, in[0]), fptr(d, in[1]), weight_ref(d, in[2], p.quant[2]),
                                          fptr(d, out[0]), p.rows, p.hidden, p.out_features, p.eps, ws, s);
        default:
            return hipErrorInvalidValue;
    }
}

// Limits of the launch paths that validation does not know about; checked
// before anything is enqueued so a rejected call still changes nothing.
bool device_limits(Device* d, const Plan& p, Error* err) {
    (void)d;
    if (p.code == SL_OP_CAUSAL_ATTENTION && p.head_dim > 256) {
        *err = Error::unimplemented("head_dim above 256 is not supported by HipDevice");
        return false;
    }
    if (p.code == SL_OP_SWIGLU && 2 * p.inter > d->workspace_floats / 2) {
        *err = Error::unimplemented("swiglu inter size exceeds the device workspace");
        return false;
    }
    if (p.code == SL_OP_RMS_NORM_MATMUL && p.hidden > d->workspace_floats / 2) {
        *err = Error::unimplemented("rms_norm_matmul hidden size exceeds the device workspace");
        return false;
    }
    return true;
}

}  // namespace
}  // namespace slhip

using slhip::Device;
using slhip::Error;

struct sl_hip_device : Device {};

extern "C" {

uint32_t sl_hip_abi_version(void) { return SL_HIP_ABI_VERSION; }

sl_status sl_hip_device_create(int ordinal, sl_hip_device** out) {
    if (out == nullptr) return SL_ERR_EXECUTION;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || ordinal < 0 || ordinal >= count) {
        (void)hipGetLastError();
        return SL_ERR_EXECUTION;
    }
    if (hipSetDevice(ordinal) != hipSuccess) return SL_ERR_EXECUTION;
    sl_hip_device* d = new (std::nothrow) sl_hip_device();
    if (d == nullptr) return SL_ERR_OUT_OF_MEMORY;
    d->ordinal = ordinal;
    if (hipStreamCreate(&d->stream) != hipSuccess) {
        delete d;
        return SL_ERR_EXECUTION;
    }
    if (hipMalloc(reinterpret_cast<void**>(&d->workspace), slhip::kWorkspaceBytes) != hipSuccess) {
        (void)hipStreamDestroy(d->stream);
        delete d;
        return SL_ERR_OUT_OF_MEMORY;
    }
    d->workspace_floats = slhip::kWorkspaceBytes / 4;
    if (hipMalloc(reinterpret_cast<void**>(&d->counters), slhip::kCounterWords * 4) != hipSuccess ||
        hipMemset(d->counters, 0, slhip::kCounterWords * 4) != hipSuccess) {
        (void)hipFree(d->workspace);
        (void)hipStreamDestroy(d->stream);
        delete d;
        return SL_ERR_OUT_OF_MEMORY;
    }
    d->id_scratch.resize(slhip::kIdScratchElements);
    *out = d;
    return SL_OK;
}

void sl_hip_device_destroy(sl_hip_device* d) {
    if (d == nullptr) return;
    (void)hipSetDevice(d->ordinal);
    (void)hipStreamSynchronize(d->stream);
    for (auto& b : d->buffers) {
        if (b.base) (void)hipFree(b.base);
        if (b.tiles) (void)hipFree(b.tiles);
    }
    if (d->workspace) (void)hipFree(d->workspace);
    if (d->counters) (void)hipFree(d->counters);
    (void)hipStreamDestroy(d->stream);
    delete d;
}

sl_status sl_hip_allocate_f32(sl_hip_device* d, size_t elements, size_t align, uint32_t* out_id) {
    return slhip::allocate(d, elements, align, SL_BUFFER_F32, out_id);
}

sl_status sl_hip_allocate_u32(sl_hip_device* d, size_t elements, size_t align, uint32_t* out_id) {
    return slhip::allocate(d, elements, align, SL_BUFFER_U32, out_id);
}

sl_status sl_hip_upload_f32(sl_hip_device* d, uint32_t buffer, const float* data, size_t len) {
    return slhip::copy_in(d, buffer, data, len, SL_BUFFER_F32);
}

sl_status sl_hip_upload_u32(sl_hip_device* d, uint32_t buffer, const uint32_t* data, size_t len) {
    return slhip::copy_in(d, buffer, data, len, SL_BUFFER_U32);
}

sl_status sl_hip_download_f32(sl_hip_device* d, uint32_t buffer, float* out, size_t len) {
    return slhip::copy_out(d, buffer, out, len, SL_BUFFER_F32);
}

sl_status sl_hip_download_u32(sl_hip_device* d, uint32_t buffer, uint32_t* out, size_t len) {
    return slhip::copy_out(d, buffer, out, len, SL_BUFFER_U32);
}

sl_status sl_hip_dispatch(sl_hip_device* d, const sl_op* op, const sl_buffer_ref* inputs,
                          const sl_value* input_values, size_t n_inputs, const sl_buffer_ref* outputs,
                          const sl_value* output_values, size_t n_outputs, const uint32_t* scalars,
                          size_t n_scalars) {
    slhip::Plan plan;
    Error err;
    if (!slhip::validate_dispatch(*d, *op, inputs, input_values, n_inputs, outputs, output_values, n_outputs,
                                  scalars, n_scalars, &plan, &err))
        return d->fail(err);
    if (!slhip::device_limits(d, plan, &err)) return d->fail(err);
    if (plan.code == SL_OP_GATHER && !slhip::gather_ids_in_range(d, inputs[1], plan.vocab, &err))
        return d->fail(err);
    hipError_t e = slhip::launch(d, plan, inputs, outputs);
    if (e != hipSuccess) return d->hip_fail(e);
    return SL_OK;
}

sl_status sl_hip_synchronize(sl_hip_device* d) {
    hipError_t e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) return d->hip_fail(e);
    return SL_OK;
}

void sl_hip_last_error(const sl_hip_device* d, sl_error* out) {
    const Error& e = d->last;
    out->status = e.status;
    out->buffer = e.buffer;
    out->offset = e.offset;
    out->len = e.len;
    out->requested = e.requested;
    out->op = e.op;
    out->reserved = 0;
    out->message = e.message;
}

sl_status sl_hip_bind_quantized(sl_hip_device* d, uint32_t payload, uint32_t scales, uint32_t qformat,
                                uint32_t group_size, uint32_t n, uint32_t k) {
    if (payload >= d->buffers.size() || d->buffers[payload].desc.kind != SL_BUFFER_U32)
        return d->fail(Error::invalid_buffer(payload));
    if (scales >= d->buffers.size() || d->buffers[scales].desc.kind != SL_BUFFER_F32)
        return d->fail(Error::invalid_buffer(scales));
    if (qformat != SL_QFORMAT_INT4 && qformat != SL_QFORMAT_INT8)
        return d->fail(Error::unimplemented("quantization format is not supported by HipDevice"));
    if (group_size == 0 || k % group_size != 0)
        return d->fail(Error::execution("quantized k must be a positive multiple of group_size"));
    slhip::Buffer& pb = d->buffers[payload];
    if (pb.desc.elements != slhip::quant_payload_words(qformat, n, k))
        return d->fail(Error::execution("quantized payload size does not match [n, k]"));
    if (d->buffers[scales].desc.elements != static_cast<uint64_t>(n) * (k / group_size))
        return d->fail(Error::execution("quantized scale count does not match [n, k / group_size]"));
    const slhip::QuantLayout layout = slhip::quant_layout_for(qformat, n, k, group_size);
    const uint64_t bytes = slhip::quant_tile_bytes(qformat, n, k, layout);
    if (pb.tiles) {
        (void)hipStreamSynchronize(d->stream);
        (void)hipFree(pb.tiles);
        pb.tiles = nullptr;
    }
    if (bytes != 0) {
        if (hipMalloc(reinterpret_cast<void**>(&pb.tiles), bytes) != hipSuccess) {
            (void)hipGetLastError();
            pb.tiles = nullptr;
            return d->fail(Error::out_of_memory(bytes / 4));
        }
    }
    pb.desc.quantized = 1;
    pb.desc.qformat = qformat;
    pb.desc.group_size = group_size;
    pb.desc.qn = n;
    pb.desc.qk = k;
    pb.scales = scales;
    pb.layout = layout;
    hipError_t e = slhip::launch_quant_repack(static_cast<const uint8_t*>(pb.ptr), pb.tiles, qformat, n, k, layout,
                                              d->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) return d->hip_fail(e);
    return SL_OK;
}

void* sl_hip_stream(const sl_hip_device* d) { return d->stream; }

void sl_hip_capabilities(sl_capabilities* out) {
    out->backend = "hip-gfx950";
    out->ir_version = SL_IR_VERSION;
    out->core_ops = (1u << slhip::kOpCount) - 1u;
    out->composite_ops =
        (1u << SL_OP_CAUSAL_ATTENTION) | (1u << SL_OP_SWIGLU) | (1u << SL_OP_RMS_NORM_MATMUL);
    out->dtypes = (1u << SL_DTYPE_F32) | (1u << SL_DTYPE_U32);
    out->min_buffer_align = 256;
    out->max_scratchpad_bytes = 64ull << 30;
    out->max_value_bytes = 64ull << 30;
    out->head_dim_multiple_of = 2;
    out->matmul_k_multiple_of = 1;
    out->max_heads = 1024;
}

}  // extern "C"
